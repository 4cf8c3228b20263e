"""ctypes side of tests/cpmath/harness.cc: runs one request through the reference's
operation core (register -> find -> prepare -> run) against the engine's CP-Math
candidates and reports the statuses. The harness library is built by `make -C oracle ref`
(__graft_entry__.build()) into oracle/_ref/."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[2]
HARNESS = ROOT / "oracle" / "_ref" / "libcpmath_harness.so"

# operation_status_code (include/Cellerator/compute/math/operation_core/operation_core.hh:133-146)
OK, INVALID_ARGUMENT, UNSUPPORTED_PROBLEM, UNSUPPORTED_NUMERIC, UNSUPPORTED_PROJECTION = 0, 1, 2, 3, 4
CAPABILITY_REJECTED, REGISTRY_FULL, DUPLICATE, STALE_STRUCTURE, INVALID_LAUNCH = 5, 6, 7, 8, 9
PREPARATION_FAILED, EXECUTION_FAILED = 10, 11
# binding_validation_code (include/Cellerator/execution/launch_bindings.hh:99-117)
B_OK, B_STALE_STRUCTURE, B_INVALID_OPERAND, B_AXIS_MISMATCH, B_STALE_VALUE = 0, 2, 3, 5, 6
B_INVALID_STREAM, B_WORKSPACE, B_STRUCTURE_COUNT, B_ALIAS = 7, 8, 11, 16
# numeric_type (include/Cellerator/execution/operands.hh:9-20)
NT_U8, NT_F16, NT_BF16, NT_F32 = 2, 6, 7, 8
# candidate_capability_flag
DETERMINISTIC, GRAPH_CAPTURE, PERSISTENT_PREPROCESSING = 1, 2, 4

KIND_QCSR, KIND_BELL, KIND_CPBP = 1, 2, 3
MUTATIONS = dict(none=0, stale_epoch=1, structure_count=2, short_workspace=4,
                 stale_generation=5, bad_numeric=6, wrong_projection_kind=7,
                 undeclared_projection=8, swapped_axes=9, output_aliases_input=10,
                 wrong_view_bytes=11, values_in_view=12, wrong_device=15,
                 wrong_dense_type=16, wrong_output_shape=17, tight_memory_policy=18,
                 retired_projection=19, missing_scalars=20, bias_numeric_mismatch=21,
                 f64_scalars=22)
B_MISSING_SCALAR = 15

p = C.c_void_p


class HCase(C.Structure):
    _fields_ = [("kind", C.c_int32), ("mutation", C.c_int32), ("view", p),
                ("view_bytes", C.c_uint64), ("variant", C.c_uint32), ("rows", C.c_uint32),
                ("cols", C.c_uint32), ("out_cols", C.c_uint32), ("block_size", C.c_uint32),
                ("sparse_type", C.c_uint32), ("dense_type", C.c_uint32),
                ("reserved", C.c_uint32), ("nnz", C.c_uint64), ("values", p),
                ("value_count", C.c_uint64), ("value_bytes", C.c_uint64), ("scales", p),
                ("offsets", p), ("w", p), ("w_ld", C.c_int64), ("y", p), ("y_ld", C.c_int64),
                ("w2", p), ("y2", p), ("workspace", p), ("workspace_bytes", C.c_uint64),
                ("stream", p), ("device", C.c_int32), ("reserved2", C.c_int32),
                ("fused", C.c_uint32), ("epilogue_kind", C.c_uint32), ("affine", C.c_uint32),
                ("reserved3", C.c_uint32), ("bias", p), ("alpha", C.c_float),
                ("beta", C.c_float), ("pairs", p), ("check_columns", C.c_uint32),
                ("repeats", C.c_uint32), ("panel", p), ("groups", p), ("exec_order", C.c_uint32),
                ("head_genes", C.c_uint32), ("reduction_view", p), ("entry_rows", p),
                ("entry_rows_capacity", C.c_uint64)]


class HResult(C.Structure):
    _fields_ = [("prepare_status", C.c_int32), ("status", C.c_int32), ("binding", C.c_int32),
                ("second_status", C.c_int32), ("kernel_low", C.c_uint64),
                ("kernel_high", C.c_uint64), ("workspace_bytes", C.c_uint64),
                ("capability_flags", C.c_uint32), ("registered", C.c_uint32),
                ("state_status", C.c_int32), ("reserved", C.c_int32),
                ("message", C.c_char * 160), ("engine", C.c_char * 256),
                ("dispatch", C.c_char * 64), ("persistent_bytes", C.c_uint64), ("launch_ms", C.c_double)]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not HARNESS.exists():
            pytest.skip("CP-Math harness not built (needs the Cellerator headers at build time)")
        _lib = C.CDLL(str(HARNESS))
        _lib.h_run.argtypes = [C.POINTER(HCase), C.POINTER(HResult)]
        _lib.h_run.restype = C.c_int
        assert _lib.h_case_size() == C.sizeof(HCase)
        assert _lib.h_result_size() == C.sizeof(HResult)
    return _lib


def run(case: HCase, mutation: str = "none") -> HResult:
    case.mutation = MUTATIONS[mutation]
    res = HResult()
    rc = lib().h_run(C.byref(case), C.byref(res))
    assert rc == 0, f"harness setup failed ({rc}): {res.message.decode()}"
    return res
