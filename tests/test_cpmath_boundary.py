"""The engine's CP-Math candidates under the reference's own operation core, on the CPU:
registration, capability query, prepare, and every rejection the core or the backend
reports before a kernel would launch. Device pointers are stand-in addresses that are
never dereferenced (each case is rejected before the engine's C-ABI is called).

Restates the boundary cases of tests/math_core/operation_core_test.cc:120-270 (stale
epoch, structure-count mismatch, insufficient workspace, numeric and projection
rejection) with real candidates, plus the backend's own launch checks."""
from __future__ import annotations

import ctypes as C

import pytest

from cellerator_amd import _native as N
from tests.cpmath import harness as H

FAKE = 0x7F0000100000  # stand-in device address, never dereferenced


def qcsr_case(bits=4, rows=1000, cols=3000, n=64, nnz=50_000, dense=H.NT_F16):
    view = N.CxQcsrMatrix(rows, cols, nnz, bits, 0, FAKE, FAKE + 0x1000, FAKE + 0x2000,
                          None, None, None, None, None, 0, 0)
    c = H.HCase(kind=H.KIND_QCSR, view=C.addressof(view), view_bytes=C.sizeof(view),
                variant=bits, rows=rows, cols=cols, out_cols=n, block_size=0,
                sparse_type=H.NT_U8 if bits else H.NT_F32, dense_type=dense, nnz=nnz,
                values=FAKE + 0x3000, value_count=nnz, value_bytes=(nnz * max(bits, 8) + 7) // 8,
                scales=FAKE + 0x4000 if bits else None, offsets=FAKE + 0x5000 if bits else None,
                w=FAKE + 0x6000, w_ld=n, y=FAKE + 0x7000, y_ld=n, stream=None, device=0)
    c._keep = view
    return c


def bell_case(n=64, dense=H.NT_BF16, rows=640, cols=2000, ell_cols=256):
    view = N.CxBellMatrix(rows, cols, 32, ell_cols, FAKE, None, 0, 0, 0, 0, None, None, None,
                          None)
    ws = ((cols + 31) // 32) * 32 * n * 2
    c = H.HCase(kind=H.KIND_BELL, view=C.addressof(view), view_bytes=C.sizeof(view), variant=0,
                rows=rows, cols=cols, out_cols=n, block_size=32, sparse_type=H.NT_BF16,
                dense_type=dense, nnz=rows * ell_cols, values=FAKE + 0x3000,
                value_count=rows * ell_cols, value_bytes=rows * ell_cols * 2, w=FAKE + 0x6000,
                w_ld=n, y=FAKE + 0x7000, y_ld=n, workspace=FAKE + 0x100000, workspace_bytes=ws,
                stream=None, device=0)
    c._keep = view
    return c


def cpbp_case(rows=640, cols=700, nnz=20_000):
    view = N.CxCpbpTiles(rows, cols, 28, 64, 10, 100, 1000, nnz, 0, 0, *([FAKE] * 8), None, FAKE)
    c = H.HCase(kind=H.KIND_CPBP, view=C.addressof(view), view_bytes=C.sizeof(view), variant=0,
                rows=rows, cols=cols, out_cols=0, block_size=0, sparse_type=H.NT_F32,
                dense_type=H.NT_F32, nnz=nnz, values=FAKE + 0x3000, value_count=nnz,
                value_bytes=nnz * 4, w=FAKE + 0x6000, w_ld=1, y=FAKE + 0x7000, y_ld=1,
                stream=None, device=0)
    c._keep = view
    return c


CASES = {"qcsr": qcsr_case, "bell": bell_case, "cpbp": cpbp_case}


@pytest.mark.parametrize("kind", CASES)
def test_registration_and_prepare(kind):
    r = H.run(CASES[kind](), "retired_projection")
    assert r.registered == 4
    assert r.capability_flags == H.DETERMINISTIC | H.GRAPH_CAPTURE
    assert r.prepare_status == H.OK, r.message
    # the projection was retired after prepare: the borrowed state is gone, run refuses
    assert r.status == H.EXECUTION_FAILED


def test_blocked_ell_kernel_selection_and_workspace():
    mfma = H.run(bell_case(n=128), "retired_projection")
    assert (mfma.kernel_low, mfma.kernel_high) == (0x4358414D4442454C, 2)
    assert mfma.workspace_bytes == ((2000 + 31) // 32) * 32 * 128 * 2
    generic = H.run(bell_case(n=96, dense=H.NT_F32), "retired_projection")
    assert (generic.kernel_low, generic.kernel_high) == (0x4358414D4442454C, 3)
    assert generic.workspace_bytes == 0


@pytest.mark.parametrize("kind", CASES)
@pytest.mark.parametrize("mutation,status,binding", [
    ("stale_epoch", H.STALE_STRUCTURE, H.B_STALE_STRUCTURE),
    ("structure_count", H.INVALID_LAUNCH, H.B_STRUCTURE_COUNT),
    ("stale_generation", H.INVALID_LAUNCH, H.B_STALE_VALUE),
    ("swapped_axes", H.INVALID_LAUNCH, H.B_AXIS_MISMATCH),
    ("output_aliases_input", H.INVALID_LAUNCH, H.B_ALIAS),
    ("wrong_device", H.INVALID_LAUNCH, H.B_INVALID_STREAM),
    ("wrong_view_bytes", H.INVALID_LAUNCH, H.B_INVALID_OPERAND),
    ("values_in_view", H.INVALID_LAUNCH, H.B_INVALID_OPERAND),
    ("wrong_dense_type", H.INVALID_LAUNCH, H.B_INVALID_OPERAND),
    ("wrong_output_shape", H.INVALID_LAUNCH, H.B_INVALID_OPERAND),
])
def test_launch_rejections(kind, mutation, status, binding):
    r = H.run(CASES[kind](), mutation)
    assert r.prepare_status == H.OK, r.message
    assert (r.status, r.binding) == (status, binding), r.message.decode()


def test_short_workspace_is_rejected():
    r = H.run(bell_case(n=64), "short_workspace")
    assert (r.status, r.binding) == (H.INVALID_LAUNCH, H.B_WORKSPACE)


@pytest.mark.parametrize("kind", CASES)
@pytest.mark.parametrize("mutation,status", [
    ("bad_numeric", H.UNSUPPORTED_NUMERIC),
    ("wrong_projection_kind", H.UNSUPPORTED_PROJECTION),
    ("undeclared_projection", H.UNSUPPORTED_PROJECTION),
])
def test_prepare_rejections(kind, mutation, status):
    r = H.run(CASES[kind](), mutation)
    assert r.prepare_status == status, r.message.decode()
    assert r.status == -1  # never ran


def test_memory_policy():
    assert H.run(bell_case(), "tight_memory_policy").prepare_status == H.CAPABILITY_REJECTED
    assert H.run(qcsr_case(), "tight_memory_policy").prepare_status == H.OK


def test_quantized_width_must_match_storage():
    c = qcsr_case(bits=4)
    c.sparse_type = H.NT_F32  # plain values with a 4-bit projection variant
    r = H.run(c, "none")
    assert r.prepare_status == H.UNSUPPORTED_NUMERIC


def test_bad_code_width_is_not_declared():
    c = qcsr_case(bits=3)
    res = H.HResult()
    c.mutation = 0
    assert H.lib().h_run(C.byref(c), C.byref(res)) == 1
    assert res.prepare_status == H.UNSUPPORTED_PROJECTION


# ---------------------------------------------------------------- fused epilogues

def _fused(case, kind, affine=False, bias=True):
    case.fused, case.epilogue_kind, case.affine = 1, kind, int(affine)
    case.alpha, case.beta = 0.5, 2.0
    if kind in (1, 5, 6, 7) and bias:
        case.bias = FAKE + 0x8000
    return case


@pytest.mark.parametrize("kind", ["qcsr", "bell"])
@pytest.mark.parametrize("epilogue", range(8))
@pytest.mark.parametrize("affine", [False, True])
def test_epilogue_prepares_on_multiplies(kind, epilogue, affine):
    r = H.run(_fused(CASES[kind](), epilogue, affine), "retired_projection")
    assert r.prepare_status == H.OK, r.message


def test_epilogue_on_the_reduction_is_unsupported():
    r = H.run(_fused(cpbp_case(), 2))
    assert r.prepare_status == H.UNSUPPORTED_PROBLEM


def test_unknown_epilogue_kind_is_unsupported():
    r = H.run(_fused(qcsr_case(), 9))
    assert r.prepare_status == H.UNSUPPORTED_PROBLEM


@pytest.mark.parametrize("kind", [1, 2])
def test_bias_numeric_must_match_the_epilogue(kind):
    """numeric_policy.bias = f32 exactly when the epilogue adds a bias."""
    r = H.run(_fused(qcsr_case(), kind), "bias_numeric_mismatch")
    assert r.prepare_status == H.UNSUPPORTED_NUMERIC


def test_bias_kind_without_a_bias_operand_is_unsupported():
    # input_count 2 with a bias epilogue (numeric bias left invalid as well)
    r = H.run(_fused(qcsr_case(), 5, bias=False))
    assert r.prepare_status == H.UNSUPPORTED_NUMERIC


def test_affine_effect_needs_both_scalars():
    """The core itself rejects an affine_accumulate launch without alpha / beta bindings."""
    r = H.run(_fused(bell_case(), 0, affine=True), "missing_scalars")
    assert r.prepare_status == H.OK
    assert (r.status, r.binding) == (H.INVALID_LAUNCH, H.B_MISSING_SCALAR)


def test_execution_order_candidate_prepare():
    """The execution-order quantized CSR candidate: registered beside the others with the
    persistent-preprocessing capability, prepared with the engine's kernel identity and the
    workspace its launch needs (W in execution order, the head's partial sums and panel,
    cx_qcsr_exec_workspace_for); f32 W, plain values and widths other than 64..256 by 64
    are numeric or shape rejections at prepare."""
    want = C.c_uint64()
    assert N.engine().cx_qcsr_exec_workspace_for(1000, 3000, 1024, 128, C.byref(want)) == 0
    c = qcsr_case(rows=1000, cols=3000, n=128)
    c.exec_order, c.head_genes = 2, 1024
    c.workspace, c.workspace_bytes = FAKE + 0x100000, want.value
    r = H.run(c, "retired_projection")
    assert r.registered == 4
    assert r.capability_flags == H.DETERMINISTIC | H.GRAPH_CAPTURE | H.PERSISTENT_PREPROCESSING
    assert r.prepare_status == H.OK, r.message
    assert (r.kernel_low, r.kernel_high) == (0x4358414D44514353, 2)
    assert r.workspace_bytes == want.value
    assert want.value >= 3000 * 128 * 2 + 1000 * 256 + 1024 * 128 * 2
    assert r.status == H.EXECUTION_FAILED  # retired after prepare: run refuses before any launch
    # the default head width is 2,048 genes (capped at the genes rounded down to 1,024)
    c = qcsr_case(rows=1000, cols=3000, n=64)
    c.exec_order = 2
    r = H.run(c, "retired_projection")
    assert N.engine().cx_qcsr_exec_workspace_for(1000, 3000, 2048, 64, C.byref(want)) == 0
    assert r.workspace_bytes == want.value
    for case in (qcsr_case(dense=H.NT_F32), qcsr_case(bits=0), qcsr_case(n=96)):
        case.exec_order = 2
        r = H.run(case)
        assert r.prepare_status == H.UNSUPPORTED_NUMERIC, r.message
