"""ctypes side of tests/cpmath/planner_harness.cc: one call of the reference's
plan_end_to_end over the engine's CP-Math candidates, with an optional Python measurement
hook. Built by `make -C oracle ref` (__graft_entry__.build()) into oracle/_ref/."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[2]
HARNESS = ROOT / "oracle" / "_ref" / "libplanner_harness.so"

QCSR, BELL, CPBP, QCSR_EXEC = 1, 2, 4, 8  # candidate_mask bits
QCSR_ID = (0x4358414D44514353, 1)
QCSR_EXEC_ID = (0x4358414D44514353, 2)
BELL_ID = (0x4358414D4442454C, 1)
CPBP_ID = (0x4358414D44435042, 1)
# candidate_rejection / selection_source / cache_state / planner_status_code
# (include/Cellerator/planner/end_to_end_planner.hh:182-223)
NONE, MALFORMED, INCORRECT, NONDETERMINISTIC, GRAPH, PERSISTENT, TRANSIENT, MEASUREMENT_FAILED, CONTAMINATED = range(9)
ANALYTICAL, EMPIRICAL, CACHE = 1, 2, 3
NOT_CONFIGURED, MISS, HIT, STALE, WINNER_UNAVAILABLE = range(5)
OK, INVALID_ARGUMENT, INVALID_COST, NO_LEGAL, NO_CORRECT_MEASUREMENT = range(5)


class PhMeasurement(C.Structure):
    _fields_ = [("ok", C.c_int32), ("correct", C.c_int32), ("contaminated", C.c_int32), ("samples", C.c_uint32),
                ("kernel_ns", C.c_double), ("spread_percent", C.c_double)]


MEASURE_FN = C.CFUNCTYPE(C.c_int, C.c_uint64, C.c_uint64, C.POINTER(PhMeasurement))


class PhCase(C.Structure):
    _fields_ = [("rows", C.c_uint64), ("cols", C.c_uint64), ("nnz", C.c_uint64), ("out_cols", C.c_uint32),
                ("bits", C.c_uint32), ("value_bytes", C.c_uint32), ("block_size", C.c_uint32),
                ("ell_columns", C.c_uint64), ("tile_blocks", C.c_uint64), ("problem_kind", C.c_uint32),
                ("candidate_mask", C.c_uint32), ("deterministic", C.c_uint32),
                ("graph_capture_required", C.c_uint32), ("max_persistent", C.c_uint64),
                ("max_transient", C.c_uint64), ("shortlist", C.c_uint32), ("max_measurements", C.c_uint32),
                ("min_tuning_work_items", C.c_uint64), ("logical_work_items", C.c_uint64),
                ("structure_reuse", C.c_uint64), ("projection_reuse", C.c_uint64),
                ("practical_tolerance", C.c_double), ("max_spread", C.c_double),
                ("min_cache_confidence", C.c_double), ("allow_fallback", C.c_uint32), ("tune_one_shot", C.c_uint32),
                ("nondeterministic_mask", C.c_uint32), ("use_cache", C.c_uint32), ("measure", MEASURE_FN),
                ("evidence_revision", C.c_uint64)]


class PhDiag(C.Structure):
    _fields_ = [("id_low", C.c_uint64), ("id_high", C.c_uint64), ("rejection", C.c_uint32),
                ("shortlisted", C.c_uint32), ("measured", C.c_uint32), ("conventional", C.c_uint32),
                ("analytical_ns", C.c_double), ("empirical_ns", C.c_double)]


class PhResult(C.Structure):
    _fields_ = [("status", C.c_int32), ("source", C.c_uint32), ("cache", C.c_uint32),
                ("tuning_skipped", C.c_uint32), ("conventional_winner", C.c_uint32), ("legal", C.c_uint32),
                ("shortlist", C.c_uint32), ("measured", C.c_uint32), ("winner_low", C.c_uint64),
                ("winner_high", C.c_uint64), ("confidence", C.c_double), ("count", C.c_uint32),
                ("stored", C.c_uint32), ("diags", PhDiag * 4), ("reason", C.c_char * 160),
                ("message", C.c_char * 160)]

    @property
    def winner(self):
        return (self.winner_low, self.winner_high)

    def diag(self, identity) -> PhDiag:
        for k in range(self.count):
            if (self.diags[k].id_low, self.diags[k].id_high) == identity:
                return self.diags[k]
        raise KeyError(identity)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not HARNESS.exists():
            pytest.skip("planner harness not built (needs the Cellerator sources at build time)")
        _lib = C.CDLL(str(HARNESS))
        _lib.ph_plan.argtypes = [C.POINTER(PhCase), C.POINTER(PhResult)]
        _lib.ph_plan.restype = C.c_int
        assert _lib.ph_case_size() == C.sizeof(PhCase)
        assert _lib.ph_result_size() == C.sizeof(PhResult)
    return _lib


def spmm_case(rows, cols, nnz, n, *, bits=4, block_size=32, ell_columns=0, value_bytes=2, mask=QCSR | BELL,
              **policy) -> PhCase:
    c = PhCase()
    c.rows, c.cols, c.nnz, c.out_cols, c.bits = rows, cols, nnz, n, bits
    c.value_bytes, c.block_size, c.ell_columns = value_bytes, block_size, ell_columns
    c.problem_kind, c.candidate_mask = 1, mask
    c.deterministic = c.graph_capture_required = 1
    c.shortlist, c.max_measurements = 3, 3
    c.min_tuning_work_items, c.logical_work_items = 4096, rows
    c.structure_reuse = c.projection_reuse = 8
    c.practical_tolerance, c.max_spread, c.min_cache_confidence = 2.0, 10.0, 0.8
    c.allow_fallback, c.evidence_revision = 1, 44
    for k, v in policy.items():
        setattr(c, k, v)
    return c


def plan(case: PhCase, measure=None) -> PhResult:
    """measure(identity) -> None (failed) or dict(kernel_ns, samples, spread_percent,
    correct=True, contaminated=False)."""
    keep = None
    if measure is not None:
        def trampoline(low, high, out):
            m = measure((low, high))
            if m is None:
                return 1
            out.contents.ok = 1
            out.contents.correct = int(m.get("correct", True))
            out.contents.contaminated = int(m.get("contaminated", False))
            out.contents.samples = m["samples"]
            out.contents.kernel_ns = m["kernel_ns"]
            out.contents.spread_percent = m["spread_percent"]
            return 0
        keep = MEASURE_FN(trampoline)
        case.measure = keep
    res = PhResult()
    assert lib().ph_plan(C.byref(case), C.byref(res)) == 0
    case.measure = MEASURE_FN()
    del keep
    return res
