"""The reference's planner choosing between the engine's two SpMM layouts with a
measurement hook that runs the real kernels: one block-structured matrix held as a plain
quantized-CSR projection (f16 values, row-group kernel) and as its Blocked-ELL lowering
(bf16, 32 x 32 blocks, the packed-panel matrix-core kernel). Each candidate's timed output
is checked against the float64 referee before its time counts; the planner's empirical
winner is the measured-faster layout (within its practical tolerance)."""
from __future__ import annotations

import statistics

import numpy as np
import pytest

from tests.cpmath import planner as P
from tests.helpers import check_against_referee

pytestmark = pytest.mark.gpu


def _block_matrix(rng, rows, cols, active, density):
    """Rows in 32-row blocks, each block using `active` random 32-column blocks."""
    offsets, ids = [0], []
    for rb in range(rows // 32):
        blocks = np.sort(rng.choice(cols // 32, active, replace=False))
        for _ in range(32):
            mask = rng.random((active, 32)) < density
            cols_r = (blocks[:, None] * 32 + np.arange(32)[None, :])[mask]
            ids.extend(cols_r.tolist())
            offsets.append(len(ids))
    # values exact in both f16 and bf16: k / 8 with |k| < 64
    values = (rng.integers(-63, 64, len(ids)) / 8.0).astype(np.float32)
    return np.asarray(offsets, np.int32), np.asarray(ids, np.int32), values


def _time(fn, reps=9):
    import torch
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    ms = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        ms.append(a.elapsed_time(b))
    ms.sort()
    med = statistics.median(ms)
    return med * 1e6, (ms[6] - ms[2]) / med * 100.0


def test_planner_measures_the_engine_kernels(oracle):
    import torch

    from cellerator_amd import BellMatrix, QcsrMatrix, bell_pack_rhs, bell_spmm_packed, qcsr_spmm
    from cellerator_amd.bell_lowering import VALUES_ROW_MAJOR, Lowering
    rng = np.random.default_rng(21)
    rows, cols, n = 8192, 4096, 64
    ro, ids, vals = _block_matrix(rng, rows, cols, 24, 0.5)
    w = (rng.integers(-127, 128, (cols, n)) / 64.0).astype(np.float32)
    ref = oracle.spmm_referee(rows, cols, n, ro, ids, vals, w)
    mag = oracle.spmm_referee(rows, cols, n, ro, ids, np.abs(vals.astype(np.float64)), np.abs(w.astype(np.float64)))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731

    # projection 1: plain quantized-CSR (f16 values)
    m = QcsrMatrix(rows, cols, 0, dev(ro), dev(ids), values=dev(vals.astype(np.float16)))
    w16 = dev(w.astype(np.float16))
    y_csr = torch.empty((rows, n), device="cuda")
    # projection 2: its Blocked-ELL lowering (identity plan and order, 32-wide feature blocks)
    bits = (vals.view(np.uint32) >> 16).astype(np.uint16)  # exact bf16
    L = Lowering(ro, ids, bits, cols, list(range(0, cols + 1, 32)), np.arange(cols), np.arange(rows))
    policy = Lowering.policy(1e6, 1e6)
    cand = L.query(policy)[2]
    view, _, bcols, bvals = L.materialize(cand, policy, VALUES_ROW_MAJOR)
    bm = BellMatrix(view.padded_row_count, view.padded_feature_count, 32, view.ell_columns,
                    dev(bcols.reshape(view.padded_row_count // 32, -1)),
                    values=dev(bvals.view(np.int16).reshape(view.padded_row_count, -1)).view(torch.bfloat16))
    panel = bell_pack_rhs(dev(w).to(torch.bfloat16))
    y_bell = torch.empty((view.padded_row_count, n), device="cuda")

    runs = {P.QCSR_ID: (lambda: qcsr_spmm(m, w16, out=y_csr), y_csr),
            P.BELL_ID: (lambda: bell_spmm_packed(bm, panel, n, out=y_bell), y_bell)}
    measured = {}

    def measure(identity):
        fn, y = runs[identity]
        ns, spread = _time(fn)
        torch.cuda.synchronize()
        try:
            check_against_referee(oracle, ref, mag, y[:rows].cpu().numpy())
            correct = True
        except AssertionError:
            correct = False
        measured[identity] = ns
        return dict(kernel_ns=ns, samples=9, spread_percent=spread, correct=correct)

    case = P.spmm_case(rows, cols, len(ids), n, bits=0, value_bytes=2, ell_columns=view.ell_columns,
                       use_cache=2, max_spread=25.0)
    r = P.plan(case, measure)
    print(f"measured ns: qcsr {measured.get(P.QCSR_ID):.0f}, bell {measured.get(P.BELL_ID):.0f}; "
          f"winner {'qcsr' if r.winner == P.QCSR_ID else 'bell'}", flush=True)
    assert r.status == P.OK, r.message
    assert r.source == P.EMPIRICAL and r.measured == 2
    assert r.diag(P.QCSR_ID).rejection == P.NONE and r.diag(P.BELL_ID).rejection == P.NONE
    loser = P.BELL_ID if r.winner == P.QCSR_ID else P.QCSR_ID
    assert measured[r.winner] <= measured[loser] * 1.02
    assert r.stored
