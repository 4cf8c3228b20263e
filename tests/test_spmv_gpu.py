"""GPU parity of the N = 1 CSR comparator cx_csr_spmv_fwd (csr_spmv_fwd_f16_f32,
src/compute/sparse/ops/ops.hh:83-90): the reference's known answer
(tests/sparse_ops_runtime_test.cu:225-245: 3x3 CSR x {1, 10, 100} -> {201, 430, 5}),
f16 and f32 values against the oracle's float64 referee with N = 1, empty rows, a long
row, and agreement with the CP-BP reduction of the same matrix."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import random_csr

pytestmark = pytest.mark.gpu


def test_reference_spmv_kat():
    import torch

    from cellerator_amd import csr_spmv
    row_ptr = torch.tensor([0, 2, 4, 5], dtype=torch.int32).cuda()
    col_idx = torch.tensor([0, 2, 1, 2, 0], dtype=torch.int32).cuda()
    values = torch.tensor([1, 2, 3, 4, 5], dtype=torch.float16).cuda()
    x = torch.tensor([1, 10, 100], dtype=torch.float32).cuda()
    y = csr_spmv(row_ptr, col_idx, values, x)
    torch.cuda.synchronize()
    assert y.cpu().tolist() == [201.0, 430.0, 5.0]


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_spmv_matches_referee(oracle, dtype):
    import torch

    from cellerator_amd import csr_spmv
    rng = np.random.default_rng(5 if dtype == np.float16 else 6)
    rows, cols = 5000, 3000
    row_ptr, col_idx = random_csr(rng, rows, cols, 60.0, empty_every=17)
    # one long row spanning many wave strides
    vals = rng.standard_normal(len(col_idx)).astype(dtype)
    x = rng.standard_normal(cols).astype(np.float32)
    y = csr_spmv(torch.from_numpy(row_ptr).cuda(), torch.from_numpy(col_idx).cuda(),
                 torch.from_numpy(vals).cuda(), torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    ref = oracle.spmm_referee(rows, cols, 1, row_ptr, col_idx, vals, x.reshape(cols, 1))[:, 0]
    mag = oracle.spmm_referee(rows, cols, 1, row_ptr, col_idx,
                              np.abs(vals.astype(np.float64)), np.abs(x.astype(np.float64)).reshape(cols, 1))[:, 0]
    got = y.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - ref) <= 1e-6 + 2.0 ** -22 * mag)
    assert np.all(got[::17] == 0.0)


def test_spmv_long_rows_and_many_rows(oracle):
    """A row of every column, and more rows than one grid pass covers (the kernel strides)."""
    import torch

    from cellerator_amd import csr_spmv
    rng = np.random.default_rng(8)
    rows, cols = 4_500_000, 700
    counts = np.zeros(rows, np.int64)
    counts[::997] = 3
    counts[7] = cols
    row_ptr = np.zeros(rows + 1, np.int64)
    row_ptr[1:] = np.cumsum(counts)
    col_idx = np.concatenate([np.arange(cols) if c == cols else np.sort(rng.choice(cols, c, replace=False))
                              for c in counts[counts > 0]]).astype(np.int32)
    vals = rng.standard_normal(len(col_idx)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    y = csr_spmv(torch.from_numpy(row_ptr.astype(np.int32)).cuda(), torch.from_numpy(col_idx).cuda(),
                 torch.from_numpy(vals).cuda(), torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    got = y.cpu().numpy().astype(np.float64)
    nz = np.nonzero(counts)[0]
    for r in nz[:2000]:
        a, b = row_ptr[r], row_ptr[r + 1]
        want = float(np.dot(vals[a:b].astype(np.float64), x[col_idx[a:b]].astype(np.float64)))
        mag = float(np.dot(np.abs(vals[a:b]).astype(np.float64), np.abs(x[col_idx[a:b]]).astype(np.float64)))
        assert abs(got[r] - want) <= 1e-6 + 2.0 ** -22 * mag, r
    assert np.all(got[counts == 0] == 0.0)


def test_spmv_agrees_with_cpbp_reduction(oracle):
    """The comparator and the CP-BP reduction compute the same per-cell weighted sum."""
    import torch

    from cellerator_amd import cpbp, cpbp_reduce, csr_spmv
    from tests.test_cpbp_build import random_csr as cpbp_csr, random_plan
    rng = np.random.default_rng(12)
    plan = random_plan(rng, 800)
    offs, feats, vals = cpbp_csr(rng, 3000, 800, 40.0, np.float32)
    w = rng.standard_normal(800).astype(np.float32)
    t = cpbp.to_device(plan, cpbp.build_tiles(plan, offs, feats, vals, group_width=64, window_size=256))
    wd = torch.from_numpy(w).cuda()
    a = cpbp_reduce(t, wd)
    b = csr_spmv(torch.from_numpy(offs.view(np.int32)).cuda(), torch.from_numpy(feats.view(np.int32)).cuda(),
                 torch.from_numpy(vals).cuda(), wd)
    torch.cuda.synchronize()
    ref, mag = oracle.cpbp_canonical_f64(offs, feats, vals, w)
    for got in (a, b):
        assert np.all(np.abs(got.cpu().numpy() - ref) <= 1e-5 + 1e-5 * np.abs(ref) + 2.0 ** -22 * mag)
