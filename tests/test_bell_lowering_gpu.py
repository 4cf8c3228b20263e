"""The lowering feeds the engine: a canonical CSR lowered on the host
(cx_bell_materialize_candidate_host, engine row-major value layout) runs through the
engine's Blocked-ELL SpMM -- the generic kernel for block sizes 8 and 16 (fp32 values),
the packed-panel matrix-core kernel for block size 32 (bf16 values) -- against weights laid
out in physical feature order by cx_bell_physical_feature_map, and every logical row of the
product (execution row order) matches the float64 referee of the canonical CSR product."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import check_against_referee
from tests.test_bell_lowering import random_case

pytestmark = pytest.mark.gpu


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    b = x.astype(np.float32).view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)  # round to nearest even


def _bf16_float(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("size,bf16", [(8, False), (16, False), (32, True)])
def test_lowered_candidate_runs_on_the_engine(oracle, size, bf16):
    import torch

    from cellerator_amd import BellMatrix, bell_pack_rhs, bell_spmm, bell_spmm_packed
    from cellerator_amd.bell_lowering import VALUES_ROW_MAJOR, Lowering
    rng = np.random.default_rng(50 + size)
    offsets, ids, values, nf, blocks, fperm, rperm = random_case(rng, 301, 517, 7, 0.06)
    if bf16:
        values = _bf16_bits(values)
    L = Lowering(offsets, ids, values, nf, blocks, fperm, rperm)
    policy = Lowering.policy(1e6, 1e6)
    cand = L.query(policy)[[8, 16, 32].index(size)]
    view, _, cols, vals = L.materialize(cand, policy, VALUES_ROW_MAJOR)
    rows_p, ell = view.padded_row_count, view.ell_columns
    dev_vals = torch.from_numpy(vals.view(np.int16 if bf16 else np.float32).reshape(rows_p, ell).copy()).cuda()
    if bf16:
        dev_vals = dev_vals.view(torch.bfloat16)
    m = BellMatrix(rows_p, view.padded_feature_count, size, ell,
                   torch.from_numpy(cols.reshape(rows_p // size, ell // size).copy()).cuda(), values=dev_vals)
    n = 64
    w = (rng.standard_normal((nf, n)) * 0.1).astype(np.float32)
    if bf16:
        w = _bf16_float(_bf16_bits(w))
    fmap = L.feature_map(view)
    w_phys = np.zeros((view.padded_feature_count, n), np.float32)
    w_phys[fmap >= 0] = w[fmap[fmap >= 0]]
    if bf16:
        panel = bell_pack_rhs(torch.from_numpy(w_phys).cuda().to(torch.bfloat16))
        y = bell_spmm_packed(m, panel, n)
    else:
        y = bell_spmm(m, torch.from_numpy(w_phys).cuda())
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert np.all(got[view.row_count:] == 0.0)  # padded rows
    vals_f = _bf16_float(values) if bf16 else values
    ro = np.asarray(offsets, np.int32)
    ref = oracle.spmm_referee(len(ro) - 1, nf, n, ro, np.asarray(ids, np.int32), vals_f, w)
    mag = oracle.spmm_referee(len(ro) - 1, nf, n, ro, np.asarray(ids, np.int32), np.abs(vals_f.astype(np.float64)),
                              np.abs(w.astype(np.float64)))
    perm = np.asarray(rperm)
    check_against_referee(oracle, ref[perm], mag[perm], got[:view.row_count])
