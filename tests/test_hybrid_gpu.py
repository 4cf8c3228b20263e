"""GPU parity of the execution-order quantized CSR SpMM with a matrix-core head
(cx_qcsr_spmm_fwd_hybrid, qcsr_hybrid.hip): the head's three-part fp16 split reproduces
every decoded value exactly (an identity weight panel), and the product over random and
C3-generated matrices -- every code width and decode policy, N = 64 and 128, fused
epilogues, ragged workgroups, empty rows and rows wholly inside or outside the head --
matches the float64 referee of the canonical matrix. Repeats are bitwise equal."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import check_against_referee, qcsr_to_host, quantized_fixture, to_device_qcsr

pytestmark = pytest.mark.gpu


def _exec(m):
    from cellerator_amd.exec_order import popularity_order, to_execution_order
    order = popularity_order(m)
    return to_execution_order(m, order), order


def _skewed(oracle, rng, rows, cols, bits, policy):
    """Row lengths from 0 to all genes, genes drawn with a Zipf-like popularity so the
    popularity order has a dense head."""
    fx = quantized_fixture(oracle, rng, rows, cols, 10.0, bits, 1 if policy == 3 else policy)
    weight = 1.0 / np.arange(1, cols + 1) ** 1.1
    weight = weight[rng.permutation(cols)]
    lengths = np.minimum(rng.lognormal(np.log(250.0), 0.8, rows).astype(np.int64), cols)
    lengths[::29] = 0
    lengths[5] = cols
    row_ptr = np.zeros(rows + 1, np.int64)
    row_ptr[1:] = np.cumsum(lengths)
    col_idx = np.empty(int(row_ptr[-1]), np.int32)
    p = weight / weight.sum()
    for r in range(rows):
        if lengths[r]:
            col_idx[row_ptr[r]:row_ptr[r + 1]] = np.sort(rng.choice(cols, lengths[r], replace=False, p=p))
    from tests.test_qcsr_parts_gpu import _rebuild
    return _rebuild(oracle, rng, fx, row_ptr.astype(np.int32), col_idx)


def _referee(oracle, fx, w):
    return oracle.qcsr_spmm_referee(fx["bits"], fx["policy"], fx["rows"], fx["cols"], fx["row_ptr"],
                                    fx["packed_row_ptr"], fx["col_idx"], fx["packed"], fx["scales"],
                                    fx["offsets"], fx["row_offsets"], w)


@pytest.mark.parametrize("bits,policy", [(4, 1), (8, 1), (2, 2), (1, 1), (4, 3), (8, 3)])
def test_hybrid_matches_referee(oracle, bits, policy):
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    rng = np.random.default_rng(2000 + 10 * bits + policy)
    fx = _skewed(oracle, rng, 700, 3100, bits, policy)
    m = to_device_qcsr(fx)
    if policy == 3:
        m = qcsr_pack_gene_affine(m)
    mx, order = _exec(m)
    w = (rng.standard_normal((3100, 64)) * 0.02).astype(np.float16)
    wx = pack_rows(order, torch.from_numpy(w).cuda())
    p = hybrid_prepare(mx, wx, 2048)
    y = hybrid_spmm(p, wx)
    y2 = hybrid_spmm(p, wx)
    torch.cuda.synchronize()
    ref, mag = _referee(oracle, dict(fx, policy=1 if policy == 3 else policy), w)
    check_against_referee(oracle, ref, mag, y.cpu().numpy())
    assert torch.equal(y.view(torch.int32), y2.view(torch.int32))


def test_identity_panel_gives_exact_decoded_values(oracle):
    """W = the identity on the first 64 execution genes: Y[r, c] is the decoded value of
    (r, gene c), through the head's split and the tail's (zero) sum -- bitwise for
    |x| >= 2^-2 and within 2^-24 below."""
    import torch

    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm
    rng = np.random.default_rng(5)
    fx = _skewed(oracle, rng, 600, 2100, 4, 1)
    mx, order = _exec(to_device_qcsr(fx))
    w = torch.zeros((2100, 64), dtype=torch.float16, device="cuda")
    w[torch.arange(64), torch.arange(64)] = 1.0
    y = hybrid_spmm(hybrid_prepare(mx, w, 1024), w)
    torch.cuda.synchronize()
    h = qcsr_to_host(mx)
    decoded = oracle.decode_csr(4, 1, h["row_ptr"], h["packed_row_ptr"], h["col_idx"], h["packed"],
                                h["scales"], h["offsets"], None)
    want = np.zeros((600, 64), np.float32)
    rows = np.repeat(np.arange(600), np.diff(h["row_ptr"]))
    sel = h["col_idx"] < 64
    want[rows[sel], h["col_idx"][sel]] = decoded[sel]
    got = y.cpu().numpy()
    big = np.abs(want) >= 0.25
    assert np.array_equal(got[big].view(np.uint32), want[big].view(np.uint32))
    assert np.all(np.abs(got[~big] - want[~big]) <= 2.0 ** -24)


@pytest.mark.parametrize("n,kind,beta", [(128, 0, 0.0), (64, 6, 0.5), (128, 2, -1.0)])
def test_hybrid_epilogue_and_wide_outputs(oracle, n, kind, beta):
    import torch

    from cellerator_amd import Epilogue
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    rng = np.random.default_rng(3000 + n + kind)
    fx = _skewed(oracle, rng, 530, 2200, 4, 1)
    mx, order = _exec(to_device_qcsr(fx))
    w = (rng.standard_normal((2200, n)) * 0.05).astype(np.float16)
    wx = pack_rows(order, torch.from_numpy(w).cuda())
    bias = (rng.standard_normal(n) * 0.3).astype(np.float32)
    c0 = rng.standard_normal((530, n)).astype(np.float32)
    y = torch.from_numpy(c0.copy()).cuda()
    ep = Epilogue(kind, 1.5, beta, torch.from_numpy(bias).cuda() if kind in (1, 5, 6, 7) else None,
                  y if beta != 0.0 else None)
    hybrid_spmm(hybrid_prepare(mx, wx, 2048), wx, out=y, epilogue=ep)
    torch.cuda.synchronize()
    decoded = oracle.decode_csr(4, 1, fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                fx["scales"], fx["offsets"], None)
    ref = oracle.spmm_referee(530, 2200, n, fx["row_ptr"], fx["col_idx"], decoded, w, alpha=1.5, beta=beta,
                              c0=c0 if beta else None, epilogue=kind,
                              bias=bias if kind in (1, 5, 6, 7) else None)
    mag = oracle.spmm_referee(530, 2200, n, fx["row_ptr"], fx["col_idx"], np.abs(decoded.astype(np.float64)),
                              np.abs(w.astype(np.float64)))
    check_against_referee(oracle, ref, 1.5 * mag + np.abs(beta * c0), y.cpu().numpy())


def test_hybrid_on_c3_rows(oracle):
    """C3-generated rows (4-bit, 33,538 genes, Zipf popularity) in popularity order with a
    4,096-gene head, several workgroups of 256 rows and a ragged last one."""
    import torch

    from cellerator_amd import qcsr_pack_gene_affine
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm, pack_rows
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    m = generate_qcsr(C3.scaled(5 * 256 + 61))
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=3)
    mx, order = _exec(qcsr_pack_gene_affine(m))
    wx = pack_rows(order, w)
    y = hybrid_spmm(hybrid_prepare(mx, wx, 4096), wx)
    torch.cuda.synchronize()
    h = qcsr_to_host(m)
    ref, mag = oracle.qcsr_spmm_referee(4, 1, m.rows, m.cols, h["row_ptr"], h["packed_row_ptr"], h["col_idx"],
                                        h["packed"], h["scales"], h["offsets"], None, w.cpu().numpy())
    check_against_referee(oracle, ref, mag, y.cpu().numpy())


def test_hybrid_rejects_unsorted_and_out_of_range_heads(oracle):
    import torch

    from cellerator_amd import _native as N
    from cellerator_amd.exec_order import hybrid_prepare, hybrid_spmm
    rng = np.random.default_rng(9)
    fx = _skewed(oracle, rng, 300, 2100, 4, 1)
    m = to_device_qcsr(fx)  # canonical order, flags 0
    w = torch.zeros((2100, 64), dtype=torch.float16, device="cuda")
    p = hybrid_prepare(m, w, 1024)
    with pytest.raises(N.EngineError, match="sorted"):
        hybrid_spmm(p, w)
    with pytest.raises(N.EngineError, match="1,024"):
        hybrid_prepare(m, w, 1000)
    big = to_device_qcsr(dict(fx, offsets=(fx["offsets"] + 40000.0).astype(np.float32)))
    with pytest.raises(N.EngineError, match="2\\^15"):
        hybrid_prepare(big, w, 1024)
