"""GPU: the device radix sort and scan, the transposed CSR build, and the backward of the
(quantized) CSR SpMM -- grad_values (csr_spmm_bwd_values_kernel_) and grad_rhs = A^T . grad_Y
(csr_spmm_bwd_rhs_kernel_) -- against numpy / scipy textbook routines and the oracle."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import check_against_referee, quantized_fixture, random_csr, to_device_qcsr

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


# ---------------------------------------------------------------- sort / scan

@pytest.mark.parametrize("count,key_bits,with_values", [
    (0, 16, False), (1, 8, False), (4095, 8, True), (4096, 16, False), (4097, 16, True),
    (100_003, 15, False), (250_000, 24, True), (70_000, 32, True)])
def test_sort_pairs_is_numpy_stable_argsort(count, key_bits, with_values):
    torch = _torch()
    from cellerator_amd import sort_pairs
    rng = np.random.default_rng(count + key_bits)
    hi = 1 << min(key_bits, 31)
    keys = rng.integers(0, hi, count, dtype=np.int64).astype(np.uint32)
    if key_bits == 32 and count:
        keys[::7] |= np.uint32(0x80000000)  # exercise the top bit
    if count > 10:
        keys[: count // 3] = keys[0]  # long runs of equal keys: stability matters
    vals = rng.integers(0, 1 << 31, count, dtype=np.int64).astype(np.uint32) if with_values else None
    kt = torch.from_numpy(keys.view(np.int32)).cuda()
    vt = None if vals is None else torch.from_numpy(vals.view(np.int32)).cuda()
    ko, vo = sort_pairs(kt, vt, key_bits)
    torch.cuda.synchronize()
    masked = keys & np.uint32((1 << key_bits) - 1 if key_bits < 32 else 0xFFFFFFFF)
    order = np.argsort(masked, kind="stable")
    assert np.array_equal(ko.cpu().numpy().view(np.uint32), keys[order])
    expect_vals = (vals if vals is not None else np.arange(count, dtype=np.uint32))[order]
    assert np.array_equal(vo.cpu().numpy().view(np.uint32), expect_vals)


def test_sort_pairs_low_bits_only():
    """Keys are ordered on their low key_bits bits; the high bits ride along."""
    torch = _torch()
    from cellerator_amd import sort_pairs
    keys = np.array([0x100 | 5, 3, 0x200 | 3, 5, 0x300 | 1], np.uint32)
    ko, vo = sort_pairs(torch.from_numpy(keys.view(np.int32)).cuda(), None, 8)
    torch.cuda.synchronize()
    assert vo.cpu().numpy().tolist() == [4, 1, 2, 0, 3]


@pytest.mark.parametrize("n", [0, 1, 255, 4096, 4097, 1_000_003])
def test_exclusive_scan_is_numpy_cumsum(n):
    torch = _torch()
    from cellerator_amd import exclusive_scan_u32
    rng = np.random.default_rng(n)
    x = rng.integers(0, 1000, n).astype(np.uint32)
    out = exclusive_scan_u32(torch.from_numpy(x.view(np.int32)).cuda())
    torch.cuda.synchronize()
    expect = (np.concatenate([[0], np.cumsum(x.astype(np.uint64))[:-1]]) % (1 << 32)).astype(np.uint32)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), expect[:n])


# ---------------------------------------------------------------- transpose

@pytest.mark.parametrize("bits,policy", [(8, 1), (4, 2), (2, 1), (1, 2), (4, 3), (0, 0)])
def test_transpose_is_scipy_transpose_with_exact_decode(oracle, bits, policy):
    torch = _torch()
    import scipy.sparse as sp

    from cellerator_amd import qcsr_pack_gene_affine, qcsr_transpose
    rng = np.random.default_rng(40 + bits * 4 + policy)
    rows, cols = 1300, 700
    if bits == 0:
        from cellerator_amd import QcsrMatrix
        row_ptr, col_idx = random_csr(rng, rows, cols, 25.0, empty_every=9)
        vals = rng.standard_normal(len(col_idx)).astype(np.float16)
        m = QcsrMatrix(rows, cols, 0, torch.from_numpy(row_ptr).cuda(),
                       torch.from_numpy(col_idx).cuda(), values=torch.from_numpy(vals).cuda())
        decoded = vals.astype(np.float32)
    else:
        fx = quantized_fixture(oracle, rng, rows, cols, 25.0, bits, 1 if policy == 3 else policy,
                               empty_every=9)
        m = to_device_qcsr(fx)
        if policy == 3:
            m = qcsr_pack_gene_affine(m)
        row_ptr, col_idx = fx["row_ptr"], fx["col_idx"]
        decoded = oracle.decode_csr(bits, fx["policy"], row_ptr, fx["packed_row_ptr"], col_idx,
                                    fx["packed"], fx["scales"], fx["offsets"], fx["row_offsets"])
    t = qcsr_transpose(m)
    torch.cuda.synchronize()
    # textbook: scipy's CSR transpose of the same matrix, with entry ids as data
    ids = sp.csr_matrix((np.arange(1, len(col_idx) + 1, dtype=np.int64), col_idx, row_ptr),
                        shape=(rows, cols)).T.tocsr()
    ids.sort_indices()
    assert (t.rows, t.cols, t.nnz) == (cols, rows, len(col_idx))
    assert np.array_equal(t.row_ptr.cpu().numpy(), ids.indptr)
    assert np.array_equal(t.col_idx.cpu().numpy(), ids.indices)
    expect = decoded[ids.data - 1]
    assert np.array_equal(t.values.cpu().numpy().view(np.uint32), expect.view(np.uint32))


def test_transpose_of_empty_and_one_gene(oracle):
    torch = _torch()
    from cellerator_amd import QcsrMatrix, qcsr_transpose
    empty = QcsrMatrix(4, 3, 0, torch.zeros(5, dtype=torch.int32).cuda(),
                       torch.zeros(0, dtype=torch.int32).cuda(),
                       values=torch.zeros(0, dtype=torch.float32).cuda())
    t = qcsr_transpose(empty)
    torch.cuda.synchronize()
    assert t.row_ptr.cpu().tolist() == [0, 0, 0, 0]
    one = QcsrMatrix(3, 1, 0, torch.tensor([0, 1, 1, 2], dtype=torch.int32).cuda(),
                     torch.tensor([0, 0], dtype=torch.int32).cuda(),
                     values=torch.tensor([2.0, 3.0]).cuda())
    t = qcsr_transpose(one)
    torch.cuda.synchronize()
    assert t.row_ptr.cpu().tolist() == [0, 2]
    assert t.col_idx.cpu().tolist() == [0, 2]
    assert t.values.cpu().tolist() == [2.0, 3.0]


# ---------------------------------------------------------------- backward

def test_backward_reference_kats(oracle):
    """tests/sparse_ops_runtime_test.cu:566-604: grad_values {5,500,110,1100,17} and
    grad_rhs {26,32,9,12,14,20} on the 3x3 f16 fixture."""
    torch = _torch()
    from cellerator_amd import QcsrMatrix, qcsr_spmm_bwd_rhs, qcsr_spmm_bwd_values, qcsr_transpose
    m = QcsrMatrix(3, 3, 0, torch.tensor([0, 2, 4, 5], dtype=torch.int32).cuda(),
                   torch.tensor([0, 2, 1, 2, 0], dtype=torch.int32).cuda(),
                   values=torch.tensor([1, 2, 3, 4, 5], dtype=torch.float16).cuda())
    rhs = torch.tensor([[1, 2], [10, 20], [100, 200]], dtype=torch.float32).cuda()
    grad = torch.tensor([[1, 2], [3, 4], [5, 6]], dtype=torch.float32).cuda()
    gv = qcsr_spmm_bwd_values(m, grad, rhs)
    gr = qcsr_spmm_bwd_rhs(qcsr_transpose(m), grad)
    torch.cuda.synchronize()
    assert gv.cpu().tolist() == [5.0, 500.0, 110.0, 1100.0, 17.0]
    assert gr.cpu().numpy().ravel().tolist() == [26.0, 32.0, 9.0, 12.0, 14.0, 20.0]


@pytest.mark.parametrize("n,rhs_dtype", [(64, np.float16), (128, np.float16), (32, np.float16),
                                         (64, np.float32), (128, np.float32), (7, np.float32),
                                         (100, np.float16)])
def test_bwd_values_matches_oracle(oracle, n, rhs_dtype):
    torch = _torch()
    from cellerator_amd import qcsr_spmm_bwd_values
    rng = np.random.default_rng(n * 3 + (rhs_dtype == np.float16))
    fx = quantized_fixture(oracle, rng, 333, 1100, 90.0, 4, 1, empty_every=8)
    g = rng.standard_normal((333, n)).astype(np.float32)
    w = (rng.standard_normal((1100, n)) * 0.1).astype(rhs_dtype)
    gv = qcsr_spmm_bwd_values(to_device_qcsr(fx), torch.from_numpy(g).cuda(), torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    ref = oracle.spmm_bwd_values(fx["row_ptr"], fx["col_idx"], g, w)
    rows_of = np.repeat(np.arange(333), np.diff(fx["row_ptr"]))
    mag = np.einsum("ij,ij->i", np.abs(g.astype(np.float64))[rows_of],
                    np.abs(w.astype(np.float64))[fx["col_idx"]])
    check_against_referee(oracle, ref, mag, gv.cpu().numpy())


@pytest.mark.parametrize("bits,policy,n", [(8, 1, 64), (4, 2, 128), (4, 1, 48), (0, 0, 64)])
def test_bwd_rhs_and_transposed_product_match_referee(oracle, bits, policy, n):
    """grad_rhs = A^T . G equals the referee's transpose_sparse product (referee.cc:170-232),
    and the transposed matrix also serves A^T . B through the plain forward."""
    torch = _torch()
    from cellerator_amd import (QcsrMatrix, qcsr_spmm, qcsr_spmm_balanced, qcsr_spmm_bwd_rhs,
                                qcsr_transpose)
    rng = np.random.default_rng(bits * 10 + policy + n)
    rows, cols = 2100, 500
    if bits == 0:
        row_ptr, col_idx = random_csr(rng, rows, cols, 30.0, empty_every=5)
        decoded = rng.standard_normal(len(col_idx)).astype(np.float32)
        m = QcsrMatrix(rows, cols, 0, torch.from_numpy(row_ptr).cuda(),
                       torch.from_numpy(col_idx).cuda(), values=torch.from_numpy(decoded).cuda())
    else:
        fx = quantized_fixture(oracle, rng, rows, cols, 30.0, bits, policy, empty_every=5)
        m = to_device_qcsr(fx)
        row_ptr, col_idx = fx["row_ptr"], fx["col_idx"]
        decoded = oracle.decode_csr(bits, policy, row_ptr, fx["packed_row_ptr"], col_idx,
                                    fx["packed"], fx["scales"], fx["offsets"], fx["row_offsets"])
    g = rng.standard_normal((rows, n)).astype(np.float32)
    t = qcsr_transpose(m)
    gr = qcsr_spmm_bwd_rhs(t, torch.from_numpy(g).cuda())
    direct = qcsr_spmm_balanced(t, torch.from_numpy(g).cuda())
    rowwave = qcsr_spmm(t, torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    ref = oracle.spmm_referee(cols, rows, n, row_ptr, col_idx, decoded, g, transpose_sparse=True)
    absx = np.abs(decoded.astype(np.float64))
    mag = oracle.spmm_referee(cols, rows, n, row_ptr, col_idx, absx, np.abs(g).astype(np.float64),
                              transpose_sparse=True)
    check_against_referee(oracle, ref, mag, gr.cpu().numpy())
    check_against_referee(oracle, ref, mag, rowwave.cpu().numpy())
    assert torch.equal(gr.view(torch.int32), direct.view(torch.int32))
    # run to run: the same bits (no atomics)
    again = qcsr_spmm_bwd_rhs(qcsr_transpose(m), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    assert torch.equal(gr.view(torch.int32), again.view(torch.int32))


# ---------------------------------------------------------------- load-balanced form

def _rows_from_lengths(oracle, rng, lengths, cols, bits=4, policy=1):
    """A quantized CSR with the given row lengths (columns sorted, distinct)."""
    from tests.helpers import quantized_fixture
    lengths = np.asarray(lengths, np.int64)
    fx = quantized_fixture(oracle, rng, len(lengths), cols, 1.0, bits, policy)
    row_ptr = np.zeros(len(lengths) + 1, np.int64)
    row_ptr[1:] = np.cumsum(lengths)
    col_idx = np.concatenate([np.sort(rng.choice(cols, size=int(c), replace=False)) for c in lengths
                              if c] or [np.zeros(0, np.int64)]).astype(np.int32)
    qmax = (1 << bits) - 1
    codes = rng.integers(0, qmax + 1, len(col_idx))
    values = (fx["offsets"][col_idx] + fx["scales"][col_idx] * codes).astype(np.float32) \
        if policy == 1 else None
    row_ptr = row_ptr.astype(np.int32)
    packed_row_ptr = oracle.build_packed_row_ptr(bits, row_ptr)
    packed = oracle.pack_csr(bits, policy, row_ptr, packed_row_ptr, col_idx, values, fx["scales"],
                             fx["offsets"], None)
    fx.update(row_ptr=row_ptr, packed_row_ptr=packed_row_ptr, col_idx=col_idx, packed=packed)
    return fx


# chunk = 1,024 entries at these sizes: rows ending exactly on a chunk edge, empty rows on
# an edge, a row spanning several chunks, trailing empty rows, a last partial chunk
EDGE_LENGTHS = [1024, 0, 0, 3000, 1, 0, 2047, 5000, 0, 1023, 1, 0, 0, 4100, 7, 0, 0]


@pytest.mark.parametrize("n,rhs_dtype", [(64, np.float16), (128, np.float32), (64, np.float32)])
def test_balanced_matches_referee_on_chunk_edges(oracle, n, rhs_dtype):
    torch = _torch()
    from cellerator_amd import Epilogue, qcsr_spmm, qcsr_spmm_balanced
    rng = np.random.default_rng(n)
    fx = _rows_from_lengths(oracle, rng, EDGE_LENGTHS, 6000)
    m = to_device_qcsr(fx)
    w = (rng.standard_normal((6000, n)) * 0.05).astype(rhs_dtype)
    wt = torch.from_numpy(w).cuda()
    out = qcsr_spmm_balanced(m, wt)
    plain = qcsr_spmm(m, wt)
    again = qcsr_spmm_balanced(m, wt)
    torch.cuda.synchronize()
    ref, mag = oracle.qcsr_spmm_referee(4, 1, len(EDGE_LENGTHS), 6000, fx["row_ptr"],
                                        fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                        fx["scales"], fx["offsets"], None, w)
    check_against_referee(oracle, ref, mag + 1e-30, out.cpu().numpy())
    check_against_referee(oracle, ref, mag + 1e-30, plain.cpu().numpy())
    assert torch.equal(out.view(torch.int32), again.view(torch.int32))
    # with an epilogue, in place
    bias = torch.randn(n, device="cuda")
    c0 = torch.randn(len(EDGE_LENGTHS), n, device="cuda")
    y = c0.clone()
    qcsr_spmm_balanced(m, wt, out=y, epilogue=Epilogue(7, 0.5, 2.0, bias, y))
    torch.cuda.synchronize()
    decoded = oracle.decode_csr(4, 1, fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                fx["scales"], fx["offsets"], None)
    ref_e = oracle.spmm_referee(len(EDGE_LENGTHS), 6000, n, fx["row_ptr"], fx["col_idx"], decoded, w,
                                alpha=0.5, beta=2.0, c0=c0.cpu().numpy(), epilogue=7,
                                bias=bias.cpu().numpy())
    cmp = oracle.compare(ref_e, y.cpu().numpy(), 1e-4, 1e-4)
    assert cmp["status"] == 0 and cmp["within_tolerance"], cmp


def test_balanced_single_row_and_empty_matrix(oracle):
    torch = _torch()
    from cellerator_amd import Epilogue, QcsrMatrix, qcsr_spmm_balanced
    rng = np.random.default_rng(3)
    fx = _rows_from_lengths(oracle, rng, [9000], 9500, bits=8)
    w = (rng.standard_normal((9500, 64)) * 0.05).astype(np.float16)
    out = qcsr_spmm_balanced(to_device_qcsr(fx), torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    ref, mag = oracle.qcsr_spmm_referee(8, 1, 1, 9500, fx["row_ptr"], fx["packed_row_ptr"],
                                        fx["col_idx"], fx["packed"], fx["scales"], fx["offsets"],
                                        None, w)
    check_against_referee(oracle, ref, mag, out.cpu().numpy())
    empty = QcsrMatrix(5, 7, 0, torch.zeros(6, dtype=torch.int32).cuda(),
                       torch.zeros(0, dtype=torch.int32).cuda(),
                       values=torch.zeros(0, dtype=torch.float32).cuda())
    bias = torch.arange(64, dtype=torch.float32, device="cuda")
    y = torch.full((5, 64), float("nan"), device="cuda")
    qcsr_spmm_balanced(empty, torch.ones(7, 64, device="cuda"), out=y,
                       epilogue=Epilogue(5, 1.0, 0.0, bias - 10.0))
    torch.cuda.synchronize()
    assert torch.equal(y, torch.relu(bias - 10.0).expand(5, 64))


def test_balanced_skewed_random_matches_row_wave(oracle):
    """Lognormal rows with a few very long ones: balanced and row-wave agree within fp32
    reordering, both within the referee's tolerance."""
    torch = _torch()
    from cellerator_amd import qcsr_spmm, qcsr_spmm_balanced
    rng = np.random.default_rng(12)
    lengths = np.minimum(rng.lognormal(3.0, 1.5, 3000).astype(np.int64), 3999)
    lengths[[5, 700, 2999]] = [3999, 3500, 3998]
    fx = _rows_from_lengths(oracle, rng, lengths, 4000, bits=4, policy=1)
    w = (rng.standard_normal((4000, 128)) * 0.05).astype(np.float16)
    m = to_device_qcsr(fx)
    a = qcsr_spmm_balanced(m, torch.from_numpy(w).cuda())
    b = qcsr_spmm(m, torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    ref, mag = oracle.qcsr_spmm_referee(4, 1, 3000, 4000, fx["row_ptr"], fx["packed_row_ptr"],
                                        fx["col_idx"], fx["packed"], fx["scales"], fx["offsets"],
                                        None, w)
    check_against_referee(oracle, ref, mag + 1e-30, a.cpu().numpy())
    check_against_referee(oracle, ref, mag + 1e-30, b.cpu().numpy())


# ---------------------------------------------------------------- panelled transpose

@pytest.mark.parametrize("panel_rows", [1, 64, 500, 5000])
def test_panelled_transpose_is_blockwise_scipy_transpose(oracle, panel_rows):
    torch = _torch()
    import scipy.sparse as sp

    from cellerator_amd import qcsr_transpose_panelled
    rng = np.random.default_rng(panel_rows)
    rows, cols = 1234, 300
    fx = quantized_fixture(oracle, rng, rows, cols, 20.0, 4, 1, empty_every=7)
    decoded = oracle.decode_csr(4, 1, fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                fx["scales"], fx["offsets"], None)
    t = qcsr_transpose_panelled(to_device_qcsr(fx), panel_rows)
    torch.cuda.synchronize()
    panels = (rows + panel_rows - 1) // panel_rows
    assert (t.rows, t.cols, t.meta["panels"]) == (panels * cols, rows, panels)
    ids = sp.csr_matrix((np.arange(1, len(fx["col_idx"]) + 1), fx["col_idx"], fx["row_ptr"]),
                        shape=(rows, cols))
    ptr, idx, val = [0], [], []
    for p in range(panels):
        block = ids[p * panel_rows:(p + 1) * panel_rows].T.tocsr()
        block.sort_indices()
        for g in range(cols):
            s, e = block.indptr[g], block.indptr[g + 1]
            idx.extend((block.indices[s:e] + p * panel_rows).tolist())
            val.extend(block.data[s:e].tolist())
            ptr.append(len(idx))
    assert np.array_equal(t.row_ptr.cpu().numpy(), np.array(ptr))
    assert np.array_equal(t.col_idx.cpu().numpy(), np.array(idx))
    expect = decoded[np.array(val, np.int64) - 1]
    assert np.array_equal(t.values.cpu().numpy().view(np.uint32), expect.view(np.uint32))


@pytest.mark.parametrize("panel_rows,n", [(256, 64), (1000, 128), (3000, 64), (64, 48)])
def test_panelled_bwd_rhs_matches_referee(oracle, panel_rows, n):
    torch = _torch()
    from cellerator_amd import qcsr_spmm_bwd_rhs, qcsr_transpose_panelled
    rng = np.random.default_rng(panel_rows + n)
    rows, cols = 2500, 400
    fx = quantized_fixture(oracle, rng, rows, cols, 30.0, 8, 1, empty_every=9)
    decoded = oracle.decode_csr(8, 1, fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                fx["scales"], fx["offsets"], None)
    g = rng.standard_normal((rows, n)).astype(np.float32)
    gt = torch.from_numpy(g).cuda()
    t = qcsr_transpose_panelled(to_device_qcsr(fx), panel_rows)
    a = qcsr_spmm_bwd_rhs(t, gt)
    b = qcsr_spmm_bwd_rhs(t, gt)
    torch.cuda.synchronize()
    ref = oracle.spmm_referee(cols, rows, n, fx["row_ptr"], fx["col_idx"], decoded, g,
                              transpose_sparse=True)
    mag = oracle.spmm_referee(cols, rows, n, fx["row_ptr"], fx["col_idx"],
                              np.abs(decoded).astype(np.float64), np.abs(g).astype(np.float64),
                              transpose_sparse=True)
    check_against_referee(oracle, ref, mag, a.cpu().numpy())
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
