"""GPU parity of the quantized CSR SpMM (cx_qcsr_spmm_fwd) against the oracle."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tests.helpers import (check_against_referee, qcsr_to_host, quantized_fixture,
                           to_device_qcsr)

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _run(m, rhs_np):
    torch = _torch()
    from cellerator_amd import qcsr_spmm
    rhs = torch.from_numpy(rhs_np).cuda()
    out = qcsr_spmm(m, rhs)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_sparse_ops_fixture_plain_csr(oracle):
    """3x3 f16 CSR x 3x2 f32 -> {201,402,430,860,5,10} (tests/sparse_ops_runtime_test.cu:279-297)."""
    torch = _torch()
    from cellerator_amd import QcsrMatrix
    m = QcsrMatrix(3, 3, 0, torch.tensor([0, 2, 4, 5], dtype=torch.int32).cuda(),
                   torch.tensor([0, 2, 1, 2, 0], dtype=torch.int32).cuda(),
                   values=torch.tensor([1, 2, 3, 4, 5], dtype=torch.float16).cuda())
    out = _run(m, np.array([[1, 2], [10, 20], [100, 200]], np.float32))
    assert out.ravel().tolist() == [201.0, 402.0, 430.0, 860.0, 5.0, 10.0]


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("policy", [1, 2])
def test_decode_bit_exact_through_identity_panel(oracle, bits, policy):
    """With W = I (64 genes, fp16 ones on the diagonal) every output element is exactly
    one decoded value, so Y must equal the oracle's decode bit for bit."""
    rng = np.random.default_rng(100 + bits * 3 + policy)
    fx = quantized_fixture(oracle, rng, 300, 64, 20.0, bits, policy, empty_every=9)
    decoded = oracle.decode_csr(bits, policy, fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"],
                                fx["packed"], fx["scales"], fx["offsets"], fx["row_offsets"])
    dense = np.zeros((300, 64), np.float32)
    for r in range(300):
        s, e = fx["row_ptr"][r], fx["row_ptr"][r + 1]
        dense[r, fx["col_idx"][s:e]] = decoded[s:e]
    out = _run(to_device_qcsr(fx), np.eye(64, dtype=np.float16))
    assert np.array_equal(out.view(np.uint32), dense.view(np.uint32))


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("policy", [1, 2])
@pytest.mark.parametrize("n,rhs_dtype", [(64, np.float16), (128, np.float16), (32, np.float16),
                                         (64, np.float32), (128, np.float32), (5, np.float16),
                                         (100, np.float32)])
def test_random_quantized_matches_referee(oracle, bits, policy, n, rhs_dtype):
    rng = np.random.default_rng(bits * 1000 + policy * 100 + n)
    fx = quantized_fixture(oracle, rng, 257, 1500, 150.0, bits, policy, empty_every=11)
    rhs = (rng.standard_normal((1500, n)) * 0.02).astype(rhs_dtype)
    ref, mag = oracle.qcsr_spmm_referee(bits, policy, 257, 1500, fx["row_ptr"],
                                        fx["packed_row_ptr"], fx["col_idx"], fx["packed"],
                                        fx["scales"], fx["offsets"], fx["row_offsets"], rhs)
    out = _run(to_device_qcsr(fx), rhs)
    check_against_referee(oracle, ref, mag, out)


def test_long_rows_and_ragged_tail(oracle):
    """Rows far longer than one 64-entry chunk, lengths not multiples of 64 or 8."""
    rng = np.random.default_rng(77)
    fx = quantized_fixture(oracle, rng, 40, 6000, 2500.0, 4, 1)
    rhs = (rng.standard_normal((6000, 64)) * 0.02).astype(np.float16)
    ref, mag = oracle.qcsr_spmm_referee(4, 1, 40, 6000, fx["row_ptr"], fx["packed_row_ptr"],
                                        fx["col_idx"], fx["packed"], fx["scales"], fx["offsets"],
                                        None, rhs)
    check_against_referee(oracle, ref, mag, _run(to_device_qcsr(fx), rhs))


def test_generated_c2_sample_matches_referee(oracle):
    """GPU-generated 8-bit matrix with the C2 distributions (2,000 x 20,000)."""
    torch = _torch()
    from cellerator_amd import qcsr_spmm
    from cellerator_amd.synth import C2, dense_normal, generate_qcsr
    m = generate_qcsr(C2.scaled(2000))
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=C2.seed + 1)
    out = qcsr_spmm(m, w)
    torch.cuda.synchronize()
    h = qcsr_to_host(m)
    assert h["row_ptr"][-1] == m.nnz and np.all(np.diff(h["row_ptr"]) >= 200)
    ref, mag = oracle.qcsr_spmm_referee(8, 1, m.rows, m.cols, h["row_ptr"], h["packed_row_ptr"],
                                        h["col_idx"], h["packed"], h["scales"], h["offsets"],
                                        None, w.cpu().numpy())
    check_against_referee(oracle, ref, mag, out.cpu().numpy())


def test_generated_c3_sample_matches_referee(oracle):
    """GPU-generated 4-bit matrix with the C3 distributions (1,500 x 33,538), N=64 and 128."""
    torch = _torch()
    from cellerator_amd import qcsr_spmm
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    m = generate_qcsr(C3.scaled(1500))
    h = qcsr_to_host(m)
    cols = h["col_idx"]
    rp = h["row_ptr"]
    for r in range(0, m.rows, 97):  # sorted, unique, in range
        seg = cols[rp[r]:rp[r + 1]]
        assert np.all(np.diff(seg) > 0) and seg.min() >= 0 and seg.max() < m.cols
    for n in (64, 128):
        w = dense_normal((m.cols, n), 0.02, torch.float16, seed=C3.seed + n)
        out = qcsr_spmm(m, w)
        torch.cuda.synchronize()
        ref, mag = oracle.qcsr_spmm_referee(4, 1, m.rows, m.cols, h["row_ptr"],
                                            h["packed_row_ptr"], h["col_idx"], h["packed"],
                                            h["scales"], h["offsets"], None, w.cpu().numpy())
        check_against_referee(oracle, ref, mag, out.cpu().numpy())


def test_generated_c1_fp32_csr(oracle):
    """C1: fp32 CSR (Poisson(200) rows, uniform genes), against the fp64 referee."""
    torch = _torch()
    from cellerator_amd import qcsr_spmm
    from cellerator_amd.synth import C1, dense_normal, generate_qcsr
    m = generate_qcsr(C1.scaled(3000))
    w = dense_normal((m.cols, 64), 0.02, torch.float32, seed=C1.seed + 1)
    out = qcsr_spmm(m, w)
    torch.cuda.synchronize()
    h = qcsr_to_host(m)
    ref = oracle.spmm_referee(m.rows, m.cols, 64, h["row_ptr"].astype(np.uint64),
                              h["col_idx"].astype(np.uint32), h["values"], w.cpu().numpy())
    rows = np.repeat(np.arange(m.rows), np.diff(h["row_ptr"]))
    mag = np.zeros((m.rows, 64))
    np.add.at(mag, rows, np.abs(h["values"][:, None].astype(np.float64)
                                * w.cpu().numpy()[h["col_idx"]].astype(np.float64)))
    check_against_referee(oracle, ref, mag, out.cpu().numpy())


def test_deterministic_repeat():
    torch = _torch()
    from cellerator_amd import qcsr_spmm
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    m = generate_qcsr(C3.scaled(800))
    w = dense_normal((m.cols, 64), 0.02, torch.float16, seed=5)
    a = qcsr_spmm(m, w).clone()
    b = qcsr_spmm(m, w)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_error_paths():
    torch = _torch()
    from cellerator_amd import QcsrMatrix, qcsr_spmm
    from cellerator_amd._native import EngineError
    m = QcsrMatrix(2, 4, 3, torch.tensor([0, 1, 2], dtype=torch.int32).cuda(),
                   torch.tensor([0, 1], dtype=torch.int32).cuda(),
                   packed_row_ptr=torch.tensor([0, 1, 2], dtype=torch.int32).cuda(),
                   packed_values=torch.zeros(16, dtype=torch.uint8).cuda())
    with pytest.raises(EngineError, match="UNSUPPORTED"):
        qcsr_spmm(m, torch.zeros((4, 8), dtype=torch.float16).cuda())
    with pytest.raises(ValueError):
        qcsr_spmm(m, torch.zeros((5, 8), dtype=torch.float16).cuda())


def test_public_abi_quantized_csr(oracle):
    """cellerator_sparse_projection_forward with the QUANTIZED_CSR layout."""
    torch = _torch()
    from cellerator_amd import _native as N
    rng = np.random.default_rng(9)
    fx = quantized_fixture(oracle, rng, 50, 300, 40.0, 4, 1)
    m = to_device_qcsr(fx)
    rhs = torch.from_numpy((rng.standard_normal((300, 64)) * 0.02).astype(np.float32)).cuda()
    out = torch.empty((50, 64), dtype=torch.float32, device="cuda")
    lib = N.engine()
    cfg = N.CelleratorExecutionConfig(1, C.sizeof(N.CelleratorExecutionConfig), 0,
                                      torch.cuda.current_stream().cuda_stream, None, 0)
    ctx = C.c_void_p()
    assert lib.cellerator_context_create(C.byref(cfg), C.byref(ctx)) == 0
    lay = N.CelleratorSparseLayoutDesc()
    lay.version, lay.size, lay.layout = 1, C.sizeof(lay), 5
    lay.rows, lay.cols, lay.nnz, lay.bits, lay.decode_policy = 50, 300, m.nnz, 4, 1
    lay.major_ptr, lay.minor_idx = m.row_ptr.data_ptr(), m.col_idx.data_ptr()
    lay.block_col_idx, lay.packed_values = m.packed_row_ptr.data_ptr(), m.packed_values.data_ptr()
    lay.column_scales, lay.column_offsets = m.column_scales.data_ptr(), m.column_offsets.data_ptr()

    def desc(t, dtype):
        d = N.CelleratorTensorDesc()
        d.version, d.size, d.data, d.dtype, d.rank = 1, C.sizeof(d), t.data_ptr(), dtype, 2
        d.shape[0], d.shape[1] = t.shape
        d.stride[0], d.stride[1] = t.stride()
        return d

    r, o = desc(rhs, N.DTYPE_F32), desc(out, N.DTYPE_F32)
    st = lib.cellerator_sparse_projection_forward(ctx, C.byref(lay), C.byref(r), C.byref(o), None)
    assert st == 0, lib.cellerator_last_error()
    assert lib.cellerator_context_synchronize(ctx) == 0
    ref, mag = oracle.qcsr_spmm_referee(4, 1, 50, 300, fx["row_ptr"], fx["packed_row_ptr"],
                                        fx["col_idx"], fx["packed"], fx["scales"], fx["offsets"],
                                        None, rhs.cpu().numpy())
    check_against_referee(oracle, ref, mag, out.cpu().numpy())
    lay.layout = 3  # SLICED_ELL -> UNSUPPORTED, as the reference
    assert lib.cellerator_sparse_projection_forward(ctx, C.byref(lay), C.byref(r), C.byref(o), None) == 3
    lib.cellerator_context_destroy(ctx)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("n,rhs_dtype", [(64, np.float16), (128, np.float16), (32, np.float16),
                                         (64, np.float32), (100, np.float32)])
def test_interleaved_gene_affine_is_bit_identical(oracle, bits, n, rhs_dtype):
    """CX_DECODE_PER_GENE_AFFINE_PAIRS decodes exactly like the separate scale/offset
    arrays: outputs equal bitwise on the fast (32/64/128) and generic shapes."""
    torch = _torch()
    from cellerator_amd import qcsr_pack_gene_affine, qcsr_spmm
    rng = np.random.default_rng(500 + bits * 10 + n)
    fx = quantized_fixture(oracle, rng, 301, 1200, 90.0, bits, oracle.PER_GENE_AFFINE, empty_every=7)
    m = to_device_qcsr(fx)
    mp = qcsr_pack_gene_affine(m)
    pairs = mp.column_scales.view(-1, 2).cpu().numpy()
    assert np.array_equal(pairs[:, 0], fx["scales"]) and np.array_equal(pairs[:, 1], fx["offsets"])
    rhs = torch.from_numpy((rng.standard_normal((1200, n)) * 0.02).astype(rhs_dtype)).cuda()
    a = qcsr_spmm(m, rhs)
    b = qcsr_spmm(mp, rhs)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_interleaved_gene_affine_defaults_and_errors():
    """NULL scales/offsets pack to (1, 0); the pairs policy rejects separate offsets."""
    torch = _torch()
    from cellerator_amd import QcsrMatrix, qcsr_pack_gene_affine, qcsr_spmm
    from cellerator_amd import _native as N
    m = QcsrMatrix(2, 4, 4, torch.tensor([0, 1, 2], dtype=torch.int32).cuda(),
                   torch.tensor([0, 3], dtype=torch.int32).cuda(),
                   packed_row_ptr=torch.tensor([0, 1, 2], dtype=torch.int32).cuda(),
                   packed_values=torch.tensor([5, 9] + [0] * 14, dtype=torch.uint8).cuda())
    mp = qcsr_pack_gene_affine(m)
    assert mp.column_scales.cpu().tolist() == [1.0, 0.0] * 4
    w = torch.arange(16, dtype=torch.float32).reshape(4, 4).cuda()
    assert torch.equal(qcsr_spmm(mp, w), qcsr_spmm(m, w))
    bad = QcsrMatrix(2, 4, 4, m.row_ptr, m.col_idx, packed_row_ptr=m.packed_row_ptr,
                     packed_values=m.packed_values, column_scales=mp.column_scales,
                     column_offsets=torch.zeros(4).cuda(),
                     decode_policy=N.DECODE_PER_GENE_AFFINE_PAIRS)
    with pytest.raises(N.EngineError, match="INVALID_ARGUMENT"):
        qcsr_spmm(bad, w)
