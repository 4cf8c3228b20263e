"""Public context ABI on the GPU: the reference's own ABI known answers
(tests/abi_runtime_test.cu:176-260: forward {201, 402, 430, ..., 10}, backward grad_values
{5, 500, 110, 1100, 17} and grad_rhs {26, 32, 9, 12, 14, 20}), the quantized-CSR backward
against the oracle, saved-state clearing and the scratch contract."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tests.helpers import check_against_referee, quantized_fixture, to_device_qcsr

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _lib():
    from cellerator_amd import _native as N
    return N, N.engine()


def _matrix(N, t, dtype=None):
    d = N.CelleratorTensorDesc()
    d.version, d.size, d.data, d.rank = 1, C.sizeof(d), t.data_ptr(), 2
    d.dtype = dtype if dtype is not None else N.DTYPE_F32
    d.shape[0], d.shape[1] = t.shape
    d.stride[0], d.stride[1] = t.stride()
    return d


def _vector(N, t):
    d = N.CelleratorTensorDesc()
    d.version, d.size, d.data, d.dtype, d.rank = 1, C.sizeof(d), t.data_ptr(), N.DTYPE_F32, 1
    d.shape[0], d.stride[0] = t.numel(), 1
    return d


def _context(N, lib, device=-1, scratch=None):
    torch = _torch()
    cfg = N.CelleratorExecutionConfig(1, C.sizeof(N.CelleratorExecutionConfig), device,
                                      torch.cuda.current_stream().cuda_stream,
                                      None if scratch is None else scratch.data_ptr(),
                                      0 if scratch is None else scratch.numel())
    ctx = C.c_void_p()
    assert lib.cellerator_context_create(C.byref(cfg), C.byref(ctx)) == 0
    return ctx


def _kat_layout(N, torch):
    """3x3 CSR, f16 values {1..5} (abi_runtime_test.cu:176-218)."""
    major = torch.tensor([0, 2, 4, 5], dtype=torch.int32).cuda()
    minor = torch.tensor([0, 2, 1, 2, 0], dtype=torch.int32).cuda()
    values = torch.tensor([1, 2, 3, 4, 5], dtype=torch.float16).cuda()
    lay = N.CelleratorSparseLayoutDesc()
    lay.version, lay.size, lay.layout = 1, C.sizeof(lay), 1
    lay.rows, lay.cols, lay.nnz, lay.value_dtype = 3, 3, 5, N.DTYPE_F16
    lay.major_ptr, lay.minor_idx, lay.values = major.data_ptr(), minor.data_ptr(), values.data_ptr()
    return lay, (major, minor, values)


def test_reference_abi_forward_backward_kats():
    torch = _torch()
    N, lib = _lib()
    ctx = _context(N, lib)  # device -1: the current device, as the reference test creates it
    lay, keep = _kat_layout(N, torch)
    rhs = torch.tensor([[1, 2], [10, 20], [100, 200]], dtype=torch.float32).cuda()
    grad = torch.tensor([[1, 2], [3, 4], [5, 6]], dtype=torch.float32).cuda()
    out = torch.empty((3, 2), dtype=torch.float32, device="cuda")
    gv = torch.empty(5, dtype=torch.float32, device="cuda")
    gr = torch.empty((3, 2), dtype=torch.float32, device="cuda")
    saved = C.c_void_p()
    r, o = _matrix(N, rhs), _matrix(N, out)
    assert lib.cellerator_sparse_projection_forward(ctx, C.byref(lay), C.byref(r), C.byref(o),
                                                    C.byref(saved)) == 0, lib.cellerator_last_error()
    assert saved.value is not None
    g, v, w = _matrix(N, grad), _vector(N, gv), _matrix(N, gr)
    st = lib.cellerator_sparse_projection_backward(ctx, C.byref(lay), C.byref(r), C.byref(g),
                                                   C.byref(v), C.byref(w))
    assert st == 0, lib.cellerator_last_error()
    assert lib.cellerator_context_synchronize(ctx) == 0
    assert out.cpu().flatten().tolist() == [201, 402, 430, 860, 5, 10]
    assert gv.cpu().tolist() == [5, 500, 110, 1100, 17]
    assert gr.cpu().flatten().tolist() == [26, 32, 9, 12, 14, 20]
    # one gradient alone, the other NULL
    gv.zero_()
    assert lib.cellerator_sparse_projection_backward(ctx, C.byref(lay), C.byref(r), C.byref(g),
                                                     C.byref(v), None) == 0
    assert lib.cellerator_context_synchronize(ctx) == 0
    assert gv.cpu().tolist() == [5, 500, 110, 1100, 17]
    # neither gradient -> INVALID_ARGUMENT; a Blocked-ELL layout -> UNSUPPORTED (abi.cu:345-350)
    assert lib.cellerator_sparse_projection_backward(ctx, C.byref(lay), C.byref(r), C.byref(g),
                                                     None, None) == 1
    lay.layout = 2
    assert lib.cellerator_sparse_projection_backward(ctx, C.byref(lay), C.byref(r), C.byref(g),
                                                     C.byref(v), C.byref(w)) == 3
    lib.cellerator_saved_state_destroy(saved)
    lib.cellerator_context_destroy(ctx)
    del keep


def test_forward_clears_saved_state_on_failure():
    """*saved_state is cleared on entry (abi.cu:285), so a failing call never leaves a stale
    pointer for the caller to destroy."""
    torch = _torch()
    N, lib = _lib()
    ctx = _context(N, lib)
    lay, keep = _kat_layout(N, torch)
    rhs = torch.zeros((4, 2), dtype=torch.float32, device="cuda")  # wrong row count
    out = torch.empty((3, 2), dtype=torch.float32, device="cuda")
    saved = C.c_void_p(0x1234)
    st = lib.cellerator_sparse_projection_forward(ctx, C.byref(lay), C.byref(_matrix(N, rhs)),
                                                  C.byref(_matrix(N, out)), C.byref(saved))
    assert st == 2  # INVALID_SHAPE
    assert saved.value is None
    lib.cellerator_context_destroy(ctx)
    del keep


@pytest.mark.parametrize("bits,policy,n,rhs_dtype", [(4, 1, 64, np.float16), (8, 1, 32, np.float32),
                                                     (2, 2, 64, np.float32)])
def test_quantized_csr_backward_matches_oracle(oracle, bits, policy, n, rhs_dtype):
    torch = _torch()
    N, lib = _lib()
    rng = np.random.default_rng(70 + bits + n)
    rows, cols = 700, 900
    fx = quantized_fixture(oracle, rng, rows, cols, 40.0, bits, policy, empty_every=9)
    m = to_device_qcsr(fx)
    w = (rng.standard_normal((cols, n)) * 0.02).astype(rhs_dtype)
    g = rng.standard_normal((rows, n)).astype(np.float32)
    rhs, grad = torch.from_numpy(w).cuda(), torch.from_numpy(g).cuda()
    lay = N.CelleratorSparseLayoutDesc()
    lay.version, lay.size, lay.layout = 1, C.sizeof(lay), 5
    lay.rows, lay.cols, lay.nnz, lay.bits, lay.decode_policy = rows, cols, m.nnz, bits, policy
    lay.major_ptr, lay.minor_idx = m.row_ptr.data_ptr(), m.col_idx.data_ptr()
    lay.block_col_idx, lay.packed_values = m.packed_row_ptr.data_ptr(), m.packed_values.data_ptr()
    lay.column_scales = m.column_scales.data_ptr()
    if policy == 1:
        lay.column_offsets = m.column_offsets.data_ptr()
    else:
        lay.row_offsets = m.row_offsets.data_ptr()
    gv = torch.empty(m.nnz, dtype=torch.float32, device="cuda")
    gr = torch.empty((cols, n), dtype=torch.float32, device="cuda")
    ctx = _context(N, lib, device=0)
    rdt = N.DTYPE_F16 if rhs_dtype == np.float16 else N.DTYPE_F32
    st = lib.cellerator_sparse_projection_backward(ctx, C.byref(lay), C.byref(_matrix(N, rhs, rdt)),
                                                   C.byref(_matrix(N, grad)), C.byref(_vector(N, gv)),
                                                   C.byref(_matrix(N, gr)))
    assert st == 0, lib.cellerator_last_error()
    assert lib.cellerator_context_synchronize(ctx) == 0
    ref = oracle.spmm_bwd_values(fx["row_ptr"], fx["col_idx"], g, w)
    mag = oracle.spmm_bwd_values(fx["row_ptr"], fx["col_idx"], np.abs(g),
                                 np.abs(w.astype(np.float64)).astype(np.float32))
    check_against_referee(oracle, ref, mag, gv.cpu().numpy())
    decoded = oracle.decode_csr(bits, policy, fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"],
                                fx["packed"], fx["scales"], fx["offsets"], fx["row_offsets"])
    refr = oracle.spmm_referee(cols, rows, n, fx["row_ptr"], fx["col_idx"], decoded, g,
                               transpose_sparse=True)
    magr = oracle.spmm_referee(cols, rows, n, fx["row_ptr"], fx["col_idx"],
                               np.abs(decoded.astype(np.float64)), np.abs(g).astype(np.float64),
                               transpose_sparse=True)
    check_against_referee(oracle, refr, magr, gr.cpu().numpy())
    lib.cellerator_context_destroy(ctx)


def test_backward_scratch_contract():
    """A config scratch that is too small is rejected; a large enough one is used as is."""
    torch = _torch()
    N, lib = _lib()
    lay, keep = _kat_layout(N, torch)
    rhs = torch.tensor([[1, 2], [10, 20], [100, 200]], dtype=torch.float32).cuda()
    grad = torch.tensor([[1, 2], [3, 4], [5, 6]], dtype=torch.float32).cuda()
    gr = torch.empty((3, 2), dtype=torch.float32, device="cuda")
    small = torch.empty(64, dtype=torch.uint8, device="cuda")
    ctx = _context(N, lib, scratch=small)
    args = (C.byref(lay), C.byref(_matrix(N, rhs)), C.byref(_matrix(N, grad)), None,
            C.byref(_matrix(N, gr)))
    assert lib.cellerator_sparse_projection_backward(ctx, *args) == 1
    assert b"scratch" in lib.cellerator_last_error()
    lib.cellerator_context_destroy(ctx)
    big = torch.empty(1 << 22, dtype=torch.uint8, device="cuda")
    ctx = _context(N, lib, scratch=big)
    assert lib.cellerator_sparse_projection_backward(ctx, *args) == 0, lib.cellerator_last_error()
    assert lib.cellerator_context_synchronize(ctx) == 0
    assert gr.cpu().flatten().tolist() == [26, 32, 9, 12, 14, 20]
    lib.cellerator_context_destroy(ctx)
    del keep
