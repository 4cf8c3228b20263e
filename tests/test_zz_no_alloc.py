"""The allocation-free balanced forward (cx_qcsr_spmm_fwd_balanced_noalloc) against the
workspace entry (cx_qcsr_spmm_fwd_balanced), through the C-ABI: bitwise equal on two calls
in a row (the second on a smaller matrix, so stale partial rows of the first would show),
with an epilogue, and the size limit rejected with a clear error."""
from __future__ import annotations

import ctypes as C
import dataclasses

import pytest

pytestmark = pytest.mark.gpu


def _run_pair(m, w, n, epilogue=None):
    import torch

    from cellerator_amd import _native as N
    from cellerator_amd import qcsr_spmm_balanced
    lib = N.engine()
    d = m.descriptor()
    ref = torch.full((m.rows, n), float("nan"), device="cuda")
    qcsr_spmm_balanced(m, w, out=ref, epilogue=epilogue)
    got = torch.full((m.rows, n), float("nan"), device="cuda")
    e = epilogue.descriptor(got) if epilogue is not None else None
    if epilogue is not None and epilogue.initial is not None:
        raise ValueError("in-place epilogues are compared through separate outputs")
    st = lib.cx_qcsr_spmm_fwd_balanced_noalloc(
        C.byref(d), w.data_ptr(), N.DTYPE_F16 if w.dtype == torch.float16 else N.DTYPE_F32,
        w.stride(0), n, got.data_ptr(), got.stride(0), C.byref(e) if e is not None else None,
        torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.cx_last_error()
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("n", [64, 128])
def test_noalloc_matches_workspace_entry_twice(n):
    import torch

    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    big = generate_qcsr(C3.scaled(20_000))      # ~3e7 entries: many chunks, rows across edges
    small = generate_qcsr(dataclasses.replace(C3.scaled(1_500), seed=77))
    for m in (big, small):
        w = dense_normal((m.cols, n), 0.02, torch.float16, seed=n)
        ref, got = _run_pair(m, w, n)
        assert torch.equal(ref.view(torch.int32), got.view(torch.int32))


def test_noalloc_epilogue_and_f32_rhs():
    import torch

    from cellerator_amd import Epilogue
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    m = generate_qcsr(C3.scaled(3_000))
    w = dense_normal((m.cols, 64), 0.02, torch.float32, seed=3)
    bias = torch.randn(64, device="cuda")
    ref, got = _run_pair(m, w, 64, Epilogue(5, 1.5, 0.0, bias, None))
    assert torch.equal(ref.view(torch.int32), got.view(torch.int32))


def test_noalloc_rejects_more_partials_than_its_scratch():
    import torch

    from cellerator_amd import _native as N
    from cellerator_amd.synth import C3, dense_normal, generate_qcsr
    m = generate_qcsr(C3.scaled(25_000))  # ~3.7e7 entries: N = 128 needs > 32 MiB
    assert m.nnz > 32768 * 1024
    w = dense_normal((m.cols, 128), 0.02, torch.float16, seed=9)
    out = torch.empty((m.rows, 128), device="cuda")
    lib = N.engine()
    d = m.descriptor()
    st = lib.cx_qcsr_spmm_fwd_balanced_noalloc(C.byref(d), w.data_ptr(), N.DTYPE_F16, w.stride(0), 128,
                                               out.data_ptr(), out.stride(0), None,
                                               torch.cuda.current_stream().cuda_stream)
    assert st == 2  # INVALID_SHAPE
    assert b"scratch" in lib.cx_last_error()
