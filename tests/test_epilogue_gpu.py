"""GPU parity of the fused SpMM epilogues (alpha, beta, bias, ReLU, exact and tanh GELU) on
the quantized CSR and Blocked-ELL paths against the oracle's restatement of the reference's
CPU referee (src/compute/math/referee.cc:75-97,170-250), whose epilogue arithmetic
tests/test_oracle.py pins against scipy's erf and numpy's tanh."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import REL_TOL, ABS_TOL_SCALED, quantized_fixture, to_device_qcsr

pytestmark = pytest.mark.gpu

BIAS_KINDS = (1, 5, 6, 7)
ALL_KINDS = list(range(8))


def _torch():
    import torch
    return torch


def _check(oracle, ref, magnitude, out):
    """Tolerance of the plain product scaled by the element's magnitude: |alpha| sum |x||w|
    plus |beta C| plus |bias| (the activations are 1-Lipschitz up to the GELU's 1.13)."""
    cmp = oracle.compare(ref, out, ABS_TOL_SCALED * 1.2, REL_TOL, magnitude)
    assert cmp["status"] == 0, cmp
    assert cmp["within_tolerance"], cmp


def _inputs(rng, rows, n, kind, beta):
    bias = (rng.standard_normal(n) * 0.5).astype(np.float32) if kind in BIAS_KINDS else None
    c0 = (rng.standard_normal((rows, n))).astype(np.float32) if beta != 0.0 else None
    return bias, c0


def _magnitude(mag, alpha, beta, c0, bias):
    m = abs(alpha) * mag
    if c0 is not None:
        m = m + abs(beta) * np.abs(c0.astype(np.float64))
    if bias is not None:
        m = m + np.abs(bias.astype(np.float64))[None, :]
    return m + 1e-6


def _qcsr_referee(oracle, fx, rhs, alpha, beta, c0, kind, bias):
    decoded = oracle.decode_csr(fx["bits"], fx["policy"], fx["row_ptr"], fx["packed_row_ptr"],
                                fx["col_idx"], fx["packed"], fx["scales"], fx["offsets"],
                                fx["row_offsets"])
    ref = oracle.spmm_referee(fx["rows"], fx["cols"], rhs.shape[1], fx["row_ptr"],
                              fx["col_idx"], decoded.astype(np.float32), rhs, alpha=alpha,
                              beta=beta, c0=c0, epilogue=kind, bias=bias)
    _, mag = oracle.qcsr_spmm_referee(fx["bits"], fx["policy"], fx["rows"], fx["cols"],
                                      fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"],
                                      fx["packed"], fx["scales"], fx["offsets"],
                                      fx["row_offsets"], rhs)
    return ref, mag


@pytest.mark.parametrize("kind", ALL_KINDS)
@pytest.mark.parametrize("n,rhs_dtype", [(64, np.float16), (128, np.float32), (48, np.float16)])
def test_qcsr_epilogue_matches_referee(oracle, kind, n, rhs_dtype):
    torch = _torch()
    from cellerator_amd import Epilogue, qcsr_spmm
    rng = np.random.default_rng(500 + kind * 10 + n)
    fx = quantized_fixture(oracle, rng, 203, 900, 60.0, 4, 1, empty_every=7)
    rhs = (rng.standard_normal((900, n)) * 0.05).astype(rhs_dtype)
    alpha, beta = 0.75, -0.5
    bias, c0 = _inputs(rng, 203, n, kind, beta)
    ref, mag = _qcsr_referee(oracle, fx, rhs, alpha, beta, c0, kind, bias)
    dev = lambda a: None if a is None else torch.from_numpy(a).cuda()  # noqa: E731
    ep = Epilogue(kind, alpha, beta, dev(bias), dev(c0))
    out = qcsr_spmm(to_device_qcsr(fx), dev(rhs), epilogue=ep)
    torch.cuda.synchronize()
    _check(oracle, ref, _magnitude(mag, alpha, beta, c0, bias), out.cpu().numpy())


@pytest.mark.parametrize("kind", [0, 5, 7])
def test_qcsr_epilogue_in_place_accumulate(oracle, kind):
    """beta * Y in place (initial == out, the affine_accumulate output effect)."""
    torch = _torch()
    from cellerator_amd import Epilogue, qcsr_spmm
    rng = np.random.default_rng(610 + kind)
    fx = quantized_fixture(oracle, rng, 150, 700, 40.0, 8, 2)
    rhs = (rng.standard_normal((700, 64)) * 0.05).astype(np.float16)
    alpha, beta = 1.5, 2.0
    bias, c0 = _inputs(rng, 150, 64, kind, beta)
    ref, mag = _qcsr_referee(oracle, fx, rhs, alpha, beta, c0, kind, bias)
    y = torch.from_numpy(c0.copy()).cuda()
    ep = Epilogue(kind, alpha, beta, None if bias is None else torch.from_numpy(bias).cuda(), y)
    out = qcsr_spmm(to_device_qcsr(fx), torch.from_numpy(rhs).cuda(), out=y, epilogue=ep)
    torch.cuda.synchronize()
    assert out.data_ptr() == y.data_ptr()
    _check(oracle, ref, _magnitude(mag, alpha, beta, c0, bias), y.cpu().numpy())


def test_qcsr_identity_epilogue_is_bitwise_plain(oracle):
    torch = _torch()
    from cellerator_amd import Epilogue, qcsr_spmm
    rng = np.random.default_rng(620)
    fx = quantized_fixture(oracle, rng, 300, 1200, 80.0, 4, 1)
    rhs = torch.from_numpy((rng.standard_normal((1200, 64)) * 0.05).astype(np.float16)).cuda()
    m = to_device_qcsr(fx)
    a = qcsr_spmm(m, rhs)
    b = qcsr_spmm(m, rhs, epilogue=Epilogue())
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_qcsr_alpha_zero_is_epilogue_only(oracle):
    """alpha == 0 is the contract's epilogue-only case (operation.cc:282-292): the product is
    skipped, so even non-finite weights leave Y = act(beta * C + bias)."""
    torch = _torch()
    from cellerator_amd import Epilogue, qcsr_spmm
    rng = np.random.default_rng(630)
    fx = quantized_fixture(oracle, rng, 64, 200, 20.0, 8, 1)
    rhs = np.full((200, 64), np.inf, np.float16)
    bias = (rng.standard_normal(64)).astype(np.float32)
    c0 = rng.standard_normal((64, 64)).astype(np.float32)
    ep = Epilogue(5, 0.0, 0.5, torch.from_numpy(bias).cuda(), torch.from_numpy(c0).cuda())
    out = qcsr_spmm(to_device_qcsr(fx), torch.from_numpy(rhs).cuda(), epilogue=ep)
    torch.cuda.synchronize()
    # the referee's own arithmetic on an empty product (nnz 0, same shape)
    ref = oracle.spmm_referee(64, 200, 64, np.zeros(65, np.int64), np.zeros(0, np.uint32),
                              np.zeros(0, np.float32), np.zeros((200, 64), np.float32),
                              alpha=0.0, beta=0.5, c0=c0, epilogue=5, bias=bias)
    assert np.allclose(out.cpu().numpy(), ref, rtol=1e-6, atol=1e-6)


def test_epilogue_rejections():
    torch = _torch()
    from cellerator_amd import Epilogue, QcsrMatrix, qcsr_spmm
    from cellerator_amd._native import EngineError
    m = QcsrMatrix(2, 2, 0, torch.tensor([0, 1, 2], dtype=torch.int32).cuda(),
                   torch.tensor([0, 1], dtype=torch.int32).cuda(),
                   values=torch.ones(2, dtype=torch.float32).cuda())
    rhs = torch.ones((2, 4), dtype=torch.float32).cuda()
    bias = torch.zeros(4, dtype=torch.float32).cuda()
    out = torch.empty((2, 4), dtype=torch.float32).cuda()
    with pytest.raises(EngineError, match="INVALID_ARGUMENT"):
        qcsr_spmm(m, rhs, out=out, epilogue=Epilogue(kind=1))              # bias kind, no bias
    with pytest.raises(EngineError, match="INVALID_ARGUMENT"):
        qcsr_spmm(m, rhs, out=out, epilogue=Epilogue(kind=2, bias=bias))   # bias on a non-bias kind
    with pytest.raises(EngineError, match="INVALID_ARGUMENT"):
        qcsr_spmm(m, rhs, out=out, epilogue=Epilogue(kind=8))              # unknown kind
    with pytest.raises(EngineError, match="INVALID_ARGUMENT"):
        qcsr_spmm(m, rhs, out=out, epilogue=Epilogue(beta=1.0))            # beta without C
    big = torch.zeros((3, 4), dtype=torch.float32).cuda()
    with pytest.raises(EngineError, match="INVALID_ARGUMENT"):             # C overlaps Y, not equal
        qcsr_spmm(m, rhs, out=big[:2], epilogue=Epilogue(beta=1.0, initial=big[1:]))
    with pytest.raises(EngineError, match="INVALID_ARGUMENT"):             # bias inside Y
        qcsr_spmm(m, rhs, out=big[:2], epilogue=Epilogue(kind=1, bias=big[1]))


# ---------------------------------------------------------------- Blocked-ELL

def _bell_as_csr(idx, vals_f32, rows, cols, bs):
    """Logical CSR of a Blocked-ELL matrix (every stored slot of a valid block, zeros
    included, in slot order) for the referee."""
    width = idx.shape[1]
    row_ptr = [0]
    col_list, val_list = [], []
    for r in range(rows):
        for s in range(width):
            bc = int(idx[r // bs, s])
            if bc == 0xFFFFFFFF:
                continue
            for kk in range(bs):
                c = bc * bs + kk
                if c >= cols:
                    break
                col_list.append(c)
                val_list.append(vals_f32[r, s * bs + kk])
        row_ptr.append(len(col_list))
    return (np.array(row_ptr, np.int64), np.array(col_list, np.uint32),
            np.array(val_list, np.float32))


@pytest.mark.parametrize("kind", ALL_KINDS)
@pytest.mark.parametrize("n", [64, 256])
def test_bell_epilogue_all_paths_match_referee(oracle, kind, n):
    """Generic, per-row-block MFMA and grouped MFMA kernels with the same epilogue."""
    torch = _torch()
    from cellerator_amd import (BellMatrix, Epilogue, bell_pack_rhs, bell_plan_groups, bell_spmm,
                                bell_spmm_grouped, bell_spmm_packed)
    from tests.test_bell_gpu import _bf16_round
    from tests.test_bell_plan import patterned
    rng = np.random.default_rng(700 + kind * 7 + n)
    rb, slots, cols = 12, 6, 32 * 40 - 3
    idx = patterned(rng, rb=rb, slots=slots, patterns=3, scatter_invalid=bool(kind % 2))
    idx[idx != 0xFFFFFFFF] %= (cols + 31) // 32
    for r in range(rb):
        v = idx[r][idx[r] != 0xFFFFFFFF]
        if len(set(v.tolist())) != len(v):
            idx[r] = 0xFFFFFFFF
    rows = rb * 32 - 9
    vals = rng.standard_normal((rb * 32, slots * 32)).astype(np.float32)
    vals *= rng.random(vals.shape) < 0.4
    vbits = _bf16_round(vals)
    vf = (vbits.astype(np.uint32) << 16).view(np.float32)
    w = (rng.standard_normal((cols, n)) * 0.05).astype(np.float32)
    wbits = _bf16_round(w)
    wf = (wbits.astype(np.uint32) << 16).view(np.float32)
    alpha, beta = 1.25, 0.5
    bias, c0 = _inputs(rng, rows, n, kind, beta)
    rp, cc, cv = _bell_as_csr(idx, vf, rows, cols, 32)
    ref = oracle.spmm_referee(rows, cols, n, rp, cc, cv, wf, alpha=alpha, beta=beta, c0=c0,
                              epilogue=kind, bias=bias)
    _, mag = oracle.bell_spmm_referee(rows, cols, 32, slots * 32, idx, vbits[:rows], wbits,
                                      value_type=oracle.BF16, rhs_type=oracle.BF16)
    magnitude = _magnitude(mag, alpha, beta, c0, bias)
    m = BellMatrix(rows, cols, 32, slots * 32, torch.from_numpy(idx.view(np.int32)).cuda(),
                   values=torch.from_numpy(vbits.view(np.int16)).view(torch.bfloat16).cuda())
    rhs = torch.from_numpy(wbits.view(np.int16)).view(torch.bfloat16).cuda()
    dev = lambda a: None if a is None else torch.from_numpy(a).cuda()  # noqa: E731
    ep = Epilogue(kind, alpha, beta, dev(bias), dev(c0))
    packed = bell_pack_rhs(rhs)
    groups = bell_plan_groups(m)
    outs = [bell_spmm(m, rhs, epilogue=ep), bell_spmm_packed(m, packed, n, epilogue=ep),
            bell_spmm_grouped(m, packed, groups, n, epilogue=ep)]
    torch.cuda.synchronize()
    for out in outs:
        _check(oracle, ref, magnitude, out.cpu().numpy())
    # grouping changes which workgroup computes a row block, never its arithmetic
    assert torch.equal(outs[1].view(torch.int32), outs[2].view(torch.int32))
