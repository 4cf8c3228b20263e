"""GPU parity of the Blocked-ELL SpMM kernels (generic and MFMA) against the oracle."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import check_against_referee

pytestmark = pytest.mark.gpu


def _bf16_round(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits (RNE) as uint16."""
    x = a.astype(np.float32).view(np.uint32)
    x = x + 0x7FFF + ((x >> 16) & 1)
    return (x >> 16).astype(np.uint16)


def random_bell(rng, rows, cols, bs, width, density=0.35):
    rb = rows // bs
    kb = (cols + bs - 1) // bs
    idx = np.full((rb, width), 0xFFFFFFFF, np.uint32)
    for b in range(rb):
        c = rng.integers(0, width + 1)
        idx[b, :c] = np.sort(rng.choice(kb, size=min(c, kb), replace=False))
    vals = rng.standard_normal((rows, width * bs)).astype(np.float32)
    vals *= rng.random(vals.shape) < density
    return idx, vals


def test_generic_sparse_ops_fixture():
    import torch

    from cellerator_amd import BellMatrix, bell_spmm
    idx = torch.tensor([[0, 2], [1, 2], [0, -1]], dtype=torch.int32).cuda()
    vals = torch.tensor([[1, 2], [3, 4], [5, 0]], dtype=torch.float16).cuda()
    m = BellMatrix(3, 3, 1, 2, idx, values=vals)
    rhs = torch.tensor([[1, 2], [10, 20], [100, 200]], dtype=torch.float32).cuda()
    out = bell_spmm(m, rhs)
    torch.cuda.synchronize()
    assert out.cpu().numpy().ravel().tolist() == [201.0, 402.0, 430.0, 860.0, 5.0, 10.0]


@pytest.mark.parametrize("n", [64, 128, 256])
def test_mfma_matches_referee(oracle, n):
    import torch

    from cellerator_amd import BellMatrix, bell_pack_rhs, bell_spmm, bell_spmm_packed
    rng = np.random.default_rng(n)
    rows, cols, bs, width = 32 * 37, 1000, 32, 9  # cols not a multiple of 32
    idx, vals = random_bell(rng, rows, cols, bs, width)
    vbits = _bf16_round(vals)
    w = (rng.standard_normal((cols, n)) * 0.02).astype(np.float32)
    wbits = _bf16_round(w)
    ref, mag = oracle.bell_spmm_referee(rows, cols, bs, width * bs, idx, vbits, wbits,
                                        value_type=oracle.BF16, rhs_type=oracle.BF16)
    m = BellMatrix(rows, cols, bs, width * bs, torch.from_numpy(idx.view(np.int32)).cuda(),
                   values=torch.from_numpy(vbits.view(np.int16)).view(torch.bfloat16).cuda())
    rhs = torch.from_numpy(wbits.view(np.int16)).view(torch.bfloat16).cuda()
    packed = bell_pack_rhs(rhs)
    out = bell_spmm_packed(m, packed, n)
    generic = bell_spmm(m, rhs)
    torch.cuda.synchronize()
    check_against_referee(oracle, ref, mag, out.cpu().numpy())
    check_against_referee(oracle, ref, mag, generic.cpu().numpy())


@pytest.mark.parametrize("bits,policy", [(8, 1), (4, 2), (2, 1), (1, 2)])
def test_quantized_bell_generic(oracle, bits, policy):
    import torch

    from cellerator_amd import BellMatrix, bell_spmm
    rng = np.random.default_rng(bits * 7 + policy)
    rows, cols, bs, width = 48, 70, 8, 4
    idx, _ = random_bell(rng, rows, cols, bs, width)
    ell_cols = width * bs
    stride = (ell_cols * bits + 7) // 8
    packed = rng.integers(0, 256, size=rows * stride).astype(np.uint8)
    scales = rng.uniform(0.1, 0.5, cols).astype(np.float32)
    offsets = rng.uniform(-0.5, 0.5, cols).astype(np.float32)
    row_off = rng.uniform(-1, 1, rows).astype(np.float32)
    rhs = rng.standard_normal((cols, 16)).astype(np.float32)
    ref, mag = oracle.bell_spmm_referee(rows, cols, bs, ell_cols, idx, None, rhs, bits=bits,
                                        policy=policy, row_stride_bytes=stride, packed=packed,
                                        scales=scales, offsets=offsets if policy == 1 else None,
                                        row_offsets=row_off if policy == 2 else None)
    t = lambda a: None if a is None else torch.from_numpy(a).cuda()  # noqa: E731
    m = BellMatrix(rows, cols, bs, ell_cols, t(idx.view(np.int32)), bits=bits,
                   decode_policy=policy, row_stride_bytes=stride, packed_values=t(packed),
                   column_scales=t(scales), column_offsets=t(offsets) if policy == 1 else None,
                   row_offsets=t(row_off) if policy == 2 else None)
    out = bell_spmm(m, t(rhs))
    torch.cuda.synchronize()
    check_against_referee(oracle, ref, mag, out.cpu().numpy())


def test_generated_c4_sample(oracle):
    import torch

    from cellerator_amd import bell_pack_rhs, bell_spmm_packed
    from cellerator_amd.synth import C4, dense_normal, generate_bell
    m = generate_bell(C4.scaled(32 * 64))
    w = dense_normal((m.cols, 256), 0.02, torch.bfloat16, seed=C4.seed + 1)
    out = bell_spmm_packed(m, bell_pack_rhs(w), 256)
    torch.cuda.synchronize()
    idx = m.block_col_idx.cpu().numpy().view(np.uint32)
    valid = (idx != 0xFFFFFFFF).sum(axis=1)
    assert valid.min() >= 24 and valid.max() <= 64
    ref, mag = oracle.bell_spmm_referee(m.rows, m.cols, 32, m.ell_cols, idx,
                                        m.values.view(torch.int16).cpu().numpy().view(np.uint16),
                                        w.view(torch.int16).cpu().numpy().view(np.uint16),
                                        value_type=oracle.BF16, rhs_type=oracle.BF16)
    check_against_referee(oracle, ref, mag, out.cpu().numpy())


@pytest.mark.parametrize("n", [64, 128, 256])
@pytest.mark.parametrize("scatter", [False, True])
@pytest.mark.parametrize("schedule", [True, False])
def test_grouped_mfma_equals_ungrouped_and_referee(oracle, n, scatter, schedule):
    """Grouped path is bitwise equal to the per-row-block MFMA kernel (same slot order per
    output) and within tolerance of the float64 referee, with valid slots contiguous or
    scattered among empty ones: the planner's groups + singletons, and its launch schedule
    (singles folded in as one-member groups, units dealt over the XCD ranges)."""
    import torch

    from cellerator_amd import (BellMatrix, bell_pack_rhs, bell_plan_groups, bell_spmm_grouped,
                                bell_spmm_packed)
    from tests.test_bell_plan import patterned
    rng = np.random.default_rng(900 + n + scatter)
    rb, slots, cols = 60, 16, 32 * 500 - 7  # K not a multiple of 32
    idx = patterned(rng, rb=rb, slots=slots, patterns=5, scatter_invalid=scatter)
    idx[:, :][idx != 0xFFFFFFFF] %= (cols + 31) // 32
    # keep each row's valid columns distinct after the modulo
    for r in range(rb):
        v = idx[r][idx[r] != 0xFFFFFFFF]
        if len(set(v.tolist())) != len(v):
            idx[r] = 0xFFFFFFFF
    rows = rb * 32 - 5  # ragged last row block
    vals = rng.standard_normal((rb * 32, slots * 32)).astype(np.float32)
    vals *= rng.random(vals.shape) < 0.35
    vbits = _bf16_round(vals)
    w = (rng.standard_normal((cols, n)) * 0.02).astype(np.float32)
    wbits = _bf16_round(w)
    m = BellMatrix(rows, cols, 32, slots * 32, torch.from_numpy(idx.view(np.int32)).cuda(),
                   values=torch.from_numpy(vbits.view(np.int16)).view(torch.bfloat16).cuda())
    rhs = torch.from_numpy(wbits.view(np.int16)).view(torch.bfloat16).cuda()
    packed = bell_pack_rhs(rhs)
    groups = bell_plan_groups(m, schedule=schedule)
    assert groups.group_count > 0 and groups.grouped_row_blocks + groups.single_count == rb
    if schedule:
        assert groups.single_count == 0 and groups.group_count == groups.planned_groups + groups.planned_singles
        assert groups.group_count >= 8 and groups.planned_singles > 0
    a = bell_spmm_packed(m, packed, n)
    b = bell_spmm_grouped(m, packed, groups, n)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    ref, mag = oracle.bell_spmm_referee(rows, cols, 32, slots * 32, idx, vbits[:rows], wbits,
                                        value_type=oracle.BF16, rhs_type=oracle.BF16)
    check_against_referee(oracle, ref, mag, b.cpu().numpy())


def test_grouped_rejects_groups_that_do_not_cover():
    import torch

    from cellerator_amd import BellGroups, BellMatrix, bell_pack_rhs, bell_spmm_grouped
    from cellerator_amd._native import EngineError
    idx = torch.zeros((2, 1), dtype=torch.int32).cuda()
    m = BellMatrix(64, 32, 32, 32, idx, values=torch.zeros((64, 32), dtype=torch.bfloat16).cuda())
    packed = bell_pack_rhs(torch.zeros((32, 64), dtype=torch.bfloat16).cuda())
    bad = BellGroups(0, 0, 1, torch.zeros(2, dtype=torch.int32).cuda(), torch.zeros(1, dtype=torch.int32).cuda())
    with pytest.raises(EngineError, match="INVALID_SHAPE"):
        bell_spmm_grouped(m, packed, bad, 64)


def test_ordered_entry_rejects_a_null_order():
    import ctypes

    import torch

    from cellerator_amd import BellMatrix
    from cellerator_amd import _native as N
    idx = torch.zeros((2, 1), dtype=torch.int32).cuda()
    m = BellMatrix(64, 32, 32, 32, idx, bits=8, decode_policy=1, row_stride_bytes=32,
                   packed_values=torch.zeros(64 * 32, dtype=torch.uint8).cuda(),
                   column_scales=torch.ones(32).cuda(), column_offsets=torch.zeros(32).cuda())
    w = torch.zeros((32, 64)).cuda()
    out = torch.empty((64, 64)).cuda()
    d = m.descriptor()
    assert N.engine().cx_bell_spmm_fwd_ordered(ctypes.byref(d), w.data_ptr(), 2, 64, 64, out.data_ptr(), 64,
                                               None, None) == 1
    assert b"null row-block order" in N.engine().cx_last_error()


def _quantized_bell_32(rng, rows, cols, width, bits, policy):
    """32x32 blocks, ragged last row block and block column, invalid slots anywhere."""
    rb, kb = (rows + 31) // 32, (cols + 31) // 32
    idx = np.full((rb, width), 0xFFFFFFFF, np.uint32)
    for b in range(rb):
        c = int(rng.integers(1 if b == 0 else 0, min(width, kb) + 1))
        picks = np.sort(rng.choice(kb, size=c, replace=False))
        if b == 0 and kb - 1 not in picks:
            picks[-1] = kb - 1  # the ragged block column in use (each block column once per row block)
        where = np.sort(rng.choice(width, size=c, replace=False))
        idx[b, where] = np.sort(picks)
    stride = width * 32 * bits // 8
    packed = rng.integers(0, 256, size=rows * stride).astype(np.uint8)
    scales = rng.uniform(0.1, 0.5, cols).astype(np.float32)
    offsets = rng.uniform(-0.5, 0.5, cols).astype(np.float32)
    row_off = rng.uniform(-1, 1, rows).astype(np.float32)
    return idx, stride, packed, scales, offsets, row_off


@pytest.mark.parametrize("bits,policy,n", [(8, 1, 256), (4, 2, 64), (2, 1, 128), (1, 2, 64), (8, 2, 192)])
def test_quantized_bell_matrix_cores(oracle, bits, policy, n):
    """Quantized Blocked-ELL with 32x32 blocks and f32 W runs on the fp32 matrix cores
    (bell_spmm_quant_lds, W tiles and metadata through LDS): within the bound of the float64
    referee for every width and policy, ragged row block and block column, invalid slots
    anywhere; a one-hot W returns every decoded value bitwise (the codec's fma(code, scale,
    offset)); a fused epilogue applies. W at an address and row stride that are not whole
    16-byte units takes the register form (bell_spmm_quant_mfma): bitwise the same sums."""
    import torch

    from cellerator_amd import BellMatrix, Epilogue, bell_spmm
    rng = np.random.default_rng(100 * bits + 10 * policy + n)
    rows, cols, width = 75, 70, 4
    idx, stride, packed, scales, offsets, row_off = _quantized_bell_32(rng, rows, cols, width, bits, policy)
    t = lambda a: None if a is None else torch.from_numpy(a).cuda()  # noqa: E731
    m = BellMatrix(rows, cols, 32, width * 32, t(idx.view(np.int32)), bits=bits, decode_policy=policy,
                   row_stride_bytes=stride, packed_values=t(packed), column_scales=t(scales),
                   column_offsets=t(offsets) if policy == 1 else None, row_offsets=t(row_off) if policy == 2 else None)
    kw = dict(bits=bits, policy=policy, row_stride_bytes=stride, packed=packed, scales=scales,
              offsets=offsets if policy == 1 else None, row_offsets=row_off if policy == 2 else None)
    rhs = rng.standard_normal((cols, n)).astype(np.float32)
    ref, mag = oracle.bell_spmm_referee(rows, cols, 32, width * 32, idx, None, rhs, **kw)
    out = bell_spmm(m, t(rhs))
    # one-hot W: column c reads gene c % cols
    onehot = np.zeros((cols, n), np.float32)
    onehot[np.arange(n) % cols, np.arange(n)] = 1.0
    dec, _ = oracle.bell_spmm_referee(rows, cols, 32, width * 32, idx, None, onehot, **kw)
    hot = bell_spmm(m, t(onehot))
    bias = rng.standard_normal(n).astype(np.float32)
    ep_out = bell_spmm(m, t(rhs), epilogue=Epilogue(kind=1, bias=t(bias)))  # bias
    wide = torch.zeros((cols, n + 1), dtype=torch.float32, device="cuda")
    wide[:, 1:] = t(rhs)
    unaligned = bell_spmm(m, wide[:, 1:])  # 4 bytes past a 16-byte boundary, row stride n + 1
    # row blocks taken in another order (cx_bell_spmm_fwd_ordered), both operand forms
    rb = (rows + 31) // 32
    order = t(np.random.default_rng(7).permutation(rb).astype(np.int32))
    ordered = bell_spmm(m, t(rhs), row_block_order=order)
    ordered_unaligned = bell_spmm(m, wide[:, 1:], row_block_order=order)
    torch.cuda.synchronize()
    check_against_referee(oracle, ref, mag, out.cpu().numpy())
    assert torch.equal(unaligned.view(torch.int32), out.view(torch.int32))
    assert torch.equal(ordered.view(torch.int32), out.view(torch.int32))
    assert torch.equal(ordered_unaligned.view(torch.int32), out.view(torch.int32))
    assert np.array_equal(hot.cpu().numpy().astype(np.float64), dec)
    check_against_referee(oracle, ref + bias[None, :].astype(np.float64), mag, ep_out.cpu().numpy())
