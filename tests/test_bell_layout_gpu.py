"""Blocked-ELL operand layouts on the GPU: the fragment-order weight panel
(cx_bell_pack_rhs), block-major values (cx_bell_block_major_values,
CX_BELL_BLOCK_MAJOR_VALUES) against numpy restatements, and every Blocked-ELL entry point
giving bitwise the same results on block-major values as on row-major ones."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import check_against_referee
from tests.test_bell_gpu import _bf16_round, random_bell

pytestmark = pytest.mark.gpu


def _panel_restatement(wbits: np.ndarray) -> np.ndarray:
    """Fragment order: element ((tile * 2 + half) * 64 + lane) * 8 + i of block column kb is
    W[32 kb + 16 half + 8 (lane // 32) + i, 32 tile + lane % 32] (0 past K)."""
    k, n = wbits.shape
    kb = (k + 31) // 32
    padded = np.zeros((kb * 32, n), np.uint16)
    padded[:k] = wbits
    out = np.zeros((kb, n // 32, 2, 64, 8), np.uint16)
    for lane in range(64):
        for i in range(8):
            for half in range(2):
                genes = np.arange(kb) * 32 + 16 * half + 8 * (lane // 32) + i
                for tile in range(n // 32):
                    out[:, tile, half, lane, i] = padded[genes, 32 * tile + lane % 32]
    return out.ravel()


@pytest.mark.parametrize("k,n", [(1000, 64), (64, 128), (77, 256)])
def test_pack_rhs_fragment_order(k, n):
    import torch

    from cellerator_amd import bell_pack_rhs
    rng = np.random.default_rng(k + n)
    wbits = _bf16_round(rng.standard_normal((k, n)).astype(np.float32))
    packed = bell_pack_rhs(torch.from_numpy(wbits.view(np.int16)).view(torch.bfloat16).cuda())
    got = packed.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got, _panel_restatement(wbits))


def test_pack_rhs_rejects_columns_not_multiple_of_32():
    import torch

    from cellerator_amd import bell_pack_rhs
    from cellerator_amd._native import EngineError
    with pytest.raises(EngineError, match="INVALID_SHAPE"):
        bell_pack_rhs(torch.zeros((64, 48), dtype=torch.bfloat16).cuda())


@pytest.mark.parametrize("bs,dtype", [(32, "bf16"), (16, "f16"), (8, "f32"), (32, "f32")])
def test_block_major_values_layout(bs, dtype):
    import torch

    from cellerator_amd import BellMatrix, bell_block_major
    rng = np.random.default_rng(bs * 7 + len(dtype))
    rows, width = bs * 11 - 3, 5  # ragged last row block
    vals = rng.standard_normal((rows, width * bs)).astype(np.float32)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    idx = torch.zeros(((rows + bs - 1) // bs, width), dtype=torch.int32).cuda()
    m = BellMatrix(rows, 8 * bs, bs, width * bs, idx, values=torch.from_numpy(vals).to(tdt).cuda())
    bm = bell_block_major(m)
    torch.cuda.synchronize()
    assert bm.block_major and bm.values.shape == (11, width, bs, bs)
    src = m.values.cpu()
    want = torch.zeros((11 * bs, width * bs), dtype=tdt)
    want[:rows] = src
    want = want.reshape(11, bs, width, bs).permute(0, 2, 1, 3)
    assert torch.equal(bm.values.cpu(), want)
    with pytest.raises(ValueError):
        bell_block_major(bm)


@pytest.mark.parametrize("n", [64, 128, 256])
def test_block_major_equals_row_major(oracle, n):
    """Per-row-block and grouped MFMA kernels, and the generic kernel, give bitwise the same
    output on block-major values as on row-major ones (ragged last row block, scattered
    empty slots), and the block-major output is within the referee's tolerance."""
    import torch

    from cellerator_amd import (BellMatrix, Epilogue, bell_block_major, bell_pack_rhs, bell_plan_groups,
                                bell_spmm, bell_spmm_grouped, bell_spmm_packed)
    from tests.test_bell_plan import patterned
    rng = np.random.default_rng(4100 + n)
    rb, slots, cols = 40, 12, 32 * 300 - 9
    idx = patterned(rng, rb=rb, slots=slots, patterns=4, scatter_invalid=True)
    idx[idx != 0xFFFFFFFF] %= (cols + 31) // 32
    for r in range(rb):
        v = idx[r][idx[r] != 0xFFFFFFFF]
        if len(set(v.tolist())) != len(v):
            idx[r] = 0xFFFFFFFF
    rows = rb * 32 - 11
    vals = rng.standard_normal((rows, slots * 32)).astype(np.float32)
    vals *= rng.random(vals.shape) < 0.35
    vbits = _bf16_round(vals)
    wbits = _bf16_round((rng.standard_normal((cols, n)) * 0.02).astype(np.float32))
    m = BellMatrix(rows, cols, 32, slots * 32, torch.from_numpy(idx.view(np.int32)).cuda(),
                   values=torch.from_numpy(vbits.view(np.int16)).view(torch.bfloat16).cuda())
    bm = bell_block_major(m)
    rhs = torch.from_numpy(wbits.view(np.int16)).view(torch.bfloat16).cuda()
    packed = bell_pack_rhs(rhs)
    groups = bell_plan_groups(m)
    pairs = [(bell_spmm_packed(m, packed, n), bell_spmm_packed(bm, packed, n)),
             (bell_spmm_grouped(m, packed, groups, n), bell_spmm_grouped(bm, packed, groups, n)),
             (bell_spmm(m, rhs), bell_spmm(bm, rhs))]
    bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).cuda()
    from cellerator_amd import _native as N
    ep = Epilogue(kind=N.EPILOGUE_BIAS_RELU, bias=bias)
    pairs.append((bell_spmm_grouped(m, packed, groups, n, epilogue=ep),
                  bell_spmm_grouped(bm, packed, groups, n, epilogue=ep)))
    torch.cuda.synchronize()
    for a, b in pairs:
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert torch.equal(pairs[0][1].view(torch.int32), pairs[1][1].view(torch.int32))
    ref, mag = oracle.bell_spmm_referee(rows, cols, 32, slots * 32, idx, vbits, wbits,
                                        value_type=oracle.BF16, rhs_type=oracle.BF16)
    check_against_referee(oracle, ref, mag, pairs[1][1].cpu().numpy())


def test_generic_block_major_small_blocks(oracle):
    """The reference-semantics kernel at block size 16 with fp32 values, block-major against
    row-major (bitwise) and against the referee."""
    import torch

    from cellerator_amd import BellMatrix, bell_block_major, bell_spmm
    rng = np.random.default_rng(77)
    rows, cols, bs, width = 16 * 23 - 5, 700, 16, 7
    idx, vals = random_bell(rng, 16 * 23, cols, bs, width)
    vals = vals[:rows]
    w = (rng.standard_normal((cols, 40)) * 0.1).astype(np.float32)
    m = BellMatrix(rows, cols, bs, width * bs, torch.from_numpy(idx.view(np.int32)).cuda(),
                   values=torch.from_numpy(vals).cuda())
    bm = bell_block_major(m)
    wt = torch.from_numpy(w).cuda()
    a, b = bell_spmm(m, wt), bell_spmm(bm, wt)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    ref, mag = oracle.bell_spmm_referee(rows, cols, bs, width * bs, idx, vals, w,
                                        value_type=oracle.F32, rhs_type=oracle.F32)
    check_against_referee(oracle, ref, mag, b.cpu().numpy())


def test_layout_flag_rejections():
    import torch

    from cellerator_amd import BellMatrix, bell_spmm
    from cellerator_amd import _native as N
    from cellerator_amd._native import EngineError
    idx = torch.zeros((2, 1), dtype=torch.int32).cuda()
    m = BellMatrix(64, 32, 32, 32, idx, values=torch.zeros((64, 32), dtype=torch.bfloat16).cuda())
    rhs = torch.zeros((32, 64), dtype=torch.float32).cuda()
    out = torch.empty((64, 64), dtype=torch.float32).cuda()
    import ctypes as C
    d = m.descriptor()
    d.value_layout_flags = 2  # unknown flag
    rc = N.engine().cx_bell_spmm_fwd(C.byref(d), rhs.data_ptr(), N.DTYPE_F32, 64, 64, out.data_ptr(), 64, None)
    assert rc == 1  # INVALID_ARGUMENT
    q = BellMatrix(64, 32, 32, 32, idx, bits=4, row_stride_bytes=16,
                   packed_values=torch.zeros(64 * 16, dtype=torch.uint8).cuda(),
                   column_scales=torch.ones(32).cuda(), column_offsets=torch.zeros(32).cuda(),
                   block_major=True)
    with pytest.raises(EngineError, match="UNSUPPORTED"):
        bell_spmm(q, rhs)
