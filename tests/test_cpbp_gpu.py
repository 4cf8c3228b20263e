"""GPU parity of the CP-BP feature-weighted row reduction (cx_cpbp_reduce) on tiles built by
the host builder, against the oracle's canonical referee
(components/CellPack/src/feature_weighted_row_reduction.cc:293-319).

Tolerance: the reference's own referee tolerance, 1e-5 absolute + 1e-5 relative
(components/CellPack/include/CellPack/feature_weighted_row_reduction.hh:13-14), widened by
2^-22 * sum|x*w| of the row: the kernel and the referee both accumulate in fp32 but in
different orders (tile/descriptor order vs canonical order).
"""
from __future__ import annotations

import numpy as np
import pytest

from cellerator_amd import cpbp
from tests.test_cpbp_build import random_csr, random_plan, reference_fixture, reference_plan

pytestmark = pytest.mark.gpu


def run_reduce(plan, tiles, weights):
    import torch

    from cellerator_amd import cpbp_reduce
    dev = cpbp.to_device(plan, tiles)
    out = cpbp_reduce(dev, torch.from_numpy(weights).cuda())
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check(oracle, offs, feats, vals, weights, got):
    vt = oracle.F16 if vals.dtype == np.float16 else oracle.F32
    ref, mag = oracle.cpbp_canonical_f64(offs, feats, vals, weights, vt)
    tol = 1e-5 + 1e-5 * np.abs(ref) + 2.0 ** -22 * mag
    bad = np.abs(got.astype(np.float64) - ref) > tol
    assert not bad.any(), f"{bad.sum()} rows differ, worst {np.max(np.abs(got - ref))}"


def test_reference_fixture_f16_width4(oracle):
    plan = reference_plan()
    offs, feats, vals, _ = reference_fixture()
    w = (np.arange(36, dtype=np.float32) * 0.0625 - 1.0).astype(np.float32)
    t = cpbp.build_tiles(plan, offs, feats, vals, kind=cpbp.ORDER_ROW_NNZ_DESCENDING,
                         window_size=8, group_width=4, threads=1)
    check(oracle, offs, feats, vals, w, run_reduce(plan, t, w))


def test_reference_fixture_all_empty(oracle):
    plan = reference_plan()
    offs, feats, vals, _ = reference_fixture(all_empty=True)
    w = np.ones(36, np.float32)
    t = cpbp.build_tiles(plan, offs, feats, vals, kind=cpbp.ORDER_ROW_NNZ_DESCENDING,
                         window_size=8, group_width=4, threads=1)
    assert np.array_equal(run_reduce(plan, t, w), np.zeros(5, np.float32))


@pytest.mark.parametrize("kind", [cpbp.ORDER_INFERRED_MINHASH, cpbp.ORDER_ORIGINAL,
                                  cpbp.ORDER_ROW_NNZ_DESCENDING])
@pytest.mark.parametrize("width,window,dtype", [(32, 1024, np.float16), (64, 1024, np.float32),
                                                (64, 128, np.float16), (7, 63, np.float32),
                                                (1, 16, np.float32)])
def test_random_tiles_match_canonical(oracle, kind, width, window, dtype):
    rng = np.random.default_rng(1000 + kind * 10 + width)
    plan = random_plan(rng, 700)
    offs, feats, vals = random_csr(rng, 1500, 700, 30.0, dtype)
    w = rng.standard_normal(700).astype(np.float32)
    t = cpbp.build_tiles(plan, offs, feats, vals, kind=kind, window_size=window,
                         group_width=width, threads=4)
    check(oracle, offs, feats, vals, w, run_reduce(plan, t, w))


def test_c5_sample_width64(oracle):
    """Config-5 distributions at 20,000 cells: module-aligned 25-gene blocks, minhash order,
    64-row tiles with u64 cell masks, fp32 values."""
    from cellerator_amd.synth import C5, generate_cpbp_host
    cfg = C5.scaled(20_000)
    offs, feats, vals = generate_cpbp_host(cfg)
    plan = cpbp.contiguous_plan(cfg.genes, cfg.block_width)
    t = cpbp.build_tiles(plan, offs, feats, vals, group_width=64, window_size=1024)
    assert t.req["cell_mask_bytes"] == 8
    w = np.random.default_rng(5).standard_normal(cfg.genes).astype(np.float32)
    check(oracle, offs, feats, vals, w, run_reduce(plan, t, w))


def test_repeat_is_bitwise_deterministic():
    rng = np.random.default_rng(3)
    plan = random_plan(rng, 400)
    offs, feats, vals = random_csr(rng, 900, 400, 25.0, np.float32)
    w = rng.standard_normal(400).astype(np.float32)
    t = cpbp.build_tiles(plan, offs, feats, vals, group_width=64, window_size=512)
    a = run_reduce(plan, t, w)
    b = run_reduce(plan, t, w)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def with_empty_descriptors(tiles, spots):
    """Copy of host tiles with a descriptor of no cells (cell mask 0, so no entries)
    inserted before descriptor `k` of tile `t` for each (t, k) in spots (k may be the
    tile's descriptor count: after its last one)."""
    import copy
    out = copy.deepcopy(tiles)
    for t, k in sorted(spots, reverse=True):
        d = int(out.tile_block_offsets[t]) + k
        assert d <= int(out.tile_block_offsets[t + 1])
        out.tile_block_ids = np.insert(out.tile_block_ids, d, out.tile_block_ids[max(d - 1, 0)])
        out.tile_block_cell_masks = np.insert(out.tile_block_cell_masks, d, 0)
        out.block_row_entry_offsets = np.insert(out.block_row_entry_offsets, d, out.block_row_entry_offsets[d])
        out.tile_block_offsets = out.tile_block_offsets.copy()
        out.tile_block_offsets[t + 1:] += 1
    out.req = dict(out.req, tile_block_count=int(out.tile_block_offsets[-1]))
    return out


@pytest.mark.parametrize("width,dtype", [(64, np.float32), (32, np.float16)])
def test_descriptors_without_cells(oracle, width, dtype):
    """A descriptor whose cell mask is 0 starts at the same entry as the next one and holds
    no entries; it contributes nothing, wherever it sits in a tile (first, between two
    descriptors, two in a row, last): the product is bitwise the one without it."""
    rng = np.random.default_rng(width)
    plan = random_plan(rng, 300)
    offs, feats, vals = random_csr(rng, 6 * width, 300, 20.0, dtype)
    w = rng.standard_normal(300).astype(np.float32)
    t = cpbp.build_tiles(plan, offs, feats, vals, group_width=width, window_size=256)
    counts = np.diff(t.tile_block_offsets)
    assert len(counts) >= 4 and (counts[:4] >= 3).all()
    spots = [(0, 0), (1, int(counts[1]) // 2), (2, 1), (2, 1), (3, int(counts[3]))]
    e = with_empty_descriptors(t, spots)
    assert int(e.tile_block_offsets[-1]) == int(t.tile_block_offsets[-1]) + len(spots)
    base = run_reduce(plan, t, w)
    got = run_reduce(plan, e, w)
    assert np.array_equal(got.view(np.uint32), base.view(np.uint32))
    check(oracle, offs, feats, vals, w, got)
