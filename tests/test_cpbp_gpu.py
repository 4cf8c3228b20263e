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


def host_entry_rows(plan, t):
    """Every entry's block start << 6 | tile row, restated on the host from the descriptors:
    the k-th entry of descriptor d sits in the tile row of the k-th set bit of d's cell mask
    (warp_tiles.hh:49-79), its block starts at feature_block_offsets[block id]."""
    fbo = plan.feature_block_offsets.astype(np.int64)
    fc = int(plan.feature_permutation.size)
    out = np.zeros(int(t.row_block_gene_masks.size), np.uint32)
    eo = t.block_row_entry_offsets.astype(np.int64)
    for d in range(int(t.tile_block_ids.size)):
        m = int(t.tile_block_cell_masks[d])
        rows = [b for b in range(64) if (m >> b) & 1]
        bb = min(int(fbo[min(int(t.tile_block_ids[d]), fbo.size - 1)]), fc)
        for k, e in enumerate(range(eo[d], eo[d + 1])):
            out[e] = (bb << 6) | rows[k]
    return out


@pytest.mark.parametrize("width,window,dtype", [(64, 1024, np.float32), (32, 1024, np.float16),
                                                (7, 63, np.float32), (1, 16, np.float16)])
def test_entry_rows_and_reduce_rows(oracle, width, window, dtype):
    """cx_cpbp_entry_rows equals the host restatement entry for entry, and cx_cpbp_reduce_rows
    over it is bitwise the reduction from the descriptors (same batches, same order)."""
    import torch

    from cellerator_amd import cpbp_entry_rows, cpbp_reduce, cpbp_reduce_rows
    rng = np.random.default_rng(2000 + width)
    plan = random_plan(rng, 700)
    offs, feats, vals = random_csr(rng, 1500, 700, 30.0, dtype)
    w = rng.standard_normal(700).astype(np.float32)
    t = cpbp.build_tiles(plan, offs, feats, vals, window_size=window, group_width=width, threads=4)
    dev = cpbp.to_device(plan, t)
    rows = cpbp_entry_rows(dev)
    n = int(t.row_block_gene_masks.size)
    assert np.array_equal(rows.cpu().numpy()[:n].view(np.uint32), host_entry_rows(plan, t))
    wd = torch.from_numpy(w).cuda()
    a = cpbp_reduce(dev, wd)
    b = cpbp_reduce_rows(dev, rows, wd)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    check(oracle, offs, feats, vals, w, b.cpu().numpy())


def test_reduce_rows_c5_sample(oracle):
    """Config-5 distributions at 20,000 cells through the per-entry rows: parity with the
    canonical referee and bitwise equal to the descriptor walk."""
    import torch

    from cellerator_amd import cpbp_entry_rows, cpbp_reduce, cpbp_reduce_rows
    from cellerator_amd.synth import C5, generate_cpbp_host
    cfg = C5.scaled(20_000)
    offs, feats, vals = generate_cpbp_host(cfg)
    plan = cpbp.contiguous_plan(cfg.genes, cfg.block_width)
    t = cpbp.build_tiles(plan, offs, feats, vals, group_width=64, window_size=1024)
    dev = cpbp.to_device(plan, t)
    rows = cpbp_entry_rows(dev)
    w = np.random.default_rng(6).standard_normal(cfg.genes).astype(np.float32)
    wd = torch.from_numpy(w).cuda()
    a = cpbp_reduce(dev, wd)
    b = cpbp_reduce_rows(dev, rows, wd)
    c = cpbp_reduce_rows(dev, rows, wd)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    assert torch.equal(b.view(torch.int32), c.view(torch.int32))
    check(oracle, offs, feats, vals, w, b.cpu().numpy())


def test_entry_rows_rejects_bad_arguments():
    import ctypes

    import torch

    from cellerator_amd import _native as N
    from cellerator_amd import cpbp_entry_rows, cpbp_reduce_rows
    rng = np.random.default_rng(77)
    plan = random_plan(rng, 100)
    offs, feats, vals = random_csr(rng, 200, 100, 10.0, np.float32)
    t = cpbp.build_tiles(plan, offs, feats, vals, window_size=64, group_width=32, threads=1)
    dev = cpbp.to_device(plan, t)
    n = int(t.row_block_gene_masks.size)
    with pytest.raises(N.EngineError, match="capacity"):
        cpbp_entry_rows(dev, out=torch.empty(n - 1, dtype=torch.int32, device="cuda"))
    rows = cpbp_entry_rows(dev)
    w = torch.ones(100, device="cuda")
    out = torch.empty(dev.row_count, device="cuda")
    d = dev.descriptor()
    lib = N.engine()
    assert lib.cx_cpbp_reduce_rows(ctypes.byref(d), None, w.data_ptr(), w.numel(), out.data_ptr(),
                                   out.numel(), None) == 1
    assert b"null entry rows" in lib.cx_last_error()
    # the output may not alias the entry rows
    assert lib.cx_cpbp_reduce_rows(ctypes.byref(d), rows.data_ptr(), w.data_ptr(), w.numel(), rows.data_ptr(),
                                   dev.row_count, None) == 1
    assert b"aliases" in lib.cx_last_error()
    with pytest.raises(ValueError):
        cpbp_reduce_rows(dev, rows[: n - 1], w)
