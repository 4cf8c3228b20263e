"""CP-BP host construction (cx_cpbp_builder_*): canonical CSR -> records -> local order ->
warp tiles. CPU tests: no GPU is touched.

Pins:
  * the reference fixture of components/CellPack/tests/feature_weighted_row_reduction_cuda_test.cu:69-151
    (36-feature plan: execution features 0..31 are canonical 31..0, 32..35 are
    canonical 35, 32, 34, 33; blocks [0, 32) and [32, 36); 5-row partition; order
    row_nnz_descending, window 8, group width 4). Its tiles follow from the reference
    algorithm by hand and are written out below;
  * exact round trip: decoding the tiles gives back every (row, feature, value);
  * the output is identical for every thread count;
  * order invariants: rows never leave their window and are sorted by
    (primary, secondary, row) inside it; equal block sets give equal minhash keys;
  * the tile referee over the built tiles agrees with the canonical referee
    (feature_weighted_row_reduction.hh:13-14 tolerance).
"""
from __future__ import annotations

import numpy as np
import pytest

from cellerator_amd import cpbp
from cellerator_amd import _native as N


def reference_plan() -> cpbp.Plan:
    perm = [31 - i for i in range(32)] + [35, 32, 34, 33]
    return cpbp.Plan(np.asarray(perm, np.uint32), np.asarray([0, 32, 36], np.uint32))


def reference_fixture(all_empty: bool = False):
    rows = [[] for _ in range(5)]
    if not all_empty:
        rows[0] = list(range(32)) + [35]
        rows[2] = [0, 5, 31, 32, 35]
        rows[3] = [3, 7]
        rows[4] = [31]
    offs, feats, vals = [0], [], []
    for r, fs in enumerate(rows):
        for f in fs:
            sign = 1.0 if (r + f) % 2 == 0 else -1.0
            feats.append(f)
            vals.append(sign * (0.25 + 0.125 * f))
        offs.append(len(feats))
    return (np.asarray(offs, np.uint32), np.asarray(feats, np.uint32),
            np.asarray(vals, np.float32).astype(np.float16), rows)


def value_of(row: int, feature: int) -> np.float16:
    sign = 1.0 if (row + feature) % 2 == 0 else -1.0
    return np.float16(sign * (0.25 + 0.125 * feature))


def test_reference_fixture_tiles():
    plan = reference_plan()
    offs, feats, vals, rows = reference_fixture()
    t = cpbp.build_tiles(plan, offs, feats, vals, kind=cpbp.ORDER_ROW_NNZ_DESCENDING,
                         window_size=8, group_width=4, threads=1)
    # row nnz 33, 0, 5, 2, 1 -> descending: canonical rows 0, 2, 3, 4, then the empty row 1
    assert t.row_permutation.tolist() == [0, 2, 3, 4, 1]
    assert t.req["tile_count"] == 2 and t.req["cell_mask_bytes"] == 4
    assert t.tile_block_offsets.tolist() == [0, 2, 2]
    assert t.tile_block_ids.tolist() == [0, 1]
    assert t.tile_block_cell_masks.tolist() == [0b1111, 0b0011]
    # block 0 locals are 31 - canonical; block 1 locals: canonical 35 -> 0, 32 -> 1
    assert t.row_block_gene_masks.tolist() == [
        0xFFFFFFFF, (1 << 0) | (1 << 26) | (1 << 31), (1 << 24) | (1 << 28), 1 << 0,
        0b01, 0b11]
    assert t.block_row_entry_offsets.tolist() == [0, 4, 6]
    assert t.row_block_value_offsets.tolist() == [0, 32, 35, 37, 38, 39, 41]
    expect = ([value_of(0, 31 - k) for k in range(32)] + [value_of(2, 31), value_of(2, 5), value_of(2, 0)]
              + [value_of(3, 7), value_of(3, 3)] + [value_of(4, 31)] + [value_of(0, 35)]
              + [value_of(2, 35), value_of(2, 32)])
    assert t.values.tolist() == [float(v) for v in expect]


def test_reference_fixture_all_empty():
    plan = reference_plan()
    offs, feats, vals, _ = reference_fixture(all_empty=True)
    t = cpbp.build_tiles(plan, offs, feats, vals, kind=cpbp.ORDER_ROW_NNZ_DESCENDING,
                         window_size=8, group_width=4, threads=1)
    assert t.req["tile_block_count"] == 0 and t.req["nnz_count"] == 0
    assert t.tile_block_offsets.tolist() == [0, 0, 0]
    assert t.row_permutation.tolist() == [0, 1, 2, 3, 4]


def random_plan(rng, features: int) -> cpbp.Plan:
    perm = rng.permutation(features).astype(np.uint32)
    offs = [0]
    while offs[-1] < features:
        offs.append(min(features, offs[-1] + int(rng.integers(1, 33))))
    return cpbp.Plan(perm, np.asarray(offs, np.uint32))


def random_csr(rng, rows: int, features: int, mean_nnz: float, dtype):
    counts = np.minimum(rng.poisson(mean_nnz, rows), features)
    counts[rng.random(rows) < 0.1] = 0  # empty rows
    offs = np.zeros(rows + 1, np.uint32)
    offs[1:] = np.cumsum(counts)
    feats = np.concatenate([np.sort(rng.choice(features, c, replace=False)) for c in counts]
                           ) if counts.sum() else np.zeros(0, np.uint32)
    vals = rng.standard_normal(int(counts.sum())).astype(dtype)
    return offs, feats.astype(np.uint32), vals


@pytest.mark.parametrize("kind", [cpbp.ORDER_INFERRED_MINHASH, cpbp.ORDER_ORIGINAL,
                                  cpbp.ORDER_DETERMINISTIC_RANDOM, cpbp.ORDER_ROW_NNZ_DESCENDING])
@pytest.mark.parametrize("width,window,dtype", [(32, 128, np.float16), (64, 256, np.float32),
                                                (7, 63, np.float32), (64, 64, np.float16)])
def test_round_trip_and_thread_invariance(kind, width, window, dtype):
    rng = np.random.default_rng(kind * 100 + width)
    plan = random_plan(rng, 300)
    offs, feats, vals = random_csr(rng, 517, 300, 12.0, dtype)
    t1 = cpbp.build_tiles(plan, offs, feats, vals, kind=kind, window_size=window, group_width=width,
                          threads=1)
    t8 = cpbp.build_tiles(plan, offs, feats, vals, kind=kind, window_size=window, group_width=width,
                          threads=8)
    for name in ("tile_block_offsets", "tile_block_ids", "tile_block_cell_masks",
                 "block_row_entry_offsets", "row_block_gene_masks", "row_block_value_offsets",
                 "values", "row_permutation", "primary_keys"):
        assert np.array_equal(getattr(t1, name), getattr(t8, name)), name
    assert t1.req["cell_mask_bytes"] == (8 if width > 32 else 4)
    decoded = cpbp.decode_tiles(plan, t1)
    for r in range(len(offs) - 1):
        src = {int(f): vals[i] for i, f in zip(range(offs[r], offs[r + 1]), feats[offs[r]:offs[r + 1]])}
        assert decoded[r].keys() == src.keys()
        assert all(decoded[r][f] == src[f] for f in src)
    # order invariants
    perm = t1.row_permutation
    assert sorted(perm.tolist()) == list(range(len(offs) - 1))
    for wb in range(0, len(perm), window):
        win = perm[wb:wb + window]
        assert win.min() >= wb and win.max() < wb + window
        keys = [(int(t1.primary_keys[r]), r) for r in win]
        prim = [k[0] for k in keys]
        assert prim == sorted(prim)


def test_minhash_equal_block_sets_share_keys():
    rng = np.random.default_rng(5)
    plan = cpbp.contiguous_plan(640, 20)
    # rows 0 and 1 touch the same blocks with different features; row 2 differs
    rows = [[0, 25, 300], [5, 39, 310], [0, 45, 300]]
    offs = np.asarray([0, 3, 6, 9], np.uint32)
    feats = np.asarray(sum(rows, []), np.uint32)
    vals = rng.standard_normal(9).astype(np.float32)
    t = cpbp.build_tiles(plan, offs, feats, vals, group_width=1, window_size=4, threads=1)
    assert t.primary_keys[0] == t.primary_keys[1] != t.primary_keys[2]


def test_tile_referee_agrees_with_canonical(oracle):
    rng = np.random.default_rng(11)
    plan = random_plan(rng, 500)
    offs, feats, vals = random_csr(rng, 700, 500, 40.0, np.float32)
    w = rng.standard_normal(500).astype(np.float32)
    canon, mag = oracle.cpbp_canonical_f64(offs, feats, vals, w)
    for width in (32, 64):
        t = cpbp.build_tiles(plan, offs, feats, vals, group_width=width, window_size=128, threads=4)
        got = oracle.cpbp_tiles(700, width, 64 if width > 32 else 32, plan.feature_block_offsets,
                                plan.feature_permutation, t.tile_block_offsets, t.tile_block_ids,
                                t.tile_block_cell_masks, t.block_row_entry_offsets,
                                t.row_block_gene_masks, t.row_block_value_offsets, t.values,
                                t.row_permutation, w)
        assert np.all(np.abs(got - canon) <= 1e-5 + 1e-5 * np.abs(canon) + 1e-6 * mag)


@pytest.mark.parametrize("case", ["unsorted", "plan_dup", "wide_block", "width", "window"])
def test_builder_rejects_bad_inputs(case):
    plan = cpbp.contiguous_plan(64, 32)
    offs = np.asarray([0, 2], np.uint32)
    feats = np.asarray([3, 9], np.uint32)
    vals = np.ones(2, np.float32)
    kw = dict(group_width=32, window_size=64)
    if case == "unsorted":
        feats = np.asarray([9, 3], np.uint32)
    elif case == "plan_dup":
        plan = cpbp.Plan(np.zeros(64, np.uint32), plan.feature_block_offsets)
    elif case == "wide_block":
        plan = cpbp.Plan(plan.feature_permutation, np.asarray([0, 64], np.uint32))
    elif case == "width":
        kw = dict(group_width=128, window_size=128)
    else:
        kw = dict(group_width=32, window_size=48)
    with pytest.raises(N.EngineError):
        cpbp.build_tiles(plan, offs, feats, vals, **kw)
