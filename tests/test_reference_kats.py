"""Known answers from the reference's own CellPack tests, restated against the engine's
host builders, plus brute-force pins of the oracle's CP-BP referees and row-parallel
baselines. CPU only.

* components/CellPack/tests/warp_tiles_test.cc:28-137 (main fixture) and :326-360 (exact
  host contract): tile offsets {0, 3, 4}, block ids {0, 1, 2, 2}, cell masks
  {0xffffffff, 3, 2, 1}, entry offsets {0, 32, 34, 35, 36}, gene masks [31] = 0x80000000,
  [32..35] = {3, 2, 1, 2}, value offsets from 0 to nnz. The reference stores 3-byte values;
  the engine's builder takes f16 / f32, so the fixture carries f32 values (the layout does
  not depend on the value width).
* components/CellPack/tests/local_cell_ordering_test.cu:62-185: 17 rows (16 alternating
  between blocks {0, 1} and {6, 7}, plus an empty tail), window 8, group width 4. The
  group block-union references are 8 for the inferred MinHash order and 16 for the original
  and row-nnz orders; the union of a group is the descriptor count of its tile.
"""
from __future__ import annotations

import numpy as np
import pytest

from cellerator_amd import cpbp


def _warp_tile_fixture():
    """make_main_fixture (warp_tiles_test.cc:96-122): identity plan of 36 features in blocks
    [0, 32), [32, 34), [34, 36); 34 rows; rows 0..31 hold feature r; row 0 also 32, 33; row
    1 also 33, 34; row 32 holds 35; row 33 is empty. Values are the entry tags as f32."""
    plan = cpbp.Plan(np.arange(36, dtype=np.uint32), np.asarray([0, 32, 34, 36], np.uint32))
    rows = []
    for r in range(34):
        if r < 32:
            feats = [(r, 10 * r)]
            if r == 0:
                feats += [(32, 1), (33, 2)]
            if r == 1:
                feats += [(33, 11), (34, 12)]
        elif r == 32:
            feats = [(35, 321)]
        else:
            feats = []
        rows.append(feats)
    offs = np.zeros(35, np.uint32)
    offs[1:] = np.cumsum([len(f) for f in rows])
    feats = np.asarray([f for row in rows for f, _ in row], np.uint32)
    vals = np.asarray([t for row in rows for _, t in row], np.float32)
    return plan, offs, feats, vals


def test_warp_tiles_exact_host_contract():
    plan, offs, feats, vals = _warp_tile_fixture()
    t = cpbp.build_tiles(plan, offs, feats, vals, kind=cpbp.ORDER_ORIGINAL, window_size=32,
                         group_width=32, global_row_begin=7, threads=1)
    assert t.tile_block_offsets.tolist() == [0, 3, 4]
    assert t.tile_block_ids.tolist() == [0, 1, 2, 2]
    assert t.tile_block_cell_masks.tolist() == [0xFFFFFFFF, 3, 2, 1]
    assert t.block_row_entry_offsets.tolist() == [0, 32, 34, 35, 36]
    gm = t.row_block_gene_masks
    assert (gm[31], gm[32], gm[33], gm[34], gm[35]) == (0x80000000, 3, 2, 1, 2)
    assert t.row_block_value_offsets[0] == 0 and t.row_block_value_offsets[-1] == len(feats)
    assert t.row_permutation.tolist() == list(range(34))
    # exact decode round trip
    want = [{int(f): float(v) for f, v in zip(feats[offs[r]:offs[r + 1]], vals[offs[r]:offs[r + 1]])}
            for r in range(34)]
    assert [{f: float(v) for f, v in row.items()} for row in cpbp.decode_tiles(plan, t)] == want
    # deterministic_random permutes the rows (warp_tiles_test.cc:362-371) and still
    # decodes exactly; the construction is deterministic
    s = cpbp.build_tiles(plan, offs, feats, vals, kind=cpbp.ORDER_DETERMINISTIC_RANDOM,
                         window_size=32, group_width=32, global_row_begin=7, threads=1)
    assert s.row_permutation.tolist() != list(range(34))
    assert [{f: float(v) for f, v in row.items()} for row in cpbp.decode_tiles(plan, s)] == want
    again = cpbp.build_tiles(plan, offs, feats, vals, kind=cpbp.ORDER_ORIGINAL, window_size=32,
                             group_width=32, global_row_begin=7, threads=4)
    for name in ("tile_block_offsets", "tile_block_ids", "tile_block_cell_masks",
                 "block_row_entry_offsets", "row_block_gene_masks", "row_block_value_offsets",
                 "values", "row_permutation"):
        assert np.array_equal(getattr(t, name), getattr(again, name)), name


def _ordering_fixture():
    """record_fixture (local_cell_ordering_test.cu:62-84): 8 blocks of 8 features; even rows
    hold local gene 0 of blocks 0 and 1, odd rows of blocks 6 and 7; row 16 is empty."""
    plan = cpbp.contiguous_plan(64, 8)
    offs, feats = [0], []
    for r in range(16):
        feats += [0, 8] if r % 2 == 0 else [48, 56]
        offs.append(len(feats))
    offs.append(len(feats))
    return (plan, np.asarray(offs, np.uint32), np.asarray(feats, np.uint32),
            np.ones(len(feats), np.float32))


@pytest.mark.parametrize("kind,union", [(cpbp.ORDER_INFERRED_MINHASH, 8), (cpbp.ORDER_ORIGINAL, 16),
                                        (cpbp.ORDER_ROW_NNZ_DESCENDING, 16)])
def test_local_order_group_unions(kind, union):
    plan, offs, feats, vals = _ordering_fixture()
    t = cpbp.build_tiles(plan, offs, feats, vals, kind=kind, window_size=8, group_width=4,
                         global_row_begin=40, threads=1)
    # rows stay in their window of 8; the inverse is a permutation
    perm = t.row_permutation
    assert sorted(perm.tolist()) == list(range(17))
    assert all(int(row) // 8 == e // 8 for e, row in enumerate(perm))
    assert int(t.tile_block_offsets[-1]) == union  # sum over groups of |block union|
    again = cpbp.build_tiles(plan, offs, feats, vals, kind=kind, window_size=8, group_width=4,
                             global_row_begin=40, threads=3)
    assert np.array_equal(perm, again.row_permutation)


def test_deterministic_random_is_seed_deterministic():
    plan, offs, feats, vals = _ordering_fixture()
    a = cpbp.build_tiles(plan, offs, feats, vals, kind=cpbp.ORDER_DETERMINISTIC_RANDOM,
                         window_size=8, group_width=4, global_row_begin=40, threads=1)
    b = cpbp.build_tiles(plan, offs, feats, vals, kind=cpbp.ORDER_DETERMINISTIC_RANDOM,
                         window_size=8, group_width=4, global_row_begin=40, threads=2)
    assert np.array_equal(a.row_permutation, b.row_permutation)


# ---------------------------------------------------------------- oracle brute force

def _dense(offs, feats, vals, cols):
    x = np.zeros((len(offs) - 1, cols), np.float64)
    for r in range(len(offs) - 1):
        x[r, feats[offs[r]:offs[r + 1]]] = vals[offs[r]:offs[r + 1]]
    return x


def test_cpbp_referees_against_dense_matvec(oracle):
    """or_cpbp_canonical, its row-parallel form and or_cpbp_tiles against a float64 dense
    mat-vec of the densified matrix; a planted wrong weight index breaks the agreement."""
    from tests.test_cpbp_build import random_csr, random_plan
    rng = np.random.default_rng(31)
    plan = random_plan(rng, 300)
    offs, feats, vals = random_csr(rng, 400, 300, 25.0, np.float32)
    w = rng.standard_normal(300).astype(np.float32)
    dense = _dense(offs, feats, vals.astype(np.float64), 300)
    truth = dense @ w.astype(np.float64)
    mag = np.abs(dense) @ np.abs(w.astype(np.float64))
    tol = 1e-6 + 2.0 ** -22 * mag
    canon = oracle.cpbp_canonical(offs, feats, vals, w)
    assert np.all(np.abs(canon - truth) <= tol)
    assert np.array_equal(oracle.cpbp_canonical_mt(offs, feats, vals, w, threads=4).view(np.uint32),
                          canon.view(np.uint32))
    c64, m64 = oracle.cpbp_canonical_f64(offs, feats, vals, w)
    assert np.all(np.abs(c64 - truth) <= 1e-9 * (1 + mag)) and np.allclose(m64, mag)
    t = cpbp.build_tiles(plan, offs, feats, vals, group_width=64, window_size=128, threads=2)
    tiles = oracle.cpbp_tiles(400, 64, 64, plan.feature_block_offsets, plan.feature_permutation,
                              t.tile_block_offsets, t.tile_block_ids, t.tile_block_cell_masks,
                              t.block_row_entry_offsets, t.row_block_gene_masks,
                              t.row_block_value_offsets, t.values, t.row_permutation, w)
    assert np.all(np.abs(tiles - truth) <= tol)
    wrong = np.roll(w, 1)  # a transposed / shifted weight index
    assert not np.all(np.abs(oracle.cpbp_canonical(offs, feats, vals, wrong) - truth) <= tol)


def test_qcsr_magnitude_is_abs_dense_product(oracle):
    """or_qcsr_spmm_f32_mt_magnitude = |decoded X| . |W| (the tolerance's magnitude term)."""
    from tests.helpers import quantized_fixture
    rng = np.random.default_rng(41)
    fx = quantized_fixture(oracle, rng, 120, 300, 30.0, 4, 1)
    w = (rng.standard_normal((300, 64)) * 0.02).astype(np.float16)
    decoded = oracle.decode_csr(4, 1, fx["row_ptr"], fx["packed_row_ptr"], fx["col_idx"],
                                fx["packed"], fx["scales"], fx["offsets"], None)
    dense = _dense(fx["row_ptr"], fx["col_idx"], decoded.astype(np.float64), 300)
    want = np.abs(dense) @ np.abs(w.astype(np.float64))
    got = oracle.qcsr_spmm_f32_mt(4, 1, 120, 300, fx["row_ptr"], fx["packed_row_ptr"],
                                  fx["col_idx"], fx["packed"], fx["scales"], fx["offsets"], None,
                                  w, threads=3, magnitude=True)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
    prod = oracle.qcsr_spmm_f32_mt(4, 1, 120, 300, fx["row_ptr"], fx["packed_row_ptr"],
                                   fx["col_idx"], fx["packed"], fx["scales"], fx["offsets"], None,
                                   w, threads=3)
    assert np.all(np.abs(prod - dense @ w.astype(np.float64)) <= 1e-5 * (1 + want))


def test_bell_bf16_mt_matches_referee(oracle):
    """The row-block-parallel Blocked-ELL baseline against the float64 referee."""
    from tests.test_bell_gpu import _bf16_round, random_bell
    rng = np.random.default_rng(43)
    idx, vals = random_bell(rng, 32 * 12, 700, 32, 7)
    vbits = _bf16_round(vals)
    w = (rng.standard_normal((700, 64)) * 0.02).astype(np.float32)
    wbits = _bf16_round(w)
    got = oracle.bell_spmm_bf16_mt(32 * 12, 700, 32, 7 * 32, idx, vbits, wbits, threads=3)
    ref, mag = oracle.bell_spmm_referee(32 * 12, 700, 32, 7 * 32, idx, vbits, wbits,
                                        value_type=oracle.BF16, rhs_type=oracle.BF16)
    assert np.all(np.abs(got - ref) <= 1e-6 + 2.0 ** -20 * mag)
