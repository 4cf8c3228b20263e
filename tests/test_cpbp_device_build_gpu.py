"""GPU: device construction of the CP-BP warp-tile projection (cx_cpbp_device_builder_*) is
bit-identical to the host builder (cx_cpbp_builder_*), whose output tests/test_cpbp_build.py
pins against the reference fixture, the decode round trip and the oracle's referees; the
reduction over device-built tiles matches the canonical referee."""
from __future__ import annotations

import numpy as np
import pytest

from cellerator_amd import _native as N
from cellerator_amd import cpbp
from tests.test_cpbp_build import random_csr, random_plan, reference_fixture, reference_plan

pytestmark = pytest.mark.gpu


def _same(host: cpbp.HostTiles, dev, primary):
    def h(t):
        return t.cpu().numpy()

    assert dev.meta["tile_requirements"] == host.req
    assert np.array_equal(h(dev.tile_block_offsets).view(np.uint32), host.tile_block_offsets)
    assert np.array_equal(h(dev.tile_block_ids).view(np.uint32), host.tile_block_ids)
    mask_t = np.uint64 if host.req["cell_mask_bytes"] == 8 else np.uint32
    assert np.array_equal(h(dev.tile_block_cell_masks).view(mask_t), host.tile_block_cell_masks)
    assert np.array_equal(h(dev.block_row_entry_offsets).view(np.uint32), host.block_row_entry_offsets)
    assert np.array_equal(h(dev.row_block_gene_masks).view(np.uint32), host.row_block_gene_masks)
    assert np.array_equal(h(dev.row_block_value_offsets).view(np.uint32), host.row_block_value_offsets)
    assert np.array_equal(h(dev.values).view(np.uint8), host.values.view(np.uint8))
    assert np.array_equal(h(dev.row_permutation).view(np.uint32), host.row_permutation)
    assert np.array_equal(h(primary).view(np.uint64), host.primary_keys)


def test_reference_fixture_matches_host(oracle):
    plan = reference_plan()
    offs, feats, vals, _ = reference_fixture()
    kw = dict(kind=cpbp.ORDER_ROW_NNZ_DESCENDING, window_size=8, group_width=4)
    host = cpbp.build_tiles(plan, offs, feats, vals, threads=1, **kw)
    dev, primary = cpbp.build_tiles_device(plan, offs, feats, vals, **kw)
    _same(host, dev, primary)


@pytest.mark.parametrize("kind", [cpbp.ORDER_INFERRED_MINHASH, cpbp.ORDER_ORIGINAL,
                                  cpbp.ORDER_DETERMINISTIC_RANDOM, cpbp.ORDER_ROW_NNZ_DESCENDING])
@pytest.mark.parametrize("width,window,dtype,rows", [
    (32, 128, np.float16, 1000), (64, 256, np.float32, 3001), (7, 63, np.float32, 500),
    (64, 1024, np.float16, 20_000), (64, 64, np.float32, 64), (1, 1, np.float16, 37)])
def test_device_build_matches_host(kind, width, window, dtype, rows):
    rng = np.random.default_rng(kind * 100 + width + rows)
    plan = random_plan(rng, 700)
    offs, feats, vals = random_csr(rng, rows, 700, 30.0, dtype)
    kw = dict(kind=kind, window_size=window, group_width=width, seed=0x1234 + kind,
              global_row_begin=77)
    host = cpbp.build_tiles(plan, offs, feats, vals, threads=4, **kw)
    dev, primary = cpbp.build_tiles_device(plan, offs, feats, vals, **kw)
    _same(host, dev, primary)


def test_device_build_edge_shapes():
    """All rows empty; a single row; rows holding every feature."""
    rng = np.random.default_rng(5)
    plan = random_plan(rng, 96)
    cases = [
        (np.zeros(10, np.uint32), np.zeros(0, np.uint32), np.zeros(0, np.float32)),
        (np.array([0, 3], np.uint32), np.array([1, 50, 95], np.uint32), np.ones(3, np.float32)),
        (np.array([0, 96, 192], np.uint32), np.tile(np.arange(96, dtype=np.uint32), 2),
         rng.standard_normal(192).astype(np.float32)),
    ]
    for offs, feats, vals in cases:
        kw = dict(kind=cpbp.ORDER_INFERRED_MINHASH, window_size=64, group_width=64)
        host = cpbp.build_tiles(plan, offs, feats, vals, threads=1, **kw)
        dev, primary = cpbp.build_tiles_device(plan, offs, feats, vals, **kw)
        _same(host, dev, primary)


@pytest.mark.parametrize("case", ["unsorted", "plan_dup", "wide_block", "width", "window",
                                  "feature_range"])
def test_device_builder_rejects_bad_inputs(case):
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
    elif case == "window":
        kw = dict(group_width=32, window_size=48)
    else:
        feats = np.asarray([3, 64], np.uint32)
    with pytest.raises(N.EngineError):
        cpbp.build_tiles_device(plan, offs, feats, vals, **kw)


def test_reduction_over_device_tiles(oracle):
    import torch

    from cellerator_amd import cpbp_reduce
    rng = np.random.default_rng(9)
    plan = random_plan(rng, 900)
    offs, feats, vals = random_csr(rng, 5000, 900, 40.0, np.float32)
    w = rng.standard_normal(900).astype(np.float32)
    dev, _ = cpbp.build_tiles_device(plan, offs, feats, vals)
    got = cpbp_reduce(dev, torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    ref, mag = oracle.cpbp_canonical_f64(offs, feats, vals, w, oracle.F32)
    tol = 1e-5 + 1e-5 * np.abs(ref) + 2.0 ** -22 * mag
    assert np.all(np.abs(got.cpu().numpy().astype(np.float64) - ref) <= tol)
