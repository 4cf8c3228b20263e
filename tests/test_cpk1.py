"""CPK1 persistent packing payload: write -> validate -> (device) upload, rebind, reduce.

Mirrors components/CellPack/tests/persistent_packing_payload_test.cu: the same 6-feature /
8-row plan fixture, partition rows [2, 6), row_nnz_descending order in windows of 4; the
image round-trips, a one-byte tamper and a wrong compatibility fingerprint are rejected,
and the reduction runs directly on the uploaded image. The identities are checked against
an independent FNV-1a (pinned by its published test vectors) and splitmix64 chain.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np
import pytest

from cellerator_amd import _native as N
from cellerator_amd import cpbp, cpk1

HEADER_BYTES = 352
SECTIONS = 15


def fnv1a64(data: bytes, h: int = 0xCBF29CE484222325) -> int:
    for b in data:
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


# The reference defines its identities with offset basis 1469598103934665603
# (persistent_packing_payload.cc:19, packing_plan.cc:11), the published basis
# 14695981039346656037 with its last decimal digit dropped; the prime is the standard one.
REFERENCE_BASIS = 1469598103934665603


def reference_fnv(data: bytes, h: int = REFERENCE_BASIS) -> int:
    return fnv1a64(data, h)


def test_fnv1a_published_vectors():
    # FNV-1a 64-bit test vectors (Fowler/Noll/Vo reference test suite)
    assert fnv1a64(b"") == 0xCBF29CE484222325
    assert fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert fnv1a64(b"foobar") == 0x85944171F73967E8


def reference_plan() -> cpbp.Plan:
    """persistent_packing_payload_test.cu:58-96"""
    return cpbp.Plan(np.array([2, 0, 4, 5, 1, 3], np.uint32), np.array([0, 3, 6], np.uint32))


def reference_source():
    """persistent_packing_payload_test.cu:98-106: 4 rows of the 8-row domain."""
    offs = np.array([0, 3, 5, 6, 9], np.uint32)
    feats = np.array([0, 2, 5, 1, 4, 3, 0, 1, 5], np.uint32)
    vals = (0.25 * np.arange(1, 10)).astype(np.float16)
    return offs, feats, vals


def reference_meta() -> cpk1.Metadata:
    return cpk1.Metadata(feature_axis_fingerprint=0x1020304050607080,
                         row_domain_identity=0x8877665544332211, full_row_count=8,
                         global_row_begin=2, evaluation_source_identity=0x1234,
                         cost_policy_identity=0x5678, row_group_width=4,
                         row_group_offsets=np.array([0, 4, 8], np.uint32),
                         maximum_feature_block_width=3, order_kind=cpbp.ORDER_ROW_NNZ_DESCENDING,
                         window_size=4, group_width=4)


def build_reference_image():
    plan = reference_plan()
    offs, feats, vals = reference_source()
    tiles = cpbp.build_tiles(plan, offs, feats, vals, kind=cpbp.ORDER_ROW_NNZ_DESCENDING,
                             window_size=4, group_width=4, threads=1)
    image, view = cpk1.write_image(plan, tiles, reference_meta())
    return plan, tiles, image, view


def section(image: np.ndarray, index: int, count: int, dtype=np.uint32) -> np.ndarray:
    offset = struct.unpack_from("<Q", image, HEADER_BYTES - 8 * SECTIONS + 8 * index)[0]
    return np.frombuffer(image, dtype, count, offset)


def test_reference_fixture_round_trips():
    plan, tiles, image, view = build_reference_image()
    assert not np.array_equal(tiles.row_permutation, np.arange(4))  # nonidentity order
    assert image.size % 64 == 0 and bytes(image[:8]) == b"CELLPK01"
    assert view.payload_identity != 0 and view.full_row_count == 8 and view.tiles.row_count == 4
    # every tile array comes back unchanged from its section
    t = view.tiles
    for idx, arr in ((0, plan.feature_permutation), (2, plan.feature_block_offsets),
                     (6, tiles.row_permutation), (8, tiles.tile_block_offsets),
                     (9, tiles.tile_block_ids), (10, tiles.tile_block_cell_masks),
                     (11, tiles.block_row_entry_offsets), (12, tiles.row_block_gene_masks),
                     (13, tiles.row_block_value_offsets)):
        assert np.array_equal(section(image, idx, arr.size), arr.astype(np.uint32)), idx
    assert np.array_equal(section(image, 14, t.nnz_count, np.float16), tiles.values)
    inv = section(image, 7, 4)
    assert np.array_equal(inv[tiles.row_permutation], np.arange(4))
    # validate again from a copy, with the writer's compatibility identity
    again = cpk1.validate(image.copy(), cpk1.expected_of(view))
    assert again.payload_identity == view.payload_identity


def test_identities_are_the_documented_hashes():
    plan, tiles, image, view = build_reference_image()
    raw = bytearray(image.tobytes())
    stored = struct.unpack_from("<Q", raw, 32)[0]
    struct.pack_into("<Q", raw, 32, 0)
    assert stored == reference_fnv(bytes(raw)) == view.payload_identity
    # geometry identity: FNV-1a of the tag, versions, counts, block offsets, permutation
    g = reference_fnv(b"cellerator_feature_block_geometry_identity_v1\x00")
    words = [1, 1, 6, 2, *plan.feature_block_offsets.tolist(), *plan.feature_permutation.tolist()]
    g = fnv1a64(b"".join(struct.pack("<I", w) for w in words), g)
    assert view.feature_block_geometry_identity == g

    def mix(v):
        v = (v + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        return v ^ (v >> 31)

    o = mix(g)
    for x in ((1 << 32) ^ 1, 0x8877665544332211, 2, (4 << 32) ^ 8, (4 << 32) ^ 4,
              0x6A09E667F3BCC909 ^ cpbp.ORDER_ROW_NNZ_DESCENDING):
        o = mix(o ^ x)
    assert view.ordering_identity == o
    t = mix(g)
    for x in ((1 << 32) ^ 1, o, 0x8877665544332211, 2, (4 << 32) ^ 8, (6 << 32) ^ 2, (4 << 32) ^ 2):
        t = mix(t ^ x)
    assert view.tile_identity == t


def test_tamper_and_mismatch_are_rejected():
    _, _, image, view = build_reference_image()
    expected = cpk1.expected_of(view)
    bad = image.copy()
    bad[-1] ^= 0x80
    with pytest.raises(N.EngineError, match="identity"):
        cpk1.validate(bad, expected)
    wrong = cpk1.expected_of(view)
    wrong.feature_axis_fingerprint ^= 1
    with pytest.raises(N.EngineError, match="compatibility"):
        cpk1.validate(image, wrong)
    with pytest.raises(N.EngineError):
        cpk1.validate(image[:-64], expected)        # wrong size
    with pytest.raises(N.EngineError):
        cpk1.validate(image[:100], expected)        # truncated header
    # a structurally wrong section with a consistent identity: rebuilt identity, bad tile
    raw = bytearray(image.tobytes())
    off = struct.unpack_from("<Q", raw, HEADER_BYTES - 8 * SECTIONS + 8 * 10)[0]
    struct.pack_into("<I", raw, off, 0)          # first cell mask = 0
    struct.pack_into("<Q", raw, 32, 0)
    ident = reference_fnv(bytes(raw))
    struct.pack_into("<Q", raw, 32, ident)
    forged = cpk1.expected_of(view)
    forged.payload_identity = ident
    with pytest.raises(N.EngineError, match="descriptor"):
        cpk1.validate(np.frombuffer(bytes(raw), np.uint8), forged)


def test_writer_rejects_wide_tiles_and_f32_values():
    plan = cpbp.contiguous_plan(64, 32)
    rng = np.random.default_rng(1)
    from tests.test_cpbp_build import random_csr
    offs, feats, vals = random_csr(rng, 100, 64, 6.0, np.float16)
    wide = cpbp.build_tiles(plan, offs, feats, vals, group_width=64, window_size=64)
    meta = cpk1.Metadata(1, 1, 100, group_width=64, window_size=64)
    with pytest.raises(N.EngineError, match="u32 cell masks"):
        cpk1.write_image(plan, wide, meta)
    offs, feats, vals = random_csr(rng, 100, 64, 6.0, np.float32)
    f32 = cpbp.build_tiles(plan, offs, feats, vals, group_width=32, window_size=64)
    with pytest.raises(N.EngineError, match="f16"):
        cpk1.write_image(plan, f32, cpk1.Metadata(1, 1, 100, group_width=32, window_size=64))


def test_rebind_moves_every_pointer_by_the_base_difference():
    _, _, image, view = build_reference_image()
    out = N.CxCpk1View()
    base = 0x7F0000000000
    assert N.engine().cx_cpk1_rebind(C.byref(view), base, view.image_bytes, C.byref(out)) == 0
    delta = base - view.image_base
    t0, t1 = view.tiles, out.tiles
    for name in ("feature_block_offsets", "feature_permutation", "tile_block_offsets",
                 "tile_block_ids", "tile_block_cell_masks", "block_row_entry_offsets",
                 "row_block_gene_masks", "row_block_value_offsets", "values", "row_permutation"):
        assert getattr(t1, name) - getattr(t0, name) == delta, name
    assert out.image_base == base
    assert N.engine().cx_cpk1_rebind(C.byref(view), base, view.image_bytes + 64, C.byref(out)) != 0


@pytest.mark.gpu
def test_reduction_runs_on_the_uploaded_image(oracle):
    """persistent_packing_payload_test.cu:294-326: upload, rebind, execute, compare with the
    canonical referee; also bitwise equal to the reduction on separately uploaded tiles."""
    import torch

    from cellerator_amd import cpbp_reduce
    plan, tiles, image, view = build_reference_image()
    dev = cpk1.upload(cpk1.validate(image, cpk1.expected_of(view)), image)
    w = (0.5 + 0.125 * np.arange(6)).astype(np.float32)
    wt = torch.from_numpy(w).cuda()
    got = cpbp_reduce(dev, wt)
    direct = cpbp_reduce(cpbp.to_device(plan, tiles), wt)
    torch.cuda.synchronize()
    offs, feats, vals = reference_source()
    ref, _ = oracle.cpbp_canonical_f64(offs, feats, vals, w, oracle.F16)
    assert np.allclose(got.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    assert torch.equal(got.view(torch.int32), direct.view(torch.int32))


@pytest.mark.gpu
def test_larger_image_on_the_device(oracle):
    import torch

    from cellerator_amd import cpbp_reduce
    from tests.test_cpbp_build import random_csr, random_plan
    rng = np.random.default_rng(44)
    plan = random_plan(rng, 500)
    offs, feats, vals = random_csr(rng, 4000, 500, 25.0, np.float16)
    tiles = cpbp.build_tiles(plan, offs, feats, vals, group_width=32, window_size=1024)
    meta = cpk1.Metadata(0xABC, 0xDEF, 10_000, global_row_begin=3000, group_width=32,
                         window_size=1024)
    image, view = cpk1.write_image(plan, tiles, meta)
    dev = cpk1.upload(cpk1.validate(image, cpk1.expected_of(view)), image)
    w = rng.standard_normal(500).astype(np.float32)
    got = cpbp_reduce(dev, torch.from_numpy(w).cuda())
    torch.cuda.synchronize()
    ref, mag = oracle.cpbp_canonical_f64(offs, feats, vals, w, oracle.F16)
    tol = 1e-5 + 1e-5 * np.abs(ref) + 2.0 ** -22 * mag
    assert np.all(np.abs(got.cpu().numpy().astype(np.float64) - ref) <= tol)


def _reduction_view(view, weight_identity=0x5EED):
    out = N.CxCpbpReductionView()
    assert N.engine().cx_cpbp_reduction_view_from_cpk1(C.byref(view), weight_identity, C.byref(out)) == 0
    return out


def test_reduction_identity_chain():
    """reduction_identity (feature_weighted_row_reduction_cuda.cu:44-55) restated here from the
    splitmix64 chain; the C-ABI's value and the view built from an image agree with it."""
    _, _, image, view = build_reference_image()
    v = _reduction_view(cpk1.validate(image, cpk1.expected_of(view)))
    M = (1 << 64) - 1

    def splitmix(x):
        x = (x + 0x9E3779B97F4A7C15) & M
        x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & M
        x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & M
        return x ^ (x >> 31)

    h = splitmix(v.tile_identity)
    h = splitmix(h ^ v.plan_geometry_identity)
    h = splitmix(h ^ 0x5EED)
    h = splitmix(h ^ (1 << 32) ^ 3)  # schema 1, storage f16 (code 3)
    h = splitmix(h ^ (4 << 32) ^ 4)  # weights and accumulation f32
    assert v.reduction_identity == h == N.engine().cx_cpbp_reduction_identity(C.byref(v))
    assert (v.storage_type_code, v.weight_type_code, v.accumulation_type_code) == (3, 4, 4)


@pytest.mark.gpu
@pytest.mark.parametrize("field,value,status", [
    (None, None, 0),
    ("schema_version", 2, "UNSUPPORTED"),
    ("order_signature_version", 2, "UNSUPPORTED"),
    ("storage_type_code", 4, "INVALID_ARGUMENT"),
    ("feature_weight_identity", 0, "INVALID_ARGUMENT"),
    ("reduction_identity", 12345, "INVALID_ARGUMENT"),
    ("tile_identity", 99, "INVALID_ARGUMENT"),  # the recomputed reduction identity no longer matches
    ("order_ordering_identity", 7, "INVALID_SHAPE"),
    ("order_group_width", 16, "INVALID_SHAPE"),
    ("order_row_count", 1, "INVALID_SHAPE"),
    ("plan_geometry_identity", 5, "INVALID_ARGUMENT"),  # part of the reduction identity too
    ("order_geometry_identity", 5, "INVALID_SHAPE"),
    ("order_row_domain_identity", 5, "INVALID_SHAPE"),
])
def test_checked_reduction_rejects_mismatched_contracts(oracle, field, value, status):
    """validate_metadata (feature_weighted_row_reduction_cuda.cu:57-136): the checked entry runs
    the reduction (bitwise equal to the plain one) only when versions, numeric contract,
    identities and the plan / order / tile domains agree; every mismatch is rejected before
    any launch."""
    import torch

    from cellerator_amd import cpbp_reduce
    _, _, image, view = build_reference_image()
    dev = cpk1.upload(cpk1.validate(image, cpk1.expected_of(view)), image)
    v = _reduction_view(dev.view)
    if field is not None:
        setattr(v, field, value)
    w = torch.from_numpy((0.5 + 0.125 * np.arange(6)).astype(np.float32)).cuda()
    out = torch.full((dev.row_count,), -7.0, device="cuda")
    rc = N.engine().cx_cpbp_reduce_checked(C.byref(v), w.data_ptr(), w.numel(), out.data_ptr(), out.numel(), None)
    torch.cuda.synchronize()
    if status == 0:
        assert rc == 0
        assert torch.equal(out.view(torch.int32), cpbp_reduce(dev, w).view(torch.int32))
    else:
        assert N.STATUS_NAMES.get(rc) == status, rc
        assert torch.all(out == -7.0)
