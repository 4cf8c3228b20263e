"""The native tile adapter (cx_*native_tile*, native_tile.cpp) against the reference's own
adapter test (tests/math_native_tile_adapter_test.cc): its 3-row, 5-feature, two-block
fixture gives union masks {0x7, 0x3}, packed offsets {0, 3, 6}, a dense workload of 10 and
the stated block metrics; every packed value decodes to the test's logical coordinates and
aliases its source value; the CPK1 form gives the same view; undersized sidecars, a
non-invertible row order, an out-of-block gene mask, corrupt sidecar offsets and an
out-of-range index are rejected. The mirrors have the reference's byte layout (sizes and
field offsets computed from the C++ rules for those structs). CPU only."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cellerator_amd import _native as N


def _u32(a):
    return np.ascontiguousarray(np.array(a, dtype=np.uint32))


class Fixture:
    """math_native_tile_adapter_test.cc:24-101."""

    def __init__(self):
        self.feature_blocks = _u32([0, 3, 5])
        self.feature_permutation = _u32([2, 0, 4, 1, 3])
        self.row_permutation = _u32([2, 0, 1])
        self.inverse_rows = _u32([1, 2, 0])
        self.tile_blocks = _u32([0, 2])
        self.block_ids = _u32([0, 1])
        self.cell_masks = _u32([0x5, 0x6])
        self.block_entries = _u32([0, 2, 4])
        self.gene_masks = _u32([0x5, 0x2, 0x3, 0x1])
        self.value_offsets = _u32([0, 2, 3, 5, 6])
        self.values = np.array([10, 11, 12, 13, 14, 15], np.float32)

    def views(self):
        p = N.CxFwrPlanView(1, 1, 5, 2, 0x1234, self.feature_blocks.ctypes.data, self.feature_permutation.ctypes.data)
        o = N.CxLocalCellOrderView()
        o.order_schema_version = o.signature_algorithm_version = 1
        o.kind, o.window_size, o.group_width = 1, 3, 3
        o.ordering_identity, o.global_row_begin, o.full_row_count, o.row_count = 0x5678, 100, 3, 3
        o.feature_block_count, o.feature_block_geometry_identity, o.row_domain_identity = 2, 0x1234, 0x9ABC
        o.row_permutation, o.inverse_row_permutation = self.row_permutation.ctypes.data, self.inverse_rows.ctypes.data
        t = N.CxWarpTileView()
        t.tile_schema_version = t.record_schema_version = t.semantic_plan_schema_version = 1
        t.geometry_identity_version = t.order_schema_version = 1
        t.tile_identity, t.feature_block_geometry_identity, t.ordering_identity = 0xDEF0, 0x1234, 0x5678
        t.global_row_begin, t.full_row_count, t.row_count, t.feature_count = 100, 3, 3, 5
        t.feature_block_count, t.tile_row_width, t.tile_count, t.nnz_count = 2, 3, 1, 6
        t.tile_block_count, t.row_block_entry_count, t.value_size_bytes = 2, 4, 4
        t.row_domain_identity = 0x9ABC
        t.tile_block_offsets, t.tile_block_ids = self.tile_blocks.ctypes.data, self.block_ids.ctypes.data
        t.tile_block_cell_masks = self.cell_masks.ctypes.data
        t.block_row_entry_offsets = self.block_entries.ctypes.data
        t.row_block_gene_masks = self.gene_masks.ctypes.data
        t.row_block_value_offsets = self.value_offsets.ctypes.data
        t.values = self.values.ctypes.data
        return p, o, t

    def cpk1(self):
        """The engine's view of a CPK1 image holding the same partition."""
        v = N.CxCpk1View()
        v.payload_identity, v.global_row_begin, v.full_row_count = 0x4242, 100, 3
        v.row_domain_identity, v.feature_block_geometry_identity = 0x9ABC, 0x1234
        v.ordering_identity, v.tile_identity = 0x5678, 0xDEF0
        v.order.kind, v.order.window_size, v.order.group_width = 1, 3, 3
        v.inverse_row_permutation = self.inverse_rows.ctypes.data
        t = v.tiles
        t.row_count, t.feature_count, t.feature_block_count, t.tile_row_width = 3, 5, 2, 3
        t.tile_count, t.tile_block_count, t.row_block_entry_count, t.nnz_count = 1, 2, 4, 6
        t.value_dtype = N.DTYPE_F32
        t.feature_block_offsets, t.feature_permutation = self.feature_blocks.ctypes.data, self.feature_permutation.ctypes.data
        t.tile_block_offsets, t.tile_block_ids = self.tile_blocks.ctypes.data, self.block_ids.ctypes.data
        t.tile_block_cell_masks = self.cell_masks.ctypes.data
        t.block_row_entry_offsets = self.block_entries.ctypes.data
        t.row_block_gene_masks = self.gene_masks.ctypes.data
        t.row_block_value_offsets = self.value_offsets.ctypes.data
        t.values = self.values.ctypes.data
        t.row_permutation = self.row_permutation.ctypes.data
        return v


class Sidecars:
    def __init__(self, req):
        self.unions = np.zeros(req.union_mask_count, np.uint32)
        self.offsets = np.zeros(req.packed_offset_count, np.uint32)
        self.metrics = (N.CxNativeTileBlockMetrics * max(req.block_metric_count, 1))()

    def buffers(self, shrink_offsets=0):
        return N.CxNativeTileBuffers(self.unions.size, self.unions.ctypes.data, self.offsets.size - shrink_offsets,
                                     self.offsets.ctypes.data, len(self.metrics), C.addressof(self.metrics))


def _lib():
    try:
        return N.engine()
    except ImportError as e:  # pragma: no cover
        pytest.skip(str(e))


def test_layout_matches_the_reference_structs():
    """Sizes and offsets of the C++ structs (natural alignment, 8-byte u64 and pointers)."""
    assert C.sizeof(N.CxFwrPlanView) == 40
    assert C.sizeof(N.CxLocalCellOrderView) == 128 and N.CxLocalCellOrderView.seed.offset == 24
    assert N.CxLocalCellOrderView.feature_block_geometry_identity.offset == 64
    assert N.CxLocalCellOrderView.row_permutation.offset == 112
    assert C.sizeof(N.CxWarpTileView) == 176 and N.CxWarpTileView.tile_identity.offset == 24
    assert N.CxWarpTileView.feature_axis_fingerprint.offset == 96
    assert N.CxWarpTileView.row_domain_identity.offset == 112 and N.CxWarpTileView.values.offset == 168
    assert C.sizeof(N.CxNativeTileView) == 384 and N.CxNativeTileView.plan.offset == 8
    assert N.CxNativeTileView.order.offset == 48 and N.CxNativeTileView.tiles.offset == 176
    assert N.CxNativeTileView.dense_workload.offset == 376
    assert C.sizeof(N.CxNativeTileBlockMetrics) == 32 and C.sizeof(N.CxNativeTileDecodedValue) == 40


def _build(lib, f):
    p, o, t = f.views()
    req = N.CxNativeTileRequirements()
    assert lib.cx_query_native_tile_requirements_host(C.byref(p), C.byref(o), C.byref(t), C.byref(req)) == 0
    side = Sidecars(req)
    view = N.CxNativeTileView()
    assert lib.cx_build_native_tile_view_host(C.byref(p), C.byref(o), C.byref(t), C.byref(side.buffers()),
                                              C.byref(view)) == 0, lib.cx_last_error()
    return req, side, view


def test_sidecars_and_aliasing():
    lib = _lib()
    f = Fixture()
    req, side, view = _build(lib, f)
    assert (req.union_mask_count, req.packed_offset_count, req.block_metric_count) == (2, 3, 2)
    assert req.sidecar_bytes == (2 + 3) * 4 + 2 * 32
    assert view.tiles.values == f.values.ctypes.data and view.tiles.tile_block_offsets == f.tile_blocks.ctypes.data
    assert side.unions.tolist() == [0x7, 0x3] and side.offsets.tolist() == [0, 3, 6]
    assert view.dense_workload == 10
    m0, m1 = side.metrics[0], side.metrics[1]
    assert (m0.active_rows, m0.active_features, m0.nnz, m0.dense_workload) == (2, 3, 3, 6)
    assert abs(m0.density - 0.5) < 1e-12 and abs(m0.feature_reuse - 1.0) < 1e-12
    assert abs(m1.density - 0.75) < 1e-12 and abs(m1.feature_reuse - 1.5) < 1e-12


@pytest.mark.parametrize("from_cpk1", [False, True])
def test_exact_decode(from_cpk1):
    lib = _lib()
    f = Fixture()
    if from_cpk1:
        cpk1 = f.cpk1()
        req = N.CxNativeTileRequirements()
        assert lib.cx_query_native_tile_requirements_from_cpk1_host(C.byref(cpk1), C.byref(req)) == 0, lib.cx_last_error()
        side = Sidecars(req)
        view = N.CxNativeTileView()
        assert lib.cx_build_native_tile_view_from_cpk1_host(C.byref(cpk1), C.byref(side.buffers()), C.byref(view)) == 0
    else:
        _, side, view = _build(lib, f)
    expected = [(0, 2, 0, 2), (0, 2, 2, 4), (2, 1, 1, 0), (1, 0, 3, 1), (1, 0, 4, 3), (2, 1, 3, 1)]
    out = N.CxNativeTileDecodedValue()
    for i, (er, cr, ef, cf) in enumerate(expected):
        assert lib.cx_decode_native_tile_value_host(C.byref(view), i, C.byref(out)) == 0, lib.cx_last_error()
        assert (out.execution_row, out.canonical_row, out.execution_feature, out.canonical_feature) == (er, cr, ef, cf)
        assert out.global_row == 100 + cr
        assert out.value == f.values.ctypes.data + 4 * i
    assert lib.cx_decode_native_tile_value_host(C.byref(view), 6, C.byref(out)) != 0
    side.offsets[1] = 4
    assert lib.cx_decode_native_tile_value_host(C.byref(view), 1, C.byref(out)) != 0
    assert b"invalid native sidecars" in lib.cx_last_error()


def test_rejections():
    lib = _lib()
    f = Fixture()
    p, o, t = f.views()
    req, side, view = _build(lib, f)
    assert lib.cx_build_native_tile_view_host(C.byref(p), C.byref(o), C.byref(t), C.byref(side.buffers(1)),
                                              C.byref(view)) == 1  # INVALID_ARGUMENT
    assert b"small sidecar buffers" in lib.cx_last_error()
    f.inverse_rows[2] = 2
    assert lib.cx_query_native_tile_requirements_host(C.byref(p), C.byref(o), C.byref(t), C.byref(req)) != 0
    assert b"invalid row permutation" in lib.cx_last_error()
    f.inverse_rows[2] = 0
    f.gene_masks[0] = 0x8
    assert lib.cx_query_native_tile_requirements_host(C.byref(p), C.byref(o), C.byref(t), C.byref(req)) == 2
    assert b"invalid gene offsets" in lib.cx_last_error()


def test_engine_tile_operand_of_a_native_view():
    """cx_cpbp_tiles_from_native_view carries plan arrays, tiles and the row permutation."""
    lib = _lib()
    f = Fixture()
    _, _, view = _build(lib, f)
    t = N.CxCpbpTiles()
    assert lib.cx_cpbp_tiles_from_native_view(C.byref(view), C.byref(t)) == 0
    assert (t.row_count, t.feature_count, t.tile_row_width, t.nnz_count, t.value_dtype) == (3, 5, 3, 6, N.DTYPE_F32)
    assert t.feature_permutation == f.feature_permutation.ctypes.data and t.row_permutation == f.row_permutation.ctypes.data
    assert t.values == f.values.ctypes.data and t.tile_block_cell_masks == f.cell_masks.ctypes.data
    view.tiles.value_size_bytes = 8
    assert lib.cx_cpbp_tiles_from_native_view(C.byref(view), C.byref(t)) == 3  # UNSUPPORTED
