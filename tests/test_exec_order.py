"""Execution feature order on the host (CPU tests): the reference's known answers of
tests/math_execution_csr_test.cu:31-224 restated against the engine's C-ABI --

* pack_dense_operand_host: plan permutation {2, 0, 3, 1} over W = [[1,2],[3,4],[5,6],[7,8]]
  gives {5, 6, 1, 2, 7, 8, 3, 4} (:96-117);
* build_execution_csr_view_host of an ordered partition maps the entries to execution
  features {0, 1, 2, 3}, aliases offsets and values, and carries a nonzero structure
  identity (:54-94); a wrong canonical id is rejected;
* the referee on the execution-order CSR and the packed W reproduces the canonical product
  {11, 14, 37, 44} (:146-176);
* materialize_execution_csr_from_cpk1_host rebuilds rows {0, 2, 4}, features {0, 1, 2, 3}
  and values {2, 1, 4, 3} from a one-tile payload (:178-224).
Plus the popularity order's tie rule and the pinned FNV identity of the packed operand.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from cellerator_amd import _native as N


def _plan():
    offsets = np.asarray([0, 2, 4], np.uint32)
    perm = np.asarray([2, 0, 3, 1], np.uint32)
    plan = N.CxCpbpPlan(4, 2, perm.ctypes.data, offsets.ctypes.data)
    plan._keep = (offsets, perm)
    return plan


GEOMETRY = 0x03030303
AXIS = 0x0303A11


def _canonical_w():
    w = np.arange(1, 9, dtype=np.float32).reshape(4, 2)
    order = N.CxFeatureOrder(1, N.FEATURE_ORDER_CANONICAL, 4, 1, AXIS, 0)
    src = N.CxDenseOperand(w.ctypes.data, 4, 4, 2, 2, 0, 0, order, 0x30303)
    src._keep = w
    return src


def _fnv_identity(values):
    h = 1469598103934665603
    for v in values:
        for b in range(8):
            h ^= (v >> (8 * b)) & 0xFF
            h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h or 1


def test_pack_dense_operand_host_kat():
    lib = N.engine()
    plan, src = _plan(), _canonical_w()
    out = np.zeros(8, np.float32)
    view = N.CxDenseOperand()
    assert lib.cx_pack_dense_operand_host(C.byref(plan), GEOMETRY, C.byref(src), out.ctypes.data,
                                          out.nbytes, C.byref(view)) == 0, lib.cx_exec_last_error()
    assert out.tolist() == [5, 6, 1, 2, 7, 8, 3, 4]
    assert view.feature_order.kind == N.FEATURE_ORDER_PACKED
    assert view.feature_order.packing_geometry_identity == GEOMETRY
    assert view.leading_dimension == 2 and view.values == out.ctypes.data
    # packed_dense_operand.cu:98-108: FNV-1a over the schema, identities, shape and value size
    assert view.operand_identity == _fnv_identity([1, 0x30303, GEOMETRY, AXIS, 1, 4, 2, 4])
    size = C.c_uint64()
    desc = N.CxDenseOperand()
    assert lib.cx_packed_dense_operand_describe(C.byref(plan), GEOMETRY, C.byref(src), C.byref(desc),
                                                C.byref(size)) == 0
    assert size.value == 32 and desc.operand_identity == view.operand_identity
    # a packed source, a zero identity, or a wrong feature count are rejected
    for field, value in (("operand_identity", 0), ("feature_count", 3)):
        bad = _canonical_w()
        setattr(bad, field, value)
        assert lib.cx_pack_dense_operand_host(C.byref(plan), GEOMETRY, C.byref(bad), out.ctypes.data,
                                              out.nbytes, C.byref(view)) == 1
    bad = _canonical_w()
    bad.feature_order.kind = N.FEATURE_ORDER_PACKED
    assert lib.cx_pack_dense_operand_host(C.byref(plan), GEOMETRY, C.byref(bad), out.ctypes.data,
                                          out.nbytes, C.byref(view)) == 1
    assert lib.cx_pack_dense_operand_host(C.byref(plan), GEOMETRY, C.byref(src), out.ctypes.data, 31,
                                          C.byref(view)) == 1


def _ordered(canonical=(2, 0, 3, 1)):
    rows = np.asarray([0, 2, 4], np.uint32)
    blocks = np.asarray([0, 0, 1, 1], np.uint32)
    locals_ = np.asarray([0, 1, 0, 1], np.uint32)
    canon = np.asarray(canonical, np.uint32)
    values = np.asarray([2.0, 1.0, 4.0, 3.0], np.float32)
    o = N.CxOrderedPartition(0, 2, 2, 4, 4, 4, 1, AXIS, 0x303, rows.ctypes.data, blocks.ctypes.data,
                             locals_.ctypes.data, canon.ctypes.data, values.ctypes.data)
    o._keep = (rows, blocks, locals_, canon, values)
    return o


def test_execution_csr_from_ordered_partition_kat(oracle):
    lib = N.engine()
    plan, ordered = _plan(), _ordered()
    ids = np.zeros(4, np.uint32)
    view = N.CxExecutionCsr()
    assert lib.cx_build_execution_csr_host(C.byref(plan), GEOMETRY, C.byref(ordered), ids.ctypes.data, 4,
                                           C.byref(view)) == 0, lib.cx_exec_last_error()
    assert ids.tolist() == [0, 1, 2, 3]
    rows, values = ordered._keep[0], ordered._keep[4]
    assert view.row_offsets == rows.ctypes.data and view.values == values.ctypes.data
    assert view.feature_order.kind == N.FEATURE_ORDER_PACKED and view.structure_identity != 0
    # physical_csr.hh:92-110: FNV over version, row domain, shape, offsets and features
    assert view.structure_identity == _fnv_identity([1, 0, 0x303, 2, 4, 4, 0, 2, 4, 0, 1, 2, 3])
    # X_exec . W_exec through the referee reproduces the canonical product (:146-176)
    packed = np.zeros(8, np.float32)
    pv = N.CxDenseOperand()
    src = _canonical_w()
    assert lib.cx_pack_dense_operand_host(C.byref(plan), GEOMETRY, C.byref(src), packed.ctypes.data, 32,
                                          C.byref(pv)) == 0
    y = oracle.spmm_referee(2, 4, 2, rows, ids, values, packed.reshape(4, 2))
    assert y.ravel().tolist() == [11.0, 14.0, 37.0, 44.0]
    # and the canonical CSR with canonical W gives the same numbers
    canon = np.asarray([2, 0, 3, 1], np.uint32)
    assert oracle.spmm_referee(2, 4, 2, rows, canon, values, src._keep).ravel().tolist() == [11, 14, 37, 44]
    # an entry whose canonical id does not map to its (block, local) is rejected
    bad = _ordered((0, 2, 3, 1))
    assert lib.cx_build_execution_csr_host(C.byref(plan), GEOMETRY, C.byref(bad), ids.ctypes.data, 4,
                                           C.byref(view)) == 1


def test_lazy_cpk1_reconstruction_kat():
    lib = N.engine()
    offs, perm = np.asarray([0, 2, 4], np.uint32), np.asarray([2, 0, 3, 1], np.uint32)
    tile_offsets = np.asarray([0, 2], np.uint32)
    blocks, masks = np.asarray([0, 1], np.uint32), np.asarray([1, 2], np.uint32)
    entries = np.asarray([0, 1, 2], np.uint32)
    genes, voffs = np.asarray([3, 3], np.uint32), np.asarray([0, 2, 4], np.uint32)
    vals = np.asarray([2.0, 1.0, 4.0, 3.0], np.float32)
    rperm = np.asarray([0, 1], np.uint32)
    v = N.CxCpk1View()
    v.payload_identity = 0xC0303
    v.full_row_count = 2
    v.feature_axis_fingerprint = AXIS
    v.feature_axis_fingerprint_version = 1
    v.row_domain_identity = 0x303
    v.feature_block_geometry_identity = GEOMETRY
    t = v.tiles
    t.row_count, t.feature_count, t.feature_block_count, t.tile_row_width = 2, 4, 2, 2
    t.tile_count, t.tile_block_count, t.row_block_entry_count, t.nnz_count = 1, 2, 2, 4
    t.value_dtype = N.DTYPE_F32
    t.feature_block_offsets, t.feature_permutation = offs.ctypes.data, perm.ctypes.data
    t.tile_block_offsets, t.tile_block_ids = tile_offsets.ctypes.data, blocks.ctypes.data
    t.tile_block_cell_masks, t.block_row_entry_offsets = masks.ctypes.data, entries.ctypes.data
    t.row_block_gene_masks, t.row_block_value_offsets = genes.ctypes.data, voffs.ctypes.data
    t.values, t.row_permutation = vals.ctypes.data, rperm.ctypes.data
    need = N.CxLazyCsrRequirements()
    assert lib.cx_lazy_execution_csr_requirements(C.byref(v), C.byref(need)) == 0
    assert (need.row_offset_count, need.execution_feature_count, need.value_bytes, need.row_cursor_count) == (3, 4, 16, 2)
    rows, feats = np.zeros(3, np.uint32), np.zeros(4, np.uint32)
    out_vals, cursors = np.zeros(4, np.float32), np.zeros(2, np.uint32)
    bufs = N.CxLazyCsrBuffers(3, 4, 16, 2, rows.ctypes.data, feats.ctypes.data, out_vals.ctypes.data,
                              cursors.ctypes.data)
    view = N.CxExecutionCsr()
    assert lib.cx_materialize_execution_csr_from_cpk1_host(C.byref(v), C.byref(bufs), C.byref(view)) == 0, \
        lib.cx_exec_last_error()
    assert rows.tolist() == [0, 2, 4] and feats.tolist() == [0, 1, 2, 3]
    assert out_vals.tolist() == [2.0, 1.0, 4.0, 3.0]
    assert view.structure_identity != 0 and view.feature_order.packing_geometry_identity == GEOMETRY
    # a cell mask naming a row past the tile is rejected
    masks[1] = 4
    assert lib.cx_materialize_execution_csr_from_cpk1_host(C.byref(v), C.byref(bufs), C.byref(view)) == 2
    masks[1] = 2
    small = N.CxLazyCsrBuffers(2, 4, 16, 2, rows.ctypes.data, feats.ctypes.data, out_vals.ctypes.data,
                               cursors.ctypes.data)
    assert lib.cx_materialize_execution_csr_from_cpk1_host(C.byref(v), C.byref(small), C.byref(view)) == 1


def test_popularity_order_ties_by_gene():
    lib = N.engine()
    counts = np.asarray([3, 9, 3, 0, 9, 1], np.uint32)
    perm, inv = np.zeros(6, np.uint32), np.zeros(6, np.uint32)
    assert lib.cx_popularity_order(counts.ctypes.data, 6, perm.ctypes.data, inv.ctypes.data) == 0
    assert perm.tolist() == [1, 4, 0, 2, 5, 3]
    assert inv[perm].tolist() == list(range(6))
