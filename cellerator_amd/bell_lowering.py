"""CSR -> Blocked-ELL lowering (bell_lowering.cpp): ctypes mirrors of the C-ABI structs and
a host-array front-end. The reference's counterparts are query_bell_candidates_host and
materialize_bell_candidate_host (include/Cellerator/compute/math/physical_bell.hh:170-193);
status codes are its bell_lowering_status_code values."""
from __future__ import annotations

import ctypes as C
from typing import Optional

import numpy as np

from . import _native as N

u32, u64, i32, p_void = C.c_uint32, C.c_uint64, C.c_int32, C.c_void_p
VALUES_BLOCK_MAJOR, VALUES_ROW_MAJOR = 0, 1
LEGAL, EMPTY_SOURCE, VALUE_EXPANSION, STORAGE_EXPANSION, PERSISTENT_BYTES, OVERFLOW_STATE = range(6)
SIZES = (8, 16, 32)


class CxBellCsrSource(C.Structure):
    _fields_ = [("row_count", u32), ("feature_count", u32), ("nnz_count", u32), ("value_size_bytes", u32),
                ("row_offsets", p_void), ("feature_ids", p_void), ("values", p_void)]


class CxBellSemanticPlan(C.Structure):
    _fields_ = [("semantic_schema_version", u32), ("full_row_count", u32), ("feature_count", u32),
                ("feature_block_count", u32), ("feature_block_geometry_identity", u64),
                ("row_domain_identity", u64), ("feature_block_offsets", p_void), ("feature_permutation", p_void),
                ("inverse_feature_permutation", p_void)]


class CxBellRowOrder(C.Structure):
    _fields_ = [("order_schema_version", u32), ("signature_algorithm_version", u32), ("kind", u32),
                ("window_size", u32), ("group_width", u32), ("full_row_count", u32), ("row_count", u32),
                ("feature_block_count", u32), ("ordering_identity", u64), ("global_row_begin", u64),
                ("feature_block_geometry_identity", u64), ("row_domain_identity", u64),
                ("row_permutation", p_void), ("inverse_row_permutation", p_void)]


class CxBellLoweringPolicy(C.Structure):
    _fields_ = [("maximum_value_slot_expansion", C.c_double), ("maximum_storage_expansion", C.c_double),
                ("maximum_persistent_bytes", u64)]


class CxBellCandidateMetrics(C.Structure):
    _fields_ = [("occupied_blocks", u64), ("stored_blocks", u64), ("dense_value_slots", u64),
                ("persistent_bytes", u64), ("source_bytes", u64), ("scalar_occupancy", C.c_double),
                ("ell_slot_utilization", C.c_double), ("value_slot_expansion", C.c_double),
                ("storage_expansion", C.c_double)]


class CxBellCandidate(C.Structure):
    _fields_ = [("state", u32), ("block_size", u32), ("row_count", u32), ("feature_count", u32),
                ("padded_row_count", u32), ("padded_feature_count", u32), ("block_row_count", u32),
                ("ell_blocks_per_row", u32), ("ell_columns", u32), ("reserved", u32),
                ("feature_block_offset_count", u64), ("column_index_count", u64), ("value_bytes", u64),
                ("candidate_identity", u64), ("metrics", CxBellCandidateMetrics)]

    def as_dict(self) -> dict:
        d = {name: getattr(self, name) for name, _ in self._fields_ if name not in ("metrics", "reserved")}
        d["metrics"] = {name: getattr(self.metrics, name) for name, _ in CxBellCandidateMetrics._fields_}
        return d


class CxBellLoweringWorkspace(C.Structure):
    _fields_ = [("marker_capacity", u64), ("markers", p_void), ("feature_block_offset_capacity", u64),
                ("feature_block_block_offsets", p_void)]


class CxBellCandidateBuffers(C.Structure):
    _fields_ = [("feature_block_offset_capacity", u64), ("padded_feature_block_offsets", p_void),
                ("column_index_capacity", u64), ("column_indices", p_void), ("value_capacity_bytes", u64),
                ("values", p_void), ("value_layout", u32)]


class CxPhysicalBellView(C.Structure):
    _fields_ = [("schema_version", u32), ("block_size", u32), ("row_count", u32), ("feature_count", u32),
                ("padded_row_count", u32), ("padded_feature_count", u32), ("ell_columns", u32),
                ("value_size_bytes", u32), ("feature_block_geometry_identity", u64), ("ordering_identity", u64),
                ("row_domain_identity", u64), ("candidate_identity", u64), ("padded_feature_block_offsets", p_void),
                ("column_indices", p_void), ("values", p_void), ("metrics", CxBellCandidateMetrics),
                ("value_layout", u32)]


_SIGS = {
    "cx_bell_lowering_workspace_requirements": (C.c_int, [C.POINTER(CxBellCsrSource), C.POINTER(CxBellSemanticPlan),
                                                          C.POINTER(CxBellRowOrder), C.POINTER(u64), C.POINTER(u64)]),
    "cx_bell_query_candidates_host": (C.c_int, [C.POINTER(CxBellCsrSource), C.POINTER(CxBellSemanticPlan),
                                                C.POINTER(CxBellRowOrder), C.POINTER(CxBellLoweringPolicy),
                                                C.POINTER(CxBellLoweringWorkspace), C.POINTER(CxBellCandidate)]),
    "cx_bell_materialize_candidate_host": (C.c_int, [C.POINTER(CxBellCsrSource), C.POINTER(CxBellSemanticPlan),
                                                     C.POINTER(CxBellRowOrder), C.POINTER(CxBellLoweringPolicy),
                                                     C.POINTER(CxBellCandidate), C.POINTER(CxBellLoweringWorkspace),
                                                     C.POINTER(CxBellCandidateBuffers),
                                                     C.POINTER(CxPhysicalBellView)]),
    "cx_bell_physical_feature_map": (C.c_int, [C.POINTER(CxPhysicalBellView), C.POINTER(CxBellSemanticPlan),
                                               p_void, u64]),
    "cx_bell_lowering_last_error": (C.c_char_p, []),
}


def _lib():
    lib = N.engine()
    if not getattr(lib, "_bell_lowering_sigs", False):
        for name, (res, args) in _SIGS.items():
            f = getattr(lib, name)
            f.restype, f.argtypes = res, args
        lib._bell_lowering_sigs = True
    return lib


class BellLoweringError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{message} (bell_lowering_status_code {code})")
        self.code = code


def _check(rc: int) -> None:
    if rc != 0:
        raise BellLoweringError(rc, _lib().cx_bell_lowering_last_error().decode())


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


class Lowering:
    """Host inputs of one lowering: canonical CSR (row_offsets, feature_ids, raw value bytes
    of value_size each), the plan's execution-order feature blocks and permutation, the local
    row order (execution row -> canonical row) and the identities the checks compare."""

    def __init__(self, row_offsets, feature_ids, values: np.ndarray, feature_count: int, block_offsets,
                 feature_permutation, row_permutation, *, geometry_identity=0x12345678,
                 row_domain_identity=0xABCDDCBA, ordering_identity=0xFEDCBA98, window_size=1024, group_width=32,
                 full_row_count: Optional[int] = None, global_row_begin: int = 0):
        self.row_offsets, self.feature_ids = _u32(row_offsets), _u32(feature_ids)
        self.values = np.ascontiguousarray(values)
        self.value_size = self.values.dtype.itemsize
        self.block_offsets = _u32(block_offsets)
        self.fperm = _u32(feature_permutation)
        self.finv = np.empty_like(self.fperm)
        self.finv[self.fperm] = np.arange(len(self.fperm), dtype=np.uint32)
        self.rperm = _u32(row_permutation)
        self.rinv = np.empty_like(self.rperm)
        self.rinv[self.rperm] = np.arange(len(self.rperm), dtype=np.uint32)
        rows = len(self.row_offsets) - 1
        self.source = CxBellCsrSource(rows, feature_count, int(self.row_offsets[-1]), self.value_size,
                                      self.row_offsets.ctypes.data, self.feature_ids.ctypes.data,
                                      self.values.ctypes.data)
        full = rows if full_row_count is None else full_row_count
        self.plan = CxBellSemanticPlan(1, full, feature_count, len(self.block_offsets) - 1, geometry_identity,
                                       row_domain_identity, self.block_offsets.ctypes.data, self.fperm.ctypes.data,
                                       self.finv.ctypes.data)
        self.order = CxBellRowOrder(1, 1, 1, window_size, group_width, full, rows, len(self.block_offsets) - 1,
                                    ordering_identity, global_row_begin, geometry_identity, row_domain_identity,
                                    self.rperm.ctypes.data, self.rinv.ctypes.data)
        mc, oc = u64(), u64()
        _check(_lib().cx_bell_lowering_workspace_requirements(C.byref(self.source), C.byref(self.plan),
                                                              C.byref(self.order), C.byref(mc), C.byref(oc)))
        self.markers = np.zeros(mc.value, np.uint32)
        self.block_scratch = np.zeros(oc.value, np.uint32)
        self.workspace = CxBellLoweringWorkspace(mc.value, self.markers.ctypes.data, oc.value,
                                                 self.block_scratch.ctypes.data)

    @staticmethod
    def policy(value_expansion=64.0, storage_expansion=64.0, persistent_bytes=(1 << 64) - 1):
        return CxBellLoweringPolicy(value_expansion, storage_expansion, persistent_bytes)

    def query(self, policy: Optional[CxBellLoweringPolicy] = None) -> list:
        out = (CxBellCandidate * 3)()
        _check(_lib().cx_bell_query_candidates_host(C.byref(self.source), C.byref(self.plan), C.byref(self.order),
                                                    C.byref(policy) if policy is not None else None,
                                                    C.byref(self.workspace), out))
        return [out[k] for k in range(3)]

    def materialize(self, candidate: CxBellCandidate, policy: Optional[CxBellLoweringPolicy] = None,
                    layout: int = VALUES_BLOCK_MAJOR):
        """(view, padded block offsets, column indices, value bytes) of a legal candidate."""
        offsets = np.zeros(max(int(candidate.feature_block_offset_count), 1), np.uint32)
        cols = np.zeros(max(int(candidate.column_index_count), 1), np.int32)
        vals = np.zeros(max(int(candidate.value_bytes), 1), np.uint8)
        bufs = CxBellCandidateBuffers(candidate.feature_block_offset_count, offsets.ctypes.data,
                                      candidate.column_index_count, cols.ctypes.data, candidate.value_bytes,
                                      vals.ctypes.data, layout)
        view = CxPhysicalBellView()
        _check(_lib().cx_bell_materialize_candidate_host(
            C.byref(self.source), C.byref(self.plan), C.byref(self.order),
            C.byref(policy) if policy is not None else None, C.byref(candidate), C.byref(self.workspace),
            C.byref(bufs), C.byref(view)))
        view._keep = (offsets, cols, vals)
        return (view, offsets[:int(candidate.feature_block_offset_count)],
                cols[:int(candidate.column_index_count)], vals[:int(candidate.value_bytes)])

    def feature_map(self, view: CxPhysicalBellView) -> np.ndarray:
        """Canonical feature of every physical feature column (-1 = padding)."""
        m = np.empty(view.padded_feature_count, np.int32)
        _check(_lib().cx_bell_physical_feature_map(C.byref(view), C.byref(self.plan), m.ctypes.data, m.size))
        return m
