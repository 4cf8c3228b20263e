"""CPU restatement of the reference's CSR -> Blocked-ELL lowering. TEST INFRASTRUCTURE
ONLY: imported by tests/ as the checker of cx_bell_query_candidates_host /
cx_bell_materialize_candidate_host; the engine never imports it. Plain Python loops, for
the small fixtures the tests use.

Follows:
  validate_bell_shapes      src/compute/math/physical_bell_candidates.cc:14-49
  validate                  src/compute/math/physical_bell.cc:27-80
  physical_block            src/compute/math/physical_bell_candidates.cc:62-91
  fill_physical_offsets     src/compute/math/physical_bell_candidates.cc:93-110
  candidate_identity        src/compute/math/physical_bell_candidates.cc:112-129
  evaluate                  src/compute/math/physical_bell_candidates.cc:131-212
  query_bell_candidates     src/compute/math/physical_bell_candidates.cc:216-238
  materialize_bell_candidate_host  src/compute/math/physical_bell.cc:98-200

Pinned by the reference's own vectors (tests/math_bell_lowering_test.cc:28-114 fixture;
:188-249 geometry {24, 48, 96} padded features, {256, 768, 3072} dense slots, BELL8 slot
utilization 0.75, the default policy rejecting only BELL32; :251-297 failure codes) and by
an independent decode of every materialized candidate back to the canonical dense matrix.
The source and candidate identity values have no reference vector: parity unpinned for the
identity numbers themselves (their equality across query and materialize is checked).
"""
from __future__ import annotations

import math

import numpy as np

# bell_lowering_status_code / bell_candidate_state (include/Cellerator/compute/math/physical_bell.hh:16-35)
OK, INVALID_ARGUMENT, INVALID_SOURCE, INCOMPATIBLE_PLAN, INCOMPATIBLE_ORDER = 0, 1, 2, 3, 4
INSUFFICIENT_CAPACITY, CANDIDATE_REJECTED, CANDIDATE_MISMATCH, OVERFLOW = 5, 6, 7, 8
LEGAL, EMPTY_SOURCE, VALUE_EXPANSION, STORAGE_EXPANSION, PERSISTENT_BYTES, STATE_OVERFLOW = 0, 1, 2, 3, 4, 5
SIZES = (8, 16, 32)
_FNV_OFFSET, _FNV_PRIME, _M64 = 1469598103934665603, 1099511628211, (1 << 64) - 1
I32_MAX, U32_MAX = (1 << 31) - 1, (1 << 32) - 1


class LoweringError(Exception):
    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


def _hash(h, item):
    for b in range(8):
        h ^= (item >> (8 * b)) & 0xFF
        h = (h * _FNV_PRIME) & _M64
    return h


def _check_shapes(src, plan, order):
    """physical_bell_candidates.cc:14-49"""
    if (plan["semantic_schema_version"] != 1 or plan["full_row_count"] == 0 or plan["feature_count"] == 0
            or plan["feature_block_count"] == 0 or plan["geometry_identity"] == 0
            or plan["row_domain_identity"] == 0):
        raise LoweringError(INCOMPATIBLE_PLAN, "semantic plan is incomplete")
    if (src["rows"] != order["row_count"] or src["features"] != plan["feature_count"]
            or not 0 < src["value_size"] <= 16):
        raise LoweringError(INVALID_SOURCE, "canonical CSR is invalid")
    if (order["order_schema_version"] != 1 or order["signature_algorithm_version"] != 1
            or order["ordering_identity"] == 0 or order["window_size"] == 0 or order["group_width"] == 0
            or order["full_row_count"] != plan["full_row_count"]
            or order["feature_block_count"] != plan["feature_block_count"]
            or order["geometry_identity"] != plan["geometry_identity"]
            or order["row_domain_identity"] != plan["row_domain_identity"]
            or order["global_row_begin"] > order["full_row_count"]
            or order["row_count"] > order["full_row_count"] - order["global_row_begin"]):
        raise LoweringError(INCOMPATIBLE_ORDER, "row order and plan disagree")
    off = plan["block_offsets"]
    if off[0] != 0 or off[plan["feature_block_count"]] != plan["feature_count"]:
        raise LoweringError(INCOMPATIBLE_PLAN, "feature-block endpoints are invalid")
    for b in range(plan["feature_block_count"]):
        if off[b] >= off[b + 1]:
            raise LoweringError(INCOMPATIBLE_PLAN, "feature block is empty")


def _validate(src, plan, order):
    """physical_bell.cc:27-80 (workspace capacity is the caller's business here)."""
    _check_shapes(src, plan, order)
    nf, nr = src["features"], src["rows"]
    fp, fi = plan["feature_permutation"], plan["inverse_feature_permutation"]
    seen = [False] * nf
    for e in range(nf):
        c = int(fp[e])
        if c >= nf or seen[c] or int(fi[c]) != e:
            raise LoweringError(INCOMPATIBLE_PLAN, "feature maps are not inverses")
        seen[c] = True
    rp, ri = order["row_permutation"], order["inverse_row_permutation"]
    seen = [False] * nr
    for e in range(nr):
        c = int(rp[e])
        if c >= nr or seen[c] or int(ri[c]) != e:
            raise LoweringError(INCOMPATIBLE_ORDER, "row maps are not inverses")
        seen[c] = True
    ro, ids = src["row_offsets"], src["feature_ids"]
    if ro[0] != 0 or ro[nr] != src["nnz"]:
        raise LoweringError(INVALID_SOURCE, "CSR offsets do not span nnz")
    h = _FNV_OFFSET
    for v in (nr, nf, src["nnz"], src["value_size"]):
        h = _hash(h, v)
    for r in range(nr):
        b, e = int(ro[r]), int(ro[r + 1])
        if b > e or e > src["nnz"]:
            raise LoweringError(INVALID_SOURCE, "CSR offsets are not monotone")
        h = _hash(h, b)
        for i in range(b, e):
            f = int(ids[i])
            if f >= nf or (i != b and f <= int(ids[i - 1])):
                raise LoweringError(INVALID_SOURCE, "CSR features are not unique and sorted")
            h = _hash(h, f)
    h = _hash(h, src["nnz"])
    return h if h != 0 else 1


def _physical_offsets(plan, size):
    """physical_bell_candidates.cc:93-110; None on int32 overflow."""
    off, count, out = plan["block_offsets"], 0, [0]
    for b in range(plan["feature_block_count"]):
        count += (int(off[b + 1]) - int(off[b]) + size - 1) // size
        if count > I32_MAX:
            return None
        out.append(count)
    return out


def _physical_block(plan, phys, size, canonical):
    """physical_bell_candidates.cc:62-91: semantic block by search, then local / size."""
    e = int(plan["inverse_feature_permutation"][canonical])
    off = plan["block_offsets"]
    b = 0
    while int(off[b + 1]) <= e:
        b += 1
    local = e - int(off[b])
    return phys[b] + local // size, local % size


def _evaluate(src, plan, order, policy, source_identity, size):
    """physical_bell_candidates.cc:131-212"""
    c = dict(state=STATE_OVERFLOW, block_size=size, row_count=src["rows"], feature_count=src["features"],
             padded_row_count=0, padded_feature_count=0, block_row_count=0, ell_blocks_per_row=0,
             ell_columns=0, feature_block_offset_count=plan["feature_block_count"] + 1, column_index_count=0,
             value_bytes=0, candidate_identity=0, metrics=None)
    phys = _physical_offsets(plan, size)
    if phys is None:
        return c
    block_rows = (src["rows"] + size - 1) // size
    if block_rows * size > U32_MAX or phys[-1] * size > U32_MAX:
        return c
    c.update(block_row_count=block_rows, padded_row_count=block_rows * size, padded_feature_count=phys[-1] * size)
    ro, ids, rp = src["row_offsets"], src["feature_ids"], order["row_permutation"]
    widest = occupied = 0
    for br in range(block_rows):
        active = set()
        for er in range(br * size, min(src["rows"], (br + 1) * size)):
            row = int(rp[er])
            for i in range(int(ro[row]), int(ro[row + 1])):
                active.add(_physical_block(plan, phys, size, int(ids[i]))[0])
        occupied += len(active)
        widest = max(widest, len(active))
    stored = block_rows * widest
    slots = stored * size * size
    nbytes = slots * src["value_size"]
    persistent = stored * 4 + nbytes + (plan["feature_block_count"] + 1) * 4
    source_bytes = (src["rows"] + 1) * 4 + src["nnz"] * (4 + src["value_size"])
    nnz = src["nnz"]
    c.update(ell_blocks_per_row=widest, ell_columns=widest * size, column_index_count=stored, value_bytes=nbytes)
    c["metrics"] = dict(occupied_blocks=occupied, stored_blocks=stored, dense_value_slots=slots,
                        persistent_bytes=persistent, source_bytes=source_bytes,
                        scalar_occupancy=0.0 if slots == 0 else nnz / slots,
                        ell_slot_utilization=0.0 if stored == 0 else occupied / stored,
                        value_slot_expansion=0.0 if nnz == 0 else slots / nnz,
                        storage_expansion=0.0 if source_bytes == 0 else persistent / source_bytes)
    m = c["metrics"]
    if nnz == 0:
        c["state"] = EMPTY_SOURCE
    elif m["value_slot_expansion"] > policy["maximum_value_slot_expansion"]:
        c["state"] = VALUE_EXPANSION
    elif m["storage_expansion"] > policy["maximum_storage_expansion"]:
        c["state"] = STORAGE_EXPANSION
    elif persistent > policy["maximum_persistent_bytes"]:
        c["state"] = PERSISTENT_BYTES
    else:
        c["state"] = LEGAL
    h = _FNV_OFFSET
    for v in (1, source_identity, plan["geometry_identity"], order["ordering_identity"],
              order["row_domain_identity"], size):
        h = _hash(h, v)
    for v in plan["block_offsets"]:
        h = _hash(h, int(v))
    for v in plan["feature_permutation"]:
        h = _hash(h, int(v))
    for v in order["row_permutation"]:
        h = _hash(h, int(v))
    c["candidate_identity"] = h if h != 0 else 1
    return c


DEFAULT_POLICY = dict(maximum_value_slot_expansion=64.0, maximum_storage_expansion=64.0,
                      maximum_persistent_bytes=(1 << 64) - 1)


def query_candidates(src, plan, order, policy=None):
    """physical_bell_candidates.cc:216-238: the three candidates (block sizes 8, 16, 32)."""
    policy = DEFAULT_POLICY if policy is None else policy
    if (not math.isfinite(policy["maximum_value_slot_expansion"])
            or not math.isfinite(policy["maximum_storage_expansion"])
            or policy["maximum_value_slot_expansion"] <= 0 or policy["maximum_storage_expansion"] <= 0):
        raise LoweringError(INVALID_ARGUMENT, "candidate policy is invalid")
    ident = _validate(src, plan, order)
    return [_evaluate(src, plan, order, policy, ident, s) for s in SIZES]


def materialize(src, plan, order, size, policy=None):
    """physical_bell.cc:98-200 for a freshly queried legal candidate: (padded block offsets,
    column indices [block_rows * ell] int32 with -1 = empty, block-major value bytes)."""
    cands = query_candidates(src, plan, order, policy)
    c = cands[SIZES.index(size)]
    if c["state"] != LEGAL:
        raise LoweringError(CANDIDATE_REJECTED, "candidate was rejected")
    phys = _physical_offsets(plan, size)
    ell = c["ell_blocks_per_row"]
    padded_offsets = np.array([p * size for p in phys], np.uint32)
    cols = np.full(c["column_index_count"], -1, np.int32)
    vs = src["value_size"]
    values = np.zeros(c["value_bytes"], np.uint8)
    raw = np.ascontiguousarray(src["values"]).view(np.uint8).reshape(-1)
    ro, ids, rp = src["row_offsets"], src["feature_ids"], order["row_permutation"]
    for br in range(c["block_row_count"]):
        begin, end = br * size, min(src["rows"], (br + 1) * size)
        blocks = set()
        for er in range(begin, end):
            row = int(rp[er])
            for i in range(int(ro[row]), int(ro[row + 1])):
                blocks.add(_physical_block(plan, phys, size, int(ids[i]))[0])
        slot_of = {}
        for slot, pb in enumerate(sorted(blocks)):
            slot_of[pb] = slot
            cols[br * ell + slot] = pb
        for er in range(begin, end):
            row = int(rp[er])
            for i in range(int(ro[row]), int(ro[row + 1])):
                pb, col = _physical_block(plan, phys, size, int(ids[i]))
                scalar = ((br * ell + slot_of[pb]) * size + (er - begin)) * size + col
                values[scalar * vs:(scalar + 1) * vs] = raw[i * vs:(i + 1) * vs]
    return c, padded_offsets, cols, values


def block_major_to_row_major(values: np.ndarray, block_rows: int, ell: int, size: int, value_size: int):
    """The engine's row-major cx_bell_matrix layout of the same candidate values."""
    v = values.reshape(block_rows, ell, size, size, value_size)
    return np.ascontiguousarray(v.transpose(0, 2, 1, 3, 4)).reshape(-1)
