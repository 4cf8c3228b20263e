// bell_lowering.cpp -- CSR -> Blocked-ELL lowering on the host: the three candidates (block
// sizes 8, 16, 32) of a canonical partition CSR under a frozen plan's feature blocks and a
// local row order, their metrics and the safety rule, and materialization into caller
// buffers (include/Cellerator/compute/math/physical_bell.hh, src/compute/math/physical_bell.cc,
// src/compute/math/physical_bell_candidates.cc).
//
// What has to match the reference does: the candidate geometry (rows in execution order
// padded to a block multiple; every semantic feature block padded on its own), the slot
// order (occupied physical blocks of a block row in increasing order), the metrics and the
// order in which the safety rule rejects, the FNV-1a source and candidate identities
// (interchanged metadata: a caller may hold a candidate from another implementation), and
// the status codes and messages. The walk is the engine's own: the semantic block of every
// execution feature is tabulated once, so an entry maps to its physical block with one
// lookup and a division instead of a search, and one pass per block row both finds the
// occupied blocks and records each entry's destination.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <new>
#include <vector>

#include "cellerator_amd.h"

namespace {

using u32 = std::uint32_t;
using u64 = std::uint64_t;

thread_local char g_error[256] = "ok";

int fail(int code, const char *message) {
    std::snprintf(g_error, sizeof(g_error), "%s", message);
    return code;
}

int ok() {
    std::snprintf(g_error, sizeof(g_error), "ok");
    return CX_BELL_LOWERING_OK;
}

// FNV-1a over the little-endian bytes of 64-bit items, with the reference's offset basis
// (the published basis with its last decimal digit dropped; kept because identities are
// compared across implementations).
constexpr u64 kFnvOffset = 1469598103934665603ull;
constexpr u64 kFnvPrime = 1099511628211ull;

void mix(u64 *h, u64 v) {
    for (u32 b = 0; b < 8u; ++b) {
        *h ^= (v >> (8u * b)) & 0xffu;
        *h *= kFnvPrime;
    }
}

constexpr u32 kSizes[CX_BELL_CANDIDATE_COUNT] = {8u, 16u, 32u};
constexpr u32 kPlanSchema = 1u, kOrderSchema = 1u, kSignatureVersion = 1u;

cx_bell_lowering_policy default_policy() {
    cx_bell_lowering_policy p{};
    p.maximum_value_slot_expansion = 64.0;
    p.maximum_storage_expansion = 64.0;
    p.maximum_persistent_bytes = std::numeric_limits<u64>::max();
    return p;
}

// validate_bell_shapes (physical_bell_candidates.cc:14-49): null pointers, versions and
// cross-identities, then the plan's block endpoints.
int check_shapes(const cx_bell_csr_source &s, const cx_bell_semantic_plan &p, const cx_bell_row_order &o) {
    if (p.semantic_schema_version != kPlanSchema || p.full_row_count == 0u || p.feature_count == 0u
        || p.feature_block_count == 0u || p.feature_block_geometry_identity == 0u || p.row_domain_identity == 0u
        || p.feature_block_offsets == nullptr || p.feature_permutation == nullptr
        || p.inverse_feature_permutation == nullptr)
        return fail(CX_BELL_LOWERING_INCOMPATIBLE_PLAN, "semantic plan is incomplete");
    if (s.row_count != o.row_count || s.feature_count != p.feature_count || s.value_size_bytes == 0u
        || s.value_size_bytes > 16u || s.row_offsets == nullptr
        || (s.nnz_count != 0u && (s.feature_ids == nullptr || s.values == nullptr)))
        return fail(CX_BELL_LOWERING_INVALID_SOURCE, "canonical CSR is invalid");
    if (o.order_schema_version != kOrderSchema || o.signature_algorithm_version != kSignatureVersion
        || o.ordering_identity == 0u || o.window_size == 0u || o.group_width == 0u
        || o.full_row_count != p.full_row_count || o.feature_block_count != p.feature_block_count
        || o.feature_block_geometry_identity != p.feature_block_geometry_identity
        || o.row_domain_identity != p.row_domain_identity || o.row_permutation == nullptr
        || o.inverse_row_permutation == nullptr || o.global_row_begin > o.full_row_count
        || o.row_count > o.full_row_count - o.global_row_begin)
        return fail(CX_BELL_LOWERING_INCOMPATIBLE_ORDER, "row order and plan disagree");
    if (p.feature_block_offsets[0] != 0u || p.feature_block_offsets[p.feature_block_count] != p.feature_count)
        return fail(CX_BELL_LOWERING_INCOMPATIBLE_PLAN, "feature-block endpoints are invalid");
    for (u32 b = 0; b < p.feature_block_count; ++b)
        if (p.feature_block_offsets[b] >= p.feature_block_offsets[b + 1u])
            return fail(CX_BELL_LOWERING_INCOMPATIBLE_PLAN, "feature block is empty");
    return CX_BELL_LOWERING_OK;
}

// physical_bell_detail::validate (physical_bell.cc:27-80): workspace capacity, both
// permutation pairs are inverses, CSR offsets span and are monotone, features sorted and
// unique; the source identity hashes the shape, every row start and every feature id.
int check_all(const cx_bell_csr_source &s, const cx_bell_semantic_plan &p, const cx_bell_row_order &o,
              const cx_bell_lowering_workspace &ws, u64 *identity) {
    int rc = check_shapes(s, p, o);
    if (rc != CX_BELL_LOWERING_OK) return rc;
    const u64 markers = std::max<u64>(s.row_count, s.feature_count);
    if (ws.marker_capacity < markers || ws.markers == nullptr
        || ws.feature_block_offset_capacity < static_cast<u64>(p.feature_block_count) + 1u
        || ws.feature_block_block_offsets == nullptr)
        return fail(CX_BELL_LOWERING_INSUFFICIENT_CAPACITY, "workspace is too small");
    u32 *seen = ws.markers;
    std::fill(seen, seen + s.feature_count, 0u);
    for (u32 e = 0; e < s.feature_count; ++e) {
        const u32 c = p.feature_permutation[e];
        if (c >= s.feature_count || seen[c] != 0u || p.inverse_feature_permutation[c] != e)
            return fail(CX_BELL_LOWERING_INCOMPATIBLE_PLAN, "feature maps are not inverses");
        seen[c] = 1u;
    }
    std::fill(seen, seen + s.row_count, 0u);
    for (u32 e = 0; e < s.row_count; ++e) {
        const u32 c = o.row_permutation[e];
        if (c >= s.row_count || seen[c] != 0u || o.inverse_row_permutation[c] != e)
            return fail(CX_BELL_LOWERING_INCOMPATIBLE_ORDER, "row maps are not inverses");
        seen[c] = 1u;
    }
    if (s.row_offsets[0] != 0u || s.row_offsets[s.row_count] != s.nnz_count)
        return fail(CX_BELL_LOWERING_INVALID_SOURCE, "CSR offsets do not span nnz");
    u64 h = kFnvOffset;
    mix(&h, s.row_count);
    mix(&h, s.feature_count);
    mix(&h, s.nnz_count);
    mix(&h, s.value_size_bytes);
    for (u32 r = 0; r < s.row_count; ++r) {
        const u32 b = s.row_offsets[r], e = s.row_offsets[r + 1u];
        if (b > e || e > s.nnz_count) return fail(CX_BELL_LOWERING_INVALID_SOURCE, "CSR offsets are not monotone");
        mix(&h, b);
        for (u32 i = b; i < e; ++i) {
            const u32 f = s.feature_ids[i];
            if (f >= s.feature_count || (i != b && f <= s.feature_ids[i - 1u]))
                return fail(CX_BELL_LOWERING_INVALID_SOURCE, "CSR features are not unique and sorted");
            mix(&h, f);
        }
    }
    mix(&h, s.nnz_count);
    *identity = h == 0u ? 1u : h;
    return CX_BELL_LOWERING_OK;
}

// Physical block offsets of every semantic block for one block size (each block padded on
// its own); false when the count leaves int32 (the column index type).
bool physical_offsets(const cx_bell_semantic_plan &p, u32 size, u32 *offsets, u32 *blocks) {
    u64 count = 0u;
    offsets[0] = 0u;
    for (u32 b = 0; b < p.feature_block_count; ++b) {
        const u64 width = p.feature_block_offsets[b + 1u] - p.feature_block_offsets[b];
        count += (width + size - 1u) / size;
        if (count > static_cast<u64>(std::numeric_limits<std::int32_t>::max())) return false;
        offsets[b + 1u] = static_cast<u32>(count);
    }
    *blocks = static_cast<u32>(count);
    return true;
}

// Semantic block of every execution feature.
std::vector<u32> semantic_table(const cx_bell_semantic_plan &p) {
    std::vector<u32> t(p.feature_count);
    for (u32 b = 0; b < p.feature_block_count; ++b)
        std::fill(t.begin() + p.feature_block_offsets[b], t.begin() + p.feature_block_offsets[b + 1u], b);
    return t;
}

struct Walk {
    const cx_bell_csr_source &s;
    const cx_bell_semantic_plan &p;
    const cx_bell_row_order &o;
    const std::vector<u32> &semantic;
    const u32 *phys;  // physical block offsets of the current size
    u32 size;

    u32 physical_block(u32 canonical_feature, u32 *column_in_block) const {
        const u32 e = p.inverse_feature_permutation[canonical_feature];
        const u32 b = semantic[e];
        const u32 local = e - p.feature_block_offsets[b];
        if (column_in_block != nullptr) *column_in_block = local % size;
        return phys[b] + local / size;
    }
};

bool mul(u64 a, u64 b, u64 *out) {
    if (a != 0u && b > std::numeric_limits<u64>::max() / a) return false;
    *out = a * b;
    return true;
}

// evaluate (physical_bell_candidates.cc:131-212).
cx_bell_candidate evaluate(const cx_bell_csr_source &s, const cx_bell_semantic_plan &p, const cx_bell_row_order &o,
                           const cx_bell_lowering_policy &policy, const cx_bell_lowering_workspace &ws,
                           const std::vector<u32> &semantic, u64 source_identity, u32 size) {
    cx_bell_candidate c{};
    c.state = CX_BELL_CANDIDATE_OVERFLOW;
    c.block_size = size;
    c.row_count = s.row_count;
    c.feature_count = s.feature_count;
    c.feature_block_offset_count = static_cast<u64>(p.feature_block_count) + 1u;
    u32 blocks = 0u;
    u32 *phys = ws.feature_block_block_offsets;
    if (!physical_offsets(p, size, phys, &blocks)) return c;
    const u64 block_rows = (static_cast<u64>(s.row_count) + size - 1u) / size;
    const u64 padded_rows = block_rows * size, padded_features = static_cast<u64>(blocks) * size;
    if (padded_rows > std::numeric_limits<u32>::max() || padded_features > std::numeric_limits<u32>::max()) return c;
    c.block_row_count = static_cast<u32>(block_rows);
    c.padded_row_count = static_cast<u32>(padded_rows);
    c.padded_feature_count = static_cast<u32>(padded_features);

    // occupied blocks per block row: markers hold the epoch (block row + 1) that last saw them
    const Walk w{s, p, o, semantic, phys, size};
    std::fill(ws.markers, ws.markers + blocks, 0u);
    u32 widest = 0u;
    u64 occupied = 0u;
    for (u32 br = 0; br < c.block_row_count; ++br) {
        const u32 epoch = br + 1u;
        u32 active = 0u;
        const u32 end = std::min<u32>(s.row_count, (br + 1u) * size);
        for (u32 er = br * size; er < end; ++er) {
            const u32 row = o.row_permutation[er];
            for (u32 i = s.row_offsets[row]; i < s.row_offsets[row + 1u]; ++i) {
                const u32 pb = w.physical_block(s.feature_ids[i], nullptr);
                if (ws.markers[pb] != epoch) {
                    ws.markers[pb] = epoch;
                    ++active;
                }
            }
        }
        occupied += active;
        widest = std::max(widest, active);
    }
    c.ell_blocks_per_row = widest;
    u64 stored = 0u, slots = 0u, bytes = 0u, persistent = 0u;
    if (!mul(block_rows, widest, &stored) || !mul(stored, size, &slots) || !mul(slots, size, &slots)
        || !mul(slots, s.value_size_bytes, &bytes) || !mul(stored, sizeof(std::int32_t), &persistent)
        || persistent > std::numeric_limits<u64>::max() - bytes || widest > std::numeric_limits<u32>::max() / size)
        return c;
    persistent += bytes;
    const u64 offset_bytes = c.feature_block_offset_count * sizeof(u32);
    if (persistent > std::numeric_limits<u64>::max() - offset_bytes) return c;
    persistent += offset_bytes;
    c.ell_columns = widest * size;
    c.column_index_count = stored;
    c.value_bytes = bytes;
    const u64 source_bytes = (static_cast<u64>(s.row_count) + 1u) * 4u
        + static_cast<u64>(s.nnz_count) * (4u + s.value_size_bytes);
    cx_bell_candidate_metrics &m = c.metrics;
    m.occupied_blocks = occupied;
    m.stored_blocks = stored;
    m.dense_value_slots = slots;
    m.persistent_bytes = persistent;
    m.source_bytes = source_bytes;
    m.scalar_occupancy = slots == 0u ? 0.0 : static_cast<double>(s.nnz_count) / static_cast<double>(slots);
    m.ell_slot_utilization = stored == 0u ? 0.0 : static_cast<double>(occupied) / static_cast<double>(stored);
    m.value_slot_expansion = s.nnz_count == 0u ? 0.0 : static_cast<double>(slots) / s.nnz_count;
    m.storage_expansion = source_bytes == 0u ? 0.0 : static_cast<double>(persistent) / static_cast<double>(source_bytes);
    // the safety rule, in the reference's order
    if (s.nnz_count == 0u) c.state = CX_BELL_CANDIDATE_EMPTY_SOURCE;
    else if (m.value_slot_expansion > policy.maximum_value_slot_expansion)
        c.state = CX_BELL_CANDIDATE_VALUE_EXPANSION_EXCEEDED;
    else if (m.storage_expansion > policy.maximum_storage_expansion)
        c.state = CX_BELL_CANDIDATE_STORAGE_EXPANSION_EXCEEDED;
    else if (persistent > policy.maximum_persistent_bytes) c.state = CX_BELL_CANDIDATE_PERSISTENT_BYTES_EXCEEDED;
    else c.state = CX_BELL_CANDIDATE_LEGAL;
    // candidate_identity (physical_bell_candidates.cc:112-129)
    u64 h = kFnvOffset;
    const u64 parts[] = {CX_BELL_LOWERING_SCHEMA_VERSION, source_identity, p.feature_block_geometry_identity,
                         o.ordering_identity, o.row_domain_identity, size};
    for (const u64 v : parts) mix(&h, v);
    for (u32 b = 0; b <= p.feature_block_count; ++b) mix(&h, p.feature_block_offsets[b]);
    for (u32 f = 0; f < p.feature_count; ++f) mix(&h, p.feature_permutation[f]);
    for (u32 r = 0; r < o.row_count; ++r) mix(&h, o.row_permutation[r]);
    c.candidate_identity = h == 0u ? 1u : h;
    return c;
}

int query(const cx_bell_csr_source *s, const cx_bell_semantic_plan *p, const cx_bell_row_order *o,
          const cx_bell_lowering_policy *policy_in, const cx_bell_lowering_workspace *ws, cx_bell_candidate *out,
          std::vector<u32> *semantic_out) {
    const cx_bell_lowering_policy policy = policy_in != nullptr ? *policy_in : default_policy();
    if (out == nullptr || !std::isfinite(policy.maximum_value_slot_expansion)
        || !std::isfinite(policy.maximum_storage_expansion) || policy.maximum_value_slot_expansion <= 0.0
        || policy.maximum_storage_expansion <= 0.0)
        return fail(CX_BELL_LOWERING_INVALID_ARGUMENT, "candidate policy is invalid");
    if (s == nullptr || p == nullptr || o == nullptr || ws == nullptr)
        return fail(CX_BELL_LOWERING_INVALID_ARGUMENT, "null source, plan, order or workspace");
    u64 source_identity = 0u;
    int rc = check_all(*s, *p, *o, *ws, &source_identity);
    if (rc != CX_BELL_LOWERING_OK) return rc;
    std::vector<u32> semantic = semantic_table(*p);
    cx_bell_candidate result[CX_BELL_CANDIDATE_COUNT];
    for (u32 k = 0; k < CX_BELL_CANDIDATE_COUNT; ++k)
        result[k] = evaluate(*s, *p, *o, policy, *ws, semantic, source_identity, kSizes[k]);
    std::copy(result, result + CX_BELL_CANDIDATE_COUNT, out);
    if (semantic_out != nullptr) *semantic_out = std::move(semantic);
    return ok();
}

bool same_geometry(const cx_bell_candidate &a, const cx_bell_candidate &b) {
    return a.candidate_identity == b.candidate_identity && a.row_count == b.row_count
        && a.feature_count == b.feature_count && a.padded_row_count == b.padded_row_count
        && a.padded_feature_count == b.padded_feature_count && a.block_row_count == b.block_row_count
        && a.ell_blocks_per_row == b.ell_blocks_per_row && a.ell_columns == b.ell_columns
        && a.feature_block_offset_count == b.feature_block_offset_count
        && a.column_index_count == b.column_index_count && a.value_bytes == b.value_bytes;
}

} // namespace

extern "C" int cx_bell_lowering_workspace_requirements(const cx_bell_csr_source *source,
                                                       const cx_bell_semantic_plan *plan,
                                                       const cx_bell_row_order *order, uint64_t *marker_count,
                                                       uint64_t *feature_block_offset_count) {
    if (source == nullptr || plan == nullptr || order == nullptr || marker_count == nullptr
        || feature_block_offset_count == nullptr || source->row_count != order->row_count
        || source->feature_count != plan->feature_count || plan->feature_count == 0u
        || plan->feature_block_count == 0u)
        return fail(CX_BELL_LOWERING_INVALID_ARGUMENT, "workspace shapes are incompatible");
    *marker_count = std::max<u64>(source->row_count, source->feature_count);
    *feature_block_offset_count = static_cast<u64>(plan->feature_block_count) + 1u;
    return ok();
}

extern "C" int cx_bell_query_candidates_host(const cx_bell_csr_source *source, const cx_bell_semantic_plan *plan,
                                             const cx_bell_row_order *order, const cx_bell_lowering_policy *policy,
                                             const cx_bell_lowering_workspace *workspace, cx_bell_candidate *out) {
    try {
        return query(source, plan, order, policy, workspace, out, nullptr);
    } catch (const std::bad_alloc &) {
        return fail(CX_BELL_LOWERING_OVERFLOW, "host memory for the lowering tables is exhausted");
    }
}

extern "C" int cx_bell_materialize_candidate_host(const cx_bell_csr_source *source,
                                                  const cx_bell_semantic_plan *plan, const cx_bell_row_order *order,
                                                  const cx_bell_lowering_policy *policy,
                                                  const cx_bell_candidate *candidate,
                                                  const cx_bell_lowering_workspace *workspace,
                                                  const cx_bell_candidate_buffers *buffers,
                                                  cx_physical_bell_view *out) try {
    if (out == nullptr) return fail(CX_BELL_LOWERING_INVALID_ARGUMENT, "output is null");
    if (candidate == nullptr || buffers == nullptr)
        return fail(CX_BELL_LOWERING_INVALID_ARGUMENT, "null candidate or buffers");
    const u32 size = candidate->block_size;
    if (size != 8u && size != 16u && size != 32u)
        return fail(CX_BELL_LOWERING_CANDIDATE_MISMATCH, "candidate block size is invalid");
    cx_bell_candidate current[CX_BELL_CANDIDATE_COUNT];
    std::vector<u32> semantic;
    int rc = query(source, plan, order, policy, workspace, current, &semantic);
    if (rc != CX_BELL_LOWERING_OK) return rc;
    const cx_bell_candidate &shape = current[size == 8u ? 0 : (size == 16u ? 1 : 2)];
    if (candidate->state != CX_BELL_CANDIDATE_LEGAL || shape.state != CX_BELL_CANDIDATE_LEGAL)
        return fail(CX_BELL_LOWERING_CANDIDATE_REJECTED, "candidate was rejected");
    if (!same_geometry(*candidate, shape))
        return fail(CX_BELL_LOWERING_CANDIDATE_MISMATCH, "candidate geometry is stale");
    if (buffers->feature_block_offset_capacity < shape.feature_block_offset_count
        || buffers->padded_feature_block_offsets == nullptr || buffers->column_index_capacity < shape.column_index_count
        || (shape.column_index_count != 0u && buffers->column_indices == nullptr)
        || buffers->value_capacity_bytes < shape.value_bytes || (shape.value_bytes != 0u && buffers->values == nullptr))
        return fail(CX_BELL_LOWERING_INSUFFICIENT_CAPACITY, "output buffers are too small");
    if (buffers->value_layout != CX_BELL_VALUES_BLOCK_MAJOR && buffers->value_layout != CX_BELL_VALUES_ROW_MAJOR)
        return fail(CX_BELL_LOWERING_INVALID_ARGUMENT, "unknown value layout");

    const cx_bell_csr_source &s = *source;
    const cx_bell_semantic_plan &p = *plan;
    const cx_bell_row_order &o = *order;
    const cx_bell_lowering_workspace &ws = *workspace;
    u32 blocks = 0u;
    if (!physical_offsets(p, size, ws.feature_block_block_offsets, &blocks))
        return fail(CX_BELL_LOWERING_OVERFLOW, "physical feature padding overflowed");
    for (u32 b = 0; b <= p.feature_block_count; ++b)
        buffers->padded_feature_block_offsets[b] = ws.feature_block_block_offsets[b] * size;
    std::fill(buffers->column_indices, buffers->column_indices + shape.column_index_count, -1);
    if (shape.value_bytes != 0u) std::memset(buffers->values, 0, shape.value_bytes);
    const auto *src = static_cast<const unsigned char *>(s.values);
    auto *dst = static_cast<unsigned char *>(buffers->values);
    const u64 vs = s.value_size_bytes;
    const u64 ell = shape.ell_blocks_per_row;
    const bool row_major = buffers->value_layout == CX_BELL_VALUES_ROW_MAJOR;
    const Walk w{s, p, o, semantic, ws.feature_block_block_offsets, size};

    // per block row: mark the occupied physical blocks, number them in increasing order
    // (markers then hold slot + 1), then place every entry
    std::fill(ws.markers, ws.markers + blocks, 0u);
    std::vector<u32> touched;
    touched.reserve(ell);
    for (u32 br = 0; br < shape.block_row_count; ++br) {
        touched.clear();
        const u32 begin = br * size, end = std::min<u32>(s.row_count, begin + size);
        for (u32 er = begin; er < end; ++er) {
            const u32 row = o.row_permutation[er];
            for (u32 i = s.row_offsets[row]; i < s.row_offsets[row + 1u]; ++i) {
                const u32 pb = w.physical_block(s.feature_ids[i], nullptr);
                if (ws.markers[pb] == 0u) {
                    ws.markers[pb] = 1u;
                    touched.push_back(pb);
                }
            }
        }
        std::sort(touched.begin(), touched.end());
        for (u32 slot = 0; slot < touched.size(); ++slot) {
            ws.markers[touched[slot]] = slot + 1u;
            buffers->column_indices[static_cast<u64>(br) * ell + slot] = static_cast<std::int32_t>(touched[slot]);
        }
        for (u32 er = begin; er < end; ++er) {
            const u32 row = o.row_permutation[er];
            for (u32 i = s.row_offsets[row]; i < s.row_offsets[row + 1u]; ++i) {
                u32 col = 0u;
                const u32 pb = w.physical_block(s.feature_ids[i], &col);
                const u64 slot = ws.markers[pb] - 1u;
                const u64 scalar = row_major
                    ? static_cast<u64>(er) * (ell * size) + slot * size + col
                    : ((static_cast<u64>(br) * ell + slot) * size + (er - begin)) * size + col;
                std::memcpy(dst + scalar * vs, src + static_cast<u64>(i) * vs, vs);
            }
        }
        for (const u32 pb : touched) ws.markers[pb] = 0u;
    }
    cx_physical_bell_view v{};
    v.schema_version = CX_BELL_LOWERING_SCHEMA_VERSION;
    v.block_size = size;
    v.row_count = s.row_count;
    v.feature_count = s.feature_count;
    v.padded_row_count = shape.padded_row_count;
    v.padded_feature_count = shape.padded_feature_count;
    v.ell_columns = shape.ell_columns;
    v.value_size_bytes = s.value_size_bytes;
    v.feature_block_geometry_identity = p.feature_block_geometry_identity;
    v.ordering_identity = o.ordering_identity;
    v.row_domain_identity = o.row_domain_identity;
    v.candidate_identity = shape.candidate_identity;
    v.padded_feature_block_offsets = buffers->padded_feature_block_offsets;
    v.column_indices = buffers->column_indices;
    v.values = buffers->values;
    v.metrics = shape.metrics;
    v.value_layout = buffers->value_layout;
    *out = v;
    return ok();
} catch (const std::bad_alloc &) {
    return fail(CX_BELL_LOWERING_OVERFLOW, "host memory for the lowering tables is exhausted");
}

extern "C" int cx_bell_physical_feature_map(const cx_physical_bell_view *view, const cx_bell_semantic_plan *plan,
                                            int32_t *map, uint64_t capacity) {
    if (view == nullptr || plan == nullptr || map == nullptr || view->padded_feature_block_offsets == nullptr
        || plan->feature_block_offsets == nullptr || plan->feature_permutation == nullptr)
        return fail(CX_BELL_LOWERING_INVALID_ARGUMENT, "null view, plan or map");
    if (capacity < view->padded_feature_count)
        return fail(CX_BELL_LOWERING_INSUFFICIENT_CAPACITY, "map is too small");
    if (view->feature_count != plan->feature_count
        || view->feature_block_geometry_identity != plan->feature_block_geometry_identity
        || view->padded_feature_block_offsets[plan->feature_block_count] != view->padded_feature_count)
        return fail(CX_BELL_LOWERING_CANDIDATE_MISMATCH, "view and plan disagree");
    for (u32 b = 0; b < plan->feature_block_count; ++b) {
        const u32 p0 = view->padded_feature_block_offsets[b], p1 = view->padded_feature_block_offsets[b + 1u];
        const u32 width = plan->feature_block_offsets[b + 1u] - plan->feature_block_offsets[b];
        if (p1 < p0 || p1 - p0 < width)
            return fail(CX_BELL_LOWERING_CANDIDATE_MISMATCH, "view and plan disagree");
        for (u32 k = 0; k < p1 - p0; ++k)
            map[p0 + k] = k < width ? static_cast<int32_t>(plan->feature_permutation[plan->feature_block_offsets[b] + k]) : -1;
    }
    return ok();
}

extern "C" const char *cx_bell_lowering_last_error(void) { return g_error; }
