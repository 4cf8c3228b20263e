// exec_csr.cpp -- host side of the execution feature order: the packed dense operand's
// descriptor and identity (include/Cellerator/compute/math/packed_dense_operand.hh:16-70),
// the execution-order CSR view of an ordered plan partition and its lazy reconstruction from
// a CPK1 image (include/Cellerator/compute/math/physical_csr.hh:40-215,
// src/compute/math/physical_csr.cc:16-240), and the gene-popularity order that puts the most
// frequently stored genes first. No device work here: the device packer and the CSR reorder
// are in exec_order.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <limits>
#include <numeric>
#include <vector>

#include "cellerator_amd.h"

namespace {

using u32 = std::uint32_t;
using u64 = std::uint64_t;

thread_local char g_error[256] = "";

int fail(int status, const char *message) {
    std::snprintf(g_error, sizeof(g_error), "%s", message);
    return status;
}

// The reference's FNV-1a constants (physical_csr.hh physical_csr_detail, packed_dense_operand.cu):
// the offset basis is the published one with its last decimal digit dropped, kept because the
// identities are part of the interchanged metadata.
constexpr u64 kFnvOffset = 1469598103934665603ull;
constexpr u64 kFnvPrime = 1099511628211ull;

void hash_u64(u64 *h, u64 v) {
    for (u32 b = 0; b < 8u; ++b) {
        *h ^= (v >> (b * 8u)) & 0xffu;
        *h *= kFnvPrime;
    }
}

bool valid_plan(const cx_cpbp_plan *plan, u64 geometry) {
    return plan != nullptr && geometry != 0u && plan->feature_block_count != 0u
        && plan->feature_block_offsets != nullptr
        && (plan->feature_count == 0u || plan->feature_permutation != nullptr)
        && plan->feature_block_offsets[0] == 0u
        && plan->feature_block_offsets[plan->feature_block_count] == plan->feature_count;
}

bool valid_value_size(u32 bytes) { return bytes == 2u || bytes == 4u || bytes == 8u; }

// validate_source + make_requirements (packed_dense_operand.cu:48-118).
int describe_packed(const cx_cpbp_plan *plan, u64 geometry, const cx_dense_operand *src,
                    cx_dense_operand *out, u64 *bytes) {
    if (src == nullptr || out == nullptr || !valid_plan(plan, geometry))
        return fail(CX_STATUS_INVALID_ARGUMENT, "packed dense operand: null descriptor or invalid plan");
    const cx_feature_order &o = src->feature_order;
    if (src->feature_count != plan->feature_count || o.schema_version != 1u
        || o.kind != CX_FEATURE_ORDER_CANONICAL || o.feature_count != src->feature_count
        || o.feature_axis_identity == 0u || o.feature_axis_identity_version == 0u
        || o.packing_geometry_identity != 0u || src->operand_identity == 0u
        || !valid_value_size(src->value_size_bytes) || src->column_major > 1u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "packed dense source metadata is invalid");
    const u64 minimum = src->column_major != 0u ? src->feature_count : src->column_count;
    if (src->feature_count != 0u && src->column_count != 0u
        && (src->values == nullptr || src->leading_dimension < minimum))
        return fail(CX_STATUS_INVALID_ARGUMENT, "packed dense source storage is invalid");
    if (src->column_count != 0u && src->feature_count > std::numeric_limits<u64>::max() / src->column_count)
        return fail(CX_STATUS_INVALID_SHAPE, "packed dense element count overflows");
    const u64 elements = static_cast<u64>(src->feature_count) * src->column_count;
    if (elements > std::numeric_limits<u64>::max() / src->value_size_bytes)
        return fail(CX_STATUS_INVALID_SHAPE, "packed dense byte count overflows");
    *bytes = elements * src->value_size_bytes;
    cx_dense_operand r = *src;
    r.values = nullptr;
    r.leading_dimension = src->column_count;
    r.column_major = 0u;
    r.feature_order.kind = CX_FEATURE_ORDER_PACKED;
    r.feature_order.packing_geometry_identity = geometry;
    u64 id = kFnvOffset;
    hash_u64(&id, 1u);  // packed_dense_operand_schema_version
    hash_u64(&id, src->operand_identity);
    hash_u64(&id, geometry);
    hash_u64(&id, o.feature_axis_identity);
    hash_u64(&id, o.feature_axis_identity_version);
    hash_u64(&id, src->feature_count);
    hash_u64(&id, src->column_count);
    hash_u64(&id, src->value_size_bytes);
    r.operand_identity = id == 0u ? 1u : id;
    *out = r;
    return CX_STATUS_SUCCESS;
}

// structure_identity (physical_csr.hh:92-110).
u64 structure_identity(u64 global_row_begin, u64 row_domain, u32 rows, u32 features, u32 nnz,
                       const u32 *row_offsets, const u32 *feature_ids) {
    u64 h = kFnvOffset;
    hash_u64(&h, 1u);  // execution_csr_structure_identity_version
    hash_u64(&h, global_row_begin);
    hash_u64(&h, row_domain);
    hash_u64(&h, rows);
    hash_u64(&h, features);
    hash_u64(&h, nnz);
    for (u32 i = 0; i <= rows; ++i) hash_u64(&h, row_offsets[i]);
    for (u32 i = 0; i < nnz; ++i) hash_u64(&h, feature_ids[i]);
    return h == 0u ? 1u : h;
}

cx_feature_order packed_order(u32 features, u64 axis, u32 axis_version, u64 geometry) {
    cx_feature_order o{};
    o.schema_version = 1u;
    o.kind = CX_FEATURE_ORDER_PACKED;
    o.feature_count = features;
    o.feature_axis_identity_version = axis_version;
    o.feature_axis_identity = axis;
    o.packing_geometry_identity = geometry;
    return o;
}

} // namespace

extern "C" {

const char *cx_exec_last_error(void) { return g_error; }

int cx_packed_dense_operand_describe(const cx_cpbp_plan *plan, uint64_t geometry_identity,
                                     const cx_dense_operand *canonical, cx_dense_operand *packed,
                                     uint64_t *value_bytes) {
    g_error[0] = '\0';
    u64 bytes = 0u;
    const int rc = describe_packed(plan, geometry_identity, canonical, packed, &bytes);
    if (rc == CX_STATUS_SUCCESS && value_bytes != nullptr) *value_bytes = bytes;
    return rc;
}

int cx_pack_dense_operand_host(const cx_cpbp_plan *plan, uint64_t geometry_identity,
                               const cx_dense_operand *canonical, void *packed, uint64_t capacity_bytes,
                               cx_dense_operand *out) {
    g_error[0] = '\0';
    cx_dense_operand r{};
    u64 bytes = 0u;
    int rc = describe_packed(plan, geometry_identity, canonical, &r, &bytes);
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (out == nullptr || (bytes != 0u && packed == canonical->values))
        return fail(CX_STATUS_INVALID_ARGUMENT, "packed dense host output is null or aliases its source");
    if (capacity_bytes < bytes || (bytes != 0u && packed == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "packed dense host buffer is too small");
    const auto *src = static_cast<const unsigned char *>(canonical->values);
    auto *dst = static_cast<unsigned char *>(packed);
    const u32 vs = canonical->value_size_bytes;
    for (u32 e = 0; e < canonical->feature_count; ++e) {
        const u32 g = plan->feature_permutation[e];
        if (g >= canonical->feature_count)
            return fail(CX_STATUS_INVALID_SHAPE, "feature permutation is out of range");
        for (u64 c = 0; c < canonical->column_count; ++c) {
            const u64 from = canonical->column_major != 0u ? c * canonical->leading_dimension + g
                                                           : static_cast<u64>(g) * canonical->leading_dimension + c;
            std::memcpy(dst + (static_cast<u64>(e) * canonical->column_count + c) * vs, src + from * vs, vs);
        }
    }
    r.values = packed;
    *out = r;
    return CX_STATUS_SUCCESS;
}

int cx_pack_dense_operand_device(const cx_cpbp_plan *device_plan, uint64_t geometry_identity,
                                 const cx_dense_operand *canonical, void *packed, uint64_t capacity_bytes,
                                 void *stream, cx_dense_operand *out) {
    g_error[0] = '\0';
    cx_dense_operand r{};
    u64 bytes = 0u;
    // The plan arrays are device-resident: validate the descriptor fields only.
    if (device_plan == nullptr || geometry_identity == 0u || device_plan->feature_block_count == 0u
        || device_plan->feature_block_offsets == nullptr
        || (device_plan->feature_count != 0u && device_plan->feature_permutation == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "packed dense device plan is invalid");
    cx_cpbp_plan shape{};
    const u32 zero_offsets[2] = {0u, device_plan->feature_count};
    shape.feature_count = device_plan->feature_count;
    shape.feature_block_count = 1u;
    shape.feature_block_offsets = zero_offsets;
    shape.feature_permutation = device_plan->feature_permutation;
    int rc = describe_packed(&shape, geometry_identity, canonical, &r, &bytes);
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (out == nullptr || (bytes != 0u && packed == canonical->values))
        return fail(CX_STATUS_INVALID_ARGUMENT, "packed dense device output is null or aliases its source");
    if (capacity_bytes < bytes || (bytes != 0u && packed == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "packed dense device buffer is too small");
    rc = cx_pack_dense_operand(device_plan->feature_permutation, canonical->feature_count, canonical->values,
                               canonical->column_count, canonical->leading_dimension, canonical->column_major,
                               canonical->value_size_bytes, packed, capacity_bytes, stream);
    if (rc != CX_STATUS_SUCCESS) return fail(rc, cx_last_error());
    r.values = packed;
    *out = r;
    return CX_STATUS_SUCCESS;
}

int cx_build_execution_csr_host(const cx_cpbp_plan *plan, uint64_t geometry_identity,
                                const cx_ordered_partition *ordered, uint32_t *execution_feature_ids,
                                uint64_t capacity, cx_execution_csr *out) {
    g_error[0] = '\0';
    if (out == nullptr || !valid_plan(plan, geometry_identity))
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution CSR requires a valid frozen plan view and output");
    if (ordered == nullptr || ordered->feature_count != plan->feature_count
        || ordered->feature_axis_fingerprint == 0u || ordered->feature_axis_fingerprint_version == 0u
        || ordered->row_offsets == nullptr || (ordered->nnz_count != 0u && ordered->value_size_bytes == 0u)
        || (ordered->nnz_count != 0u
            && (ordered->block_ids == nullptr || ordered->local_feature_ids == nullptr
                || ordered->canonical_feature_ids == nullptr || ordered->values == nullptr)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "ordered partition disagrees with the frozen feature plan");
    if (capacity < ordered->nnz_count || (ordered->nnz_count != 0u && execution_feature_ids == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution feature buffer is too small");
    if (ordered->row_offsets[0] != 0u || ordered->row_offsets[ordered->row_count] != ordered->nnz_count)
        return fail(CX_STATUS_INVALID_SHAPE, "ordered CSR row offsets do not span nnz");
    for (u32 row = 0; row < ordered->row_count; ++row) {
        const u32 begin = ordered->row_offsets[row], end = ordered->row_offsets[row + 1u];
        if (end < begin || end > ordered->nnz_count)
            return fail(CX_STATUS_INVALID_SHAPE, "ordered CSR row offsets are not monotonic");
        u32 previous = 0u;
        for (u32 i = begin; i < end; ++i) {
            const u32 block = ordered->block_ids[i];
            if (block >= plan->feature_block_count)
                return fail(CX_STATUS_INVALID_SHAPE, "ordered feature block is out of range");
            const u32 b0 = plan->feature_block_offsets[block], b1 = plan->feature_block_offsets[block + 1u];
            const u32 local = ordered->local_feature_ids[i];
            if (local >= b1 - b0) return fail(CX_STATUS_INVALID_SHAPE, "ordered local feature is out of range");
            const u32 e = b0 + local;
            if (plan->feature_permutation[e] != ordered->canonical_feature_ids[i] || (i != begin && e <= previous))
                return fail(CX_STATUS_INVALID_ARGUMENT, "ordered feature identity does not map to packed order");
            execution_feature_ids[i] = e;
            previous = e;
        }
    }
    cx_execution_csr r{};
    r.global_row_begin = ordered->global_row_begin;
    r.full_row_count = ordered->full_row_count;
    r.row_count = ordered->row_count;
    r.feature_count = ordered->feature_count;
    r.nnz_count = ordered->nnz_count;
    r.value_size_bytes = ordered->value_size_bytes;
    r.row_domain_identity = ordered->row_domain_identity;
    r.feature_order = packed_order(ordered->feature_count, ordered->feature_axis_fingerprint,
                                   ordered->feature_axis_fingerprint_version, geometry_identity);
    r.row_offsets = ordered->row_offsets;
    r.execution_feature_ids = execution_feature_ids;
    r.values = ordered->values;
    r.structure_identity = structure_identity(r.global_row_begin, r.row_domain_identity, r.row_count,
                                              r.feature_count, r.nnz_count, r.row_offsets, execution_feature_ids);
    *out = r;
    return CX_STATUS_SUCCESS;
}

int cx_lazy_execution_csr_requirements(const cx_cpk1_view *payload, cx_lazy_csr_requirements *out) {
    g_error[0] = '\0';
    if (out == nullptr || payload == nullptr || payload->payload_identity == 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "lazy CSR requirements need a validated host CPK1 view");
    const cx_cpbp_tiles &t = payload->tiles;
    const u64 vs = t.value_dtype == CELLERATOR_DTYPE_F32 ? 4u : 2u;
    cx_lazy_csr_requirements r{};
    r.row_offset_count = static_cast<u64>(t.row_count) + 1u;
    r.execution_feature_count = t.nnz_count;
    r.value_bytes = static_cast<u64>(t.nnz_count) * vs;
    r.row_cursor_count = t.row_count;
    r.total_bytes = (r.row_offset_count + r.execution_feature_count + r.row_cursor_count) * 4u + r.value_bytes;
    *out = r;
    return CX_STATUS_SUCCESS;
}

int cx_materialize_execution_csr_from_cpk1_host(const cx_cpk1_view *payload, const cx_lazy_csr_buffers *buffers,
                                                cx_execution_csr *out) {
    g_error[0] = '\0';
    cx_lazy_csr_requirements need{};
    int rc = cx_lazy_execution_csr_requirements(payload, &need);
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (out == nullptr || buffers == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "lazy CSR output is null");
    if (buffers->row_offset_capacity < need.row_offset_count
        || buffers->execution_feature_capacity < need.execution_feature_count
        || buffers->value_capacity_bytes < need.value_bytes || buffers->row_cursor_capacity < need.row_cursor_count
        || buffers->row_offsets == nullptr
        || (need.execution_feature_count != 0u && (buffers->execution_feature_ids == nullptr || buffers->values == nullptr))
        || (need.row_cursor_count != 0u && buffers->row_cursors == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "lazy CSR caller-owned buffers are too small");
    const cx_cpbp_tiles &t = payload->tiles;
    const u32 width = t.tile_row_width;
    if (width == 0u || width > 64u || t.feature_block_offsets == nullptr || t.tile_block_offsets == nullptr
        || t.block_row_entry_offsets == nullptr || t.row_block_value_offsets == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1 tile metadata is invalid");
    const bool wide = width > 32u;
    auto mask_of = [&](u32 d) -> u64 {
        return wide ? static_cast<const u64 *>(t.tile_block_cell_masks)[d]
                    : static_cast<const u32 *>(t.tile_block_cell_masks)[d];
    };
    const u64 vs = t.value_dtype == CELLERATOR_DTYPE_F32 ? 4u : 2u;
    u32 *rows = buffers->row_offsets;
    std::fill(rows, rows + need.row_offset_count, 0u);
    for (u32 tile = 0; tile < t.tile_count; ++tile) {
        const u32 d0 = t.tile_block_offsets[tile], d1 = t.tile_block_offsets[tile + 1u];
        const u32 lanes = std::min(width, t.row_count - tile * width);
        const u64 valid_cells = lanes == 64u ? ~0ull : (1ull << lanes) - 1ull;
        if (d1 < d0 || d1 > t.tile_block_count)
            return fail(CX_STATUS_INVALID_SHAPE, "CPK1 tile descriptor offsets are invalid");
        u32 previous = 0u;
        for (u32 d = d0; d < d1; ++d) {
            const u32 block = t.tile_block_ids[d];
            const u64 cells = mask_of(d);
            u32 entry = t.block_row_entry_offsets[d];
            const u32 entry_end = t.block_row_entry_offsets[d + 1u];
            if (block >= t.feature_block_count || cells == 0u || (d != d0 && block <= previous)
                || (cells & ~valid_cells) != 0u || entry_end < entry || entry_end > t.row_block_entry_count)
                return fail(CX_STATUS_INVALID_SHAPE, "CPK1 tile descriptor is invalid");
            previous = block;
            const u32 b0 = t.feature_block_offsets[block], b1 = t.feature_block_offsets[block + 1u];
            if (b1 <= b0 || b1 - b0 > 32u) return fail(CX_STATUS_INVALID_SHAPE, "CPK1 feature-block width is invalid");
            const u32 valid_genes = b1 - b0 == 32u ? ~0u : (1u << (b1 - b0)) - 1u;
            for (u32 lane = 0; lane < width; ++lane) {
                if (((cells >> lane) & 1u) == 0u) continue;
                const u32 row = tile * width + lane;
                if (row >= t.row_count || entry >= entry_end)
                    return fail(CX_STATUS_INVALID_SHAPE, "CPK1 tile row entry is invalid");
                const u32 genes = t.row_block_gene_masks[entry];
                const u32 v0 = t.row_block_value_offsets[entry], v1 = t.row_block_value_offsets[++entry];
                const u32 count = static_cast<u32>(__builtin_popcount(genes));
                if (genes == 0u || (genes & ~valid_genes) != 0u || v1 < v0 || v1 > t.nnz_count || v1 - v0 != count)
                    return fail(CX_STATUS_INVALID_SHAPE, "CPK1 row-block gene/value geometry is invalid");
                if (rows[row + 1u] > t.nnz_count || count > t.nnz_count - rows[row + 1u])
                    return fail(CX_STATUS_INVALID_SHAPE, "CPK1 row nnz count overflows");
                rows[row + 1u] += count;
            }
            if (entry != entry_end)
                return fail(CX_STATUS_INVALID_SHAPE, "CPK1 row-entry count disagrees with the cell mask");
        }
    }
    for (u32 r = 0; r < t.row_count; ++r) {
        rows[r + 1u] += rows[r];
        buffers->row_cursors[r] = rows[r];
    }
    if (rows[t.row_count] != t.nnz_count)
        return fail(CX_STATUS_INVALID_SHAPE, "CPK1 decoded row counts do not span nnz");
    const auto *src = static_cast<const unsigned char *>(t.values);
    auto *dst = static_cast<unsigned char *>(buffers->values);
    for (u32 tile = 0; tile < t.tile_count; ++tile) {
        for (u32 d = t.tile_block_offsets[tile]; d < t.tile_block_offsets[tile + 1u]; ++d) {
            const u32 b0 = t.feature_block_offsets[t.tile_block_ids[d]];
            const u64 cells = mask_of(d);
            u32 entry = t.block_row_entry_offsets[d];
            for (u32 lane = 0; lane < width; ++lane) {
                if (((cells >> lane) & 1u) == 0u) continue;
                const u32 row = tile * width + lane;
                const u32 genes = t.row_block_gene_masks[entry];
                u32 v = t.row_block_value_offsets[entry++];
                for (u32 local = 0; local < 32u; ++local) {
                    if (((genes >> local) & 1u) == 0u) continue;
                    const u32 to = buffers->row_cursors[row]++;
                    buffers->execution_feature_ids[to] = b0 + local;
                    std::memcpy(dst + static_cast<u64>(to) * vs, src + static_cast<u64>(v++) * vs, vs);
                }
            }
        }
    }
    cx_execution_csr r{};
    r.global_row_begin = payload->global_row_begin;
    r.full_row_count = payload->full_row_count;
    r.row_count = t.row_count;
    r.feature_count = t.feature_count;
    r.nnz_count = t.nnz_count;
    r.value_size_bytes = static_cast<u32>(vs);
    r.row_domain_identity = payload->row_domain_identity;
    r.feature_order = packed_order(t.feature_count, payload->feature_axis_fingerprint,
                                   payload->feature_axis_fingerprint_version,
                                   payload->feature_block_geometry_identity);
    r.row_offsets = rows;
    r.execution_feature_ids = buffers->execution_feature_ids;
    r.values = buffers->values;
    r.structure_identity = structure_identity(r.global_row_begin, r.row_domain_identity, r.row_count,
                                              r.feature_count, r.nnz_count, rows, buffers->execution_feature_ids);
    *out = r;
    return CX_STATUS_SUCCESS;
}

int cx_popularity_order(const uint32_t *counts, uint32_t genes, uint32_t *feature_permutation,
                        uint32_t *inverse_permutation) {
    g_error[0] = '\0';
    if (genes != 0u && (counts == nullptr || feature_permutation == nullptr || inverse_permutation == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_popularity_order: null argument");
    std::vector<u32> order(genes);
    std::iota(order.begin(), order.end(), 0u);
    std::stable_sort(order.begin(), order.end(), [&](u32 a, u32 b) { return counts[a] > counts[b]; });
    for (u32 e = 0; e < genes; ++e) {
        feature_permutation[e] = order[e];
        inverse_permutation[order[e]] = e;
    }
    return CX_STATUS_SUCCESS;
}

} // extern "C"
