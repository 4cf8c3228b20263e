// native_tile.cpp -- the reference's native tile adapter on the host: a read-only math
// projection of a CP-BP partition (plan, local cell order, warp tiles) with three sidecars
// per tile-block descriptor (union gene mask, packed value offset, block metrics), and the
// decoder from a packed value index back to its logical coordinate. Restates
// include/Cellerator/compute/math/native_tile_view.hh:78-136 and
// src/compute/math/native_tile_view.cc:33-251 on the engine's layout-identical mirrors of the
// reference's views (cx_fwr_plan_view, cx_local_cell_order_view, cx_warp_tile_view,
// cx_native_tile_view); the checks run in the reference's order with its messages, so a
// caller that compares messages sees the same ones. Host only: no device work.
#include "cx_common.hpp"

#include <cstring>
#include <limits>
#include <type_traits>

namespace {

using u32 = std::uint32_t;
using u64 = std::uint64_t;

// CellPack's schema versions (packing_plan.hh:9-10, local_cell_ordering.hh:9-10,
// warp_tiles.hh:10-11, cell_block_records.hh:9): all version 1.
constexpr u32 kPlanSchema = 1u, kGeometryVersion = 1u, kOrderSchema = 1u, kSignatureVersion = 1u;
constexpr u32 kTileSchema = 1u, kRecordSchema = 1u, kCellMaskBits = 32u;

// physical_view_status_code (include/Cellerator/compute/math/physical_csr.hh:17-26) as the
// engine's statuses.
int invalid_argument(const char *m) { return cx::fail(CX_STATUS_INVALID_ARGUMENT, m); }
int incompatible_identity(const char *m) { return cx::fail(CX_STATUS_INVALID_ARGUMENT, m); }
int invalid_geometry(const char *m) { return cx::fail(CX_STATUS_INVALID_SHAPE, m); }
int overflow(const char *m) { return cx::fail(CX_STATUS_INVALID_SHAPE, m); }
int insufficient_capacity(const char *m) { return cx::fail(CX_STATUS_INVALID_ARGUMENT, m); }

u32 popcount(u32 v) { return static_cast<u32>(__builtin_popcount(v)); }
u32 low_mask(u32 width) { return width >= 32u ? std::numeric_limits<u32>::max() : (1u << width) - 1u; }

// physical_csr_detail::valid_plan (physical_csr.hh:126-138)
bool valid_plan(const cx_fwr_plan_view &p) {
    return p.semantic_plan_schema_version == kPlanSchema && p.geometry_identity_version == kGeometryVersion
        && p.feature_block_geometry_identity != 0u && (p.feature_count == 0u || p.feature_permutation != nullptr)
        && p.feature_block_count != 0u && p.feature_block_offsets != nullptr && p.feature_block_offsets[0] == 0u
        && p.feature_block_offsets[p.feature_block_count] == p.feature_count;
}

// native_tile_detail::validate_source (native_tile_view.cc:33-148)
int validate_source(const cx_fwr_plan_view &plan, const cx_local_cell_order_view &order,
                    const cx_warp_tile_view &tiles) {
    if (!valid_plan(plan)) return invalid_argument("invalid native plan");
    if (order.order_schema_version != kOrderSchema || order.signature_algorithm_version != kSignatureVersion
        || order.ordering_identity == 0u || order.group_width == 0u || order.group_width > kCellMaskBits
        || order.row_count != tiles.row_count || order.feature_block_count != plan.feature_block_count
        || order.feature_block_geometry_identity != plan.feature_block_geometry_identity
        || order.ordering_identity != tiles.ordering_identity || order.global_row_begin != tiles.global_row_begin
        || order.full_row_count != tiles.full_row_count || order.row_domain_identity != tiles.row_domain_identity
        || (order.row_count != 0u && (order.row_permutation == nullptr || order.inverse_row_permutation == nullptr)))
        return incompatible_identity("incompatible native order");
    if (tiles.tile_schema_version != kTileSchema || tiles.record_schema_version != kRecordSchema
        || tiles.semantic_plan_schema_version != plan.semantic_plan_schema_version
        || tiles.geometry_identity_version != plan.geometry_identity_version
        || tiles.order_schema_version != order.order_schema_version || tiles.tile_identity == 0u
        || tiles.feature_block_geometry_identity != plan.feature_block_geometry_identity
        || tiles.feature_count != plan.feature_count || tiles.feature_block_count != plan.feature_block_count
        || tiles.tile_row_width != order.group_width
        || tiles.tile_count != tiles.row_count / tiles.tile_row_width + (tiles.row_count % tiles.tile_row_width != 0u ? 1u : 0u)
        || tiles.value_size_bytes == 0u || tiles.tile_block_offsets == nullptr || tiles.block_row_entry_offsets == nullptr
        || tiles.row_block_value_offsets == nullptr || tiles.tile_block_offsets[0] != 0u
        || tiles.tile_block_offsets[tiles.tile_count] != tiles.tile_block_count || tiles.block_row_entry_offsets[0] != 0u
        || tiles.block_row_entry_offsets[tiles.tile_block_count] != tiles.row_block_entry_count
        || tiles.row_block_value_offsets[0] != 0u
        || tiles.row_block_value_offsets[tiles.row_block_entry_count] != tiles.nnz_count
        || (tiles.tile_block_count != 0u && (tiles.tile_block_ids == nullptr || tiles.tile_block_cell_masks == nullptr))
        || (tiles.row_block_entry_count != 0u && tiles.row_block_gene_masks == nullptr)
        || (tiles.nnz_count != 0u && tiles.values == nullptr))
        return invalid_geometry("invalid native metadata");
    if (tiles.nnz_count != 0u && tiles.value_size_bytes > std::numeric_limits<std::size_t>::max() / tiles.nnz_count)
        return overflow("native value size overflow");
    for (u32 e = 0u; e < order.row_count; ++e) {
        const u32 c = order.row_permutation[e];
        if (c >= order.row_count || order.inverse_row_permutation[c] != e)
            return incompatible_identity("invalid row permutation");
    }
    for (u32 tile = 0u; tile < tiles.tile_count; ++tile) {
        const u32 begin = tiles.tile_block_offsets[tile], end = tiles.tile_block_offsets[tile + 1u];
        if (end < begin || end > tiles.tile_block_count) return invalid_geometry("invalid tile offsets");
        const u32 rows_left = tiles.row_count - tile * tiles.tile_row_width;
        const u32 valid_cells = low_mask(rows_left < tiles.tile_row_width ? rows_left : tiles.tile_row_width);
        u32 previous = std::numeric_limits<u32>::max();
        for (u32 d = begin; d < end; ++d) {
            const u32 block = tiles.tile_block_ids[d], cells = tiles.tile_block_cell_masks[d];
            const u32 e0 = tiles.block_row_entry_offsets[d], e1 = tiles.block_row_entry_offsets[d + 1u];
            if (block >= plan.feature_block_count || cells == 0u || (cells & ~valid_cells) != 0u
                || (d != begin && block <= previous) || e1 < e0 || e1 > tiles.row_block_entry_count
                || e1 - e0 != popcount(cells))
                return invalid_geometry("invalid block descriptor");
            previous = block;
            const u32 b0 = plan.feature_block_offsets[block], b1 = plan.feature_block_offsets[block + 1u];
            if (b1 <= b0 || b1 - b0 > 32u) return invalid_geometry("invalid block width");
            const u32 valid_genes = low_mask(b1 - b0);
            for (u32 e = e0; e < e1; ++e) {
                const u32 genes = tiles.row_block_gene_masks[e];
                const u32 v0 = tiles.row_block_value_offsets[e], v1 = tiles.row_block_value_offsets[e + 1u];
                if (genes == 0u || (genes & ~valid_genes) != 0u || v1 < v0 || v1 > tiles.nnz_count
                    || v1 - v0 != popcount(genes))
                    return invalid_geometry("invalid gene offsets");
            }
        }
    }
    return CX_STATUS_SUCCESS;
}

// The reference's views of a CPK1 payload, from the engine's view of the image
// (persistent_packing_payload_view's plan, order and tiles, persistent_packing_payload.hh:35-56).
int views_of_cpk1(const cx_cpk1_view *p, cx_fwr_plan_view *plan, cx_local_cell_order_view *order,
                  cx_warp_tile_view *tiles) {
    if (p == nullptr || p->payload_identity == 0u) return invalid_argument("invalid CPK1 view");
    const cx_cpbp_tiles &t = p->tiles;
    if (t.tile_row_width == 0u || t.tile_row_width > kCellMaskBits) return invalid_argument("invalid CPK1 view");
    *plan = cx_fwr_plan_view{};
    plan->semantic_plan_schema_version = kPlanSchema;
    plan->geometry_identity_version = kGeometryVersion;
    plan->feature_count = t.feature_count;
    plan->feature_block_count = t.feature_block_count;
    plan->feature_block_geometry_identity = p->feature_block_geometry_identity;
    plan->feature_block_offsets = t.feature_block_offsets;
    plan->feature_permutation = t.feature_permutation;
    if (!valid_plan(*plan)) return invalid_argument("invalid CPK1 view");
    *order = cx_local_cell_order_view{};
    order->order_schema_version = kOrderSchema;
    order->signature_algorithm_version = kSignatureVersion;
    order->kind = p->order.kind;
    order->window_size = p->order.window_size;
    order->group_width = p->order.group_width;
    order->seed = p->order.seed;
    order->ordering_identity = p->ordering_identity;
    order->global_row_begin = p->global_row_begin;
    order->full_row_count = p->full_row_count;
    order->row_count = t.row_count;
    order->feature_block_count = t.feature_block_count;
    order->feature_block_geometry_identity = p->feature_block_geometry_identity;
    order->row_domain_identity = p->row_domain_identity;
    order->row_permutation = t.row_permutation;
    order->inverse_row_permutation = p->inverse_row_permutation;
    *tiles = cx_warp_tile_view{};
    tiles->tile_schema_version = kTileSchema;
    tiles->record_schema_version = kRecordSchema;
    tiles->semantic_plan_schema_version = kPlanSchema;
    tiles->geometry_identity_version = kGeometryVersion;
    tiles->order_schema_version = kOrderSchema;
    tiles->tile_identity = p->tile_identity;
    tiles->feature_block_geometry_identity = p->feature_block_geometry_identity;
    tiles->ordering_identity = p->ordering_identity;
    tiles->global_row_begin = p->global_row_begin;
    tiles->full_row_count = p->full_row_count;
    tiles->row_count = t.row_count;
    tiles->feature_count = t.feature_count;
    tiles->feature_block_count = t.feature_block_count;
    tiles->tile_row_width = t.tile_row_width;
    tiles->tile_count = t.tile_count;
    tiles->nnz_count = t.nnz_count;
    tiles->tile_block_count = t.tile_block_count;
    tiles->row_block_entry_count = t.row_block_entry_count;
    tiles->value_size_bytes = t.value_dtype == CELLERATOR_DTYPE_F32 ? 4u : 2u;
    tiles->feature_axis_fingerprint = p->feature_axis_fingerprint;
    tiles->feature_axis_fingerprint_version = p->feature_axis_fingerprint_version;
    tiles->row_domain_identity = p->row_domain_identity;
    tiles->tile_block_offsets = t.tile_block_offsets;
    tiles->tile_block_ids = t.tile_block_ids;
    tiles->tile_block_cell_masks = static_cast<const u32 *>(t.tile_block_cell_masks);
    tiles->block_row_entry_offsets = t.block_row_entry_offsets;
    tiles->row_block_gene_masks = t.row_block_gene_masks;
    tiles->row_block_value_offsets = t.row_block_value_offsets;
    tiles->values = t.values;
    return CX_STATUS_SUCCESS;
}

} // namespace

extern "C" int cx_query_native_tile_requirements_host(const cx_fwr_plan_view *plan, const cx_local_cell_order_view *order,
                                                      const cx_warp_tile_view *tiles, cx_native_tile_requirements *out) {
    cx::clear_error();
    if (out == nullptr) return invalid_argument("null requirements output");
    if (plan == nullptr || order == nullptr || tiles == nullptr) return invalid_argument("invalid native plan");
    const int rc = validate_source(*plan, *order, *tiles);
    if (rc != CX_STATUS_SUCCESS) return rc;
    cx_native_tile_requirements r{};
    r.union_mask_count = tiles->tile_block_count;
    r.packed_offset_count = static_cast<u64>(tiles->tile_block_count) + 1u;
    r.block_metric_count = tiles->tile_block_count;
    r.sidecar_bytes = (r.union_mask_count + r.packed_offset_count) * sizeof(u32)
        + r.block_metric_count * sizeof(cx_native_tile_block_metrics);
    *out = r;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_build_native_tile_view_host(const cx_fwr_plan_view *plan, const cx_local_cell_order_view *order,
                                              const cx_warp_tile_view *tiles, const cx_native_tile_buffers *buffers,
                                              cx_native_tile_view *out) {
    cx_native_tile_requirements need{};
    int rc = cx_query_native_tile_requirements_host(plan, order, tiles, &need);
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (out == nullptr) return invalid_argument("null native output");
    if (buffers == nullptr || buffers->union_mask_capacity < need.union_mask_count
        || buffers->packed_offset_capacity < need.packed_offset_count
        || buffers->block_metric_capacity < need.block_metric_count
        || (need.union_mask_count != 0u && buffers->union_gene_masks == nullptr)
        || buffers->packed_value_offsets == nullptr
        || (need.block_metric_count != 0u && buffers->block_metrics == nullptr))
        return insufficient_capacity("small sidecar buffers");
    const cx_warp_tile_view &t = *tiles;
    u64 total = 0u;
    for (u32 d = 0u; d < t.tile_block_count; ++d) {
        const u32 e0 = t.block_row_entry_offsets[d], e1 = t.block_row_entry_offsets[d + 1u];
        u32 mask = 0u;
        for (u32 e = e0; e < e1; ++e) mask |= t.row_block_gene_masks[e];
        const u32 v0 = t.row_block_value_offsets[e0], v1 = t.row_block_value_offsets[e1];
        const u32 rows = popcount(t.tile_block_cell_masks[d]), features = popcount(mask), nnz = v1 - v0;
        const u32 work = rows * features;
        buffers->union_gene_masks[d] = mask;
        buffers->packed_value_offsets[d] = v0;
        buffers->block_metrics[d] = {rows, features, nnz, work,
                                     work == 0u ? 0.0 : static_cast<double>(nnz) / work,
                                     features == 0u ? 0.0 : static_cast<double>(nnz) / features};
        total += work;
    }
    buffers->packed_value_offsets[t.tile_block_count] = t.nnz_count;
    cx_native_tile_view v{};
    v.schema_version = CX_NATIVE_TILE_VIEW_SCHEMA;
    v.plan = *plan;
    v.order = *order;
    v.tiles = t;
    v.union_gene_masks = buffers->union_gene_masks;
    v.packed_value_offsets = buffers->packed_value_offsets;
    v.block_metrics = buffers->block_metrics;
    v.dense_workload = total;
    *out = v;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_query_native_tile_requirements_from_cpk1_host(const cx_cpk1_view *payload,
                                                                cx_native_tile_requirements *out) {
    cx::clear_error();
    cx_fwr_plan_view plan;
    cx_local_cell_order_view order;
    cx_warp_tile_view tiles;
    const int rc = views_of_cpk1(payload, &plan, &order, &tiles);
    if (rc != CX_STATUS_SUCCESS) return rc;
    return cx_query_native_tile_requirements_host(&plan, &order, &tiles, out);
}

extern "C" int cx_build_native_tile_view_from_cpk1_host(const cx_cpk1_view *payload, const cx_native_tile_buffers *buffers,
                                                        cx_native_tile_view *out) {
    cx::clear_error();
    cx_fwr_plan_view plan;
    cx_local_cell_order_view order;
    cx_warp_tile_view tiles;
    const int rc = views_of_cpk1(payload, &plan, &order, &tiles);
    if (rc != CX_STATUS_SUCCESS) return rc;
    return cx_build_native_tile_view_host(&plan, &order, &tiles, buffers, out);
}

// decode_native_tile_value_host (native_tile_view.cc:197-249)
extern "C" int cx_decode_native_tile_value_host(const cx_native_tile_view *view, uint32_t value_index,
                                                cx_native_tile_decoded_value *out) {
    cx::clear_error();
    if (out == nullptr || view == nullptr || view->schema_version != CX_NATIVE_TILE_VIEW_SCHEMA
        || value_index >= view->tiles.nnz_count)
        return invalid_argument("invalid decode request");
    int rc = validate_source(view->plan, view->order, view->tiles);
    if (rc != CX_STATUS_SUCCESS) return rc;
    const cx_warp_tile_view &t = view->tiles;
    if (view->packed_value_offsets == nullptr) return invalid_geometry("invalid native sidecars");
    for (u32 d = 0u; d <= t.tile_block_count; ++d)
        if (view->packed_value_offsets[d] != t.row_block_value_offsets[t.block_row_entry_offsets[d]])
            return invalid_geometry("invalid native sidecars");
    u32 d = 0u;
    while (view->packed_value_offsets[d + 1u] <= value_index) ++d;
    if (d >= t.tile_block_count) return invalid_geometry("invalid packed offsets");
    u32 tile = 0u;
    while (t.tile_block_offsets[tile + 1u] <= d) ++tile;
    u32 entry = t.block_row_entry_offsets[d];
    while (t.row_block_value_offsets[entry + 1u] <= value_index) ++entry;
    const u32 entry_rank = entry - t.block_row_entry_offsets[d];
    const u32 cells = t.tile_block_cell_masks[d];
    u32 lane = 0u;
    for (u32 seen = 0u; lane < t.tile_row_width; ++lane) {
        if ((cells & (1u << lane)) == 0u) continue;
        if (seen++ == entry_rank) break;
    }
    u32 gene_rank = value_index - t.row_block_value_offsets[entry];
    u32 gene = 0u;
    for (u32 mask = t.row_block_gene_masks[entry]; mask != 0u; ++gene, mask >>= 1u)
        if ((mask & 1u) != 0u && gene_rank-- == 0u) break;
    const u32 execution_row = tile * t.tile_row_width + lane;
    const u32 execution_feature = view->plan.feature_block_offsets[t.tile_block_ids[d]] + gene;
    cx_native_tile_decoded_value r{};
    r.value_index = value_index;
    r.execution_row = execution_row;
    r.canonical_row = view->order.row_permutation[execution_row];
    r.global_row = t.global_row_begin + r.canonical_row;
    r.execution_feature = execution_feature;
    r.canonical_feature = view->plan.feature_permutation[execution_feature];
    r.value = static_cast<const unsigned char *>(t.values) + static_cast<std::size_t>(value_index) * t.value_size_bytes;
    *out = r;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_cpbp_tiles_from_native_view(const cx_native_tile_view *view, cx_cpbp_tiles *out) {
    cx::clear_error();
    if (view == nullptr || out == nullptr || view->schema_version != CX_NATIVE_TILE_VIEW_SCHEMA)
        return invalid_argument("cx_cpbp_tiles_from_native_view: not a native tile view");
    const cx_warp_tile_view &t = view->tiles;
    if (t.value_size_bytes != 2u && t.value_size_bytes != 4u)
        return cx::fail(CX_STATUS_UNSUPPORTED, "cx_cpbp_tiles_from_native_view: values of 2 (f16) or 4 (f32) bytes only");
    if (t.tile_row_width == 0u || t.tile_row_width > kCellMaskBits)
        return invalid_geometry("cx_cpbp_tiles_from_native_view: tile_row_width must be 1..32");
    cx_cpbp_tiles r{};
    r.row_count = t.row_count;
    r.feature_count = t.feature_count;
    r.feature_block_count = t.feature_block_count;
    r.tile_row_width = t.tile_row_width;
    r.tile_count = t.tile_count;
    r.tile_block_count = t.tile_block_count;
    r.row_block_entry_count = t.row_block_entry_count;
    r.nnz_count = t.nnz_count;
    r.value_dtype = t.value_size_bytes == 4u ? CELLERATOR_DTYPE_F32 : CELLERATOR_DTYPE_F16;
    r.feature_block_offsets = view->plan.feature_block_offsets;
    r.feature_permutation = view->plan.feature_permutation;
    r.tile_block_offsets = t.tile_block_offsets;
    r.tile_block_ids = t.tile_block_ids;
    r.tile_block_cell_masks = t.tile_block_cell_masks;
    r.block_row_entry_offsets = t.block_row_entry_offsets;
    r.row_block_gene_masks = t.row_block_gene_masks;
    r.row_block_value_offsets = t.row_block_value_offsets;
    r.values = t.values;
    r.row_permutation = view->order.row_permutation;
    *out = r;
    return CX_STATUS_SUCCESS;
}

// A view built on a validated host image, moved to an equal copy of the image (the device
// upload): every plan, order and tile pointer inside [old_base, old_base + bytes) moves by
// new_base - old_base, as rebind_persistent_packing_payload moves the payload view's; the
// caller's sidecars and pointers outside the image stay.
extern "C" int cx_native_tile_view_rebind(const cx_native_tile_view *view, const void *old_base, uint64_t bytes,
                                          const void *new_base, cx_native_tile_view *out) {
    cx::clear_error();
    if (view == nullptr || out == nullptr || old_base == nullptr || new_base == nullptr
        || view->schema_version != CX_NATIVE_TILE_VIEW_SCHEMA)
        return invalid_argument("cx_native_tile_view_rebind: null argument or not a native tile view");
    const auto lo = reinterpret_cast<std::uintptr_t>(old_base);
    const auto to = reinterpret_cast<std::uintptr_t>(new_base);
    auto move = [&](auto *&ptr) {
        const auto at = reinterpret_cast<std::uintptr_t>(ptr);
        if (ptr != nullptr && at >= lo && at - lo < bytes)
            ptr = reinterpret_cast<std::remove_reference_t<decltype(ptr)>>(to + (at - lo));
    };
    cx_native_tile_view v = *view;
    move(v.plan.feature_block_offsets);
    move(v.plan.feature_permutation);
    move(v.order.primary_keys);
    move(v.order.secondary_keys);
    move(v.order.active_block_counts);
    move(v.order.row_nnz_counts);
    move(v.order.row_permutation);
    move(v.order.inverse_row_permutation);
    move(v.tiles.tile_block_offsets);
    move(v.tiles.tile_block_ids);
    move(v.tiles.tile_block_cell_masks);
    move(v.tiles.block_row_entry_offsets);
    move(v.tiles.row_block_gene_masks);
    move(v.tiles.row_block_value_offsets);
    move(v.tiles.values);
    *out = v;
    return CX_STATUS_SUCCESS;
}
