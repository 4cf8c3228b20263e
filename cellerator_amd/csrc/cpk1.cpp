// cpk1.cpp -- CPK1 persistent packing payload: write, validate, and rebind to a device copy.
//
// CPK1 is the reference's pointer-free on-disk / in-memory image of one packed partition
// (components/CellPack/include/CellPack/persistent_packing_payload.hh,
// components/CellPack/src/persistent_packing_payload.cc): a fixed header, then fifteen
// 64-byte-aligned sections (plan permutations and maps, row groups, row permutations, the
// warp tiles and their values). The format is external, so the header fields, section order,
// alignment, identity hashes (FNV-1a over the image with the identity field zeroed; FNV-1a
// geometry identity; splitmix64 chains for the ordering and tile identities) and the
// validation rules follow the reference exactly; the code is this engine's own.
//
// The flow mirrors the reference's: validate the image once on the host, upload its bytes
// to the device in one copy, then rebind -- every pointer of the view becomes
// device_base + section offset -- and hand the view's cx_cpbp_tiles to cx_cpbp_reduce. The
// rebind performs no copy, allocation, checksum or dereference of the new base.
// CPK1 v1 stores u32 cell masks (tile widths up to 32) and 2-byte (f16) values.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <type_traits>
#include <vector>

#include "cellerator_amd.h"

namespace {

using u32 = std::uint32_t;
using u64 = std::uint64_t;

constexpr unsigned char kMagic[8] = {'C', 'E', 'L', 'L', 'P', 'K', '0', '1'};
constexpr u32 kEndian = 0x01020304u;
constexpr u32 kAlign = 64u;
constexpr u32 kSchema = 1u;
// versions the image records (packing_plan.hh:9-10, cell_block_records.hh:9,
// local_cell_ordering.hh:9-10, warp_tiles.hh:10)
constexpr u32 kPlanSchema = 1u, kGeometryVersion = 1u, kRecordSchema = 1u, kOrderSchema = 1u,
              kSignatureVersion = 1u, kTileSchema = 1u;
// The reference's FNV-1a offset basis is 1469598103934665603 (persistent_packing_payload.cc:19,
// packing_plan.cc:11): the published 64-bit basis 14695981039346656037 with its last decimal
// digit dropped. Image identities are defined with this value, so it is kept as is.
constexpr u64 kFnvOffset = 1469598103934665603ull;
constexpr u64 kFnvPrime = 1099511628211ull;

enum Section : u32 {
    kFeaturePermutation, kInverseFeaturePermutation, kFeatureBlockOffsets, kFeatureToBlock,
    kFeatureToLocal, kRowGroupOffsets, kRowPermutation, kInverseRowPermutation,
    kTileBlockOffsets, kTileBlockIds, kTileBlockCellMasks, kBlockRowEntryOffsets,
    kRowBlockGeneMasks, kRowBlockValueOffsets, kValues, kSectionCount
};

struct Header {
    unsigned char magic[8];
    u32 schema_version, header_bytes, endian, alignment;
    u64 image_bytes, payload_identity;
    u32 semantic_plan_schema_version, geometry_identity_version, order_schema_version,
        signature_algorithm_version, tile_schema_version, record_schema_version, objective_kind,
        row_domain_kind;
    u32 full_row_count, row_count, feature_count, feature_block_count, row_group_count,
        maximum_feature_block_width, row_group_width, feature_axis_fingerprint_version;
    u64 feature_block_geometry_identity, feature_axis_fingerprint, row_domain_identity,
        evaluation_source_identity, sampling_provenance_identity, cost_policy_identity;
    u32 order_kind, order_window_size, order_group_width, reserved0;
    u64 order_seed, ordering_identity;
    u64 tile_identity, global_row_begin;
    u32 tile_row_width, tile_count, nnz_count, tile_block_count, row_block_entry_count,
        value_size_bytes, reserved1, reserved2;
    u64 offsets[kSectionCount];
};
static_assert(std::is_trivially_copyable<Header>::value, "header is copied by bytes");
static_assert(sizeof(Header) == 352u, "CPK1 header is 352 bytes");

thread_local char g_error[256] = "";

int fail(int status, const char *message) {
    std::snprintf(g_error, sizeof(g_error), "%s", message);
    return status;
}

// ---- layout -------------------------------------------------------------------------------

struct Layout {
    u64 offsets[kSectionCount]{};
    u64 total = 0u;
};

bool add(u64 *cursor, u64 count, u64 element, u64 *offset) {
    const u64 aligned = (*cursor + (kAlign - 1u)) & ~static_cast<u64>(kAlign - 1u);
    if (aligned < *cursor || (element != 0u && count > (std::numeric_limits<u64>::max() - aligned) / element))
        return false;
    *offset = aligned;
    *cursor = aligned + count * element;
    return true;
}

bool make_layout(u32 rows, u32 features, u32 blocks, u32 groups, u32 tiles, u32 tile_blocks,
                 u32 entries, u32 nnz, u32 value_bytes, Layout *out) {
    Layout l;
    u64 c = sizeof(Header);
    const u64 counts[kSectionCount] = {
        features, features, blocks + 1ull, features, features, groups + 1ull, rows, rows,
        tiles + 1ull, tile_blocks, tile_blocks, tile_blocks + 1ull, entries, entries + 1ull, nnz};
    for (u32 s = 0; s < kSectionCount; ++s)
        if (!add(&c, counts[s], s == kValues ? value_bytes : 4u, &l.offsets[s])) return false;
    l.total = (c + (kAlign - 1u)) & ~static_cast<u64>(kAlign - 1u);
    *out = l;
    return true;
}

// ---- identities ---------------------------------------------------------------------------

u64 fnv_bytes(u64 h, const void *data, u64 bytes) {
    const auto *p = static_cast<const unsigned char *>(data);
    for (u64 i = 0; i < bytes; ++i) {
        h ^= p[i];
        h *= kFnvPrime;
    }
    return h;
}

void fnv_u32(u64 *h, u32 v) {
    for (u32 b = 0; b < 4u; ++b) {
        *h ^= static_cast<unsigned char>(v >> (8u * b));
        *h *= kFnvPrime;
    }
}

u64 geometry_identity(u32 features, u32 blocks, const u32 *block_offsets, const u32 *perm) {
    u64 h = kFnvOffset;
    const char *tag = "cellerator_feature_block_geometry_identity_v1";
    h = fnv_bytes(h, tag, std::strlen(tag) + 1u);  // the literal and its terminating zero
    fnv_u32(&h, kGeometryVersion);
    fnv_u32(&h, kPlanSchema);
    fnv_u32(&h, features);
    fnv_u32(&h, blocks);
    for (u32 b = 0; b <= blocks; ++b) fnv_u32(&h, block_offsets[b]);
    for (u32 e = 0; e < features; ++e) fnv_u32(&h, perm[e]);
    return h == 0u ? 1u : h;
}

u64 image_identity(const void *image, u64 bytes) {
    Header h;
    std::memcpy(&h, image, sizeof(h));
    h.payload_identity = 0u;
    u64 id = fnv_bytes(kFnvOffset, &h, sizeof(h));
    id = fnv_bytes(id, static_cast<const unsigned char *>(image) + sizeof(h), bytes - sizeof(h));
    return id == 0u ? 1u : id;
}

u64 splitmix64(u64 v) {
    v += 0x9e3779b97f4a7c15ull;
    v = (v ^ (v >> 30u)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27u)) * 0x94d049bb133111ebull;
    return v ^ (v >> 31u);
}

// local_cell_ordering.cc compute_ordering_identity
u64 ordering_identity(u64 geometry, u64 row_domain, u64 global_row_begin, u32 rows, u32 full_rows,
                      const cx_cpbp_order_config &cfg) {
    u64 id = splitmix64(geometry);
    id = splitmix64(id ^ (static_cast<u64>(kOrderSchema) << 32u) ^ kSignatureVersion);
    id = splitmix64(id ^ row_domain);
    id = splitmix64(id ^ global_row_begin);
    id = splitmix64(id ^ (static_cast<u64>(rows) << 32u) ^ full_rows);
    id = splitmix64(id ^ (static_cast<u64>(cfg.window_size) << 32u) ^ cfg.group_width);
    id = splitmix64(id ^ cfg.seed ^ static_cast<u32>(cfg.kind));
    return id == 0u ? 1u : id;
}

// warp_tiles.cc compute_tile_identity
u64 tile_identity(u64 geometry, u64 ordering, u64 row_domain, u64 global_row_begin, u32 rows,
                  u32 full_rows, u32 features, u32 blocks, u32 group_width, u32 value_bytes) {
    u64 id = splitmix64(geometry);
    id = splitmix64(id ^ (static_cast<u64>(kTileSchema) << 32u) ^ kRecordSchema);
    id = splitmix64(id ^ ordering);
    id = splitmix64(id ^ row_domain);
    id = splitmix64(id ^ global_row_begin);
    id = splitmix64(id ^ (static_cast<u64>(rows) << 32u) ^ full_rows);
    id = splitmix64(id ^ (static_cast<u64>(features) << 32u) ^ blocks);
    id = splitmix64(id ^ (static_cast<u64>(group_width) << 32u) ^ value_bytes);
    return id == 0u ? 1u : id;
}

// ---- view ---------------------------------------------------------------------------------

template<typename T>
const T *at(const void *base, u64 offset) {
    return reinterpret_cast<const T *>(static_cast<const unsigned char *>(base) + offset);
}

void populate(const Header &h, const void *base, cx_cpk1_view *v) {
    *v = cx_cpk1_view{};
    v->payload_identity = h.payload_identity;
    v->image_base = base;
    v->image_bytes = h.image_bytes;
    v->global_row_begin = h.global_row_begin;
    v->full_row_count = h.full_row_count;
    v->row_group_count = h.row_group_count;
    v->row_group_width = h.row_group_width;
    v->maximum_feature_block_width = h.maximum_feature_block_width;
    v->feature_axis_fingerprint = h.feature_axis_fingerprint;
    v->feature_axis_fingerprint_version = h.feature_axis_fingerprint_version;
    v->row_domain_kind = h.row_domain_kind;
    v->row_domain_identity = h.row_domain_identity;
    v->feature_block_geometry_identity = h.feature_block_geometry_identity;
    v->ordering_identity = h.ordering_identity;
    v->tile_identity = h.tile_identity;
    v->order.kind = h.order_kind;
    v->order.window_size = h.order_window_size;
    v->order.group_width = h.order_group_width;
    v->order.seed = h.order_seed;
    v->order.global_row_begin = h.global_row_begin;
    v->inverse_feature_permutation = at<u32>(base, h.offsets[kInverseFeaturePermutation]);
    v->feature_to_block = at<u32>(base, h.offsets[kFeatureToBlock]);
    v->feature_to_local = at<u32>(base, h.offsets[kFeatureToLocal]);
    v->row_group_offsets = at<u32>(base, h.offsets[kRowGroupOffsets]);
    v->inverse_row_permutation = at<u32>(base, h.offsets[kInverseRowPermutation]);
    cx_cpbp_tiles &t = v->tiles;
    t.row_count = h.row_count;
    t.feature_count = h.feature_count;
    t.feature_block_count = h.feature_block_count;
    t.tile_row_width = h.tile_row_width;
    t.tile_count = h.tile_count;
    t.tile_block_count = h.tile_block_count;
    t.row_block_entry_count = h.row_block_entry_count;
    t.nnz_count = h.nnz_count;
    t.value_dtype = CELLERATOR_DTYPE_F16;
    t.feature_block_offsets = at<u32>(base, h.offsets[kFeatureBlockOffsets]);
    t.feature_permutation = at<u32>(base, h.offsets[kFeaturePermutation]);
    t.tile_block_offsets = at<u32>(base, h.offsets[kTileBlockOffsets]);
    t.tile_block_ids = at<u32>(base, h.offsets[kTileBlockIds]);
    t.tile_block_cell_masks = at<void>(base, h.offsets[kTileBlockCellMasks]);
    t.block_row_entry_offsets = at<u32>(base, h.offsets[kBlockRowEntryOffsets]);
    t.row_block_gene_masks = at<u32>(base, h.offsets[kRowBlockGeneMasks]);
    t.row_block_value_offsets = at<u32>(base, h.offsets[kRowBlockValueOffsets]);
    t.values = at<void>(base, h.offsets[kValues]);
    t.row_permutation = at<u32>(base, h.offsets[kRowPermutation]);
}

u32 lane_mask(u32 lanes) { return lanes >= 32u ? 0xffffffffu : ((1u << lanes) - 1u); }

// validate_plan_arrays / validate_tile_arrays (persistent_packing_payload.cc:317-418)
int check_arrays(const cx_cpk1_view &v) {
    const cx_cpbp_tiles &t = v.tiles;
    const u32 features = t.feature_count, blocks = t.feature_block_count;
    const u32 *boffs = t.feature_block_offsets, *perm = t.feature_permutation;
    if (boffs[0] != 0u || boffs[blocks] != features || v.row_group_offsets[0] != 0u
        || v.row_group_offsets[v.row_group_count] != v.full_row_count
        || geometry_identity(features, blocks, boffs, perm) != v.feature_block_geometry_identity)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: plan boundaries are invalid");
    for (u32 e = 0; e < features; ++e)
        if (perm[e] >= features || v.inverse_feature_permutation[perm[e]] != e)
            return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: feature permutations do not round trip");
    for (u32 b = 0; b < blocks; ++b) {
        const u32 lo = boffs[b], hi = boffs[b + 1u];
        if (hi <= lo || hi > features || hi - lo > v.maximum_feature_block_width)
            return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: feature-block width is invalid");
        for (u32 e = lo; e < hi; ++e)
            if (v.feature_to_block[perm[e]] != b || v.feature_to_local[perm[e]] != e - lo)
                return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: canonical feature maps disagree");
    }
    for (u32 g = 0; g < v.row_group_count; ++g) {
        const u32 lo = v.row_group_offsets[g], hi = v.row_group_offsets[g + 1u];
        if (hi <= lo || hi - lo > v.row_group_width || (g + 1u < v.row_group_count && hi - lo != v.row_group_width))
            return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: row-group geometry is invalid");
    }
    for (u32 r = 0; r < t.row_count; ++r)
        if (t.row_permutation[r] >= t.row_count || v.inverse_row_permutation[t.row_permutation[r]] != r)
            return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: row permutations do not round trip");
    const auto *masks = static_cast<const u32 *>(t.tile_block_cell_masks);
    if (t.tile_row_width == 0u || t.tile_row_width > 32u
        || t.tile_count != t.row_count / t.tile_row_width + (t.row_count % t.tile_row_width != 0u ? 1u : 0u)
        || t.tile_block_offsets[0] != 0u || t.tile_block_offsets[t.tile_count] != t.tile_block_count
        || t.block_row_entry_offsets[0] != 0u
        || t.block_row_entry_offsets[t.tile_block_count] != t.row_block_entry_count
        || t.row_block_value_offsets[0] != 0u
        || t.row_block_value_offsets[t.row_block_entry_count] != t.nnz_count)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: tile terminal geometry is invalid");
    for (u32 tile = 0; tile < t.tile_count; ++tile) {
        const u32 begin = t.tile_block_offsets[tile], end = t.tile_block_offsets[tile + 1u];
        if (end < begin || end > t.tile_block_count)
            return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: tile descriptor range is invalid");
        const u32 lanes = std::min(t.tile_row_width, t.row_count - tile * t.tile_row_width);
        u32 previous = 0u;
        for (u32 d = begin; d < end; ++d) {
            const u32 block = t.tile_block_ids[d], mask = masks[d];
            const u32 eb = t.block_row_entry_offsets[d], ee = t.block_row_entry_offsets[d + 1u];
            if (block >= blocks || (d != begin && block <= previous) || mask == 0u
                || (mask & ~lane_mask(lanes)) != 0u || ee < eb || ee > t.row_block_entry_count
                || ee - eb != static_cast<u32>(__builtin_popcount(mask)))
                return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: tile descriptor is invalid");
            const u32 width = boffs[block + 1u] - boffs[block];
            for (u32 e = eb; e < ee; ++e) {
                const u32 gm = t.row_block_gene_masks[e];
                const u32 vb = t.row_block_value_offsets[e], ve = t.row_block_value_offsets[e + 1u];
                if (gm == 0u || (gm & ~lane_mask(width)) != 0u || ve < vb || ve > t.nnz_count
                    || ve - vb != static_cast<u32>(__builtin_popcount(gm)))
                    return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: tile row-block entry is invalid");
            }
            previous = block;
        }
    }
    return CX_STATUS_SUCCESS;
}

} // namespace

extern "C" {

const char *cx_cpk1_last_error(void) { return g_error; }

int cx_cpk1_image_bytes(const cx_cpbp_tile_requirements *req, uint32_t row_group_count, uint64_t *bytes) {
    g_error[0] = '\0';
    if (req == nullptr || bytes == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: null argument");
    Layout l;
    if (!make_layout(req->row_count, req->feature_count, req->feature_block_count, row_group_count,
                     req->tile_count, req->tile_block_count, req->row_block_entry_count, req->nnz_count,
                     req->value_size_bytes, &l))
        return fail(CX_STATUS_INVALID_SHAPE, "CPK1: image size overflows");
    *bytes = l.total;
    return CX_STATUS_SUCCESS;
}

int cx_cpk1_validate(const void *image, uint64_t image_bytes, const cx_cpk1_expected *expected,
                     cx_cpk1_view *out) {
    g_error[0] = '\0';
    if (image == nullptr || out == nullptr || expected == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: null image, expectation or output");
    if (image_bytes < sizeof(Header)) return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: image is truncated");
    Header h;
    std::memcpy(&h, image, sizeof(h));
    if (std::memcmp(h.magic, kMagic, sizeof(kMagic)) != 0 || h.schema_version != kSchema
        || h.header_bytes != sizeof(Header) || h.endian != kEndian || h.alignment != kAlign
        || h.image_bytes != image_bytes || h.payload_identity == 0u
        || h.payload_identity != image_identity(image, image_bytes))
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: header or identity is invalid");
    if (h.semantic_plan_schema_version != kPlanSchema || h.geometry_identity_version != kGeometryVersion
        || h.order_schema_version != kOrderSchema || h.signature_algorithm_version != kSignatureVersion
        || h.tile_schema_version != kTileSchema || h.record_schema_version != kRecordSchema
        || h.feature_block_geometry_identity == 0u || h.ordering_identity == 0u || h.tile_identity == 0u
        || h.cost_policy_identity == 0u || h.full_row_count == 0u || h.row_count == 0u
        || h.feature_count == 0u || h.feature_block_count == 0u || h.row_group_count == 0u
        || h.maximum_feature_block_width == 0u || h.row_group_width == 0u
        || h.feature_axis_fingerprint == 0u || h.feature_axis_fingerprint_version == 0u
        || h.row_domain_identity == 0u || h.value_size_bytes != 2u
        || h.global_row_begin > h.full_row_count || h.row_count > h.full_row_count - h.global_row_begin
        || h.objective_kind < 1u || h.objective_kind > 3u
        || (h.row_domain_kind != 1u && h.row_domain_kind != 2u) || h.order_kind < 1u || h.order_kind > 4u
        || h.reserved0 != 0u || h.reserved1 != 0u || h.reserved2 != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: semantic metadata is invalid");
    Layout l;
    if (!make_layout(h.row_count, h.feature_count, h.feature_block_count, h.row_group_count, h.tile_count,
                     h.tile_block_count, h.row_block_entry_count, h.nnz_count, h.value_size_bytes, &l)
        || l.total != image_bytes || !std::equal(l.offsets, l.offsets + kSectionCount, h.offsets))
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: section offsets are invalid");
    if (expected->global_row_begin != h.global_row_begin || expected->row_count != h.row_count
        || expected->feature_count != h.feature_count
        || expected->feature_axis_fingerprint != h.feature_axis_fingerprint
        || expected->feature_axis_fingerprint_version != h.feature_axis_fingerprint_version
        || expected->row_domain_identity != h.row_domain_identity
        || expected->payload_identity != h.payload_identity)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: compatibility identity mismatches");
    cx_cpk1_view v;
    populate(h, image, &v);
    const int rc = check_arrays(v);
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (h.order_group_width != h.tile_row_width)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: plan/order/tile domains disagree");
    *out = v;
    return CX_STATUS_SUCCESS;
}

int cx_cpk1_rebind(const cx_cpk1_view *validated, const void *new_base, uint64_t new_bytes,
                   cx_cpk1_view *out) {
    g_error[0] = '\0';
    if (validated == nullptr || validated->image_base == nullptr || new_base == nullptr || out == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: rebind pointer is null");
    if (new_bytes != validated->image_bytes) return fail(CX_STATUS_INVALID_SHAPE, "CPK1: rebind size differs");
    const auto *old_b = static_cast<const unsigned char *>(validated->image_base);
    const auto *new_b = static_cast<const unsigned char *>(new_base);
    auto rebase = [&](const void *p) -> const void * {
        return p == nullptr ? nullptr : new_b + (static_cast<const unsigned char *>(p) - old_b);
    };
    cx_cpk1_view v = *validated;
    v.image_base = new_base;
    v.inverse_feature_permutation = static_cast<const uint32_t *>(rebase(v.inverse_feature_permutation));
    v.feature_to_block = static_cast<const uint32_t *>(rebase(v.feature_to_block));
    v.feature_to_local = static_cast<const uint32_t *>(rebase(v.feature_to_local));
    v.row_group_offsets = static_cast<const uint32_t *>(rebase(v.row_group_offsets));
    v.inverse_row_permutation = static_cast<const uint32_t *>(rebase(v.inverse_row_permutation));
    cx_cpbp_tiles &t = v.tiles;
    t.feature_block_offsets = static_cast<const uint32_t *>(rebase(t.feature_block_offsets));
    t.feature_permutation = static_cast<const uint32_t *>(rebase(t.feature_permutation));
    t.tile_block_offsets = static_cast<const uint32_t *>(rebase(t.tile_block_offsets));
    t.tile_block_ids = static_cast<const uint32_t *>(rebase(t.tile_block_ids));
    t.tile_block_cell_masks = rebase(t.tile_block_cell_masks);
    t.block_row_entry_offsets = static_cast<const uint32_t *>(rebase(t.block_row_entry_offsets));
    t.row_block_gene_masks = static_cast<const uint32_t *>(rebase(t.row_block_gene_masks));
    t.row_block_value_offsets = static_cast<const uint32_t *>(rebase(t.row_block_value_offsets));
    t.values = rebase(t.values);
    t.row_permutation = static_cast<const uint32_t *>(rebase(t.row_permutation));
    *out = v;
    return CX_STATUS_SUCCESS;
}

int cx_cpk1_write(const cx_cpbp_plan *plan, const cx_cpk1_metadata *meta,
                  const cx_cpbp_tile_requirements *req, const cx_cpbp_tile_buffers *tiles, void *image,
                  uint64_t capacity, cx_cpk1_view *out) {
    g_error[0] = '\0';
    if (plan == nullptr || meta == nullptr || req == nullptr || tiles == nullptr || image == nullptr
        || out == nullptr || plan->feature_permutation == nullptr || plan->feature_block_offsets == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: null argument");
    if (req->tile_row_width == 0u || req->tile_row_width > 32u || req->cell_mask_bytes != 4u)
        return fail(CX_STATUS_UNSUPPORTED, "CPK1 v1 stores u32 cell masks: tile widths 1..32");
    if (req->value_size_bytes != 2u) return fail(CX_STATUS_UNSUPPORTED, "CPK1 v1 stores f16 values");
    if (req->feature_count != plan->feature_count || req->feature_block_count != plan->feature_block_count)
        return fail(CX_STATUS_INVALID_SHAPE, "CPK1: tiles and plan disagree");
    if (meta->order.group_width != req->tile_row_width)
        return fail(CX_STATUS_INVALID_SHAPE, "CPK1: order group width differs from the tile width");
    if (meta->full_row_count == 0u || meta->global_row_begin > meta->full_row_count
        || req->row_count > meta->full_row_count - meta->global_row_begin)
        return fail(CX_STATUS_INVALID_SHAPE, "CPK1: partition is outside the full row domain");
    if (meta->row_group_width == 0u) return fail(CX_STATUS_INVALID_SHAPE, "CPK1: row group width is zero");
    const u32 features = plan->feature_count, blocks = plan->feature_block_count;
    // row groups: given, or uniform groups of row_group_width over the full row domain
    std::vector<u32> groups;
    if (meta->row_group_offsets != nullptr) {
        groups.assign(meta->row_group_offsets, meta->row_group_offsets + meta->row_group_count + 1u);
    } else {
        for (u32 r = 0; r < meta->full_row_count; r += meta->row_group_width) groups.push_back(r);
        groups.push_back(meta->full_row_count);
    }
    const u32 group_count = static_cast<u32>(groups.size() - 1u);
    Layout l;
    if (!make_layout(req->row_count, features, blocks, group_count, req->tile_count, req->tile_block_count,
                     req->row_block_entry_count, req->nnz_count, 2u, &l))
        return fail(CX_STATUS_INVALID_SHAPE, "CPK1: image size overflows");
    if (capacity < l.total) return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: image buffer is too small");
    // derived plan maps and the inverse row permutation
    std::vector<u32> inv_feat(features, 0xffffffffu), to_block(features, 0u), to_local(features, 0u);
    for (u32 b = 0; b < blocks; ++b)
        for (u32 e = plan->feature_block_offsets[b]; e < plan->feature_block_offsets[b + 1u] && e < features; ++e) {
            const u32 c = plan->feature_permutation[e];
            if (c >= features) return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: plan permutation is out of range");
            inv_feat[c] = e;
            to_block[c] = b;
            to_local[c] = e - plan->feature_block_offsets[b];
        }
    std::vector<u32> inv_row(req->row_count, 0xffffffffu);
    for (u32 r = 0; r < req->row_count; ++r) {
        const u32 c = tiles->row_permutation[r];
        if (c >= req->row_count) return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1: row permutation is out of range");
        inv_row[c] = r;
    }
    u32 max_width = 0u;
    for (u32 b = 0; b < blocks; ++b)
        max_width = std::max(max_width, plan->feature_block_offsets[b + 1u] - plan->feature_block_offsets[b]);
    if (meta->maximum_feature_block_width != 0u) max_width = meta->maximum_feature_block_width;

    std::memset(image, 0, l.total);
    Header h{};
    std::memcpy(h.magic, kMagic, sizeof(kMagic));
    h.schema_version = kSchema;
    h.header_bytes = sizeof(Header);
    h.endian = kEndian;
    h.alignment = kAlign;
    h.image_bytes = l.total;
    h.semantic_plan_schema_version = kPlanSchema;
    h.geometry_identity_version = kGeometryVersion;
    h.order_schema_version = kOrderSchema;
    h.signature_algorithm_version = kSignatureVersion;
    h.tile_schema_version = kTileSchema;
    h.record_schema_version = kRecordSchema;
    h.objective_kind = meta->objective_kind;
    h.row_domain_kind = meta->row_domain_kind;
    h.full_row_count = meta->full_row_count;
    h.row_count = req->row_count;
    h.feature_count = features;
    h.feature_block_count = blocks;
    h.row_group_count = group_count;
    h.maximum_feature_block_width = max_width;
    h.row_group_width = meta->row_group_width;
    h.feature_axis_fingerprint_version = meta->feature_axis_fingerprint_version;
    h.feature_block_geometry_identity = geometry_identity(features, blocks, plan->feature_block_offsets,
                                                          plan->feature_permutation);
    h.feature_axis_fingerprint = meta->feature_axis_fingerprint;
    h.row_domain_identity = meta->row_domain_identity;
    h.evaluation_source_identity = meta->evaluation_source_identity;
    h.sampling_provenance_identity = meta->sampling_provenance_identity;
    h.cost_policy_identity = meta->cost_policy_identity;
    h.order_kind = meta->order.kind;
    h.order_window_size = meta->order.window_size;
    h.order_group_width = meta->order.group_width;
    h.order_seed = meta->order.seed;
    h.ordering_identity = ordering_identity(h.feature_block_geometry_identity, meta->row_domain_identity,
                                            meta->global_row_begin, req->row_count, meta->full_row_count,
                                            meta->order);
    h.tile_identity = tile_identity(h.feature_block_geometry_identity, h.ordering_identity,
                                    meta->row_domain_identity, meta->global_row_begin, req->row_count,
                                    meta->full_row_count, features, blocks, req->tile_row_width, 2u);
    h.global_row_begin = meta->global_row_begin;
    h.tile_row_width = req->tile_row_width;
    h.tile_count = req->tile_count;
    h.nnz_count = req->nnz_count;
    h.tile_block_count = req->tile_block_count;
    h.row_block_entry_count = req->row_block_entry_count;
    h.value_size_bytes = 2u;
    std::copy(l.offsets, l.offsets + kSectionCount, h.offsets);

    auto *base = static_cast<unsigned char *>(image);
    auto put = [&](Section s, const void *src, u64 bytes) {
        if (bytes != 0u) std::memcpy(base + l.offsets[s], src, bytes);
    };
    put(kFeaturePermutation, plan->feature_permutation, features * 4ull);
    put(kInverseFeaturePermutation, inv_feat.data(), features * 4ull);
    put(kFeatureBlockOffsets, plan->feature_block_offsets, (blocks + 1ull) * 4u);
    put(kFeatureToBlock, to_block.data(), features * 4ull);
    put(kFeatureToLocal, to_local.data(), features * 4ull);
    put(kRowGroupOffsets, groups.data(), (group_count + 1ull) * 4u);
    put(kRowPermutation, tiles->row_permutation, req->row_count * 4ull);
    put(kInverseRowPermutation, inv_row.data(), req->row_count * 4ull);
    put(kTileBlockOffsets, tiles->tile_block_offsets, (req->tile_count + 1ull) * 4u);
    put(kTileBlockIds, tiles->tile_block_ids, req->tile_block_count * 4ull);
    put(kTileBlockCellMasks, tiles->tile_block_cell_masks, req->tile_block_count * 4ull);
    put(kBlockRowEntryOffsets, tiles->block_row_entry_offsets, (req->tile_block_count + 1ull) * 4u);
    put(kRowBlockGeneMasks, tiles->row_block_gene_masks, req->row_block_entry_count * 4ull);
    put(kRowBlockValueOffsets, tiles->row_block_value_offsets, (req->row_block_entry_count + 1ull) * 4u);
    put(kValues, tiles->values, req->nnz_count * 2ull);
    std::memcpy(image, &h, sizeof(h));
    h.payload_identity = image_identity(image, l.total);
    std::memcpy(image, &h, sizeof(h));
    const cx_cpk1_expected expected{meta->global_row_begin, req->row_count, features, 0u,
                                    meta->feature_axis_fingerprint, meta->feature_axis_fingerprint_version, 0u,
                                    meta->row_domain_identity, h.payload_identity};
    return cx_cpk1_validate(image, l.total, &expected, out);
}

} // extern "C"
