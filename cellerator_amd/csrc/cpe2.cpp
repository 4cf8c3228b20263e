// cpe2.cpp -- the CPE2 execution image (schema v2): a pointer-free container holding one
// biological relation / semantic geometry and a directory of concrete projections of it
// (components/CellPack/include/CellPack/persistence/EXECUTION_IMAGE_V2.md,
// execution_image_v2.hh, src/persistence/execution_image_v2.cc and
// execution_image_v2_cpk1.cc).
//
// The byte format is the reference's because images are interchanged: the 256-byte header
// (magic "CELLEX02", schema 2, endian marker, 64-byte alignment, identities, axis records,
// directory offsets), 64-byte section and projection entries, sections placed in directory
// order each at its own power-of-two alignment after the 64-aligned directories, the image
// padded to 64 bytes, a nonzero FNV-1a checksum per section and an FNV-1a image identity
// over the whole image with its identity field read as zero (the reference's offset basis).
// The checks are the reference's too, with its messages: foundational section cardinality,
// unknown kinds only when optional, alignment and bounds, non-overlap, unique identities,
// projection references, lazy projections without bytes, caller identities.
//
// Device use: the whole image goes to the device in one opaque copy; cx_cpe2_rebind moves
// the directory pointers, and cx_cpe2_prebind_for_base forms a projection's hot pointers
// as destination base + validated section offset without touching the destination. A
// native row-masked projection whose payload is a CPK1 section (cx_cpe2_load_cpk1) is
// consumed by the CP-BP reduction after cx_cpk1_rebind to that device address.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <limits>

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
    return CX_STATUS_SUCCESS;
}

static_assert(sizeof(cx_cpe2_header) == 256u, "the CPE2 header is 256 bytes");
static_assert(sizeof(cx_cpe2_section_entry) == 64u && sizeof(cx_cpe2_projection_entry) == 64u,
              "CPE2 directory entries are 64 bytes");
static_assert(offsetof(cx_cpe2_header, image_identity) == 32u, "image identity field offset");

constexpr unsigned char kMagic[8] = {'C', 'E', 'L', 'L', 'E', 'X', '0', '2'};
constexpr u64 kFnvOffset = 1469598103934665603ull;  // the reference's basis (published one, last digit dropped)
constexpr u64 kFnvPrime = 1099511628211ull;
constexpr u32 kMaxSectionAlignment = 4096u;

u64 fnv(u64 h, const void *data, std::size_t n) {
    const auto *p = static_cast<const unsigned char *>(data);
    for (std::size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= kFnvPrime;
    }
    return h;
}

u64 checksum(const void *data, std::size_t n) {
    const u64 h = fnv(kFnvOffset, data, n);
    return h == 0u ? 1u : h;
}

// FNV-1a of the image with the 8 identity bytes read as zero.
u64 image_identity(const void *image, std::size_t bytes) {
    constexpr std::size_t at = offsetof(cx_cpe2_header, image_identity);
    const auto *b = static_cast<const unsigned char *>(image);
    const u64 zero = 0u;
    u64 h = fnv(kFnvOffset, b, at);
    h = fnv(h, &zero, sizeof(zero));
    h = fnv(h, b + at + 8u, bytes - at - 8u);
    return h == 0u ? 1u : h;
}

bool pow2(u32 v) { return v != 0u && (v & (v - 1u)) == 0u; }
bool present(u64 lo, u64 hi) { return lo != 0u || hi != 0u; }
bool present(const cx_cpe2_id &id) { return present(id.low, id.high); }
bool same(u64 a_lo, u64 a_hi, u64 b_lo, u64 b_hi) { return a_lo == b_lo && a_hi == b_hi; }
bool known_section(u32 k) { return k >= CX_CPE2_SECTION_DOMAIN_TABLE && k <= CX_CPE2_SECTION_CPK1_V1_COMPATIBILITY; }
bool known_projection(u32 k) { return k >= CX_CPE2_PROJECTION_NATIVE_ROW_MASKED && k <= CX_CPE2_PROJECTION_ARCHITECTURE_SPECIFIC; }

bool add(std::size_t a, std::size_t b, std::size_t *out) {
    if (b > std::numeric_limits<std::size_t>::max() - a) return false;
    *out = a + b;
    return true;
}

bool mul(std::size_t a, std::size_t b, std::size_t *out) {
    if (a != 0u && b > std::numeric_limits<std::size_t>::max() / a) return false;
    *out = a * b;
    return true;
}

bool align_up(std::size_t at, u32 alignment, std::size_t *out) {
    if (!pow2(alignment)) return false;
    const std::size_t m = alignment - 1u;
    if (at > std::numeric_limits<std::size_t>::max() - m) return false;
    *out = (at + m) & ~m;
    return true;
}

// validate_persistent_axis_identity (include/Cellerator/execution/identity.hh:183-196).
bool valid_axis(const cx_cpe2_axis_identity &a) {
    return a.schema_version == 1u && a.record_kind == 1u && a.byte_count == sizeof(cx_cpe2_axis_identity)
        && present(a.domain) && present(a.order) && present(a.geometry) && present(a.partition);
}

cx_cpe2_axis_record record_of(const cx_cpe2_axis_identity &a) {
    return {a.domain.low, a.domain.high, a.order.low, a.order.high, a.geometry.low, a.geometry.high,
            a.partition.low, a.partition.high};
}

u32 count_kind(const cx_cpe2_section_source *s, u32 n, u32 kind) {
    u32 c = 0u;
    for (u32 i = 0; i < n; ++i) c += s[i].kind == kind ? 1u : 0u;
    return c;
}

bool is_payload_kind(u32 kind) {
    return kind == CX_CPE2_SECTION_PROJECTION_PAYLOAD || kind == CX_CPE2_SECTION_CPK1_V1_COMPATIBILITY;
}

// The projection's section references, given a lookup of section kinds.
template<typename KindOf>
int check_projection(const cx_cpe2_projection_entry &e, u32 section_count, KindOf kind_of, bool image) {
    if (!present(e.identity_low, e.identity_high) || e.schema_version == 0u
        || (!known_projection(e.kind) && (e.flags & CX_CPE2_DIRECTORY_OPTIONAL) == 0u))
        return fail(CX_STATUS_INVALID_ARGUMENT, image ? "execution image projection directory is invalid"
                                                      : "execution image projection descriptor is invalid");
    const bool has_payload = e.payload_section != CX_CPE2_INVALID_INDEX;
    const bool payload_ok = e.payload_section < section_count && is_payload_kind(kind_of(e.payload_section));
    if (has_payload != payload_ok)
        return fail(CX_STATUS_INVALID_ARGUMENT, image ? "execution image projection payload is invalid"
                                                      : "execution image projection payload reference is invalid");
    if (!has_payload && (e.flags & CX_CPE2_PROJECTION_LAZY_CONSTRUCTIBLE) == 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, image ? "execution image projection payload is invalid"
                                                      : "projection without bytes must be lazy-constructible");
    auto ref = [&](u32 index, u32 kind) {
        return index == CX_CPE2_INVALID_INDEX || (index < section_count && kind_of(index) == kind);
    };
    if (!ref(e.forward_map_section, CX_CPE2_SECTION_FORWARD_VALUE_MAP))
        return fail(CX_STATUS_INVALID_ARGUMENT, image ? "execution image forward map is invalid"
                                                      : "projection forward map reference is invalid");
    if (!ref(e.transpose_map_section, CX_CPE2_SECTION_TRANSPOSE_VALUE_MAP))
        return fail(CX_STATUS_INVALID_ARGUMENT, image ? "execution image transpose map is invalid"
                                                      : "projection transpose map reference is invalid");
    if (!ref(e.scheduling_summary_section, CX_CPE2_SECTION_SCHEDULING_SUMMARY))
        return fail(CX_STATUS_INVALID_ARGUMENT, image ? "execution image scheduling summary is invalid"
                                                      : "projection scheduling summary reference is invalid");
    if (e.capability_section != CX_CPE2_INVALID_INDEX && e.capability_section >= section_count)
        return fail(CX_STATUS_INVALID_ARGUMENT, image ? "execution image projection capability is invalid"
                                                      : "projection capability reference is invalid");
    return CX_STATUS_SUCCESS;
}

// validate_request (execution_image_v2.cc:120-211).
int check_request(const cx_cpe2_build_request &r) {
    if (!present(r.structure_identity) || r.structure_epoch == 0u || !present(r.semantic_geometry_identity)
        || !present(r.projection_catalog_identity))
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image semantic identity is invalid");
    if (!valid_axis(r.source_axis) || !valid_axis(r.destination_axis))
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image axis identity is invalid");
    if (r.sections == nullptr || r.section_count == 0u || r.projections == nullptr || r.projection_count == 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image requires section and projection directories");
    const u32 n = r.section_count;
    const u32 initial = count_kind(r.sections, n, CX_CPE2_SECTION_INITIAL_VALUES);
    if (count_kind(r.sections, n, CX_CPE2_SECTION_DOMAIN_TABLE) != 1u
        || count_kind(r.sections, n, CX_CPE2_SECTION_ORDER_PARTITION_TABLE) != 1u
        || count_kind(r.sections, n, CX_CPE2_SECTION_RELATION_STRUCTURE) != 1u
        || count_kind(r.sections, n, CX_CPE2_SECTION_SEMANTIC_GEOMETRY) != 1u || initial > 1u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image foundational sections are incomplete or duplicated");
    if ((initial == 0u) != (r.initial_value_generation == 0u))
        return fail(CX_STATUS_INVALID_ARGUMENT, "initial values and value generation must be present together");
    for (u32 i = 0; i < n; ++i) {
        const cx_cpe2_section_source &s = r.sections[i];
        if ((!known_section(s.kind) && (s.flags & CX_CPE2_DIRECTORY_OPTIONAL) == 0u) || s.schema_version == 0u
            || !pow2(s.alignment) || s.alignment > kMaxSectionAlignment || !present(s.identity_low, s.identity_high)
            || s.data == nullptr || s.bytes == 0u)
            return fail(CX_STATUS_INVALID_ARGUMENT, "execution image section source is invalid");
        if ((s.element_count == 0u) != (s.element_bytes == 0u))
            return fail(CX_STATUS_INVALID_ARGUMENT, "execution image section element shape is partial");
        std::size_t shaped = 0u;
        if (s.element_count != 0u && (!mul(s.element_count, s.element_bytes, &shaped) || shaped != s.bytes))
            return fail(CX_STATUS_INVALID_ARGUMENT, "execution image section element shape mismatches bytes");
        for (u32 j = 0; j < i; ++j)
            if (same(s.identity_low, s.identity_high, r.sections[j].identity_low, r.sections[j].identity_high))
                return fail(CX_STATUS_INVALID_ARGUMENT, "execution image section identity is duplicated");
    }
    auto kind_of = [&](u32 index) { return r.sections[index].kind; };
    for (u32 i = 0; i < r.projection_count; ++i) {
        const cx_cpe2_projection_entry &e = r.projections[i];
        const int rc = check_projection(e, n, kind_of, false);
        if (rc != CX_STATUS_SUCCESS) return rc;
        for (u32 j = 0; j < i; ++j)
            if (same(e.identity_low, e.identity_high, r.projections[j].identity_low, r.projections[j].identity_high))
                return fail(CX_STATUS_INVALID_ARGUMENT, "execution image projection identity is duplicated");
    }
    return CX_STATUS_SUCCESS;
}

struct Layout {
    std::size_t projection_offset, first_section, image_bytes, directory_bytes, section_bytes, padding;
};

// compute_layout (execution_image_v2.cc:213-252): header, section directory, projection
// directory at 64, sections each at its own alignment, image rounded up to 64.
int layout_of(const cx_cpe2_build_request &r, Layout *out) {
    std::size_t sdir = 0u, pdir = 0u;
    if (!mul(r.section_count, sizeof(cx_cpe2_section_entry), &sdir)
        || !mul(r.projection_count, sizeof(cx_cpe2_projection_entry), &pdir))
        return fail(CX_STATUS_INVALID_SHAPE, "execution image directory byte count overflows");
    Layout L{};
    std::size_t at = sizeof(cx_cpe2_header);
    if (!add(at, sdir, &at) || !align_up(at, CX_CPE2_ALIGNMENT, &L.projection_offset)
        || !add(L.projection_offset, pdir, &at) || !align_up(at, CX_CPE2_ALIGNMENT, &L.first_section))
        return fail(CX_STATUS_INVALID_SHAPE, "execution image directory layout overflows");
    at = L.first_section;
    L.padding = L.first_section - sizeof(cx_cpe2_header) - sdir - pdir;
    for (u32 i = 0; i < r.section_count; ++i) {
        std::size_t aligned = 0u;
        if (!align_up(at, r.sections[i].alignment, &aligned))
            return fail(CX_STATUS_INVALID_SHAPE, "execution image section alignment overflows");
        L.padding += aligned - at;
        if (!add(L.section_bytes, static_cast<std::size_t>(r.sections[i].bytes), &L.section_bytes)
            || !add(aligned, static_cast<std::size_t>(r.sections[i].bytes), &at))
            return fail(CX_STATUS_INVALID_SHAPE, "execution image section byte count overflows");
    }
    std::size_t end = 0u;
    if (!align_up(at, CX_CPE2_ALIGNMENT, &end))
        return fail(CX_STATUS_INVALID_SHAPE, "execution image terminal alignment overflows");
    L.padding += end - at;
    L.image_bytes = end;
    L.directory_bytes = sdir + pdir;
    *out = L;
    return CX_STATUS_SUCCESS;
}

bool in_range(u64 offset, u64 bytes, u64 total) { return offset <= total && bytes <= total - offset; }

} // namespace

extern "C" int cx_cpe2_query_requirements(const cx_cpe2_build_request *request, cx_cpe2_requirements *out) {
    if (out == nullptr || request == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image requirements output is null");
    int rc = check_request(*request);
    if (rc != CX_STATUS_SUCCESS) return rc;
    Layout L;
    rc = layout_of(*request, &L);
    if (rc != CX_STATUS_SUCCESS) return rc;
    *out = {L.image_bytes, L.directory_bytes, L.section_bytes, L.padding};
    return ok();
}

extern "C" int cx_cpe2_build(const cx_cpe2_build_request *request, void *image, uint64_t capacity,
                             cx_cpe2_view *out) {
    if (image == nullptr || out == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image buffer or output is null");
    cx_cpe2_requirements req;
    int rc = cx_cpe2_query_requirements(request, &req);
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (capacity < req.image_bytes) return fail(CX_STATUS_INVALID_SHAPE, "execution image buffer is too small");
    const cx_cpe2_build_request &r = *request;
    Layout L;
    (void)layout_of(r, &L);
    auto *base = static_cast<unsigned char *>(image);
    std::memset(base, 0, L.image_bytes);
    cx_cpe2_header h{};
    std::memcpy(h.magic, kMagic, sizeof(kMagic));
    h.schema_version = CX_CPE2_SCHEMA_VERSION;
    h.header_bytes = sizeof(h);
    h.endian = CX_CPE2_ENDIAN_MARKER;
    h.alignment = CX_CPE2_ALIGNMENT;
    h.image_bytes = L.image_bytes;
    h.structure_identity_low = r.structure_identity.low;
    h.structure_identity_high = r.structure_identity.high;
    h.structure_epoch = r.structure_epoch;
    h.semantic_geometry_identity_low = r.semantic_geometry_identity.low;
    h.semantic_geometry_identity_high = r.semantic_geometry_identity.high;
    h.projection_catalog_identity_low = r.projection_catalog_identity.low;
    h.projection_catalog_identity_high = r.projection_catalog_identity.high;
    h.initial_value_generation = r.initial_value_generation;
    h.source_axis = record_of(r.source_axis);
    h.destination_axis = record_of(r.destination_axis);
    h.section_count = r.section_count;
    h.projection_count = r.projection_count;
    h.section_directory_offset = sizeof(h);
    h.projection_directory_offset = L.projection_offset;
    std::size_t at = L.first_section;
    for (u32 i = 0; i < r.section_count; ++i) {
        const cx_cpe2_section_source &s = r.sections[i];
        (void)align_up(at, s.alignment, &at);
        const cx_cpe2_section_entry e{s.kind, s.schema_version, s.flags, s.alignment, s.identity_low,
                                      s.identity_high, at, s.bytes, checksum(s.data, static_cast<std::size_t>(s.bytes)),
                                      s.element_count, s.element_bytes};
        std::memcpy(base + h.section_directory_offset + i * sizeof(e), &e, sizeof(e));
        std::memcpy(base + at, s.data, static_cast<std::size_t>(s.bytes));
        at += static_cast<std::size_t>(s.bytes);
    }
    std::memcpy(base + h.projection_directory_offset, r.projections,
                static_cast<std::size_t>(r.projection_count) * sizeof(cx_cpe2_projection_entry));
    std::memcpy(base, &h, sizeof(h));
    h.image_identity = image_identity(base, L.image_bytes);
    std::memcpy(base, &h, sizeof(h));
    const cx_cpe2_expected expected{r.structure_identity, r.structure_epoch, r.semantic_geometry_identity,
                                    r.projection_catalog_identity, h.image_identity};
    return cx_cpe2_validate(image, L.image_bytes, &expected, out);
}

extern "C" int cx_cpe2_validate(const void *image, uint64_t image_bytes, const cx_cpe2_expected *expected,
                                cx_cpe2_view *out) {
    if (image == nullptr || out == nullptr || expected == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image or output is null");
    if (image_bytes < sizeof(cx_cpe2_header)) return fail(CX_STATUS_INVALID_ARGUMENT, "execution image is truncated");
    cx_cpe2_header h;
    std::memcpy(&h, image, sizeof(h));
    if (std::memcmp(h.magic, kMagic, sizeof(kMagic)) != 0 || h.schema_version != CX_CPE2_SCHEMA_VERSION
        || h.header_bytes != sizeof(h) || h.endian != CX_CPE2_ENDIAN_MARKER || h.alignment != CX_CPE2_ALIGNMENT
        || h.image_bytes != image_bytes || h.image_identity == 0u
        || h.image_identity != image_identity(image, static_cast<std::size_t>(image_bytes)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image header or checksum is invalid");
    const cx_cpe2_expected &x = *expected;
    if (!present(x.structure_identity) || x.structure_epoch == 0u || !present(x.semantic_geometry_identity)
        || !present(x.projection_catalog_identity)
        || !same(h.structure_identity_low, h.structure_identity_high, x.structure_identity.low, x.structure_identity.high)
        || h.structure_epoch != x.structure_epoch
        || !same(h.semantic_geometry_identity_low, h.semantic_geometry_identity_high, x.semantic_geometry_identity.low,
                 x.semantic_geometry_identity.high)
        || !same(h.projection_catalog_identity_low, h.projection_catalog_identity_high,
                 x.projection_catalog_identity.low, x.projection_catalog_identity.high)
        || (x.image_identity != 0u && h.image_identity != x.image_identity))
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image compatibility identity mismatches");
    if (h.section_count == 0u || h.projection_count == 0u || h.section_directory_offset != sizeof(h)
        || h.projection_directory_offset % CX_CPE2_ALIGNMENT != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image directory metadata is invalid");
    const u64 sdir = static_cast<u64>(h.section_count) * sizeof(cx_cpe2_section_entry);
    const u64 pdir = static_cast<u64>(h.projection_count) * sizeof(cx_cpe2_projection_entry);
    if (!in_range(h.section_directory_offset, sdir, image_bytes) || !in_range(h.projection_directory_offset, pdir, image_bytes))
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image directory range is invalid");
    const auto *b = static_cast<const unsigned char *>(image);
    const auto *sections = reinterpret_cast<const cx_cpe2_section_entry *>(b + h.section_directory_offset);
    const auto *projections = reinterpret_cast<const cx_cpe2_projection_entry *>(b + h.projection_directory_offset);
    const u64 directory_end = std::max(h.section_directory_offset + sdir, h.projection_directory_offset + pdir);
    u32 counts[6] = {0u, 0u, 0u, 0u, 0u, 0u};
    for (u32 i = 0; i < h.section_count; ++i) {
        const cx_cpe2_section_entry &s = sections[i];
        if ((!known_section(s.kind) && (s.flags & CX_CPE2_DIRECTORY_OPTIONAL) == 0u) || s.schema_version == 0u
            || !pow2(s.alignment) || s.alignment > kMaxSectionAlignment || !present(s.identity_low, s.identity_high)
            || s.bytes == 0u || s.offset < directory_end || s.offset % s.alignment != 0u
            || !in_range(s.offset, s.bytes, image_bytes)
            || s.checksum != checksum(b + s.offset, static_cast<std::size_t>(s.bytes)))
            return fail(CX_STATUS_INVALID_ARGUMENT, "execution image section directory is invalid");
        if ((s.element_count == 0u) != (s.element_bytes == 0u)
            || (s.element_count != 0u && static_cast<u64>(s.element_count) * s.element_bytes != s.bytes))
            return fail(CX_STATUS_INVALID_ARGUMENT, "execution image section element shape is invalid");
        for (u32 j = 0; j < i; ++j) {
            const cx_cpe2_section_entry &o = sections[j];
            const bool overlap = s.offset < o.offset + o.bytes && o.offset < s.offset + s.bytes;
            if (overlap || same(s.identity_low, s.identity_high, o.identity_low, o.identity_high))
                return fail(CX_STATUS_INVALID_ARGUMENT, "execution image sections overlap or duplicate identity");
        }
        if (s.kind >= CX_CPE2_SECTION_DOMAIN_TABLE && s.kind <= CX_CPE2_SECTION_INITIAL_VALUES) ++counts[s.kind];
    }
    if (counts[CX_CPE2_SECTION_DOMAIN_TABLE] != 1u || counts[CX_CPE2_SECTION_ORDER_PARTITION_TABLE] != 1u
        || counts[CX_CPE2_SECTION_RELATION_STRUCTURE] != 1u || counts[CX_CPE2_SECTION_SEMANTIC_GEOMETRY] != 1u
        || counts[CX_CPE2_SECTION_INITIAL_VALUES] > 1u
        || ((counts[CX_CPE2_SECTION_INITIAL_VALUES] == 0u) != (h.initial_value_generation == 0u)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image foundational section set is invalid");
    auto kind_of = [&](u32 index) { return sections[index].kind; };
    for (u32 i = 0; i < h.projection_count; ++i) {
        const int rc = check_projection(projections[i], h.section_count, kind_of, true);
        if (rc != CX_STATUS_SUCCESS) return rc;
        for (u32 j = 0; j < i; ++j)
            if (same(projections[i].identity_low, projections[i].identity_high, projections[j].identity_low,
                     projections[j].identity_high))
                return fail(CX_STATUS_INVALID_ARGUMENT, "execution image projection identity is duplicated");
    }
    *out = {h, image, image_bytes, sections, projections};
    return ok();
}

extern "C" int cx_cpe2_rebind(const cx_cpe2_view *validated, const void *new_base, uint64_t new_bytes,
                              cx_cpe2_view *out) {
    if (validated == nullptr || validated->image_base == nullptr || new_base == nullptr || out == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image rebind pointer is null");
    if (new_bytes != validated->image_bytes || validated->header.image_bytes != new_bytes)
        return fail(CX_STATUS_INVALID_ARGUMENT, "execution image rebind size differs");
    cx_cpe2_view v = *validated;
    const auto *b = static_cast<const unsigned char *>(new_base);
    v.image_base = new_base;
    v.image_bytes = new_bytes;
    v.sections = reinterpret_cast<const cx_cpe2_section_entry *>(b + v.header.section_directory_offset);
    v.projections = reinterpret_cast<const cx_cpe2_projection_entry *>(b + v.header.projection_directory_offset);
    *out = v;
    return ok();
}

extern "C" int cx_cpe2_prebind_for_base(const cx_cpe2_view *validated_host, uint32_t projection_index,
                                        const void *destination_base, uint64_t destination_bytes,
                                        cx_cpe2_prebound_projection *out) {
    if (validated_host == nullptr || validated_host->image_base == nullptr || validated_host->sections == nullptr
        || validated_host->projections == nullptr || destination_base == nullptr || out == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "projection prebind image or output is null");
    if (destination_bytes != validated_host->image_bytes || validated_host->header.image_bytes != destination_bytes)
        return fail(CX_STATUS_INVALID_ARGUMENT, "projection prebind destination size differs");
    if (projection_index >= validated_host->header.projection_count)
        return fail(CX_STATUS_INVALID_ARGUMENT, "projection prebind index is out of range");
    const cx_cpe2_projection_entry &e = validated_host->projections[projection_index];
    cx_cpe2_prebound_projection p{};
    p.descriptor = e;
    const std::uintptr_t base = reinterpret_cast<std::uintptr_t>(destination_base);
    bool fits = true;
    auto bind = [&](u32 index, const void **ptr, uint64_t *bytes) {
        if (index == CX_CPE2_INVALID_INDEX || !fits) return;
        const u64 offset = validated_host->sections[index].offset;
        if (offset > std::numeric_limits<std::uintptr_t>::max() - base) {
            fits = false;
            return;
        }
        *ptr = reinterpret_cast<const void *>(base + static_cast<std::uintptr_t>(offset));
        *bytes = validated_host->sections[index].bytes;
    };
    bind(e.payload_section, &p.payload, &p.payload_bytes);
    bind(e.forward_map_section, &p.forward_map, &p.forward_map_bytes);
    bind(e.transpose_map_section, &p.transpose_map, &p.transpose_map_bytes);
    bind(e.scheduling_summary_section, &p.scheduling_summary, &p.scheduling_summary_bytes);
    if (!fits) return fail(CX_STATUS_INVALID_ARGUMENT, "projection prebind destination pointer overflows");
    *out = p;
    return ok();
}

extern "C" int cx_cpe2_prebind(const cx_cpe2_view *validated_host, uint32_t projection_index,
                               cx_cpe2_prebound_projection *out) {
    if (validated_host == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "projection prebind image or output is null");
    return cx_cpe2_prebind_for_base(validated_host, projection_index, validated_host->image_base,
                                    validated_host->image_bytes, out);
}

extern "C" int cx_cpe2_load_cpk1(const cx_cpe2_view *validated_host, uint32_t projection_index,
                                 const cx_cpk1_expected *expected, cx_cpk1_view *out) {
    if (out == nullptr || validated_host == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1 compatibility output is null");
    if (projection_index >= validated_host->header.projection_count)
        return fail(CX_STATUS_INVALID_ARGUMENT, "CPK1 compatibility projection index is out of range");
    const cx_cpe2_projection_entry &p = validated_host->projections[projection_index];
    if (p.kind != CX_CPE2_PROJECTION_NATIVE_ROW_MASKED || p.payload_section == CX_CPE2_INVALID_INDEX
        || p.payload_section >= validated_host->header.section_count
        || validated_host->sections[p.payload_section].kind != CX_CPE2_SECTION_CPK1_V1_COMPATIBILITY)
        return fail(CX_STATUS_INVALID_ARGUMENT, "projection does not contain a CPK1 compatibility section");
    const cx_cpe2_section_entry &s = validated_host->sections[p.payload_section];
    const int rc = cx_cpk1_validate(static_cast<const unsigned char *>(validated_host->image_base) + s.offset,
                                    s.bytes, expected, out);
    if (rc != CX_STATUS_SUCCESS)
        return fail(rc, cx_cpk1_last_error());
    return ok();
}

extern "C" const char *cx_cpe2_last_error(void) { return g_error; }
