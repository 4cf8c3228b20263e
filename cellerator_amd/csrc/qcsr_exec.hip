// qcsr_exec.hip -- a prepared execution-order projection of a quantized CSR, owned by one
// object: the popularity order of the genes, the per-gene metadata in that order, the dense
// head layout for the matrix cores and the prepared tail stream, built once per structure
// and code generation. A launch gathers the caller's canonical W into execution order in
// its workspace and runs the hybrid product (head + tail stream), so callers that bind
// canonical operands -- the CP-Math plug-in, any C caller -- get the prepared path without
// handling relabelled arrays. The relabelled column indices and codes are needed only while
// the head and the stream are built, and are freed before prepare returns.
//
// Engine addition: the reference's quantized CSR projection has no prepared
// execution-order form. The value semantics are the reference codec's
// (fma(code, scale, offset), include/Cellerator/quantized/access.cuh:81-91) and the
// product is the referee's (src/compute/math/referee.cc:101-253) up to fp32 summation order.
#include "qcsr_common.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <new>
#include <numeric>
#include <vector>

struct cx_qcsr_exec_projection {
    cx_qcsr_matrix shape;        // rows, cols, nnz, bits, decode policy, flags, metadata (owned); no structure
    std::uint32_t *perm;         // [cols]: canonical gene at execution position
    float *meta;                 // execution-order metadata: (scale, offset) pairs, or scales
    float *row_offsets;          // [rows] (column-scale / row-offset policy) or NULL
    void *head_storage;
    void *plan_storage;
    void *entries;
    cx_qcsr_hybrid_layout layout;
    cx_qcsr_tail_stream tail;
    std::uint64_t persistent_bytes;
};

namespace cx {
namespace {

constexpr std::uint64_t align256(std::uint64_t b) { return (b + 255u) & ~std::uint64_t{255u}; }
constexpr std::uint32_t kExecPartGenes = 1024u;

// Device memory that is freed when the owner goes out of scope (preparation temporaries).
struct DeviceBuffer {
    void *p = nullptr;
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    ~DeviceBuffer() {
        if (p != nullptr) (void)hipFree(p);
    }
    int allocate(std::uint64_t bytes, const char *who) {
        const hipError_t e = hipMalloc(&p, bytes == 0u ? 256u : bytes);
        if (e != hipSuccess) {
            p = nullptr;
            return hip_fail(e, who);
        }
        return CX_STATUS_SUCCESS;
    }
    void *release() {
        void *q = p;
        p = nullptr;
        return q;
    }
};

void destroy(cx_qcsr_exec_projection *p) {
    if (p == nullptr) return;
    for (void *q : {static_cast<void *>(p->perm), static_cast<void *>(p->meta), static_cast<void *>(p->row_offsets),
                    p->head_storage, p->plan_storage, p->entries})
        if (q != nullptr) (void)hipFree(q);
    delete p;
}

bool valid_out_cols(std::int64_t n) { return n > 0 && n % 64 == 0 && n <= 256; }

constexpr int kNever = INT_MAX;  // no layout exponent (at most 100) carries the gene exactly

// Exponent of the lowest set bit of a finite nonzero float: x = m 2^e with m odd.
int low_bit(float x) {
    std::uint32_t b;
    std::memcpy(&b, &x, 4);
    const std::uint32_t field = (b >> 23) & 0xffu;
    std::uint32_t m = b & 0x7fffffu;
    int e = -149;
    if (field != 0u) {
        m |= 0x800000u;
        e = static_cast<int>(field) - 150;
    }
    return e + __builtin_ctz(m);
}

// Smallest layout exponent k under which the head carries every value of a per-gene-policy
// gene exactly (the conditions head_exact_kernel checks, qcsr_hybrid.hip): 2^k s and 2^k o
// stay normal floats (or zero), and every decoded value x = fma(c, s, o) is a multiple of
// 2^(-14-k), i.e. 2^k x lies on the 2^-14 grid. Both hold for every larger k, so the
// smallest suffices; kNever for non-finite metadata or values, or when k would exceed 100.
int gene_min_exp(float s, float o, std::uint32_t qmax) {
    if (!std::isfinite(s) || !std::isfinite(o)) return kNever;
    int need = INT_MIN;
    if (s != 0.0f) need = std::max(need, -126 - std::ilogb(s));
    if (o != 0.0f) need = std::max(need, -126 - std::ilogb(o));
    for (std::uint32_t c = 0; c <= qmax; ++c) {
        const float x = std::fma(static_cast<float>(c), s, o);
        if (!std::isfinite(x)) return kNever;
        if (x != 0.0f) need = std::max(need, -14 - low_bit(x));
    }
    return need > 100 ? kNever : need;
}

// The same under the row-offset policy, for the gene's scale alone: 2^k s on the 2^-14 grid
// (and normal). The row offsets add one condition shared by every gene (rows_min_exp).
int scale_min_exp(float s) {
    if (!std::isfinite(s)) return kNever;
    if (s == 0.0f) return INT_MIN;
    const int need = -14 - low_bit(s);
    return need > 100 ? kNever : need;
}

// Smallest k putting every 2^k r on the 2^-14 grid; the largest |r| in *largest.
int rows_min_exp(const float *r, std::uint32_t rows, float *largest) {
    int need = INT_MIN;
    float big = 0.0f;
    for (std::uint32_t i = 0; r != nullptr && i < rows; ++i) {
        if (!std::isfinite(r[i])) return kNever;
        big = std::max(big, std::fabs(r[i]));
        if (r[i] != 0.0f) need = std::max(need, -14 - low_bit(r[i]));
    }
    *largest = big;
    return need > 100 ? kNever : need;
}

std::uint64_t weights_bytes(const cx_qcsr_exec_projection *p, std::int64_t out_cols) {
    return align256(static_cast<std::uint64_t>(p->shape.cols) * static_cast<std::uint64_t>(out_cols) * 2u);
}

int build(const cx_qcsr_matrix *a, std::uint32_t head_cols, cx_qcsr_exec_projection *p, hipStream_t s) {
    constexpr const char *who = "cx_qcsr_exec_prepare";
    const std::uint32_t rows = a->rows, cols = a->cols;
    // 1. the popularity order of the genes (stored entries per gene, descending; ties by gene)
    //    with the genes the head cannot carry exactly moved after it (cx_qcsr_head_order)
    DeviceBuffer counts, inverse, err, col_x, packed_x, pairs_canon;
    int rc = counts.allocate(static_cast<std::uint64_t>(cols) * 4u, who);
    if (rc == CX_STATUS_SUCCESS) rc = cx_qcsr_column_counts(a, static_cast<std::uint32_t *>(counts.p), s);
    if (rc != CX_STATUS_SUCCESS) return rc;
    std::vector<std::uint32_t> host_counts(cols), perm(cols), inv(cols);
    const bool pairs = a->decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS;
    const bool row_policy = a->decode_policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET;
    std::vector<float> scales(a->column_scales != nullptr ? static_cast<std::size_t>(cols) * (pairs ? 2u : 1u) : 0u);
    std::vector<float> offsets(!row_policy && !pairs && a->column_offsets != nullptr ? cols : 0u);
    std::vector<float> row_offsets(row_policy && a->row_offsets != nullptr ? rows : 0u);
    std::int32_t packed_total = 0;
    hipError_t e = hipMemcpyAsync(host_counts.data(), counts.p, static_cast<std::size_t>(cols) * 4u,
                                  hipMemcpyDeviceToHost, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(&packed_total, a->packed_row_ptr + rows, 4u, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && !scales.empty())
        e = hipMemcpyAsync(scales.data(), a->column_scales, scales.size() * 4u, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && !offsets.empty())
        e = hipMemcpyAsync(offsets.data(), a->column_offsets, offsets.size() * 4u, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess && !row_offsets.empty())
        e = hipMemcpyAsync(row_offsets.data(), a->row_offsets, row_offsets.size() * 4u, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, who);
    std::uint32_t head = 0u;
    rc = cx_qcsr_head_order(host_counts.data(), cols, a->bits, a->decode_policy, scales.empty() ? nullptr : scales.data(),
                            offsets.empty() ? nullptr : offsets.data(), row_offsets.empty() ? nullptr : row_offsets.data(),
                            rows, head_cols, perm.data(), inv.data(), &head);
    if (rc != CX_STATUS_SUCCESS) return rc;
    DeviceBuffer perm_d;
    rc = perm_d.allocate(static_cast<std::uint64_t>(cols) * 4u, who);
    if (rc == CX_STATUS_SUCCESS) rc = inverse.allocate(static_cast<std::uint64_t>(cols) * 4u, who);
    if (rc != CX_STATUS_SUCCESS) return rc;
    e = hipMemcpyAsync(perm_d.p, perm.data(), static_cast<std::size_t>(cols) * 4u, hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(inverse.p, inv.data(), static_cast<std::size_t>(cols) * 4u, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return hip_fail(e, who);

    // 2. the matrix relabelled into that order, rows re-sorted with their codes (temporary)
    const std::uint64_t packed_bytes = static_cast<std::uint64_t>(packed_total < 0 ? 0 : packed_total) + 64u;
    rc = col_x.allocate(a->nnz * 4u, who);
    if (rc == CX_STATUS_SUCCESS) rc = packed_x.allocate(packed_bytes, who);
    if (rc == CX_STATUS_SUCCESS) rc = err.allocate(4u, who);
    if (rc != CX_STATUS_SUCCESS) return rc;
    e = hipMemsetAsync(packed_x.p, 0, packed_bytes, s);
    if (e == hipSuccess) e = hipMemsetAsync(err.p, 0, 4u, s);
    if (e != hipSuccess) return hip_fail(e, who);
    rc = cx_qcsr_to_execution_order(a, static_cast<const std::uint32_t *>(inverse.p), static_cast<std::int32_t *>(col_x.p),
                                    static_cast<std::uint8_t *>(packed_x.p), nullptr, static_cast<std::uint32_t *>(err.p), s);
    if (rc != CX_STATUS_SUCCESS) return rc;
    std::uint32_t bad = 0u;
    e = hipMemcpyAsync(&bad, err.p, 4u, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, who);
    if (bad != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_exec_prepare: a row repeats a gene or holds a column outside [0, cols)");

    // 3. per-gene metadata in execution order: (scale, offset) pairs for the per-gene
    //    policies (decoded bit-identically to separate arrays), scales for row offsets
    p->shape = *a;
    p->shape.row_ptr = p->shape.packed_row_ptr = p->shape.col_idx = nullptr;
    p->shape.packed_values = nullptr;
    p->shape.values = nullptr;
    p->shape.column_offsets = nullptr;
    p->shape.row_offsets = nullptr;
    p->shape.column_scales = nullptr;
    p->shape.flags = CX_QCSR_COLUMNS_SORTED;
    DeviceBuffer meta, row_off;
    if (a->decode_policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET) {
        if (a->column_scales != nullptr) {
            rc = meta.allocate(static_cast<std::uint64_t>(cols) * 4u, who);
            if (rc == CX_STATUS_SUCCESS)
                rc = cx_pack_dense_operand(static_cast<const std::uint32_t *>(perm_d.p), cols, a->column_scales, 1u, 1u,
                                           0u, 4u, meta.p, static_cast<std::uint64_t>(cols) * 4u, s);
            if (rc != CX_STATUS_SUCCESS) return rc;
        }
        if (a->row_offsets != nullptr) {
            rc = row_off.allocate(static_cast<std::uint64_t>(rows) * 4u, who);
            if (rc != CX_STATUS_SUCCESS) return rc;
            e = hipMemcpyAsync(row_off.p, a->row_offsets, static_cast<std::size_t>(rows) * 4u, hipMemcpyDeviceToDevice, s);
            if (e != hipSuccess) return hip_fail(e, who);
        }
        p->shape.column_scales = static_cast<const float *>(meta.p);
        p->shape.row_offsets = static_cast<const float *>(row_off.p);
    } else {
        const float *canon = a->column_scales;
        if (a->decode_policy == CX_DECODE_PER_GENE_AFFINE) {
            rc = pairs_canon.allocate(static_cast<std::uint64_t>(cols) * 8u, who);
            if (rc == CX_STATUS_SUCCESS)
                rc = cx_qcsr_pack_gene_affine(a->column_scales, a->column_offsets, cols,
                                              static_cast<float *>(pairs_canon.p), s);
            if (rc != CX_STATUS_SUCCESS) return rc;
            canon = static_cast<const float *>(pairs_canon.p);
        }
        rc = meta.allocate(static_cast<std::uint64_t>(cols) * 8u, who);
        if (rc == CX_STATUS_SUCCESS)
            rc = cx_pack_dense_operand(static_cast<const std::uint32_t *>(perm_d.p), cols, canon, 1u, 1u, 0u, 8u, meta.p,
                                       static_cast<std::uint64_t>(cols) * 8u, s);
        if (rc != CX_STATUS_SUCCESS) return rc;
        p->shape.decode_policy = CX_DECODE_PER_GENE_AFFINE_PAIRS;
        p->shape.column_scales = static_cast<const float *>(meta.p);
    }

    // 4. the dense head and the tail stream of the relabelled matrix
    cx_qcsr_matrix mx = p->shape;
    mx.row_ptr = a->row_ptr;
    mx.packed_row_ptr = a->packed_row_ptr;
    mx.col_idx = static_cast<const std::int32_t *>(col_x.p);
    mx.packed_values = static_cast<const std::uint8_t *>(packed_x.p);
    std::uint64_t bytes = 0u;
    rc = cx_qcsr_hybrid_layout_bytes(&mx, head, &bytes);
    DeviceBuffer head_storage, plan, entries;
    if (rc == CX_STATUS_SUCCESS) rc = head_storage.allocate(bytes, who);
    if (rc == CX_STATUS_SUCCESS) rc = cx_qcsr_hybrid_prepare(&mx, head, head_storage.p, bytes, &p->layout, s);
    if (rc != CX_STATUS_SUCCESS) return rc;
    std::uint64_t plan_bytes = 0u, entry_bytes = 0u;
    rc = cx_qcsr_tail_plan_bytes(&mx, &p->layout, &plan_bytes);
    if (rc == CX_STATUS_SUCCESS) rc = plan.allocate(plan_bytes, who);
    if (rc == CX_STATUS_SUCCESS) rc = cx_qcsr_tail_plan(&mx, &p->layout, plan.p, plan_bytes, &p->tail, &entry_bytes, s);
    if (rc == CX_STATUS_SUCCESS) rc = entries.allocate(entry_bytes, who);
    if (rc == CX_STATUS_SUCCESS) rc = cx_qcsr_tail_fill(&mx, &p->layout, &p->tail, entries.p, entry_bytes, s);
    if (rc != CX_STATUS_SUCCESS) return rc;
    e = hipStreamSynchronize(s);  // the temporaries are read until here
    if (e != hipSuccess) return hip_fail(e, who);
    p->layout.tail = &p->tail;
    p->perm = static_cast<std::uint32_t *>(perm_d.release());
    p->meta = static_cast<float *>(meta.release());
    p->row_offsets = static_cast<float *>(row_off.release());
    p->head_storage = head_storage.release();
    p->plan_storage = plan.release();
    p->entries = entries.release();
    p->persistent_bytes = static_cast<std::uint64_t>(cols) * 4u
        + (p->meta != nullptr ? static_cast<std::uint64_t>(cols) * (p->shape.decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS ? 8u : 4u) : 0u)
        + (p->row_offsets != nullptr ? static_cast<std::uint64_t>(rows) * 4u : 0u) + bytes + plan_bytes + entry_bytes;
    return CX_STATUS_SUCCESS;
}

} // namespace
} // namespace cx

extern "C" int cx_qcsr_head_order(const uint32_t *counts, uint32_t cols, uint32_t bits, uint32_t decode_policy,
                                  const float *scales, const float *offsets, const float *row_offsets, uint32_t rows,
                                  uint32_t head_cols, uint32_t *feature_permutation, uint32_t *inverse_permutation,
                                  uint32_t *head_out) {
    using namespace cx;
    clear_error();
    if (head_out == nullptr || (cols != 0u && (counts == nullptr || feature_permutation == nullptr
                                               || inverse_permutation == nullptr)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_head_order: null argument");
    if (bits != 1u && bits != 2u && bits != 4u && bits != 8u)
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_head_order: quantized codes of 1, 2, 4 or 8 bits only");
    if (decode_policy != CX_DECODE_PER_GENE_AFFINE && decode_policy != CX_DECODE_PER_GENE_AFFINE_PAIRS
        && decode_policy != CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_head_order: unknown decode policy");
    if (decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS && scales == nullptr && cols != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_head_order: the pairs policy needs scales");
    if (head_cols % kExecPartGenes != 0u)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_head_order: head_cols must be a multiple of 1,024");
    std::vector<std::uint32_t> order(cols);
    std::iota(order.begin(), order.end(), 0u);
    std::stable_sort(order.begin(), order.end(), [&](std::uint32_t x, std::uint32_t y) { return counts[x] > counts[y]; });
    const std::uint32_t qmax = (1u << bits) - 1u;
    const float qmax_f = static_cast<float>(qmax);
    const bool row_policy = decode_policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET;
    float roff = 0.0f;
    const int rows_need = row_policy ? rows_min_exp(row_offsets, rows, &roff) : INT_MIN;
    const std::uint32_t want = std::min(head_cols, cols / kExecPartGenes * kExecPartGenes);
    // Per gene, in popularity order: the smallest exponent carrying its values exactly (lo)
    // and the largest its magnitude allows (hi: the bound head_range_kernel computes, plus the
    // largest |row offset| under that policy, below 2^(15 - k)).
    std::vector<int> lo(cols, kNever), hi(cols, INT_MIN);
    for (std::uint32_t e = 0; e < cols && want != 0u; ++e) {
        const std::uint32_t g = order[e];
        float sg, og;
        if (decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS) {
            sg = scales[2u * g];
            og = scales[2u * g + 1u];
        } else {
            sg = scales != nullptr ? scales[g] : 1.0f;
            og = !row_policy && offsets != nullptr ? offsets[g] : 0.0f;
        }
        const float b = row_policy ? std::fabs(sg) * qmax_f : std::max(std::fabs(og), std::fabs(std::fma(qmax_f, sg, og)));
        const float total = row_policy ? b + roff : b;
        lo[e] = row_policy ? scale_min_exp(sg) : gene_min_exp(sg, og, qmax);
        if (!std::isfinite(total)) lo[e] = kNever;
        hi[e] = total > 0.0f ? 14 - std::ilogb(total) : INT_MAX;
    }
    // The layout exponent K under which the head takes the most stored entries: the head is
    // the most popular genes with lo <= K <= hi (whole 1,024-gene parts of them, at most
    // `want`). The layout's own exponent (head_scale_exp of the head's largest bound) is then
    // at least K, so every head gene stays exact under it.
    std::uint64_t best = 0u;
    int best_k = INT_MIN;
    std::uint32_t head = 0u;
    for (int K = std::max(-100, rows_need); K <= 100 && want != 0u && rows_need != kNever; ++K) {
        std::uint32_t n = 0u;
        for (std::uint32_t e = 0; e < cols && n < want; ++e) n += lo[e] <= K && K <= hi[e] ? 1u : 0u;
        const std::uint32_t h = n / kExecPartGenes * kExecPartGenes;
        std::uint64_t covered = 0u;
        for (std::uint32_t e = 0, taken = 0u; e < cols && taken < h; ++e)
            if (lo[e] <= K && K <= hi[e]) {
                covered += static_cast<std::uint64_t>(counts[order[e]]) + 1u;  // + 1: of equal heads, the wider
                ++taken;
            }
        if (h > 0u && covered > best) {
            best = covered;
            best_k = K;
            head = h;
        }
    }
    std::vector<std::uint8_t> in_head(cols, 0u);
    for (std::uint32_t e = 0, taken = 0u; e < cols && taken < head; ++e)
        if (lo[e] <= best_k && best_k <= hi[e]) {
            in_head[order[e]] = 1u;
            ++taken;
        }
    std::uint32_t at = 0u;
    for (int pass = 0; pass < 2; ++pass)
        for (std::uint32_t e = 0; e < cols; ++e) {
            const std::uint32_t g = order[e];
            if ((in_head[g] != 0u) == (pass == 0)) {
                feature_permutation[at] = g;
                inverse_permutation[g] = at++;
            }
        }
    *head_out = head;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_exec_prepare(const cx_qcsr_matrix *a, uint32_t head_cols, cx_qcsr_exec_projection **out,
                                    void *stream) {
    using namespace cx;
    clear_error();
    if (out == nullptr || a == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_exec_prepare: null argument");
    *out = nullptr;
    if (a->bits != 1u && a->bits != 2u && a->bits != 4u && a->bits != 8u)
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_exec_prepare: quantized codes of 1, 2, 4 or 8 bits only");
    if (a->decode_policy != CX_DECODE_PER_GENE_AFFINE && a->decode_policy != CX_DECODE_PER_GENE_AFFINE_PAIRS
        && a->decode_policy != CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_exec_prepare: unknown decode policy");
    if (a->decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS && a->column_scales == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_exec_prepare: the pairs policy needs column_scales");
    if (a->rows == 0u || a->cols == 0u) return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_exec_prepare: empty matrix");
    if (a->row_ptr == nullptr || a->packed_row_ptr == nullptr
        || (a->nnz != 0u && (a->col_idx == nullptr || a->packed_values == nullptr)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_exec_prepare: null structure or codes");
    if (a->nnz > static_cast<std::uint64_t>(INT32_MAX) || a->cols > static_cast<std::uint32_t>(INT32_MAX))
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_exec_prepare: nnz exceeds int32 row offsets");
    if (head_cols % kExecPartGenes != 0u)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_exec_prepare: head_cols must be a multiple of 1,024");
    const std::uint32_t head = std::min(head_cols, a->cols / kExecPartGenes * kExecPartGenes);
    auto *p = new (std::nothrow) cx_qcsr_exec_projection{};
    if (p == nullptr) return fail(CX_STATUS_HIP_ERROR, "cx_qcsr_exec_prepare: out of host memory");
    const int rc = build(a, head, p, static_cast<hipStream_t>(stream));
    if (rc != CX_STATUS_SUCCESS) {
        destroy(p);
        return rc;
    }
    *out = p;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_exec_query(const cx_qcsr_exec_projection *p, cx_qcsr_exec_info *info) {
    using namespace cx;
    clear_error();
    if (p == nullptr || info == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_exec_query: null argument");
    cx_qcsr_exec_info i{};
    i.rows = p->shape.rows;
    i.cols = p->shape.cols;
    i.bits = p->shape.bits;
    i.head_cols = p->layout.head_cols;
    i.nnz = p->shape.nnz;
    i.tail_fills = p->tail.fills;
    i.persistent_bytes = p->persistent_bytes;
    i.head_form = p->layout.head_form;
    i.tail_blocks = p->tail.blocks;
    *info = i;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_exec_workspace_bytes(const cx_qcsr_exec_projection *p, int64_t out_cols, uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (p == nullptr || bytes == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_exec_workspace_bytes: null argument");
    if (!valid_out_cols(out_cols))
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_exec_workspace_bytes: out_cols must be 64, 128, 192 or 256");
    std::uint64_t hybrid = 0u;
    const int rc = cx_qcsr_hybrid_workspace(&p->shape, p->layout.head_cols, out_cols, &hybrid);
    if (rc != CX_STATUS_SUCCESS) return rc;
    *bytes = weights_bytes(p, out_cols) + hybrid;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_exec_workspace_for(uint32_t rows, uint32_t cols, uint32_t head_cols, int64_t out_cols,
                                          uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (bytes == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_exec_workspace_for: null bytes");
    if (!valid_out_cols(out_cols))
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_exec_workspace_for: out_cols must be 64, 128, 192 or 256");
    if (head_cols % kExecPartGenes != 0u)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_exec_workspace_for: head_cols must be a multiple of 1,024");
    cx_qcsr_matrix m{};
    m.rows = rows;
    m.cols = cols;
    m.bits = 8u;  // the code width is not known here: size for the words-form head, the larger need
    const std::uint32_t head = std::min(head_cols, cols / kExecPartGenes * kExecPartGenes);
    std::uint64_t hybrid = 0u;
    const int rc = cx_qcsr_hybrid_workspace(&m, head, out_cols, &hybrid);
    if (rc != CX_STATUS_SUCCESS) return rc;
    *bytes = align256(static_cast<std::uint64_t>(cols) * static_cast<std::uint64_t>(out_cols) * 2u) + hybrid;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_exec_spmm(const cx_qcsr_exec_projection *p, const void *rhs, int64_t rhs_ld, int64_t out_cols,
                                 float *out, int64_t out_ld, const cx_spmm_epilogue *epilogue, void *workspace,
                                 uint64_t workspace_bytes, void *stream) {
    using namespace cx;
    clear_error();
    if (p == nullptr || rhs == nullptr || out == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_exec_spmm: null projection, rhs or output");
    if (!valid_out_cols(out_cols) || rhs_ld < out_cols || out_ld < out_cols)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_exec_spmm: out_cols must be 64, 128, 192 or 256 within the row strides");
    if ((reinterpret_cast<std::uintptr_t>(out) & 15u) != 0u || (out_ld * 4) % 16 != 0
        || (reinterpret_cast<std::uintptr_t>(rhs) & 1u) != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_exec_spmm: the output must be 16-byte aligned (row stride too)");
    if (static_cast<const void *>(out) == rhs)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_exec_spmm: output aliases the rhs");
    std::uint64_t need = 0u;
    int rc = cx_qcsr_exec_workspace_bytes(p, out_cols, &need);
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (workspace == nullptr || workspace_bytes < need || (reinterpret_cast<std::uintptr_t>(workspace) & 255u) != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_exec_spmm: needs a 256-byte aligned workspace of cx_qcsr_exec_workspace_bytes");
    const std::uint64_t wb = weights_bytes(p, out_cols);
    // W rows into execution order (the packed dense operand), out_cols wide
    rc = cx_pack_dense_operand(p->perm, p->shape.cols, rhs, static_cast<std::uint64_t>(out_cols),
                               static_cast<std::uint64_t>(rhs_ld), 0u, 2u, workspace, wb, stream);
    if (rc != CX_STATUS_SUCCESS) return rc;
    return launch_hybrid(p->shape, p->layout, workspace, out_cols, out_cols, out, out_ld, epilogue,
                         static_cast<unsigned char *>(workspace) + wb, workspace_bytes - wb,
                         static_cast<hipStream_t>(stream), "cx_qcsr_exec_spmm");
}

extern "C" int cx_qcsr_exec_destroy(cx_qcsr_exec_projection *p) {
    cx::clear_error();
    cx::destroy(p);
    return CX_STATUS_SUCCESS;
}
