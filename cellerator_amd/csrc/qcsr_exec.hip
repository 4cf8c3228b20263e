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

#include <new>
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

std::uint64_t weights_bytes(const cx_qcsr_exec_projection *p, std::int64_t out_cols) {
    return align256(static_cast<std::uint64_t>(p->shape.cols) * static_cast<std::uint64_t>(out_cols) * 2u);
}

int build(const cx_qcsr_matrix *a, std::uint32_t head, cx_qcsr_exec_projection *p, hipStream_t s) {
    constexpr const char *who = "cx_qcsr_exec_prepare";
    const std::uint32_t rows = a->rows, cols = a->cols;
    // 1. the popularity order of the genes (stored entries per gene, descending; ties by gene)
    DeviceBuffer counts, inverse, err, col_x, packed_x, pairs_canon;
    int rc = counts.allocate(static_cast<std::uint64_t>(cols) * 4u, who);
    if (rc == CX_STATUS_SUCCESS) rc = cx_qcsr_column_counts(a, static_cast<std::uint32_t *>(counts.p), s);
    if (rc != CX_STATUS_SUCCESS) return rc;
    std::vector<std::uint32_t> host_counts(cols), perm(cols), inv(cols);
    std::int32_t packed_total = 0;
    hipError_t e = hipMemcpyAsync(host_counts.data(), counts.p, static_cast<std::size_t>(cols) * 4u,
                                  hipMemcpyDeviceToHost, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(&packed_total, a->packed_row_ptr + rows, 4u, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, who);
    rc = cx_popularity_order(host_counts.data(), cols, perm.data(), inv.data());
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
