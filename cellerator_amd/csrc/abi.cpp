// abi.cpp -- public context ABI (include/cellerator_amd.h, part 2), layout-compatible
// with the reference's include/Cellerator/abi.h. Validation order and status mapping
// follow src/abi/abi.cu:62-218 and :278-400; dispatch goes to the cx_* launch layer.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <new>

#include "cellerator_amd.h"

struct cellerator_context {
    int device = -1;  // < 0: the calling thread's current device (the reference's default)
    hipStream_t stream = nullptr;
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    bool owns_scratch = false;  // grown on demand when the config brings no scratch
};

struct cellerator_saved_state {
    uint32_t version = CELLERATOR_ABI_VERSION;
    cellerator_saved_state_kind kind = CELLERATOR_SAVED_STATE_NONE;
    cellerator_sparse_layout layout = CELLERATOR_LAYOUT_CSR;
    uint32_t rows = 0u;
    uint32_t cols = 0u;
    uint32_t nnz = 0u;
    uint32_t out_cols = 0u;
};

namespace {

thread_local char g_abi_error[512] = {0};

cellerator_status fail(cellerator_status status, const char *message) {
    std::snprintf(g_abi_error, sizeof(g_abi_error), "%s", message);
    return status;
}

cellerator_status from_cx(int status) {
    if (status == CX_STATUS_SUCCESS) return CELLERATOR_STATUS_SUCCESS;
    std::snprintf(g_abi_error, sizeof(g_abi_error), "%s", cx_last_error());
    return static_cast<cellerator_status>(status);
}

bool versioned(uint32_t version, size_t size, size_t minimum) {
    return version == CELLERATOR_ABI_VERSION && size >= minimum;
}

cellerator_status validate_layout(const cellerator_sparse_layout_desc *layout) {
    if (layout == nullptr) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "layout descriptor is null");
    if (!versioned(layout->version, layout->size, sizeof(cellerator_sparse_layout_desc)))
        return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "layout descriptor version or size mismatch");
    if (layout->rows == 0u || layout->cols == 0u)
        return fail(CELLERATOR_STATUS_INVALID_SHAPE, "layout rows and columns must be nonzero");
    return CELLERATOR_STATUS_SUCCESS;
}

// Leading dimension of a rank-2 descriptor: a zero row stride means compact rows, as in
// the reference (abi.cu matrix_ld_).
int64_t matrix_ld(const cellerator_tensor_desc *t) {
    return t->stride[0] == 0 ? static_cast<int64_t>(t->shape[1]) : t->stride[0];
}

// Rank-2 row-major matrix [rows x cols] (cols == 0: any column count). Column stride 1
// (or 0, the reference's "compact"), leading dimension at least the column count.
cellerator_status validate_dense(const cellerator_tensor_desc *t, uint64_t rows, uint64_t cols,
                                 const char *null_message) {
    if (t == nullptr) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor descriptor is null");
    if (!versioned(t->version, t->size, sizeof(cellerator_tensor_desc)))
        return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor descriptor version or size mismatch");
    if (t->data == nullptr) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, null_message);
    if (t->rank != 2u) return fail(CELLERATOR_STATUS_INVALID_SHAPE, "tensor rank mismatch");
    if (t->shape[0] != rows) return fail(CELLERATOR_STATUS_INVALID_SHAPE, "tensor row dimension mismatch");
    if (cols != 0u && t->shape[1] != cols)
        return fail(CELLERATOR_STATUS_INVALID_SHAPE, "tensor column dimension mismatch");
    if ((t->stride[1] != 1 && t->stride[1] != 0) || matrix_ld(t) < static_cast<int64_t>(t->shape[1]))
        return fail(CELLERATOR_STATUS_INVALID_SHAPE, "tensor must be row-major with unit column stride");
    return CELLERATOR_STATUS_SUCCESS;
}

// Rank-1 F32 vector of `count` elements (abi.cu validate_vector_tensor_).
cellerator_status validate_vector(const cellerator_tensor_desc *t, uint64_t count,
                                  const char *null_message) {
    if (t == nullptr) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor descriptor is null");
    if (!versioned(t->version, t->size, sizeof(cellerator_tensor_desc)))
        return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor descriptor version or size mismatch");
    if (t->data == nullptr) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, null_message);
    if (t->dtype != CELLERATOR_DTYPE_F32) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor dtype mismatch");
    if (t->rank != 1u) return fail(CELLERATOR_STATUS_INVALID_SHAPE, "tensor rank mismatch");
    if (t->shape[0] != count) return fail(CELLERATOR_STATUS_INVALID_SHAPE, "tensor row dimension mismatch");
    if (t->stride[0] != 1 && t->stride[0] != 0)
        return fail(CELLERATOR_STATUS_INVALID_SHAPE, "vector tensor must be contiguous");
    return CELLERATOR_STATUS_SUCCESS;
}

// The CSR layouts as the engine's matrix view (plain CSR: F16/F32 values; quantized CSR:
// codes + metadata, block_col_idx carrying the packed row byte offsets).
cellerator_status csr_view(const cellerator_sparse_layout_desc *layout, cx_qcsr_matrix *m) {
    *m = cx_qcsr_matrix{};
    m->rows = layout->rows;
    m->cols = layout->cols;
    m->nnz = layout->nnz;
    m->row_ptr = reinterpret_cast<const int32_t *>(layout->major_ptr);
    m->col_idx = reinterpret_cast<const int32_t *>(layout->minor_idx);
    if (layout->layout == CELLERATOR_LAYOUT_CSR) {
        if (layout->major_ptr == nullptr || layout->minor_idx == nullptr || layout->values == nullptr)
            return fail(CELLERATOR_STATUS_INVALID_ARGUMENT,
                        "CSR layout requires row offsets, column indices, and values");
        m->bits = 0u;
        m->values = layout->values;
        m->value_dtype = layout->value_dtype;
    } else {
        m->bits = layout->bits;
        m->decode_policy = layout->decode_policy;
        m->packed_row_ptr = reinterpret_cast<const int32_t *>(layout->block_col_idx);
        m->packed_values = layout->packed_values;
        m->column_scales = layout->column_scales;
        m->column_offsets = layout->column_offsets;
        m->row_offsets = layout->row_offsets;
    }
    return CELLERATOR_STATUS_SUCCESS;
}

uint64_t align256(uint64_t bytes) { return (bytes + 255u) & ~static_cast<uint64_t>(255u); }

// At least `bytes` of device scratch for this call: the config's scratch when it brought
// one (too small is an error), else the context's own, grown on demand. Growing frees the
// old block after the stream's earlier work is done.
cellerator_status context_scratch(cellerator_context *ctx, uint64_t bytes, void **out) {
    *out = nullptr;
    if (bytes == 0u) return CELLERATOR_STATUS_SUCCESS;
    if (!ctx->owns_scratch && ctx->scratch != nullptr) {
        if (ctx->scratch_bytes < bytes)
            return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "context scratch is smaller than the operation needs");
        *out = ctx->scratch;
        return CELLERATOR_STATUS_SUCCESS;
    }
    if (ctx->scratch_bytes < bytes) {
        if (ctx->scratch != nullptr) {
            if (hipStreamSynchronize(ctx->stream) != hipSuccess || hipFree(ctx->scratch) != hipSuccess)
                return fail(CELLERATOR_STATUS_CUDA_ERROR, "releasing the context scratch failed");
            ctx->scratch = nullptr;
            ctx->scratch_bytes = 0u;
        }
        void *p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess)
            return fail(CELLERATOR_STATUS_CUDA_ERROR, "context scratch allocation failed");
        ctx->scratch = p;
        ctx->scratch_bytes = bytes;
        ctx->owns_scratch = true;
    }
    *out = ctx->scratch;
    return CELLERATOR_STATUS_SUCCESS;
}

} // namespace

extern "C" {

const char *cellerator_status_string(cellerator_status status) {
    switch (status) {
    case CELLERATOR_STATUS_SUCCESS: return "success";
    case CELLERATOR_STATUS_INVALID_ARGUMENT: return "invalid argument";
    case CELLERATOR_STATUS_INVALID_SHAPE: return "invalid shape";
    case CELLERATOR_STATUS_UNSUPPORTED: return "unsupported";
    case CELLERATOR_STATUS_CUDA_ERROR: return "device runtime error";
    case CELLERATOR_STATUS_INTERNAL_ERROR: return "internal error";
    }
    return "unknown status";
}

const char *cellerator_last_error(void) { return g_abi_error; }

cellerator_status cellerator_context_create(const cellerator_execution_config *config,
                                            cellerator_context **out_context) {
    g_abi_error[0] = '\0';
    if (out_context == nullptr) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "context output is null");
    *out_context = nullptr;
    cellerator_context *ctx = new (std::nothrow) cellerator_context();
    if (ctx == nullptr) return fail(CELLERATOR_STATUS_INTERNAL_ERROR, "context allocation failed");
    if (config != nullptr) {
        if (!versioned(config->version, config->size, sizeof(cellerator_execution_config))) {
            delete ctx;
            return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "execution config version or size mismatch");
        }
        ctx->device = config->device;
        ctx->stream = static_cast<hipStream_t>(config->stream);
        ctx->scratch = config->scratch;
        ctx->scratch_bytes = config->scratch != nullptr ? config->scratch_bytes : 0u;
    }
    *out_context = ctx;
    return CELLERATOR_STATUS_SUCCESS;
}

cellerator_status cellerator_context_synchronize(cellerator_context *context) {
    if (context == nullptr) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "Cellerator ABI requires a context");
    const hipError_t status = context->stream != nullptr ? hipStreamSynchronize(context->stream)
                                                         : hipDeviceSynchronize();
    if (status != hipSuccess) return fail(CELLERATOR_STATUS_CUDA_ERROR, hipGetErrorString(status));
    return CELLERATOR_STATUS_SUCCESS;
}

void cellerator_context_destroy(cellerator_context *context) {
    if (context == nullptr) return;
    if (context->owns_scratch && context->scratch != nullptr) {
        (void)hipStreamSynchronize(context->stream);
        (void)hipFree(context->scratch);
    }
    delete context;
}

void cellerator_saved_state_destroy(cellerator_saved_state *saved_state) { delete saved_state; }

cellerator_status cellerator_sparse_projection_forward(cellerator_context *context,
                                                       const cellerator_sparse_layout_desc *layout,
                                                       const cellerator_tensor_desc *rhs,
                                                       cellerator_tensor_desc *out,
                                                       cellerator_saved_state **saved_state) {
    g_abi_error[0] = '\0';
    if (saved_state != nullptr) *saved_state = nullptr;
    if (context == nullptr) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "Cellerator ABI requires a context");
    cellerator_status status = validate_layout(layout);
    if (status != CELLERATOR_STATUS_SUCCESS) return status;
    if (rhs == nullptr || out == nullptr)
        return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor descriptor is null");
    status = validate_dense(rhs, layout->cols, 0u, "rhs tensor data is null");
    if (status != CELLERATOR_STATUS_SUCCESS) return status;
    const uint64_t n = rhs->shape[1];
    status = validate_dense(out, layout->rows, n, "output tensor data is null");
    if (status != CELLERATOR_STATUS_SUCCESS) return status;
    if (out->dtype != CELLERATOR_DTYPE_F32) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor dtype mismatch");
    if (rhs->dtype != CELLERATOR_DTYPE_F32 && rhs->dtype != CELLERATOR_DTYPE_F16
        && rhs->dtype != CELLERATOR_DTYPE_BF16)
        return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor dtype mismatch");
    if (context->device >= 0 && hipSetDevice(context->device) != hipSuccess)
        return fail(CELLERATOR_STATUS_CUDA_ERROR, "hipSetDevice failed");

    int rc = CX_STATUS_SUCCESS;
    switch (layout->layout) {
    case CELLERATOR_LAYOUT_CSR:
    case CELLERATOR_LAYOUT_QUANTIZED_CSR: {
        if (rhs->dtype == CELLERATOR_DTYPE_BF16)
            return fail(CELLERATOR_STATUS_UNSUPPORTED, "CSR projection takes F32 or F16 rhs");
        cx_qcsr_matrix m;
        status = csr_view(layout, &m);
        if (status != CELLERATOR_STATUS_SUCCESS) return status;
        rc = cx_qcsr_spmm_fwd(&m, rhs->data, rhs->dtype, matrix_ld(rhs), static_cast<int64_t>(n),
                              static_cast<float *>(out->data), matrix_ld(out), context->stream);
        break;
    }
    case CELLERATOR_LAYOUT_BLOCKED_ELL:
    case CELLERATOR_LAYOUT_QUANTIZED_BLOCKED_ELL: {
        cx_bell_matrix m{};
        m.rows = layout->rows;
        m.cols = layout->cols;
        m.block_size = layout->block_size;
        m.ell_cols = layout->ell_cols;
        m.block_col_idx = layout->block_col_idx;
        if (layout->layout == CELLERATOR_LAYOUT_BLOCKED_ELL) {
            m.values = layout->values;
            m.value_dtype = layout->value_dtype;
        } else {
            m.bits = layout->bits;
            m.decode_policy = layout->decode_policy;
            m.row_stride_bytes = layout->row_stride_bytes;
            m.packed_values = layout->packed_values;
            m.column_scales = layout->column_scales;
            m.column_offsets = layout->column_offsets;
            m.row_offsets = layout->row_offsets;
        }
        rc = cx_bell_spmm_fwd(&m, rhs->data, rhs->dtype, matrix_ld(rhs), static_cast<int64_t>(n),
                              static_cast<float *>(out->data), matrix_ld(out), context->stream);
        break;
    }
    default:
        return fail(CELLERATOR_STATUS_UNSUPPORTED, "sparse layout is not supported by the projection forward");
    }
    if (rc != CX_STATUS_SUCCESS) return from_cx(rc);
    if (saved_state != nullptr) {
        cellerator_saved_state *state = new (std::nothrow) cellerator_saved_state();
        if (state == nullptr) return fail(CELLERATOR_STATUS_INTERNAL_ERROR, "saved state allocation failed");
        state->kind = CELLERATOR_SAVED_STATE_SPARSE_PROJECTION;
        state->layout = layout->layout;
        state->rows = layout->rows;
        state->cols = layout->cols;
        state->nnz = layout->nnz;
        state->out_cols = static_cast<uint32_t>(n);
        *saved_state = state;
    }
    return CELLERATOR_STATUS_SUCCESS;
}

cellerator_status cellerator_sparse_projection_backward(cellerator_context *context,
                                                        const cellerator_sparse_layout_desc *layout,
                                                        const cellerator_tensor_desc *rhs,
                                                        const cellerator_tensor_desc *grad_out,
                                                        cellerator_tensor_desc *grad_values,
                                                        cellerator_tensor_desc *grad_rhs) {
    g_abi_error[0] = '\0';
    if (context == nullptr) return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "Cellerator ABI requires a context");
    cellerator_status status = validate_layout(layout);
    if (status != CELLERATOR_STATUS_SUCCESS) return status;
    if (layout->layout != CELLERATOR_LAYOUT_CSR && layout->layout != CELLERATOR_LAYOUT_QUANTIZED_CSR)
        return fail(CELLERATOR_STATUS_UNSUPPORTED, "operator currently requires CSR layout");
    if (layout->layout == CELLERATOR_LAYOUT_CSR && layout->value_dtype != CELLERATOR_DTYPE_F16
        && layout->value_dtype != CELLERATOR_DTYPE_F32)
        return fail(CELLERATOR_STATUS_UNSUPPORTED, "operator currently requires fp16 or fp32 sparse values");
    cx_qcsr_matrix m;
    status = csr_view(layout, &m);
    if (status != CELLERATOR_STATUS_SUCCESS) return status;
    status = validate_dense(rhs, layout->cols, 0u, "rhs data is null");
    if (status != CELLERATOR_STATUS_SUCCESS) return status;
    if (rhs->dtype != CELLERATOR_DTYPE_F32 && rhs->dtype != CELLERATOR_DTYPE_F16)
        return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor dtype mismatch");
    const uint64_t n = rhs->shape[1];
    status = validate_dense(grad_out, layout->rows, n, "grad_out data is null");
    if (status != CELLERATOR_STATUS_SUCCESS) return status;
    if (grad_out->dtype != CELLERATOR_DTYPE_F32)
        return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor dtype mismatch");
    if (grad_values == nullptr && grad_rhs == nullptr)
        return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "projection backward requires at least one gradient output");
    if (grad_values != nullptr) {
        status = validate_vector(grad_values, layout->nnz, "grad_values data is null");
        if (status != CELLERATOR_STATUS_SUCCESS) return status;
    }
    if (grad_rhs != nullptr) {
        status = validate_dense(grad_rhs, layout->cols, n, "grad_rhs data is null");
        if (status != CELLERATOR_STATUS_SUCCESS) return status;
        if (grad_rhs->dtype != CELLERATOR_DTYPE_F32)
            return fail(CELLERATOR_STATUS_INVALID_ARGUMENT, "tensor dtype mismatch");
    }
    if (context->device >= 0 && hipSetDevice(context->device) != hipSuccess)
        return fail(CELLERATOR_STATUS_CUDA_ERROR, "hipSetDevice failed");

    if (grad_values != nullptr) {
        const int rc = cx_qcsr_spmm_bwd_values(&m, static_cast<const float *>(grad_out->data),
                                               matrix_ld(grad_out), rhs->data, rhs->dtype, matrix_ld(rhs),
                                               static_cast<int64_t>(n),
                                               static_cast<float *>(grad_values->data), context->stream);
        if (rc != CX_STATUS_SUCCESS) return from_cx(rc);
    }
    if (grad_rhs != nullptr) {
        // grad_rhs = A^T . grad_out: the transpose (decoded f32 values) into the scratch,
        // then the deterministic balanced SpMM over it; both workspaces share one region.
        uint64_t t_ws = 0u, b_ws = 0u;
        int rc = cx_qcsr_transpose_workspace(&m, &t_ws);
        if (rc != CX_STATUS_SUCCESS) return from_cx(rc);
        cx_qcsr_matrix t{};
        t.rows = m.cols;
        t.cols = m.rows;
        t.nnz = m.nnz;
        t.bits = 0u;
        t.value_dtype = CELLERATOR_DTYPE_F32;
        rc = cx_qcsr_spmm_balanced_workspace(&t, static_cast<int64_t>(n), &b_ws);
        if (rc != CX_STATUS_SUCCESS) return from_cx(rc);
        const uint64_t ptr_bytes = align256((static_cast<uint64_t>(m.cols) + 1u) * 4u);
        const uint64_t arr_bytes = align256(m.nnz * 4u);
        const uint64_t work = t_ws > b_ws ? t_ws : b_ws;
        void *scratch = nullptr;
        status = context_scratch(context, ptr_bytes + 2u * arr_bytes + work, &scratch);
        if (status != CELLERATOR_STATUS_SUCCESS) return status;
        auto *base = static_cast<unsigned char *>(scratch);
        auto *t_row_ptr = reinterpret_cast<int32_t *>(base);
        auto *t_col_idx = reinterpret_cast<int32_t *>(base + ptr_bytes);
        auto *t_values = reinterpret_cast<float *>(base + ptr_bytes + arr_bytes);
        void *ws = base + ptr_bytes + 2u * arr_bytes;
        rc = cx_qcsr_transpose(&m, t_row_ptr, t_col_idx, t_values, ws, work, context->stream);
        if (rc != CX_STATUS_SUCCESS) return from_cx(rc);
        t.row_ptr = t_row_ptr;
        t.col_idx = t_col_idx;
        t.values = t_values;
        rc = cx_qcsr_spmm_bwd_rhs(&t, static_cast<const float *>(grad_out->data), matrix_ld(grad_out),
                                  static_cast<int64_t>(n), static_cast<float *>(grad_rhs->data),
                                  matrix_ld(grad_rhs), ws, work, context->stream);
        if (rc != CX_STATUS_SUCCESS) return from_cx(rc);
    }
    return CELLERATOR_STATUS_SUCCESS;
}

} // extern "C"
