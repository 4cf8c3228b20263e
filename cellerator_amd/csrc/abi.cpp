// abi.cpp -- public context ABI (include/cellerator_amd.h, part 2), layout-compatible
// with the reference's include/Cellerator/abi.h. Validation order and status mapping
// follow src/abi/abi.cu:62-218 and :278-330; dispatch goes to the cx_* launch layer.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <new>

#include "cellerator_amd.h"

struct cellerator_context {
    int device = 0;
    hipStream_t stream = nullptr;
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
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
    if (t->stride[1] != 1 || t->stride[0] < static_cast<int64_t>(t->shape[1]))
        return fail(CELLERATOR_STATUS_INVALID_SHAPE, "tensor must be row-major with unit column stride");
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
        ctx->scratch_bytes = config->scratch_bytes;
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

void cellerator_context_destroy(cellerator_context *context) { delete context; }

void cellerator_saved_state_destroy(cellerator_saved_state *saved_state) { delete saved_state; }

cellerator_status cellerator_sparse_projection_forward(cellerator_context *context,
                                                       const cellerator_sparse_layout_desc *layout,
                                                       const cellerator_tensor_desc *rhs,
                                                       cellerator_tensor_desc *out,
                                                       cellerator_saved_state **saved_state) {
    g_abi_error[0] = '\0';
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
    if (hipSetDevice(context->device) != hipSuccess)
        return fail(CELLERATOR_STATUS_CUDA_ERROR, "hipSetDevice failed");

    int rc = CX_STATUS_SUCCESS;
    switch (layout->layout) {
    case CELLERATOR_LAYOUT_CSR:
    case CELLERATOR_LAYOUT_QUANTIZED_CSR: {
        if (rhs->dtype == CELLERATOR_DTYPE_BF16)
            return fail(CELLERATOR_STATUS_UNSUPPORTED, "CSR projection takes F32 or F16 rhs");
        cx_qcsr_matrix m{};
        m.rows = layout->rows;
        m.cols = layout->cols;
        m.nnz = layout->nnz;
        m.row_ptr = reinterpret_cast<const int32_t *>(layout->major_ptr);
        m.col_idx = reinterpret_cast<const int32_t *>(layout->minor_idx);
        if (layout->layout == CELLERATOR_LAYOUT_CSR) {
            m.bits = 0u;
            m.values = layout->values;
            m.value_dtype = layout->value_dtype;
        } else {
            m.bits = layout->bits;
            m.decode_policy = layout->decode_policy;
            m.packed_row_ptr = reinterpret_cast<const int32_t *>(layout->block_col_idx);
            m.packed_values = layout->packed_values;
            m.column_scales = layout->column_scales;
            m.column_offsets = layout->column_offsets;
            m.row_offsets = layout->row_offsets;
        }
        rc = cx_qcsr_spmm_fwd(&m, rhs->data, rhs->dtype, rhs->stride[0], static_cast<int64_t>(n),
                              static_cast<float *>(out->data), out->stride[0], context->stream);
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
        rc = cx_bell_spmm_fwd(&m, rhs->data, rhs->dtype, rhs->stride[0], static_cast<int64_t>(n),
                              static_cast<float *>(out->data), out->stride[0], context->stream);
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

} // extern "C"
