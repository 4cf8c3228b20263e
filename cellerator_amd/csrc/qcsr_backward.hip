// qcsr_backward.hip -- transpose and backward of the (quantized) CSR SpMM Y = A . W.
//
//   grad_values = (grad_Y . W^T) sampled at A's nonzeros: one dot product of length N per
//                 stored entry (csr_spmm_bwd_values_kernel_,
//                 src/compute/sparse/ops/kernels/base_sparse/csr_spmm_bwd_values_kernel_.cuh).
//   grad_W      = A^T . grad_Y (csr_spmm_bwd_rhs_kernel_, same directory). The reference
//                 scatters with float atomics after a memset, so its summation order varies
//                 from run to run. Here A^T is built once per structure (and value
//                 generation) as a plain f32 CSR -- genes x cells, cells ascending in each
//                 row, values decoded exactly as the forward decodes them -- and grad_W is
//                 the forward row-wave SpMM on it: a fixed order, no atomics, no memset.
//
// Transpose build: stable radix sort of the column indices with the entry index as payload
// (sort.hip), row pointers by binary search of each gene in the sorted keys, then one pass
// that maps every sorted entry back to its cell row (binary search of the CSR row pointers)
// and decodes its value.
#include "qcsr_common.hpp"

namespace cx {
namespace {

// ---- grad_values ------------------------------------------------------------------------

struct BwdValuesArgs {
    const std::int32_t *row_ptr;
    const std::int32_t *col_idx;
    const float *grad_out;
    std::int64_t grad_out_ld;
    const void *rhs;
    std::int64_t rhs_ld;
    float *grad_values;
    std::uint32_t rows;
};

// Row per wave; lane group g (kLpe lanes) takes entry s + g of the staged 64, each lane
// holding kCpl consecutive columns of the row's grad_Y segment in registers and reading
// 16 B of the entry's weight row; the group's partial dots are summed with a butterfly.
template<typename RhsT, int kN>
__global__ __launch_bounds__(kWave *kWavesPerBlock) void qcsr_bwd_values_rowwave(BwdValuesArgs a) {
    constexpr int kCpl = 16 / static_cast<int>(sizeof(RhsT));
    constexpr int kLpe = kN / kCpl;
    constexpr int kEps = kWave / kLpe;
    constexpr int kLastBit = __builtin_ctz(kLpe) - 1;
    static_assert(kN % kCpl == 0 && kLpe <= kWave && kWave % kLpe == 0 && kLpe >= 2, "bad shape");
    __shared__ int stage[kWavesPerBlock][kWave];
    __shared__ float result[kWavesPerBlock][kWave];

    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t row = blockIdx.x * kWavesPerBlock + wave;
    if (row >= a.rows) return;
    const int g = lane / kLpe;
    const int j = lane % kLpe;
    const std::int64_t begin = a.row_ptr[row];
    const std::int64_t end = a.row_ptr[row + 1];

    float go[kCpl];
    {
        const float4 *src = reinterpret_cast<const float4 *>(
            a.grad_out + static_cast<std::int64_t>(row) * a.grad_out_ld + j * kCpl);
#pragma unroll
        for (int k = 0; k < kCpl / 4; ++k) {
            const float4 v = src[k];
            go[4 * k] = v.x; go[4 * k + 1] = v.y; go[4 * k + 2] = v.z; go[4 * k + 3] = v.w;
        }
    }
    const RhsT *rhs = static_cast<const RhsT *>(a.rhs) + j * kCpl;

    for (std::int64_t c0 = begin; c0 < end; c0 += kWave) {
        const std::int64_t i = c0 + lane;
        stage[wave][lane] = i < end ? a.col_idx[i] : 0;
        wave_sync();
        const int count = end - c0 < kWave ? static_cast<int>(end - c0) : kWave;
        for (int s = 0; s < count; s += kEps) {
            const int e = s + g;  // < 64; entries past `count` read gene 0 and are not stored
            const RhsT *w = rhs + static_cast<std::int64_t>(stage[wave][e]) * a.rhs_ld;
            float dot = 0.0f;
            if constexpr (sizeof(RhsT) == 2) {
                const uint4 raw = *reinterpret_cast<const uint4 *>(w);
                const unsigned words[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    dot = __builtin_fmaf(go[2 * k], h2f(static_cast<std::uint16_t>(words[k] & 0xffffu)), dot);
                    dot = __builtin_fmaf(go[2 * k + 1], h2f(static_cast<std::uint16_t>(words[k] >> 16)), dot);
                }
            } else {
                const float4 v = *reinterpret_cast<const float4 *>(w);
                dot = __builtin_fmaf(go[0], v.x, dot);
                dot = __builtin_fmaf(go[1], v.y, dot);
                dot = __builtin_fmaf(go[2], v.z, dot);
                dot = __builtin_fmaf(go[3], v.w, dot);
            }
            dot = xor_reduce<0, kLastBit>(dot);
            if (j == 0) result[wave][e] = dot;
        }
        wave_sync();
        if (lane < count) a.grad_values[c0 + lane] = result[wave][lane];
        wave_sync();
    }
}

// Any N / alignment: lanes over the row's entries, columns in order (grad_Y row read
// uniformly by the wave).
template<typename RhsT>
__global__ __launch_bounds__(kWave *kWavesPerBlock) void qcsr_bwd_values_generic(BwdValuesArgs a,
                                                                                std::int64_t n) {
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint32_t row = blockIdx.x * kWavesPerBlock + wave;
    if (row >= a.rows) return;
    const std::int64_t begin = a.row_ptr[row];
    const std::int64_t end = a.row_ptr[row + 1];
    const float *go = a.grad_out + static_cast<std::int64_t>(row) * a.grad_out_ld;
    for (std::int64_t i = begin + lane; i < end; i += kWave) {
        const RhsT *w = static_cast<const RhsT *>(a.rhs) + static_cast<std::int64_t>(a.col_idx[i]) * a.rhs_ld;
        float dot = 0.0f;
        for (std::int64_t c = 0; c < n; ++c) {
            float wf;
            if constexpr (sizeof(RhsT) == 2) wf = h2f(w[c]);
            else wf = w[c];
            dot = __builtin_fmaf(go[c], wf, dot);
        }
        a.grad_values[i] = dot;
    }
}

template<typename RhsT>
int launch_bwd_values(const BwdValuesArgs &a, std::int64_t n, bool aligned, hipStream_t s) {
    const dim3 grid((a.rows + kWavesPerBlock - 1) / kWavesPerBlock), block(kWave * kWavesPerBlock);
    constexpr bool kHalf = sizeof(RhsT) == 2;
    if (aligned && n == 64) {
        hipLaunchKernelGGL((qcsr_bwd_values_rowwave<RhsT, 64>), grid, block, 0, s, a);
    } else if (aligned && n == 128) {
        hipLaunchKernelGGL((qcsr_bwd_values_rowwave<RhsT, 128>), grid, block, 0, s, a);
    } else if (aligned && kHalf && n == 32) {
        hipLaunchKernelGGL((qcsr_bwd_values_rowwave<RhsT, kHalf ? 32 : 64>), grid, block, 0, s, a);
    } else {
        hipLaunchKernelGGL(qcsr_bwd_values_generic<RhsT>, grid, block, 0, s, a, n);
    }
    return check_launch("qcsr_bwd_values");
}

// ---- transpose ----------------------------------------------------------------------------

__global__ void transpose_row_ptr_kernel(const std::uint32_t *sorted_genes, std::uint32_t nnz,
                                         std::uint32_t cols, std::int32_t *t_row_ptr) {
    const std::uint32_t gene = blockIdx.x * blockDim.x + threadIdx.x;
    if (gene > cols) return;
    std::uint32_t lo = 0u, hi = nnz;  // first position whose gene >= `gene`
    while (lo < hi) {
        const std::uint32_t mid = lo + (hi - lo) / 2u;
        if (sorted_genes[mid] < gene) lo = mid + 1u;
        else hi = mid;
    }
    t_row_ptr[gene] = static_cast<std::int32_t>(lo);
}

// t_col_idx holds the sorted entry indices on entry and the cell rows on exit.
template<int kBits, int kPolicy, ValueMode kMode>
__global__ void transpose_finalize_kernel(QcsrArgs a, std::uint32_t nnz, std::int32_t *t_col_idx,
                                          float *t_values) {
    const std::uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nnz) return;
    const std::int32_t e = t_col_idx[t];
    std::uint32_t lo = 0u, hi = a.rows;  // last row whose start <= e
    while (hi - lo > 1u) {
        const std::uint32_t mid = lo + (hi - lo) / 2u;
        if (a.row_ptr[mid] <= e) lo = mid;
        else hi = mid;
    }
    const std::uint32_t row = lo;
    const std::uint8_t *pbase = nullptr;
    float row_offset = 0.0f;
    if constexpr (kMode == ValueMode::quantized) {
        pbase = a.packed + a.packed_row_ptr[row];
        if constexpr (kPolicy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
            row_offset = a.row_offsets != nullptr ? a.row_offsets[row] : 0.0f;
    }
    int col;
    t_values[t] = load_entry<kBits, kPolicy, kMode>(a, e, a.row_ptr[row], pbase, row_offset, col);
    t_col_idx[t] = static_cast<std::int32_t>(row);
}

template<int kBits, int kPolicy, ValueMode kMode>
void launch_finalize(const QcsrArgs &a, std::uint32_t nnz, std::int32_t *t_col_idx, float *t_values,
                     hipStream_t s) {
    hipLaunchKernelGGL((transpose_finalize_kernel<kBits, kPolicy, kMode>), dim3((nnz + 255u) / 256u),
                       dim3(256), 0, s, a, nnz, t_col_idx, t_values);
}

template<int kPolicy>
int finalize_bits(const QcsrArgs &a, std::uint32_t bits, std::uint32_t nnz, std::int32_t *tc,
                  float *tv, hipStream_t s) {
    switch (bits) {
    case 1: launch_finalize<1, kPolicy, ValueMode::quantized>(a, nnz, tc, tv, s); break;
    case 2: launch_finalize<2, kPolicy, ValueMode::quantized>(a, nnz, tc, tv, s); break;
    case 4: launch_finalize<4, kPolicy, ValueMode::quantized>(a, nnz, tc, tv, s); break;
    case 8: launch_finalize<8, kPolicy, ValueMode::quantized>(a, nnz, tc, tv, s); break;
    default: return fail(CX_STATUS_UNSUPPORTED, "quantized CSR bits must be 1, 2, 4 or 8");
    }
    return check_launch("qcsr_transpose_finalize");
}

// Checks shared by the transpose: the structure and value arrays the decode reads.
int validate_matrix(const cx_qcsr_matrix *m, const char *who) {
    if (m == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, who);
    if (m->nnz > static_cast<std::uint64_t>(INT32_MAX))
        return fail(CX_STATUS_INVALID_SHAPE, "quantized CSR: nnz exceeds int32 row offsets");
    if (m->rows != 0u && m->row_ptr == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "quantized CSR: null row_ptr");
    if (m->nnz != 0u && m->col_idx == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "quantized CSR: null col_idx");
    if (m->bits != 0u) {
        if (m->packed_row_ptr == nullptr || (m->nnz != 0u && m->packed_values == nullptr))
            return fail(CX_STATUS_INVALID_ARGUMENT, "quantized CSR: needs packed_row_ptr and packed_values");
        if (m->decode_policy != CX_DECODE_PER_GENE_AFFINE && m->decode_policy != CX_DECODE_COLUMN_SCALE_ROW_OFFSET
            && m->decode_policy != CX_DECODE_PER_GENE_AFFINE_PAIRS)
            return fail(CX_STATUS_UNSUPPORTED, "quantized CSR: unknown decode policy");
        if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS
            && (m->column_scales == nullptr || m->column_offsets != nullptr
                || (reinterpret_cast<std::uintptr_t>(m->column_scales) & 7u) != 0u))
            return fail(CX_STATUS_INVALID_ARGUMENT, "quantized CSR: interleaved metadata needs 8-byte aligned pairs");
    } else {
        if (m->nnz != 0u && m->values == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "CSR: null values");
        if (m->value_dtype != CELLERATOR_DTYPE_F16 && m->value_dtype != CELLERATOR_DTYPE_F32)
            return fail(CX_STATUS_UNSUPPORTED, "CSR: value dtype must be F16 or F32");
    }
    return CX_STATUS_SUCCESS;
}

std::uint32_t key_bits_for(std::uint32_t cols) {
    std::uint32_t b = 1u;
    while (b < 32u && (cols - 1u) >> b != 0u) ++b;
    return b;
}

std::uint64_t align256(std::uint64_t b) { return (b + 255u) & ~static_cast<std::uint64_t>(255u); }

// Rows of the (panelled) transpose: panel p, gene g -> row p * cols + g.
std::uint64_t panel_count(const cx_qcsr_matrix *m, std::uint32_t panel_rows) {
    return panel_rows == 0u ? 1u : (static_cast<std::uint64_t>(m->rows) + panel_rows - 1u) / panel_rows;
}

std::uint64_t transpose_workspace(const cx_qcsr_matrix *m, std::uint32_t panel_rows) {
    const std::uint64_t out_rows = panel_count(m, panel_rows) * m->cols;
    std::uint64_t bytes = align256(m->nnz * 4u)
        + sort_pairs_workspace_bytes(m->nnz, key_bits_for(static_cast<std::uint32_t>(out_rows)));
    if (panel_rows != 0u) bytes += align256(m->nnz * 4u);  // the computed keys
    return bytes;
}

// key[i] = panel(row of i) * cols + col[i], one wave per row (coalesced).
__global__ __launch_bounds__(256) void panel_key_kernel(const std::int32_t *row_ptr, const std::int32_t *col_idx,
                                                        std::uint32_t rows, std::uint32_t cols,
                                                        std::uint32_t panel_rows, std::uint32_t *key) {
    const std::uint32_t row = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    if (row >= rows) return;
    const std::uint32_t base = (row / panel_rows) * cols;
    for (std::int64_t i = row_ptr[row] + lane; i < row_ptr[row + 1]; i += kWave)
        key[i] = base + static_cast<std::uint32_t>(col_idx[i]);
}

// grad_rhs[g, c] = sum over panels p (in order) of z[(p * cols + g) * n + c].
__global__ void panel_reduce_kernel(const float *z, std::uint32_t panels, std::uint32_t cols,
                                    std::int64_t n, float *out, std::int64_t out_ld) {
    const std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x;
    if (i >= static_cast<std::uint64_t>(cols) * n) return;
    const std::uint64_t g = i / n, c = i % n;
    float v = 0.0f;
    for (std::uint32_t p = 0; p < panels; ++p) v += z[(static_cast<std::uint64_t>(p) * cols + g) * n + c];
    out[g * out_ld + c] = v;
}

int transpose_impl(const cx_qcsr_matrix *m, std::uint32_t panel_rows, std::int32_t *t_row_ptr,
                   std::int32_t *t_col_idx, float *t_values, void *workspace,
                   std::uint64_t workspace_bytes, hipStream_t s);

bool aligned16(const void *p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0u; }

} // namespace
} // namespace cx

extern "C" int cx_qcsr_transpose_workspace(const cx_qcsr_matrix *m, uint64_t *bytes) {
    return cx_qcsr_transpose_panelled_workspace(m, 0u, bytes);
}

extern "C" int cx_qcsr_transpose_panelled_workspace(const cx_qcsr_matrix *m, uint32_t panel_rows,
                                                    uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (bytes == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_transpose_workspace: null bytes");
    const int rc = validate_matrix(m, "cx_qcsr_transpose_workspace: null matrix");
    if (rc != CX_STATUS_SUCCESS) return rc;
    *bytes = transpose_workspace(m, panel_rows);
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_transpose(const cx_qcsr_matrix *m, int32_t *t_row_ptr, int32_t *t_col_idx,
                                 float *t_values, void *workspace, uint64_t workspace_bytes,
                                 void *stream) {
    cx::clear_error();
    return cx::transpose_impl(m, 0u, t_row_ptr, t_col_idx, t_values, workspace, workspace_bytes,
                              static_cast<hipStream_t>(stream));
}

extern "C" int cx_qcsr_transpose_panelled(const cx_qcsr_matrix *m, uint32_t panel_rows,
                                          int32_t *t_row_ptr, int32_t *t_col_idx, float *t_values,
                                          void *workspace, uint64_t workspace_bytes, void *stream) {
    cx::clear_error();
    if (panel_rows == 0u)
        return cx::fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_transpose_panelled: panel_rows must be positive");
    return cx::transpose_impl(m, panel_rows, t_row_ptr, t_col_idx, t_values, workspace, workspace_bytes,
                              static_cast<hipStream_t>(stream));
}

namespace cx {
namespace {

int transpose_impl(const cx_qcsr_matrix *m, std::uint32_t panel_rows, std::int32_t *t_row_ptr,
                   std::int32_t *t_col_idx, float *t_values, void *workspace,
                   std::uint64_t workspace_bytes, hipStream_t s) {
    int rc = validate_matrix(m, "cx_qcsr_transpose: null matrix");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (m->cols == 0u) return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_transpose: the matrix has no columns");
    const std::uint64_t out_rows = panel_count(m, panel_rows) * m->cols;
    if (out_rows >= 0xFFFFFFFFull)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_transpose: panels x genes exceeds u32 row ids");
    if (t_row_ptr == nullptr || (m->nnz != 0u && (t_col_idx == nullptr || t_values == nullptr)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_transpose: null output");
    if (workspace_bytes < transpose_workspace(m, panel_rows) || (workspace == nullptr && workspace_bytes != 0u))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_transpose: workspace smaller than cx_qcsr_transpose_workspace");
    const std::uint32_t nnz = static_cast<std::uint32_t>(m->nnz);
    auto *ws = static_cast<unsigned char *>(workspace);
    auto *sorted_keys = reinterpret_cast<std::uint32_t *>(ws);
    ws += align256(m->nnz * 4u);
    std::uint64_t left = workspace_bytes - align256(m->nnz * 4u);
    const std::uint32_t *keys = reinterpret_cast<const std::uint32_t *>(m->col_idx);
    if (panel_rows != 0u) {
        auto *computed = reinterpret_cast<std::uint32_t *>(ws);
        ws += align256(m->nnz * 4u);
        left -= align256(m->nnz * 4u);
        if (nnz != 0u) {
            const std::uint64_t threads = static_cast<std::uint64_t>(m->rows) * kWave;
            hipLaunchKernelGGL(panel_key_kernel, dim3(static_cast<unsigned>((threads + 255u) / 256u)), dim3(256),
                               0, s, m->row_ptr, m->col_idx, m->rows, m->cols, panel_rows, computed);
            rc = check_launch("qcsr_transpose_panel_keys");
            if (rc != CX_STATUS_SUCCESS) return rc;
        }
        keys = computed;
    }
    if (nnz != 0u) {
        rc = sort_pairs(keys, nullptr, sorted_keys, reinterpret_cast<std::uint32_t *>(t_col_idx), nnz,
                        key_bits_for(static_cast<std::uint32_t>(out_rows)), ws, left, s);
        if (rc != CX_STATUS_SUCCESS) return rc;
    }
    const std::uint32_t rows_out = static_cast<std::uint32_t>(out_rows);
    hipLaunchKernelGGL(transpose_row_ptr_kernel, dim3((rows_out + 1u + 255u) / 256u), dim3(256), 0, s,
                       sorted_keys, nnz, rows_out, t_row_ptr);
    rc = check_launch("qcsr_transpose_row_ptr");
    if (rc != CX_STATUS_SUCCESS || nnz == 0u) return rc;

    QcsrArgs a{};
    a.row_ptr = m->row_ptr;
    a.packed_row_ptr = m->packed_row_ptr;
    a.col_idx = m->col_idx;
    a.packed = m->packed_values;
    a.scales = m->column_scales;
    a.offsets = m->column_offsets;
    a.row_offsets = m->row_offsets;
    a.values = m->values;
    a.rows = m->rows;
    a.cols = m->cols;
    if (m->bits == 0u) {
        if (m->value_dtype == CELLERATOR_DTYPE_F16)
            launch_finalize<0, CX_DECODE_PER_GENE_AFFINE, ValueMode::f16>(a, nnz, t_col_idx, t_values, s);
        else
            launch_finalize<0, CX_DECODE_PER_GENE_AFFINE, ValueMode::f32>(a, nnz, t_col_idx, t_values, s);
        return check_launch("qcsr_transpose_finalize");
    }
    if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE)
        return finalize_bits<CX_DECODE_PER_GENE_AFFINE>(a, m->bits, nnz, t_col_idx, t_values, s);
    if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS)
        return finalize_bits<CX_DECODE_PER_GENE_AFFINE_PAIRS>(a, m->bits, nnz, t_col_idx, t_values, s);
    return finalize_bits<CX_DECODE_COLUMN_SCALE_ROW_OFFSET>(a, m->bits, nnz, t_col_idx, t_values, s);
}

} // namespace
} // namespace cx

extern "C" int cx_qcsr_spmm_bwd_values(const cx_qcsr_matrix *m, const float *grad_out,
                                       int64_t grad_out_ld, const void *rhs, uint32_t rhs_dtype,
                                       int64_t rhs_ld, int64_t out_cols, float *grad_values,
                                       void *stream) {
    using namespace cx;
    clear_error();
    if (m == nullptr || grad_out == nullptr || rhs == nullptr || (m->nnz != 0u && grad_values == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_bwd_values: null argument");
    if (rhs_dtype != CELLERATOR_DTYPE_F16 && rhs_dtype != CELLERATOR_DTYPE_F32)
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_spmm_bwd_values: rhs dtype must be F16 or F32");
    if (out_cols <= 0 || grad_out_ld < out_cols || rhs_ld < out_cols)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_spmm_bwd_values: bad out_cols or leading dimension");
    if (m->nnz > static_cast<std::uint64_t>(INT32_MAX))
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_spmm_bwd_values: nnz exceeds int32 row offsets");
    if (m->rows == 0u || m->nnz == 0u) return CX_STATUS_SUCCESS;
    if (m->row_ptr == nullptr || m->col_idx == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_bwd_values: null row_ptr or col_idx");
    BwdValuesArgs a{m->row_ptr, m->col_idx, grad_out, grad_out_ld, rhs, rhs_ld, grad_values, m->rows};
    const std::size_t esize = rhs_dtype == CELLERATOR_DTYPE_F16 ? 2u : 4u;
    const bool aligned = aligned16(grad_out) && aligned16(rhs) && (grad_out_ld * 4) % 16 == 0
        && (rhs_ld * static_cast<std::int64_t>(esize)) % 16 == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (bwd_values_parts_applicable(m->rows, m->cols, rhs_dtype, out_cols, aligned, rhs_ld))
        return launch_bwd_values_parts(m->row_ptr, m->col_idx, grad_out, grad_out_ld, rhs, rhs_ld, grad_values,
                                       m->rows, m->cols, (m->flags & CX_QCSR_COLUMNS_SORTED) != 0u, s);
    if (rhs_dtype == CELLERATOR_DTYPE_F16) return launch_bwd_values<std::uint16_t>(a, out_cols, aligned, s);
    return launch_bwd_values<float>(a, out_cols, aligned, s);
}

extern "C" int cx_qcsr_spmm_bwd_rhs(const cx_qcsr_matrix *transposed, const float *grad_out,
                                    int64_t grad_out_ld, int64_t out_cols, float *grad_rhs,
                                    int64_t grad_rhs_ld, void *workspace,
                                    uint64_t workspace_bytes, void *stream) {
    using namespace cx;
    clear_error();
    if (transposed == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_bwd_rhs: null transposed matrix");
    if (transposed->bits != 0u || transposed->value_dtype != CELLERATOR_DTYPE_F32)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_spmm_bwd_rhs: expects the f32 transpose built by cx_qcsr_transpose");
    // gene rows of an expression matrix are heavily skewed: the balanced form
    return cx_qcsr_spmm_fwd_balanced(transposed, grad_out, CELLERATOR_DTYPE_F32, grad_out_ld,
                                     out_cols, grad_rhs, grad_rhs_ld, nullptr, workspace,
                                     workspace_bytes, stream);
}

extern "C" int cx_qcsr_spmm_bwd_rhs_panelled_workspace(const cx_qcsr_matrix *panelled, uint32_t panels,
                                                      int64_t out_cols, uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (panelled == nullptr || bytes == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_bwd_rhs_panelled_workspace: null argument");
    if (panels == 0u || out_cols <= 0 || panelled->rows % panels != 0u)
        return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_spmm_bwd_rhs_panelled_workspace: bad panels or columns");
    std::uint64_t balanced = 0u;
    const int rc = cx_qcsr_spmm_balanced_workspace(panelled, out_cols, &balanced);
    if (rc != CX_STATUS_SUCCESS) return rc;
    *bytes = align256(static_cast<std::uint64_t>(panelled->rows) * static_cast<std::uint64_t>(out_cols) * 4u)
        + align256(balanced);
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_spmm_bwd_rhs_panelled(const cx_qcsr_matrix *panelled, uint32_t panels,
                                             const float *grad_out, int64_t grad_out_ld, int64_t out_cols,
                                             float *grad_rhs, int64_t grad_rhs_ld, void *workspace,
                                             uint64_t workspace_bytes, void *stream) {
    using namespace cx;
    clear_error();
    if (panelled == nullptr || grad_rhs == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_spmm_bwd_rhs_panelled: null argument");
    if (panelled->bits != 0u || panelled->value_dtype != CELLERATOR_DTYPE_F32)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_spmm_bwd_rhs_panelled: expects the f32 transpose built by cx_qcsr_transpose_panelled");
    std::uint64_t need = 0u;
    int rc = cx_qcsr_spmm_bwd_rhs_panelled_workspace(panelled, panels, out_cols, &need);
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (workspace == nullptr || workspace_bytes < need || (reinterpret_cast<std::uintptr_t>(workspace) & 15u) != 0u)
        return fail(CX_STATUS_INVALID_ARGUMENT,
                    "cx_qcsr_spmm_bwd_rhs_panelled: workspace (16-byte aligned) smaller than the query");
    if (grad_rhs_ld < out_cols) return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_spmm_bwd_rhs_panelled: bad grad_rhs_ld");
    const std::uint32_t genes = panelled->rows / panels;
    auto *z = static_cast<float *>(workspace);
    const std::uint64_t z_bytes = align256(static_cast<std::uint64_t>(panelled->rows) * out_cols * 4u);
    rc = cx_qcsr_spmm_fwd_balanced(panelled, grad_out, CELLERATOR_DTYPE_F32, grad_out_ld, out_cols, z, out_cols,
                                   nullptr, static_cast<unsigned char *>(workspace) + z_bytes,
                                   workspace_bytes - z_bytes, stream);
    if (rc != CX_STATUS_SUCCESS) return rc;
    const std::uint64_t total = static_cast<std::uint64_t>(genes) * static_cast<std::uint64_t>(out_cols);
    if (total == 0u) return CX_STATUS_SUCCESS;
    hipLaunchKernelGGL(panel_reduce_kernel, dim3(static_cast<unsigned>((total + 255u) / 256u)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), z, panels, genes, out_cols, grad_rhs, grad_rhs_ld);
    return check_launch("qcsr_bwd_rhs_panel_reduce");
}
