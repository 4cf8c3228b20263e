// exec_order.hip -- the execution feature order on the device: the packed dense operand
// (W rows gathered into execution order), per-gene column counts, and the reordering of a
// quantized CSR's columns into execution order.
//
// An execution order is a permutation of the gene axis: feature_permutation[e] is the
// canonical gene at execution position e (the frozen packing plan's convention,
// components/CellPack/include/CellPack/packing_plan.hh:39-128). X . W is invariant under
// relabelling the genes of X and the rows of W together, so a projection may run on
// (X_exec, W_exec) and give the same Y. The engine uses this to put the most frequently
// stored genes first, where the head kernel turns them into dense matrix-core tiles.
#include "cx_common.hpp"

#include <algorithm>

namespace cx {
namespace {

// packed[e][c] = source[perm[e]][c] (row-major source) or source[c][perm[e]] (column-major),
// packed contiguous row-major features x columns: pack_dense_rows_kernel of
// src/compute/math/packed_dense_operand.cu:131-151, one element per thread (grid-stride).
template<typename T>
__global__ __launch_bounds__(256) void pack_dense_kernel(const std::uint32_t *perm, const T *source,
                                                         std::uint32_t features, std::uint64_t columns,
                                                         std::uint64_t ld, std::uint32_t column_major,
                                                         T *packed) {
    const std::uint64_t count = static_cast<std::uint64_t>(features) * columns;
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    for (std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const std::uint64_t e = i / columns;
        const std::uint64_t c = i - e * columns;
        const std::uint64_t g = perm[e];
        packed[i] = source[column_major != 0u ? c * ld + g : g * ld + c];
    }
}

__global__ __launch_bounds__(256) void fill_u32_kernel(std::uint32_t *p, std::uint64_t n, std::uint32_t v) {
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    for (std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        p[i] = v;
}

// Column histogram: each workgroup counts a contiguous slice of the entries into LDS bins
// (one u32 per gene), then adds its nonzero bins to the global counts. Columns outside
// [0, cols) are not counted.
__global__ __launch_bounds__(1024) void column_counts_lds(const std::int32_t *col_idx, std::uint64_t nnz,
                                                          std::uint32_t cols, std::uint64_t per_block,
                                                          std::uint32_t *counts) {
    extern __shared__ std::uint32_t bins[];
    for (std::uint32_t g = threadIdx.x; g < cols; g += blockDim.x) bins[g] = 0u;
    __syncthreads();
    const std::uint64_t begin = static_cast<std::uint64_t>(blockIdx.x) * per_block;
    const std::uint64_t end = begin + per_block < nnz ? begin + per_block : nnz;
    for (std::uint64_t i = begin + threadIdx.x; i < end; i += blockDim.x) {
        const std::uint32_t g = static_cast<std::uint32_t>(col_idx[i]);
        if (g < cols) atomicAdd(&bins[g], 1u);
    }
    __syncthreads();
    for (std::uint32_t g = threadIdx.x; g < cols; g += blockDim.x)
        if (bins[g] != 0u) atomicAdd(&counts[g], bins[g]);
}

__global__ __launch_bounds__(256) void column_counts_global(const std::int32_t *col_idx, std::uint64_t nnz,
                                                            std::uint32_t cols, std::uint32_t *counts) {
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    for (std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nnz; i += stride) {
        const std::uint32_t g = static_cast<std::uint32_t>(col_idx[i]);
        if (g < cols) atomicAdd(&counts[g], 1u);
    }
}

// Reorders one row per workgroup (grid-stride over rows) into execution order: every entry's
// execution gene e = inverse[canonical gene] is marked in an LDS bitmap of the genes; the
// exclusive prefix of the bitmap's popcounts gives each entry its output position (the rank
// of e among the row's genes), so the row comes out sorted by e with its codes carried along.
// Codes are staged in LDS words (kBits per entry, little-endian in a byte, as the input) and
// written out byte by byte over the row's unchanged byte range. A repeated gene in a row, or a
// column outside [0, cols), sets *error (output undefined).
template<int kBits, typename ValueT>
__global__ __launch_bounds__(256) void reorder_rows_kernel(const std::int32_t *row_ptr, const std::int32_t *packed_row_ptr,
                                                           const std::int32_t *col_idx, const std::uint8_t *packed,
                                                           const ValueT *values, const std::uint32_t *inverse,
                                                           std::uint32_t rows, std::uint32_t cols,
                                                           std::int32_t *col_out, std::uint8_t *packed_out,
                                                           ValueT *values_out, std::uint32_t *error) {
    extern __shared__ std::uint32_t lds[];
    const std::uint32_t words = (cols + 31u) / 32u;
    std::uint32_t *bitmap = lds;
    std::uint32_t *prefix = lds + words;
    std::uint32_t *stage = lds + 2u * words;
    __shared__ std::uint32_t wave_sums[4];
    const std::uint32_t tid = threadIdx.x;
    const std::uint32_t per = (words + 255u) / 256u;  // bitmap words per thread in the scan
    for (std::uint32_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const std::int64_t begin = row_ptr[row], end = row_ptr[row + 1];
        const std::uint32_t n = static_cast<std::uint32_t>(end - begin);
        if (n == 0u) continue;  // uniform across the workgroup
        const std::uint32_t row_bytes = kBits == 0 ? 0u : static_cast<std::uint32_t>(packed_row_ptr[row + 1] - packed_row_ptr[row]);
        const std::uint32_t stage_words = (row_bytes + 3u) / 4u;
        for (std::uint32_t w = tid; w < words; w += 256u) bitmap[w] = 0u;
        for (std::uint32_t w = tid; w < stage_words; w += 256u) stage[w] = 0u;
        __syncthreads();
        bool bad = false;
        for (std::uint32_t i = tid; i < n; i += 256u) {
            const std::uint32_t g = static_cast<std::uint32_t>(col_idx[begin + i]);
            if (g >= cols) { bad = true; continue; }
            const std::uint32_t e = inverse[g];
            if (e >= cols) { bad = true; continue; }
            const std::uint32_t bit = 1u << (e & 31u);
            if ((atomicOr(&bitmap[e >> 5], bit) & bit) != 0u) bad = true;
        }
        __syncthreads();
        // exclusive scan of the words' popcounts: thread t sums words [t per, t per + per)
        std::uint32_t local = 0u;
        for (std::uint32_t k = 0; k < per; ++k) {
            const std::uint32_t w = tid * per + k;
            if (w < words) local += __popc(bitmap[w]);
        }
        std::uint32_t incl = local;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const std::uint32_t up = __shfl_up(incl, d, kWave);
            if (static_cast<int>(tid % kWave) >= d) incl += up;
        }
        if (tid % kWave == kWave - 1) wave_sums[tid / kWave] = incl;
        __syncthreads();
        std::uint32_t base = 0u;
        for (std::uint32_t v = 0; v < tid / kWave; ++v) base += wave_sums[v];
        std::uint32_t run = base + incl - local;
        for (std::uint32_t k = 0; k < per; ++k) {
            const std::uint32_t w = tid * per + k;
            if (w < words) {
                prefix[w] = run;
                run += __popc(bitmap[w]);
            }
        }
        __syncthreads();
        const std::uint8_t *pin = kBits == 0 ? nullptr : packed + packed_row_ptr[row];
        for (std::uint32_t i = tid; i < n; i += 256u) {
            const std::uint32_t g = static_cast<std::uint32_t>(col_idx[begin + i]);
            if (g >= cols) continue;
            const std::uint32_t e = inverse[g];
            if (e >= cols) continue;
            const std::uint32_t below = bitmap[e >> 5] & ((1u << (e & 31u)) - 1u);
            const std::uint32_t pos = prefix[e >> 5] + __popc(below);
            if (pos >= n) continue;  // only with repeated genes (flagged above)
            col_out[begin + pos] = static_cast<std::int32_t>(e);
            if constexpr (kBits == 0) {
                values_out[begin + pos] = values[begin + i];
            } else {
                const std::uint32_t bit_in = i * kBits;
                const std::uint32_t code = (static_cast<std::uint32_t>(pin[bit_in >> 3]) >> (bit_in & 7u)) & ((1u << kBits) - 1u);
                const std::uint32_t bit_out = pos * kBits;
                atomicOr(&stage[bit_out >> 5], code << (bit_out & 31u));
            }
        }
        if (__syncthreads_or(bad ? 1 : 0) != 0 && tid == 0) atomicOr(error, 1u);
        if constexpr (kBits != 0) {
            std::uint8_t *pout = packed_out + packed_row_ptr[row];
            for (std::uint32_t b = tid; b < row_bytes; b += 256u)
                pout[b] = static_cast<std::uint8_t>(stage[b >> 2] >> (8u * (b & 3u)));
        }
        __syncthreads();  // the next row reuses the LDS
    }
}

bool valid_value_size(std::uint32_t bytes) { return bytes == 1u || bytes == 2u || bytes == 4u || bytes == 8u; }

unsigned grid_for(std::uint64_t count) {
    const std::uint64_t blocks = (count + 255u) / 256u;
    return static_cast<unsigned>(std::min<std::uint64_t>(std::max<std::uint64_t>(blocks, 1u), 65536u));
}

} // namespace
} // namespace cx

extern "C" int cx_pack_dense_operand(const uint32_t *feature_permutation, uint32_t feature_count,
                                     const void *canonical, uint64_t column_count, uint64_t leading_dimension,
                                     uint32_t column_major, uint32_t value_size_bytes, void *packed,
                                     uint64_t packed_capacity_bytes, void *stream) {
    using namespace cx;
    clear_error();
    if (!valid_value_size(value_size_bytes))
        return fail(CX_STATUS_UNSUPPORTED, "cx_pack_dense_operand: value size must be 1, 2, 4 or 8 bytes");
    const std::uint64_t count = static_cast<std::uint64_t>(feature_count) * column_count;
    if (count == 0u) return CX_STATUS_SUCCESS;
    if (feature_permutation == nullptr || canonical == nullptr || packed == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_pack_dense_operand: null argument");
    if (packed == canonical)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_pack_dense_operand: output aliases its source");
    if (leading_dimension < (column_major != 0u ? feature_count : column_count))
        return fail(CX_STATUS_INVALID_SHAPE, "cx_pack_dense_operand: leading dimension below the row length");
    if (packed_capacity_bytes < count * value_size_bytes)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_pack_dense_operand: packed buffer is too small");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(grid_for(count)), block(256);
    switch (value_size_bytes) {
    case 1: hipLaunchKernelGGL(pack_dense_kernel<std::uint8_t>, grid, block, 0, s, feature_permutation,
                               static_cast<const std::uint8_t *>(canonical), feature_count, column_count,
                               leading_dimension, column_major, static_cast<std::uint8_t *>(packed)); break;
    case 2: hipLaunchKernelGGL(pack_dense_kernel<std::uint16_t>, grid, block, 0, s, feature_permutation,
                               static_cast<const std::uint16_t *>(canonical), feature_count, column_count,
                               leading_dimension, column_major, static_cast<std::uint16_t *>(packed)); break;
    case 4: hipLaunchKernelGGL(pack_dense_kernel<std::uint32_t>, grid, block, 0, s, feature_permutation,
                               static_cast<const std::uint32_t *>(canonical), feature_count, column_count,
                               leading_dimension, column_major, static_cast<std::uint32_t *>(packed)); break;
    default: hipLaunchKernelGGL(pack_dense_kernel<std::uint64_t>, grid, block, 0, s, feature_permutation,
                                static_cast<const std::uint64_t *>(canonical), feature_count, column_count,
                                leading_dimension, column_major, static_cast<std::uint64_t *>(packed)); break;
    }
    return check_launch("cx_pack_dense_operand");
}

extern "C" int cx_qcsr_column_counts(const cx_qcsr_matrix *m, uint32_t *counts, void *stream) {
    using namespace cx;
    clear_error();
    if (m == nullptr || counts == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_column_counts: null argument");
    if (m->cols == 0u) return CX_STATUS_SUCCESS;
    if (m->nnz != 0u && m->col_idx == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_column_counts: null col_idx");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(m->cols)), dim3(256), 0, s, counts,
                       static_cast<std::uint64_t>(m->cols), 0u);
    if (m->nnz != 0u) {
        const std::uint64_t lds = static_cast<std::uint64_t>(m->cols) * 4u;
        if (lds <= 150u * 1024u) {
            const std::uint64_t per_block = 1u << 20;
            const unsigned blocks = static_cast<unsigned>((m->nnz + per_block - 1u) / per_block);
            if (lds > 64u * 1024u)
                (void)hipFuncSetAttribute(reinterpret_cast<const void *>(column_counts_lds),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
            hipLaunchKernelGGL(column_counts_lds, dim3(blocks), dim3(1024), static_cast<unsigned>(lds), s,
                               m->col_idx, m->nnz, m->cols, per_block, counts);
        } else {
            hipLaunchKernelGGL(column_counts_global, dim3(grid_for(m->nnz)), dim3(256), 0, s, m->col_idx,
                               m->nnz, m->cols, counts);
        }
    }
    return check_launch("cx_qcsr_column_counts");
}

extern "C" int cx_qcsr_execution_order_lds_bytes(const cx_qcsr_matrix *m, uint64_t *bytes) {
    using namespace cx;
    clear_error();
    if (m == nullptr || bytes == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_execution_order_lds_bytes: null argument");
    const std::uint64_t words = (static_cast<std::uint64_t>(m->cols) + 31u) / 32u;
    const std::uint64_t stage = (static_cast<std::uint64_t>(m->cols) * m->bits + 31u) / 32u;
    *bytes = (2u * words + stage) * 4u;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_to_execution_order(const cx_qcsr_matrix *m, const uint32_t *inverse_permutation,
                                          int32_t *col_idx_out, uint8_t *packed_out, void *values_out,
                                          uint32_t *device_error, void *stream) {
    using namespace cx;
    clear_error();
    if (m == nullptr || inverse_permutation == nullptr || device_error == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_to_execution_order: null argument");
    if (!(m->bits == 0u || m->bits == 1u || m->bits == 2u || m->bits == 4u || m->bits == 8u))
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_to_execution_order: bits must be 0, 1, 2, 4 or 8");
    if (m->rows != 0u && (m->row_ptr == nullptr || (m->nnz != 0u && (m->col_idx == nullptr || col_idx_out == nullptr))))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_to_execution_order: null structure or output");
    if (m->bits != 0u && m->nnz != 0u && (m->packed_row_ptr == nullptr || m->packed_values == nullptr || packed_out == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_to_execution_order: null codes");
    if (m->bits == 0u && m->nnz != 0u
        && (m->values == nullptr || values_out == nullptr
            || (m->value_dtype != CELLERATOR_DTYPE_F16 && m->value_dtype != CELLERATOR_DTYPE_F32)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_to_execution_order: plain values need F16/F32 values and an output");
    if (col_idx_out == m->col_idx || (packed_out != nullptr && packed_out == m->packed_values)
        || (values_out != nullptr && values_out == m->values))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_to_execution_order: outputs alias the inputs");
    std::uint64_t lds = 0u;
    (void)cx_qcsr_execution_order_lds_bytes(m, &lds);
    if (lds > 150u * 1024u)
        return fail(CX_STATUS_UNSUPPORTED, "cx_qcsr_to_execution_order: too many genes for the LDS bitmap");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(256), 0, s, device_error, static_cast<std::uint64_t>(1u), 0u);
    if (m->rows == 0u || m->nnz == 0u) return check_launch("cx_qcsr_to_execution_order");
    const dim3 grid(std::min<std::uint32_t>(m->rows, 1u << 20)), block(256);
    const unsigned shared = static_cast<unsigned>(lds);
#define CX_REORDER(B, T)                                                                                       \
    do {                                                                                                       \
        if (shared > 64u * 1024u)                                                                              \
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(reorder_rows_kernel<B, T>),               \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(shared));   \
        hipLaunchKernelGGL((reorder_rows_kernel<B, T>), grid, block, shared, s, m->row_ptr, m->packed_row_ptr, \
                           m->col_idx, m->packed_values, static_cast<const T *>(m->values), inverse_permutation,\
                           m->rows, m->cols, col_idx_out, packed_out, static_cast<T *>(values_out),            \
                           device_error);                                                                      \
    } while (0)
    switch (m->bits) {
    case 0:
        if (m->value_dtype == CELLERATOR_DTYPE_F16) CX_REORDER(0, std::uint16_t);
        else CX_REORDER(0, std::uint32_t);
        break;
    case 1: CX_REORDER(1, std::uint8_t); break;
    case 2: CX_REORDER(2, std::uint8_t); break;
    case 4: CX_REORDER(4, std::uint8_t); break;
    default: CX_REORDER(8, std::uint8_t); break;
    }
#undef CX_REORDER
    return check_launch("cx_qcsr_to_execution_order");
}
