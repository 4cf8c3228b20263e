// qcsr_codec.hip -- the quantized CSR codec as standalone device passes over a row block:
// quantize (values -> packed codes) and dequantize (packed codes -> values), the work of the
// reference's launch_quantize_block / launch_dequantize_block
// (include/Cellerator/quantized/dispatch.cuh:36-86) with pack_row_values / unpack_row_values
// per row (include/Cellerator/quantized/packing.cuh:13-146, 148-260).
//
// Semantics kept from the reference: codes of a row packed low bits first, a row's bytes
// starting at packed_row_ptr[row] with the unused high bits of its last byte zero; the
// portable encode rule (include/Cellerator/quantized/access.cuh:104-131: subtract the offset,
// IEEE-divide by the scale, round half away from zero, clamp to [0, 2^bits - 1]; scale 0
// gives code 0) and the decode fma(code, scale, offset) (:81-91); values indexed from the
// block's first entry. Per-gene affine, interleaved (scale, offset) pairs and column scale
// with row offset metadata; a null scale reads 1, a null offset 0.
//
// Layout of the work: one wave per row, lanes over the row's packed bytes (quantize: each lane
// assembles a whole byte, so there is no read-modify-write of shared bytes and adjacent lanes
// store adjacent bytes) or over its entries (dequantize: adjacent lanes store adjacent fp32
// values); four rows per workgroup, rows of the block strided over the grid.
#include "qcsr_common.hpp"

namespace cx {
namespace {

constexpr int kCodecWaves = 4;

struct CodecArgs {
    const std::int32_t *row_ptr;
    const std::int32_t *packed_row_ptr;
    const std::int32_t *col_idx;
    const float *scales;
    const float *offsets;
    const float *row_offsets;
    std::uint32_t policy;
    std::uint32_t cols;
    std::int32_t row_begin;
    std::int32_t row_end;
    std::int64_t nnz_begin;  // values are indexed from this entry
};

__device__ __forceinline__ float2 entry_meta(const CodecArgs &a, std::int32_t row, std::int32_t col) {
    if (a.policy == CX_DECODE_PER_GENE_AFFINE_PAIRS) return reinterpret_cast<const float2 *>(a.scales)[col];
    const float s = a.scales != nullptr ? a.scales[col] : 1.0f;
    float o;
    if (a.policy == CX_DECODE_COLUMN_SCALE_ROW_OFFSET) o = a.row_offsets != nullptr ? a.row_offsets[row] : 0.0f;
    else o = a.offsets != nullptr ? a.offsets[col] : 0.0f;
    return make_float2(s, o);
}

template<int kBits>
__device__ __forceinline__ std::uint32_t encode(float value, float2 md) {
    if (md.x == 0.0f) return 0u;
    const float q = (value - md.y) / md.x;  // correctly rounded divide (HIP's default)
    const int r = q >= 0.0f ? static_cast<int>(q + 0.5f) : static_cast<int>(q - 0.5f);
    if (r < 0) return 0u;
    return static_cast<std::uint32_t>(r > (1 << kBits) - 1 ? (1 << kBits) - 1 : r);
}

template<int kBits>
__global__ __launch_bounds__(kCodecWaves * kWave) void quantize_rows_kernel(CodecArgs a, const float *values,
                                                                            std::uint8_t *packed) {
    constexpr int kPerByte = 8 / kBits;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    for (std::int64_t row = a.row_begin + static_cast<std::int64_t>(blockIdx.x) * kCodecWaves + threadIdx.x / kWave;
         row < a.row_end; row += static_cast<std::int64_t>(gridDim.x) * kCodecWaves) {
        const std::int64_t begin = a.row_ptr[row], end = a.row_ptr[row + 1];
        const std::int64_t out0 = a.packed_row_ptr[row];
        const std::int64_t bytes = (end - begin + kPerByte - 1) / kPerByte;
        for (std::int64_t b = lane; b < bytes; b += kWave) {
            std::uint32_t byte = 0u;
#pragma unroll
            for (int k = 0; k < kPerByte; ++k) {
                const std::int64_t i = begin + b * kPerByte + k;
                if (i < end) {
                    // a column outside [0, cols) (a broken structure) encodes as code 0
                    const std::int32_t col = a.col_idx[i];
                    if (static_cast<std::uint32_t>(col) < a.cols)
                        byte |= encode<kBits>(values[i - a.nnz_begin], entry_meta(a, static_cast<std::int32_t>(row), col))
                            << (k * kBits);
                }
            }
            packed[out0 + b] = static_cast<std::uint8_t>(byte);
        }
    }
}

template<int kBits>
__global__ __launch_bounds__(kCodecWaves * kWave) void dequantize_rows_kernel(CodecArgs a, const std::uint8_t *packed,
                                                                              float *values) {
    constexpr int kPerByte = 8 / kBits;
    constexpr std::uint32_t kMask = (1u << kBits) - 1u;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    for (std::int64_t row = a.row_begin + static_cast<std::int64_t>(blockIdx.x) * kCodecWaves + threadIdx.x / kWave;
         row < a.row_end; row += static_cast<std::int64_t>(gridDim.x) * kCodecWaves) {
        const std::int64_t begin = a.row_ptr[row], end = a.row_ptr[row + 1];
        const std::uint8_t *in = packed + a.packed_row_ptr[row];
        for (std::int64_t i = begin + lane; i < end; i += kWave) {
            const std::int64_t local = i - begin;
            const std::uint32_t code = (static_cast<std::uint32_t>(in[local / kPerByte]) >> ((local % kPerByte) * kBits)) & kMask;
            const std::int32_t col = a.col_idx[i];
            // a column outside [0, cols) (a broken structure) decodes as 0
            const float2 md = static_cast<std::uint32_t>(col) < a.cols
                ? entry_meta(a, static_cast<std::int32_t>(row), col) : make_float2(0.0f, 0.0f);
            values[i - a.nnz_begin] = __builtin_fmaf(static_cast<float>(code), md.x, md.y);
        }
    }
}

int prepare(const cx_qcsr_matrix *m, const cx_qcsr_block *block, CodecArgs *a, const char *who) {
    if (m == nullptr) return fail(CX_STATUS_INVALID_ARGUMENT, who);
    if (m->bits != 1u && m->bits != 2u && m->bits != 4u && m->bits != 8u)
        return fail(CX_STATUS_UNSUPPORTED, "quantized codec: codes of 1, 2, 4 or 8 bits only");
    if (m->decode_policy != CX_DECODE_PER_GENE_AFFINE && m->decode_policy != CX_DECODE_PER_GENE_AFFINE_PAIRS
        && m->decode_policy != CX_DECODE_COLUMN_SCALE_ROW_OFFSET)
        return fail(CX_STATUS_UNSUPPORTED, "quantized codec: unknown decode policy");
    if (m->decode_policy == CX_DECODE_PER_GENE_AFFINE_PAIRS && m->column_scales == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "quantized codec: the pairs policy needs column_scales");
    if (m->rows != 0u && (m->row_ptr == nullptr || m->packed_row_ptr == nullptr || (m->nnz != 0u && m->col_idx == nullptr)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "quantized codec: null structure");
    CodecArgs c{};
    c.row_ptr = m->row_ptr;
    c.packed_row_ptr = m->packed_row_ptr;
    c.col_idx = m->col_idx;
    c.scales = m->column_scales;
    c.offsets = m->column_offsets;
    c.row_offsets = m->row_offsets;
    c.policy = m->decode_policy;
    c.cols = m->cols;
    if (block == nullptr) {
        c.row_begin = 0;
        c.row_end = static_cast<std::int32_t>(m->rows);
        c.nnz_begin = 0;
    } else {
        if (block->row_begin < 0 || block->row_end < block->row_begin
            || static_cast<std::uint32_t>(block->row_end) > m->rows || block->nnz_begin < 0)
            return fail(CX_STATUS_INVALID_SHAPE, "quantized codec: the block's rows lie outside the matrix");
        c.row_begin = block->row_begin;
        c.row_end = block->row_end;
        c.nnz_begin = block->nnz_begin;
    }
    *a = c;
    return CX_STATUS_SUCCESS;
}

unsigned codec_grid(const CodecArgs &a) {
    const std::int64_t rows = static_cast<std::int64_t>(a.row_end) - a.row_begin;
    return static_cast<unsigned>(std::min<std::int64_t>((rows + kCodecWaves - 1) / kCodecWaves, 1 << 20));
}

} // namespace
} // namespace cx

extern "C" int cx_qcsr_get_block(const int32_t *block_row_ptr, int32_t block_count, const int32_t *row_ptr,
                                 const int32_t *packed_row_ptr, int32_t rows, int32_t block_index,
                                 cx_qcsr_block *out) {
    using namespace cx;
    clear_error();
    if (out == nullptr || row_ptr == nullptr || packed_row_ptr == nullptr || rows < 0)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_get_block: null argument");
    cx_qcsr_block b{};
    b.block_index = block_index;
    if (block_row_ptr == nullptr || block_count <= 0) {
        b.block_index = 0;
        b.row_begin = 0;
        b.row_end = rows;
    } else {
        if (block_index < 0 || block_index >= block_count) {
            *out = b;  // the reference returns an empty block
            return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_get_block: block index out of range");
        }
        b.row_begin = block_row_ptr[block_index];
        b.row_end = block_row_ptr[block_index + 1];
        if (b.row_begin < 0 || b.row_end < b.row_begin || b.row_end > rows)
            return fail(CX_STATUS_INVALID_SHAPE, "cx_qcsr_get_block: block rows outside the matrix");
    }
    b.nnz_begin = row_ptr[b.row_begin];
    b.nnz_end = row_ptr[b.row_end];
    b.packed_begin = packed_row_ptr[b.row_begin];
    b.packed_end = packed_row_ptr[b.row_end];
    *out = b;
    return CX_STATUS_SUCCESS;
}

extern "C" int cx_qcsr_quantize_block(const cx_qcsr_matrix *m, const cx_qcsr_block *block,
                                      const float *values_by_nnz_block, uint8_t *packed_out, void *stream) {
    using namespace cx;
    clear_error();
    CodecArgs a;
    int rc = prepare(m, block, &a, "cx_qcsr_quantize_block: null matrix");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (a.row_end == a.row_begin) return CX_STATUS_SUCCESS;
    if (packed_out == nullptr || (m->nnz != 0u && values_by_nnz_block == nullptr))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_quantize_block: null values or packed output");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(codec_grid(a)), threads(kCodecWaves * kWave);
    switch (m->bits) {
    case 1: hipLaunchKernelGGL(quantize_rows_kernel<1>, grid, threads, 0, s, a, values_by_nnz_block, packed_out); break;
    case 2: hipLaunchKernelGGL(quantize_rows_kernel<2>, grid, threads, 0, s, a, values_by_nnz_block, packed_out); break;
    case 4: hipLaunchKernelGGL(quantize_rows_kernel<4>, grid, threads, 0, s, a, values_by_nnz_block, packed_out); break;
    default: hipLaunchKernelGGL(quantize_rows_kernel<8>, grid, threads, 0, s, a, values_by_nnz_block, packed_out); break;
    }
    return check_launch("cx_qcsr_quantize_block");
}

extern "C" int cx_qcsr_dequantize_block(const cx_qcsr_matrix *m, const cx_qcsr_block *block,
                                        float *values_by_nnz_block, void *stream) {
    using namespace cx;
    clear_error();
    CodecArgs a;
    int rc = prepare(m, block, &a, "cx_qcsr_dequantize_block: null matrix");
    if (rc != CX_STATUS_SUCCESS) return rc;
    if (a.row_end == a.row_begin) return CX_STATUS_SUCCESS;
    if ((m->nnz != 0u && (values_by_nnz_block == nullptr || m->packed_values == nullptr)))
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_qcsr_dequantize_block: null values or codes");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(codec_grid(a)), threads(kCodecWaves * kWave);
    const std::uint8_t *p = m->packed_values;
    switch (m->bits) {
    case 1: hipLaunchKernelGGL(dequantize_rows_kernel<1>, grid, threads, 0, s, a, p, values_by_nnz_block); break;
    case 2: hipLaunchKernelGGL(dequantize_rows_kernel<2>, grid, threads, 0, s, a, p, values_by_nnz_block); break;
    case 4: hipLaunchKernelGGL(dequantize_rows_kernel<4>, grid, threads, 0, s, a, p, values_by_nnz_block); break;
    default: hipLaunchKernelGGL(dequantize_rows_kernel<8>, grid, threads, 0, s, a, p, values_by_nnz_block); break;
    }
    return check_launch("cx_qcsr_dequantize_block");
}
