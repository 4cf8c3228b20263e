// csr_spmv.hip -- N = 1 CSR comparator for the CP-BP reduction: y[r] = sum fp32(v) x[col]
// (the operation of csr_spmv_fwd_f16_f32, src/compute/sparse/ops/ops.hh:83-90). One
// wave per row (grid-stride over rows, 64-bit wave index), lanes stride the row's entries
// with coalesced loads, butterfly sum.
#include "cx_common.hpp"

namespace cx {
namespace {

template<typename ValT>
__global__ __launch_bounds__(256) void csr_spmv_kernel(std::uint32_t rows, const std::uint32_t *row_ptr,
                                                       const std::uint32_t *col_idx,
                                                       const ValT *values, const float *x, float *y) {
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const std::uint64_t waves = static_cast<std::uint64_t>(gridDim.x) * (blockDim.x / kWave);
    for (std::uint64_t row = (static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
         row < rows; row += waves) {
        const std::uint32_t begin = row_ptr[row], end = row_ptr[row + 1];
        float sum = 0.0f;
        for (std::uint32_t i = begin + lane; i < end; i += kWave) {
            float v;
            if constexpr (sizeof(ValT) == 2) v = h2f(values[i]);
            else v = values[i];
            sum = __builtin_fmaf(v, x[col_idx[i]], sum);
        }
        sum = xor_reduce<0, 5>(sum);
        if (lane == 0) y[row] = sum;
    }
}

} // namespace
} // namespace cx

extern "C" int cx_csr_spmv_fwd(uint32_t rows, const uint32_t *row_ptr, const uint32_t *col_idx,
                               const void *values, uint32_t value_dtype, const float *x, float *y,
                               void *stream) {
    using namespace cx;
    clear_error();
    if (rows == 0u) return CX_STATUS_SUCCESS;
    if (row_ptr == nullptr || col_idx == nullptr || values == nullptr || x == nullptr || y == nullptr)
        return fail(CX_STATUS_INVALID_ARGUMENT, "cx_csr_spmv_fwd: null argument");
    // 4 rows per block, at most 2^20 blocks; the kernel strides over the rest
    const std::uint64_t blocks = (static_cast<std::uint64_t>(rows) + 3u) / 4u;
    const dim3 grid(static_cast<unsigned>(blocks < (1u << 20) ? blocks : (1u << 20))), block(256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (value_dtype == CELLERATOR_DTYPE_F16)
        hipLaunchKernelGGL(csr_spmv_kernel<std::uint16_t>, grid, block, 0, s, rows, row_ptr, col_idx,
                           static_cast<const std::uint16_t *>(values), x, y);
    else if (value_dtype == CELLERATOR_DTYPE_F32)
        hipLaunchKernelGGL(csr_spmv_kernel<float>, grid, block, 0, s, rows, row_ptr, col_idx,
                           static_cast<const float *>(values), x, y);
    else
        return fail(CX_STATUS_UNSUPPORTED, "cx_csr_spmv_fwd: values must be F16 or F32");
    return check_launch("csr_spmv");
}
