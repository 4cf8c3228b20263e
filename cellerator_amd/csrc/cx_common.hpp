// cx_common.hpp -- shared device helpers and the error channel of the HIP layer.
// gfx950 only: wave64, 160 KB LDS per CU, MFMA; no other target is compiled.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "cellerator_amd.h"

namespace cx {

constexpr int kWave = 64;

// Thread-local last-error text behind cx_last_error(); set by every failing entry.
void set_error(const char *fmt, ...);
void clear_error();

// Maps a HIP runtime status to CX_STATUS_HIP_ERROR with the runtime's message.
int hip_fail(hipError_t status, const char *what);

inline int fail(int status, const char *message) {
    set_error("%s", message);
    return status;
}

// Returns CX_STATUS_HIP_ERROR if the last launch on this thread failed.
int check_launch(const char *kernel);

// Column-contiguous 16-bit weight panel [ceil(k/32)][n][32] (genes past k zero), the matrix-
// core operand of the quantized CSR path's dense head (bell_spmm.hip).
int pack_panel_columns(const std::uint16_t *rhs, std::int64_t rhs_ld, std::uint32_t k, std::uint32_t n,
                       std::uint16_t *packed, hipStream_t stream);

// Exact fp16 -> fp32 widening on the device.
__device__ __forceinline__ float h2f(std::uint16_t bits) {
    _Float16 h;
    __builtin_memcpy(&h, &bits, 2);
    return static_cast<float>(h);
}

__device__ __forceinline__ float bf2f(std::uint16_t bits) {
    return __uint_as_float(static_cast<std::uint32_t>(bits) << 16);
}

// Device primitives of sort.hip (stream-ordered; workspace sized by the *_bytes helpers).
std::uint64_t scan_workspace_bytes(std::uint64_t n);
int exclusive_scan_u32(const std::uint32_t *in, std::uint32_t *out, std::uint64_t n,
                       void *workspace, hipStream_t stream);
std::uint64_t sort_pairs_workspace_bytes(std::uint64_t count, std::uint32_t key_bits);
int sort_pairs(const std::uint32_t *keys_in, const std::uint32_t *vals_in, std::uint32_t *keys_out,
               std::uint32_t *vals_out, std::uint64_t count, std::uint32_t key_bits,
               void *workspace, std::uint64_t workspace_bytes, hipStream_t stream);

// Device form of cx_spmm_epilogue. `active` == 0 means a plain store of the accumulator.
struct Epilogue {
    const float *bias;
    const float *initial;
    std::int64_t initial_ld;
    float alpha;
    float beta;
    std::uint32_t kind;
    std::uint32_t active;
};

// Validates `ep` (NULL = none) for an fp32 output of rows x cols at `out` (leading
// dimension out_ld) and fills `dev`; `who` prefixes the error text.
int make_epilogue(const cx_spmm_epilogue *ep, std::uint64_t rows, std::int64_t cols,
                  const float *out, std::int64_t out_ld, Epilogue *dev, const char *who);

__device__ __forceinline__ bool bias_kind(std::uint32_t kind) {
    return kind == CX_EPILOGUE_BIAS || kind == CX_EPILOGUE_BIAS_RELU
        || kind == CX_EPILOGUE_BIAS_GELU_ERF || kind == CX_EPILOGUE_BIAS_GELU_TANH;
}

// act(alpha * acc + beta * C[row, col] + bias[col]) in fp32, in the referee's order
// (src/compute/math/referee.cc:81-97): scale and accumulate, add the bias, then activate.
__device__ __forceinline__ float epilogue_value(const Epilogue &e, float acc, std::int64_t row,
                                                std::int64_t col) {
    float v = e.alpha == 0.0f ? 0.0f : e.alpha * acc;
    if (e.beta != 0.0f) v = __builtin_fmaf(e.beta, e.initial[row * e.initial_ld + col], v);
    if (bias_kind(e.kind)) v += e.bias[col];
    switch (e.kind) {
    case CX_EPILOGUE_RELU:
    case CX_EPILOGUE_BIAS_RELU: return fmaxf(v, 0.0f);
    case CX_EPILOGUE_GELU_ERF:
    case CX_EPILOGUE_BIAS_GELU_ERF: return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
    case CX_EPILOGUE_GELU_TANH:
    case CX_EPILOGUE_BIAS_GELU_TANH:
        return 0.5f * v * (1.0f + tanhf(0.79788456080286536f * (v + 0.044715f * v * v * v)));
    default: return v;
    }
}

// Sum over the lanes that differ only in the bits of `mask_bits` (xor butterfly).
template<int kFirstBit, int kLastBit>
__device__ __forceinline__ float xor_reduce(float v) {
#pragma unroll
    for (int b = kFirstBit; b <= kLastBit; ++b) v += __shfl_xor(v, 1 << b, kWave);
    return v;
}

} // namespace cx
