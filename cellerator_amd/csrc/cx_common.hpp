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

// Exact fp16 -> fp32 widening on the device.
__device__ __forceinline__ float h2f(std::uint16_t bits) {
    _Float16 h;
    __builtin_memcpy(&h, &bits, 2);
    return static_cast<float>(h);
}

__device__ __forceinline__ float bf2f(std::uint16_t bits) {
    return __uint_as_float(static_cast<std::uint32_t>(bits) << 16);
}

// Sum over the lanes that differ only in the bits of `mask_bits` (xor butterfly).
template<int kFirstBit, int kLastBit>
__device__ __forceinline__ float xor_reduce(float v) {
#pragma unroll
    for (int b = kFirstBit; b <= kLastBit; ++b) v += __shfl_xor(v, 1 << b, kWave);
    return v;
}

} // namespace cx
