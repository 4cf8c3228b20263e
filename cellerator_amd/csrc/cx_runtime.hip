// cx_runtime.hip -- error channel and build identity of the HIP layer.
#include "cx_common.hpp"

#include <cstdarg>
#include <cstdio>

namespace cx {
namespace {
thread_local char g_last_error[512] = {0};
} // namespace

void set_error(const char *fmt, ...) {
    va_list args;
    va_start(args, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, args);
    va_end(args);
}

void clear_error() { g_last_error[0] = '\0'; }

int hip_fail(hipError_t status, const char *what) {
    set_error("%s: %s", what, hipGetErrorString(status));
    return CX_STATUS_HIP_ERROR;
}

int check_launch(const char *kernel) {
    const hipError_t status = hipGetLastError();
    if (status != hipSuccess) return hip_fail(status, kernel);
    return CX_STATUS_SUCCESS;
}

namespace {

// Byte range [begin, end) of a row-major rows x cols f32 matrix with leading dimension ld.
struct Span {
    std::uintptr_t begin, end;
};

Span matrix_span(const float *p, std::uint64_t rows, std::int64_t cols, std::int64_t ld) {
    const std::uintptr_t b = reinterpret_cast<std::uintptr_t>(p);
    if (rows == 0u || cols <= 0) return {b, b};
    const std::uint64_t elems = (rows - 1u) * static_cast<std::uint64_t>(ld)
        + static_cast<std::uint64_t>(cols);
    return {b, b + elems * sizeof(float)};
}

bool overlap(Span x, Span y) { return x.begin < y.end && y.begin < x.end; }

} // namespace

int make_epilogue(const cx_spmm_epilogue *ep, std::uint64_t rows, std::int64_t cols,
                  const float *out, std::int64_t out_ld, Epilogue *dev, const char *who) {
    *dev = Epilogue{};
    dev->alpha = 1.0f;
    if (ep == nullptr) return CX_STATUS_SUCCESS;
    if (ep->reserved != 0u || ep->kind > CX_EPILOGUE_BIAS_GELU_TANH) {
        set_error("%s: unknown epilogue kind or nonzero reserved field", who);
        return CX_STATUS_INVALID_ARGUMENT;
    }
    const bool bias = ep->kind == CX_EPILOGUE_BIAS || ep->kind == CX_EPILOGUE_BIAS_RELU
        || ep->kind == CX_EPILOGUE_BIAS_GELU_ERF || ep->kind == CX_EPILOGUE_BIAS_GELU_TANH;
    if (bias != (ep->bias != nullptr)) {
        set_error("%s: the bias kinds need bias values and the others must not carry any", who);
        return CX_STATUS_INVALID_ARGUMENT;
    }
    const Span out_span = matrix_span(out, rows, cols, out_ld);
    if (bias && overlap(matrix_span(ep->bias, 1u, cols, cols), out_span)) {
        set_error("%s: the bias overlaps the output", who);
        return CX_STATUS_INVALID_ARGUMENT;
    }
    if (ep->beta != 0.0f) {
        if (ep->initial == nullptr || ep->initial_ld < cols) {
            set_error("%s: beta != 0 needs the initial output C with initial_ld >= out_cols", who);
            return CX_STATUS_INVALID_ARGUMENT;
        }
        const bool in_place = ep->initial == out && ep->initial_ld == out_ld;
        if (!in_place && overlap(matrix_span(ep->initial, rows, cols, ep->initial_ld), out_span)) {
            set_error("%s: the initial output overlaps the output without being it", who);
            return CX_STATUS_INVALID_ARGUMENT;
        }
    }
    dev->bias = ep->bias;
    dev->initial = ep->beta != 0.0f ? ep->initial : nullptr;
    dev->initial_ld = ep->initial_ld;
    dev->alpha = ep->alpha;
    dev->beta = ep->beta;
    dev->kind = ep->kind;
    dev->active = (ep->kind != CX_EPILOGUE_NONE || ep->alpha != 1.0f || ep->beta != 0.0f) ? 1u : 0u;
    return CX_STATUS_SUCCESS;
}

} // namespace cx

extern "C" const char *cx_last_error(void) { return cx::g_last_error; }

extern "C" const char *cx_build_info(void) { return "cellerator_amd gfx950 wave64"; }
