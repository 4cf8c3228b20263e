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

} // namespace cx

extern "C" const char *cx_last_error(void) { return cx::g_last_error; }

extern "C" const char *cx_build_info(void) { return "cellerator_amd gfx950 wave64"; }
