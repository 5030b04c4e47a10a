// Host-side status plumbing of the C ABI: a thread-local last-error message, status helpers and
// the version string. Pure host code (no kernels).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "clk.h"

namespace clk {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

clk_status fail(clk_status code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

clk_status ok() {
    g_last_error[0] = '\0';
    return CLK_OK;
}

// Maps a launch failure to CLK_INTERNAL, as the reference maps cudaGetLastError to
// ffi::Error::Internal (cuda/volta_mma_attn.cu:297-300).
clk_status check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return fail(CLK_INTERNAL, "%s launch: %s", what, hipGetErrorString(err));
    }
    return ok();
}

const char* dtype_name(clk_dtype t) {
    switch (t) {
        case CLK_U8: return "u8";
        case CLK_F16: return "f16";
        case CLK_F32: return "f32";
        case CLK_BF16: return "bf16";
    }
    return "invalid";
}

}  // namespace clk

extern "C" const char* clk_last_error(void) { return clk::g_last_error; }

extern "C" const char* clk_version(void) { return "colabfold-legacy-kernels gfx950 0.2.0"; }
