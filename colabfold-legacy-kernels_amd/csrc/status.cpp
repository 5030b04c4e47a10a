// Host-side status plumbing of the C ABI: a thread-local last-error message, status helpers and
// the version string. Pure host code (no kernels).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <vector>

#include "common.hpp"

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

namespace {
struct LaunchRecord {
    const char* name;
    hipEvent_t start, stop;
};
thread_local bool g_profile = false;
thread_local std::vector<LaunchRecord> g_records;
}  // namespace

KernelTimer::KernelTimer(const char* name, hipStream_t stream) : name_(name), stream_(stream) {
    if (!g_profile) return;
    if (hipEventCreate(&start_) != hipSuccess) {
        start_ = nullptr;
        return;
    }
    hipEventRecord(start_, stream_);
}

KernelTimer::~KernelTimer() {
    if (!start_) return;
    hipEvent_t stop = nullptr;
    if (hipEventCreate(&stop) != hipSuccess) {
        hipEventDestroy(start_);
        return;
    }
    hipEventRecord(stop, stream_);
    g_records.push_back({name_, start_, stop});
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

extern "C" void clk_profile_enable(int on) { clk::g_profile = on != 0; }

extern "C" int clk_profile_collect(const char** names, float* ms, int max) {
    const int n = (int)clk::g_records.size();
    for (int i = 0; i < n; ++i) {
        auto& r = clk::g_records[i];
        float t = -1.f;
        if (hipEventSynchronize(r.stop) == hipSuccess) hipEventElapsedTime(&t, r.start, r.stop);
        if (i < max) {
            if (names) names[i] = r.name;
            if (ms) ms[i] = t;
        }
        hipEventDestroy(r.start);
        hipEventDestroy(r.stop);
    }
    clk::g_records.clear();
    return n;
}

extern "C" const char* clk_version(void) { return "colabfold-legacy-kernels gfx950 0.2.0"; }
