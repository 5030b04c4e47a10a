// Attention backward for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc): clk_attention_bwd with its
// workspace taken from a fixed, file-scope device array instead of a caller-provided buffer.
// No reference counterpart.
//
// The array `scratch` holds kScratchBytes per GPU for the life of the process. In host code its
// name is only a host-side stand-in, so its device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and that address is what reaches the kernels.
// Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams, two
// threads) race on it and must be serialised by the caller. Nothing in it needs to start at zero:
// the backward writes every byte of its workspace that it later reads (transposed bias, per-row
// logits and statistics, dBias and dQ partials) before reading it, in every call.
#include <mutex>

#include "common.hpp"

namespace clk {
namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;  // 64 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, once looked up

// The device address of this device's `scratch`, looked up on first use with `dev` current.
clk_status scratch_for(int dev, void** out) {
    if (dev < 0 || dev >= kMaxDevices)
        return fail(CLK_INVALID_ARGUMENT, "attention_bwd_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess)
            return fail(CLK_INTERNAL, "attention_bwd_noalloc: hipGetDevice failed");
        if (cur != dev && hipSetDevice(dev) != hipSuccess)
            return fail(CLK_INTERNAL, "attention_bwd_noalloc: hipSetDevice(%d) failed", dev);
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != dev) (void)hipSetDevice(cur);
        if (e != hipSuccess || !p)
            return fail(CLK_INTERNAL, "attention_bwd_noalloc: hipGetSymbolAddress: %s",
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return CLK_OK;
}

}  // namespace
}  // namespace clk

using namespace clk;

extern "C" size_t clk_attention_bwd_noalloc_limit(void) { return kScratchBytes; }

extern "C" clk_status clk_attention_bwd_noalloc(hipStream_t stream, clk_dtype dtype,
                                                const void* q, const void* k, const void* v,
                                                const void* bias, const uint8_t* kmask,
                                                const void* out, const void* dout,
                                                const float* lse, void* dq, void* dk, void* dv,
                                                float* dbias, int64_t N, int64_t H, int64_t Sq,
                                                int64_t Sk, int64_t D, float scale) {
    // Sizes first, on the host alone: a problem whose workspace exceeds the array is refused
    // before any device call.
    if (N < 0 || H < 0 || Sq < 0 || Sk < 0)
        return fail(CLK_INVALID_ARGUMENT, "attention_bwd_noalloc: negative dimension");
    const size_t need = clk_attention_bwd_workspace_size(N, H, Sq, Sk, D);
    if (need > kScratchBytes)
        return fail(CLK_INVALID_ARGUMENT,
                    "attention_bwd_noalloc: these sizes need %zu bytes of scratch, more than its "
                    "fixed %zu (use clk_attention_bwd with a caller workspace)",
                    need, kScratchBytes);
    int dev = -1;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess)
        return fail(CLK_INTERNAL, "attention_bwd_noalloc: hipStreamGetDevice failed");
    void* ws = nullptr;
    const clk_status s = scratch_for(dev, &ws);
    if (s != CLK_OK) return s;
    return clk_attention_bwd(stream, dtype, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv,
                             dbias, ws, kScratchBytes, N, H, Sq, Sk, D, scale);
}
