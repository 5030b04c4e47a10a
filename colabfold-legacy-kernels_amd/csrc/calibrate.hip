// Instruction-issue calibration: fixed instruction mixes that measure, on the device at hand,
// what one wave instruction of each kind costs a SIMD -- a float32 FMA, a float32 exponential
// (v_exp_f32, the transcendental of every softmax) and a 16x16x32 bf16 MFMA -- alone and mixed,
// at one to a few waves per SIMD. The benchmark's instruction-issue floor of the attention
// kernels uses these costs. No reference counterpart (measurement only).
#include "common.hpp"

namespace clk {
namespace {

using bf16x8 = __attribute__((ext_vector_type(8))) __bf16;

// One round: NM independent MFMA chains (one MFMA each), NV x 32 independent FMAs, NE x 32
// independent exponentials; `iters` rounds of two unrolled copies. Every result feeds the one
// float each thread writes, so nothing is dead code, and every chain stays finite (v -> v*s + 1
// with s < 1; w -> 2^-w, a source modifier, converges).
template <int NM, int NV, int NE>
__global__ __launch_bounds__(1024) void issue_mix_kernel(float* __restrict__ sink, int iters,
                                                         float s) {
    static_assert(NM <= 4, "four MFMA chains");
    f32x4 acc[4] = {};
    bf16x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = (__bf16)(threadIdx.x * 1e-3f + j);
        b[j] = (__bf16)(s + j);
    }
    float v[32], w[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        v[j] = threadIdx.x * 1e-3f + j;
        w[j] = -1e-3f * j;
    }
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
#pragma unroll
            for (int m = 0; m < NM; ++m)
                acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[m], 0, 0, 0);
#pragma unroll
            for (int k = 0; k < NV; ++k)
#pragma unroll
                for (int j = 0; j < 32; ++j) v[j] = fmaf(v[j], s, 1.f);
#pragma unroll
            for (int k = 0; k < NE; ++k)
#pragma unroll
                for (int j = 0; j < 32; ++j) w[j] = __builtin_amdgcn_exp2f(-w[j]);  // bounded
        }
    }
    float t = 0.f;
#pragma unroll
    for (int m = 0; m < 4; ++m) t += acc[m][0] + acc[m][1] + acc[m][2] + acc[m][3];
#pragma unroll
    for (int j = 0; j < 32; ++j) t += v[j] + w[j];
    sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = t;
}

template <int NM, int NV, int NE>
void launch_mix(hipStream_t st, int blocks, int threads, int iters, float* sink) {
    issue_mix_kernel<NM, NV, NE><<<blocks, threads, 0, st>>>(sink, iters, 0.999f);
}

}  // namespace
}  // namespace clk

using namespace clk;

extern "C" clk_status clk_issue_calibration(hipStream_t stream, int kind, int blocks,
                                            int threads, int iters, float* sink) {
    if (kind < 0 || kind > 6)
        return fail(CLK_INVALID_ARGUMENT, "issue_calibration: kind %d not in 0..6", kind);
    if (blocks < 1 || blocks > 65535 || threads < 64 || threads > 1024 || threads % 64 ||
        iters < 1)
        return fail(CLK_INVALID_ARGUMENT,
                    "issue_calibration: blocks %d (1..65535), threads %d (64..1024, a multiple "
                    "of 64), iters %d (>= 1)", blocks, threads, iters);
    if (!sink) return fail(CLK_INVALID_ARGUMENT, "issue_calibration: null sink");
    switch (kind) {
        case 0: launch_mix<0, 1, 0>(stream, blocks, threads, iters, sink); break;
        case 1: launch_mix<0, 0, 1>(stream, blocks, threads, iters, sink); break;
        case 2: launch_mix<4, 0, 0>(stream, blocks, threads, iters, sink); break;
        case 3: launch_mix<0, 1, 1>(stream, blocks, threads, iters, sink); break;
        case 4: launch_mix<4, 1, 0>(stream, blocks, threads, iters, sink); break;
        case 5: launch_mix<4, 0, 1>(stream, blocks, threads, iters, sink); break;
        default: launch_mix<4, 1, 1>(stream, blocks, threads, iters, sink); break;
    }
    return check_launch("issue_calibration");
}
