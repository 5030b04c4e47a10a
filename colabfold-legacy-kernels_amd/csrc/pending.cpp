// Entry points whose kernels are not written yet: they return CLK_UNIMPLEMENTED.
#include "common.hpp"

using namespace clk;

extern "C" clk_status clk_gated_dual_proj(hipStream_t, clk_dtype, const void*, const void*,
                                          const void*, const void*, const void*, const void*,
                                          void*, int64_t, int64_t, int64_t) {
    return fail(CLK_UNIMPLEMENTED, "gated_dual_proj: not built yet");
}
extern "C" clk_status clk_ln_gated_dual_proj(hipStream_t, clk_dtype, const void*, const float*,
                                             const float*, const void*, const void*, const void*,
                                             const void*, const void*, const void*, const void*,
                                             const void*, const void*, void*, void*, int64_t,
                                             int64_t, int64_t, float) {
    return fail(CLK_UNIMPLEMENTED, "ln_gated_dual_proj: not built yet");
}
