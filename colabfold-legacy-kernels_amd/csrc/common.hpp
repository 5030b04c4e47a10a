// Shared helpers for the gfx950 Evoformer kernels: vector types, MFMA wrappers, element
// conversions, the LDS transpose read and the host-side status plumbing.
//
// MFMA register layouts used throughout (measured on gfx950 with an in-bounds probe):
//   v_mfma_f32_16x16x32_{bf16,f16}: A[16 x 32] lane l holds row l%16, 8 k-slots of group l/16;
//   B[32 x 16] lane l holds column l%16, the same 8 k-slots; C[16 x 16] lane l holds column
//   l%16, rows 4*(l/16)+i for i = 0..3. A and B share the k-slot map, so any permutation of the
//   contraction index that is applied to both operands is exact.
//   ds_read_b64_tr_b16: within each 16-lane group, lane r supplies an 8-byte address; lane i
//   receives element i%4 of the read of lane 4*j + i/4 as its element j. With lane 4*j+t
//   pointing at row j, columns c0+4t..c0+4t+3 of a row-major tile, lane i gets column c0+i of
//   rows 0..3: a transposed 4x16 block.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <cstdarg>
#include <string>
#include <type_traits>

#include "clk.h"

namespace clk {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kMaskedLogit = -1.0e9f;

// ---------------------------------------------------------------------------------------------
// Element traits: storage type <-> float, and the 8-wide MFMA operand type.
// ---------------------------------------------------------------------------------------------
struct BF16 {
    using elem = __bf16;
    using vec8 = bf16x8;
    using vec4 = bf16x4;
    static __device__ __forceinline__ float to_f(elem x) { return (float)x; }
    static __device__ __forceinline__ elem from_f(float x) { return (elem)x; }
    static __device__ __forceinline__ f32x4 mfma(vec8 a, vec8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

struct F16 {
    using elem = _Float16;
    using vec8 = f16x8;
    using vec4 = f16x4;
    static __device__ __forceinline__ float to_f(elem x) { return (float)x; }
    static __device__ __forceinline__ elem from_f(float x) { return (elem)x; }
    static __device__ __forceinline__ f32x4 mfma(vec8 a, vec8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

struct F32 {
    using elem = float;
    static __device__ __forceinline__ float to_f(elem x) { return x; }
    static __device__ __forceinline__ elem from_f(float x) { return x; }
};

// 16-byte global load/store of 8 half-width elements, as raw bits.
__device__ __forceinline__ u32x4 ld16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x2 ld8(const void* p) {
    return *reinterpret_cast<const u32x2*>(p);
}
__device__ __forceinline__ void st8(void* p, u32x2 v) { *reinterpret_cast<u32x2*>(p) = v; }

template <typename V>
__device__ __forceinline__ V bits_as(u32x4 v) {
    return __builtin_bit_cast(V, v);
}

// Two 4-element LDS transpose reads -> one 8-slot MFMA operand.
__device__ __forceinline__ i16x4 lds_tr4(const void* lds_ptr) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(lds_ptr));
}
template <typename V>
__device__ __forceinline__ V lds_tr8(const void* p_lo, const void* p_hi) {
    i16x4 a = lds_tr4(p_lo);
    i16x4 b = lds_tr4(p_hi);
    typedef short i16x8 __attribute__((ext_vector_type(8)));
    i16x8 r = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(V, r);
}

// Eight 2-byte elements (one 16-byte load) as floats.
template <typename TR>
__device__ __forceinline__ void unpack8(u32x4 raw, float* out) {
    typename TR::elem e[8];
    __builtin_memcpy(e, &raw, 16);
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = TR::to_f(e[j]);
}

// Eight floats rounded to the 2-byte element type, as one 16-byte value.
template <typename TR>
__device__ __forceinline__ u32x4 pack8(const float* v) {
    typename TR::elem e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = TR::from_f(v[j]);
    u32x4 raw;
    __builtin_memcpy(&raw, e, 16);
    return raw;
}

// a.x * b.x + a.y * b.y + c for two packed 16-bit pairs, in fp32.
template <typename TR>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    if constexpr (std::is_same_v<typename TR::elem, __bf16>) {
        typedef __bf16 p2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(p2, a), __builtin_bit_cast(p2, b),
                                               c, false);
    } else {
        typedef _Float16 p2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(p2, a), __builtin_bit_cast(p2, b), c,
                                      false);
    }
}

// The pair (1, 1) in the 2-byte element type: dot2 with it sums a packed pair.
template <typename TR>
constexpr uint32_t kOnePair = std::is_same_v<typename TR::elem, __bf16> ? 0x3F803F80u : 0x3C003C00u;

// Raw buffer resource over `bytes` bytes at `base` (stride 0). Buffer loads check the whole
// offset (VGPR offset + SGPR offset) against `bytes` and return zeros past it, so tiles that run
// off the end of a slice need no per-lane selects, and the per-lane offsets stay the same from
// tile to tile (only the scalar offset moves).
using Rsrc = __amdgpu_buffer_rsrc_t;
__device__ __forceinline__ Rsrc buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
// A per-lane offset that every slice resource treats as out of range (resources cover < 2^30).
constexpr int kPastEnd = 1 << 30;

// Direct buffer->LDS loads: lane i's 16 (4) bytes at byte voff + soff of the resource land at
// lds_window + 16*i (4*i); lds_window must be wave-uniform.
__device__ __forceinline__ void buf_dma16(Rsrc r, int voff, int soff, char* lds_window) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)lds_window, 16, voff, soff, 0, 0);
}
// The same with the non-temporal cache policy, for rows read once.
__device__ __forceinline__ void buf_dma16_nt(Rsrc r, int voff, int soff, char* lds_window) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)lds_window, 16, voff, soff, 0, 2);
}
__device__ __forceinline__ void buf_dma4(Rsrc r, int voff, int soff, char* lds_window) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)lds_window, 4, voff, soff, 0, 0);
}

// Waits for this thread's outstanding global loads (including async LDS fills).
__device__ __forceinline__ void async_wait() { __builtin_amdgcn_s_waitcnt(0); }

// Waits until at most N of this thread's vector memory operations (loads, direct-to-LDS loads
// and stores, which retire in issue order for this count) are outstanding. Memory accesses stay
// on their side of the wait.
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The LDS address (byte offset in the workgroup's LDS) of a __shared__ pointer, for explicit LDS
// instructions.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// 16-byte buffer store; a store whose offset falls past the resource's range is dropped.
__device__ __forceinline__ void buf_st16(Rsrc r, int voff, int soff, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, soff, 0);
}
// The same with the non-temporal cache policy. Pays where one wave instruction writes whole
// 128-byte lines (a line written in pieces by several waves is evicted part-written).
__device__ __forceinline__ void buf_st16_nt(Rsrc r, int voff, int soff, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, soff, 2);
}

// Stores a tile of R rows x W 2-byte columns staged in LDS (row stride OSTR bytes) to the rows of
// `ro` (row stride W elements; rows past the resource are dropped) as whole rows: wave `wave` of
// NW takes 64 consecutive 16-byte pieces per instruction, non-temporal. An MFMA wave's own
// output is 16 rows x 64 bytes (half lines); staging it lets one instruction write whole lines.
template <int R, int W, int OSTR, int NW>
__device__ __forceinline__ void store_staged_rows(Rsrc ro, const char* ob, int wave, int lane) {
    constexpr int PPR = W / 8, NI = R * PPR / (64 * NW);
    static_assert(W % 8 == 0 && NI * 64 * NW == R * PPR, "whole store rounds");
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int f = (i * NW + wave) * 64 + lane;
        const int row = f / PPR, piece = f % PPR;
        buf_st16_nt(ro, (row * W + piece * 8) * 2, 0,
                    *reinterpret_cast<const u32x4*>(ob + row * OSTR + piece * 16));
    }
}

// Workgroup barrier that publishes LDS only: waits for this wave's LDS operations, not for its
// outstanding global loads and stores (the fence of __syncthreads waits for those too, so a
// barrier right after a batch of stores would stall for their write-back).
__device__ __forceinline__ void lds_barrier() {
    // Compiler-only fences keep memory accesses on their side of the barrier; the hardware wait
    // is for LDS (lgkmcnt) alone: vmcnt and expcnt fields at their maxima in the encoding.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Cross-lane reductions among the four lanes l, l^16, l^32, l^48 (same column of a C tile).
// v_permlane32_swap / v_permlane16_swap with both operands = v return, in each lane, v of that
// lane and of the lane 32 (16) apart, as a pair: two VALU ops per step, no LDS round trip.
__device__ __forceinline__ u32x2 pair_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return u32x2{r[0], r[1]};
}
__device__ __forceinline__ u32x2 pair_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return u32x2{r[0], r[1]};
}
__device__ __forceinline__ float xgroup_max(float v) {
    u32x2 p = pair_xor32(v);
    v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    p = pair_xor16(v);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float xgroup_sum(float v) {
    u32x2 p = pair_xor32(v);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    p = pair_xor16(v);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Lane exchanges for reductions over aligned groups of G lanes (G a power of two, 2..64), as
// (own value, partner value) pairs. Step s pairs the lanes s apart in the butterfly sense. Steps
// 1 and 2 are DPP quad permutations (lane ^ 1, lane ^ 2); steps 4 and 8 are row_half_mirror and
// row_mirror, which pair a lane with one of the other quad (half row) -- equivalent to lane ^ 4
// (^ 8) once the earlier steps have made every quad (half row) hold identical values; steps 16
// and 32 are permlane swaps. All are VALU moves, no LDS round trip. A reduction that combines
// each pair symmetrically (a + b, max, Chan's merge) therefore leaves identical bits in every
// lane of the group.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int STEP>
__device__ __forceinline__ u32x2 lane_pair(float v) {
    static_assert(STEP == 1 || STEP == 2 || STEP == 4 || STEP == 8 || STEP == 16 || STEP == 32,
                  "butterfly step");
    if constexpr (STEP == 16) return pair_xor16(v);
    else if constexpr (STEP == 32) return pair_xor32(v);
    else {
        constexpr int ctrl = STEP == 1 ? 0xB1 : STEP == 2 ? 0x4E : STEP == 4 ? 0x141 : 0x140;
        return u32x2{__float_as_uint(v), __float_as_uint(dpp_move<ctrl>(v))};
    }
}
template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "group of 2^k lanes");
    if constexpr (G >= 2) {
        const u32x2 p = lane_pair<G / 2>(group_sum<G / 2>(v));
        return __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    return v;
}

// Work item of workgroup L out of T so that each XCD runs a contiguous range of work items.
// The dispatcher hands workgroup L to XCD L % 8 (each XCD has its own L2), so with the identity
// mapping neighbouring work items -- which share inputs -- land on different L2s. A bijection
// of [0, T): results never depend on it, only the L2 hit rate does.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_contiguous(int L, int T) {
    const int xcd = L % kXcds, slot = L / kXcds;
    const int per = T / kXcds, rem = T % kXcds;
    return xcd * per + min(xcd, rem) + slot;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// ---------------------------------------------------------------------------------------------
// Host side: thread-local last-error message and status helpers.
// ---------------------------------------------------------------------------------------------
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
clk_status fail(clk_status code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
clk_status ok();
clk_status check_launch(const char* what);

// Brackets one kernel launch with HIP events when per-launch timing is enabled on this thread.
class KernelTimer {
   public:
    KernelTimer(const char* name, hipStream_t stream);
    ~KernelTimer();
    KernelTimer(const KernelTimer&) = delete;
    KernelTimer& operator=(const KernelTimer&) = delete;

   private:
    const char* name_;
    hipStream_t stream_;
    hipEvent_t start_ = nullptr;
};

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline size_t elem_size(clk_dtype t) {
    return t == CLK_F32 ? 4 : (t == CLK_U8 ? 1 : 2);
}
const char* dtype_name(clk_dtype t);

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

}  // namespace clk
