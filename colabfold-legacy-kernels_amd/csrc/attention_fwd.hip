// Flash attention forward with a per-head pair bias and a per-row key mask, for gfx950.
// Replaces VoltaMma (cuda/volta_mma_attn.cu:70-351) and VoltaWmma (cuda/volta_wmma_attn.cu:
// 47-311) with one kernel for f16 and bf16 on MFMA 16x16x32 with float32 accumulation.
//
// Work split: a block of 4 waves owns (query tile of 64*QT rows, head h, row n); each wave owns
// 16*QT queries and streams the keys in tiles of 64 through double-buffered LDS: tile kt+1 is
// fetched with direct global->LDS loads (and its bias rows into registers) while tile kt is
// computed, so each tile costs one barrier. Which tiles contain an absent key is worked out once
// per block from the mask row; the others skip the mask entirely.
//
// Per 64-key tile and 16-query sub-tile a wave computes S^T = K . Q^T with the keys of each
// 32-key chunk permuted so that lane l's accumulator holds keys 8*(l/16)+0..7 of the chunk for
// query l%16. Those eight values are exactly the B operand of O^T = V^T . P^T for that chunk, so
// P never leaves registers; V^T comes from LDS with ds_read_b64_tr_b16 (two 4x16 transposed
// reads per operand). O^T accumulates four consecutive head dims per lane, stored as 8 bytes.
//
// Numerics (volta_mma_attn.cu:137,174-272): logit = scale*(q.k) + bias in float32; a key with
// kmask == 0 gets the logit -1e9 (the float32 value of the caller's additive 1e9*(mask-1)), a
// key past Sk gets -inf; online softmax in the exp2 domain; P rounded to the input type for the
// P.V product (as the reference rounds it to f16, :221); O = acc / max(l, 1e-30) (:265).
// A row whose keys are all masked gets the logit 0 for them instead: its softmax is the same
// (uniform over the Sk keys), but float32 cannot subtract a running max of -1e9 exactly (its
// rounding unit there is 128), which would scale P by up to 2^64.
// lse = m + log(l) (natural log) is written when requested, for the backward pass; for an
// all-masked row it is therefore ln(Sk), relative to the masked logit.
#include "attention_common.hpp"

namespace clk {
namespace {

// Per-tile "some key absent or past Sk" flags of one mask row, for up to kMaxFlagTiles tiles of
// 64 keys (beyond that every tile takes the checked path). Also returns the row's masked logit.
constexpr int kMaxFlagTiles = 128;

__device__ __forceinline__ float tile_flags(const uint8_t* mrow, int Sk, int* flags) {
    const int ntiles = (Sk + 63) / 64;
    for (int t = threadIdx.x; t < kMaxFlagTiles; t += blockDim.x)
        flags[t] = (t >= ntiles || 64 * (t + 1) > Sk) ? 1 : 0;
    __syncthreads();
    int any = 0;
    if (mrow) {
        for (int i = threadIdx.x; i < Sk; i += blockDim.x) {
            const bool present = mrow[i] != 0;
            any |= present;
            if (!present && i / 64 < kMaxFlagTiles) flags[i / 64] = 1;
        }
    }
    any = __syncthreads_or(any);
    return (mrow && !any) ? 0.f : kMaskedLogit;
}

// Eight consecutive keys' bias values and mask bytes of one tile, as loaded. VEC: 16-byte bias
// and 8-byte mask loads (Sk % 8 == 0, 8-byte aligned mask rows); a lane whose eight keys lie past
// Sk reads the last eight instead (those keys are forced to -inf). Otherwise element loads.
template <typename TR, bool VEC>
struct KeyChunk {
    u32x4 bias;
    u32x2 mask;
    __device__ __forceinline__ void load(const typename TR::elem* brow, const uint8_t* mrow,
                                         int kk, int Sk) {
        using E = typename TR::elem;
        if constexpr (VEC) {
            const int kc = min(kk, Sk - 8);
            bias = ld16(brow + kc);
            mask = mrow ? *reinterpret_cast<const u32x2*>(mrow + kc) : u32x2{~0u, ~0u};
        } else {
            E e[8];
            uint8_t m[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const bool in = kk + j < Sk;
                e[j] = in ? brow[kk + j] : E(0.f);
                m[j] = in ? (mrow ? mrow[kk + j] : uint8_t(1)) : uint8_t(0);
            }
            __builtin_memcpy(&bias, e, 16);
            __builtin_memcpy(&mask, m, 8);
        }
    }
    // Bit j set when key kk + j is present.
    __device__ __forceinline__ unsigned valid() const {
        unsigned bits = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bits |= (((mask[0] >> (8 * j)) & 0xffu) != 0u ? 1u : 0u) << j;
            bits |= (((mask[1] >> (8 * j)) & 0xffu) != 0u ? 1u : 0u) << (4 + j);
        }
        return bits;
    }
};

template <typename TR, int D, int QT, bool VEC>
__global__ __launch_bounds__(256) void attn_fwd_kernel(
    const typename TR::elem* __restrict__ q, const typename TR::elem* __restrict__ k,
    const typename TR::elem* __restrict__ v, const typename TR::elem* __restrict__ bias,
    const uint8_t* __restrict__ kmask, typename TR::elem* __restrict__ out,
    float* __restrict__ lse, int H, int Sq, int Sk, float scale) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    using G = AttnGeom<D>;
    using T = SwzTile<D>;
    using KC = KeyChunk<TR, VEC>;
    constexpr int BQ = 4 * 16 * QT;
    constexpr int BK = G::BK;
    constexpr int TILE = BK * T::ROWB;  // bytes of one K or V tile

    __shared__ __attribute__((aligned(16))) char kv_lds[2][2][TILE];  // [buffer][K, V]
    __shared__ int flags[kMaxFlagTiles];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int q0 = blockIdx.x * BQ, h = blockIdx.y, n = blockIdx.z;
    const size_t nh = (size_t)n * H + h;
    const E* qp = q + nh * Sq * D;
    const E* kp = k + nh * Sk * D;
    const E* vp = v + nh * Sk * D;
    const E* bp = bias + (size_t)h * Sq * Sk;
    const uint8_t* mp = kmask ? kmask + (size_t)n * Sk : nullptr;
    const int qbase = q0 + wave * 16 * QT;
    const int ntiles = (Sk + BK - 1) / BK;

    if (ntiles > 0) {
        stage_rows_async<D, BK, 256>(kp, 0, Sk, kv_lds[0][0]);
        stage_rows_async<D, BK, 256>(vp, 0, Sk, kv_lds[0][1]);
    }
    const float masked_logit = tile_flags(mp, Sk, flags);

    // B operand Q^T: lane (query r16, group g) holds head dims 32*ks + 8*g + 0..7.
    V8 qf[QT][G::KS];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int row = qbase + qt * 16 + r16;
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            const int d0 = ks * 32 + g * 8;
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (row < Sq && d0 < D) raw = ld16(qp + (size_t)row * D + d0);
            qf[qt][ks] = bits_as<V8>(raw);
        }
    }

    // Bias rows of the lane's queries (clamped inside [0, Sq)), keys 32c + 8g + 0..7 per tile.
    const E* brow[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) brow[qt] = bp + (size_t)min(qbase + qt * 16 + r16, Sq - 1) * Sk;
    KC cur[QT][2], nxt[QT][2];
    auto load_chunks = [&](int k0, KC (&kc)[QT][2]) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
            for (int c = 0; c < 2; ++c) kc[qt][c].load(brow[qt], mp, k0 + 32 * c + 8 * g, Sk);
    };
    if (ntiles > 0) load_chunks(0, cur);

    float m_run[QT], l_run[QT];
    f32x4 acc[QT][G::DT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        m_run[qt] = -INFINITY;
        l_run[qt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) acc[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    for (int kt = 0; kt < ntiles; ++kt) {
        const int k0 = kt * BK;
        const char* k_lds = kv_lds[kt & 1][0];
        const char* v_lds = kv_lds[kt & 1][1];
        async_wait();
        __syncthreads();  // tile kt visible; every wave is done with the other buffer

        // Everything this tile needs from LDS is read before the next tile's direct-to-LDS
        // loads are issued, so no LDS read waits for them.
        const bool need_mask = kt >= kMaxFlagTiles || flags[kt] != 0;
        V8 kf[4][G::KS];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int ks = 0; ks < G::KS; ++ks)
                kf[t][ks] = swz_row_operand<V8, D>(k_lds, perm_key(t, r16), ks, g);
        V8 vf[G::DT][2];
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
            for (int c = 0; c < 2; ++c) vf[dt][c] = swz_tr_operand<V8, D>(v_lds, 32 * c, dt, r16, g);

        if (kt + 1 < ntiles) {
            stage_rows_async<D, BK, 256>(kp, k0 + BK, Sk, kv_lds[(kt + 1) & 1][0]);
            stage_rows_async<D, BK, 256>(vp, k0 + BK, Sk, kv_lds[(kt + 1) & 1][1]);
            load_chunks(k0 + BK, nxt);
        }

        // S^T = K . Q^T for the four 16-key sub-tiles (chunk c = t/2, half t%2).
        f32x4 s[QT][4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int ks = 0; ks < G::KS; ++ks)
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
                    s[qt][t] = TR::mfma(kf[t][ks], qf[qt][ks],
                                        ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[qt][t]);

#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            float x[2][8];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                float bv[8];
                unpack8<TR>(cur[qt][c].bias, bv);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[c][j] = fmaf(s[qt][2 * c][j], scale, bv[j]);
                    x[c][4 + j] = fmaf(s[qt][2 * c + 1][j], scale, bv[4 + j]);
                }
            }
            if (need_mask) {
                // Opaque to speculation: keeps the selects out of the unmasked path.
                asm volatile("");
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const unsigned valid = cur[qt][c].valid();
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int key = k0 + 32 * c + 8 * g + j;
                        x[c][j] = key >= Sk ? -INFINITY
                                            : (((valid >> j) & 1u) ? x[c][j] : masked_logit);
                    }
                }
            }
            float mt = x[0][0];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int j = 0; j < 8; ++j) mt = fmaxf(mt, x[c][j]);
            mt = xgroup_max(mt);
            const float m_new = fmaxf(m_run[qt], mt);
            const float alpha = fast_exp2((m_run[qt] - m_new) * kLog2e);
            const float neg = -m_new * kLog2e;
            float psum = 0.f;
            V8 pf[2];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float p = fast_exp2(fmaf(x[c][j], kLog2e, neg));
                    psum += p;
                    pf[c][j] = TR::from_f(p);
                }
            l_run[qt] = l_run[qt] * alpha + psum;
            m_run[qt] = m_new;
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
                acc[qt][dt] *= alpha;
#pragma unroll
                for (int c = 0; c < 2; ++c) acc[qt][dt] = TR::mfma(vf[dt][c], pf[c], acc[qt][dt]);
            }
        }
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
            for (int c = 0; c < 2; ++c) cur[qt][c] = nxt[qt][c];
    }

    // Normalise and store: lane holds O[row][16*dt + 4*g + i], i = 0..3.
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float l_tot = xgroup_sum(l_run[qt]);
        const float inv = 1.0f / fmaxf(l_tot, 1e-30f);
        const int row = qbase + qt * 16 + r16;
        if (row >= Sq) continue;
        E* orow = out + (nh * Sq + row) * D;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
            const int d = 16 * dt + 4 * g;
            if (d < D) store4<TR>(orow + d, acc[qt][dt] * inv);
        }
        if (lse && g == 0) lse[nh * Sq + row] = m_run[qt] + logf(l_tot);
    }
}

template <typename TR, int D, int QT>
void launch_fwd_qt(hipStream_t st, const void* q, const void* k, const void* v, const void* bias,
                   const uint8_t* kmask, void* out, float* lse, int N, int H, int Sq, int Sk,
                   float scale) {
    using E = typename TR::elem;
    const dim3 grid(ceil_div(Sq, 64 * QT), H, N);
    const bool vec = Sk % 8 == 0 && (reinterpret_cast<uintptr_t>(kmask) & 7u) == 0;
    if (vec)
        attn_fwd_kernel<TR, D, QT, true><<<grid, 256, 0, st>>>(
            (const E*)q, (const E*)k, (const E*)v, (const E*)bias, kmask, (E*)out, lse, H, Sq, Sk,
            scale);
    else
        attn_fwd_kernel<TR, D, QT, false><<<grid, 256, 0, st>>>(
            (const E*)q, (const E*)k, (const E*)v, (const E*)bias, kmask, (E*)out, lse, H, Sq, Sk,
            scale);
}

template <typename TR, int D>
void launch_fwd(hipStream_t st, const void* q, const void* k, const void* v, const void* bias,
                const uint8_t* kmask, void* out, float* lse, int N, int H, int Sq, int Sk,
                float scale) {
    KernelTimer timer("attn_fwd", st);
    if (Sq <= 64)
        launch_fwd_qt<TR, D, 1>(st, q, k, v, bias, kmask, out, lse, N, H, Sq, Sk, scale);
    else
        launch_fwd_qt<TR, D, 2>(st, q, k, v, bias, kmask, out, lse, N, H, Sq, Sk, scale);
}

template <typename TR>
void dispatch_fwd(hipStream_t st, int64_t D, const void* q, const void* k, const void* v,
                  const void* bias, const uint8_t* kmask, void* out, float* lse, int N, int H,
                  int Sq, int Sk, float scale) {
    switch (D) {
        case 8: launch_fwd<TR, 8>(st, q, k, v, bias, kmask, out, lse, N, H, Sq, Sk, scale); break;
        case 16: launch_fwd<TR, 16>(st, q, k, v, bias, kmask, out, lse, N, H, Sq, Sk, scale); break;
        case 32: launch_fwd<TR, 32>(st, q, k, v, bias, kmask, out, lse, N, H, Sq, Sk, scale); break;
        default: launch_fwd<TR, 64>(st, q, k, v, bias, kmask, out, lse, N, H, Sq, Sk, scale); break;
    }
}

}  // namespace
}  // namespace clk

using namespace clk;

extern "C" clk_status clk_attention_fwd(hipStream_t stream, clk_dtype dtype, const void* q,
                                        const void* k, const void* v, const void* bias,
                                        const uint8_t* kmask, void* out, float* lse, int64_t N,
                                        int64_t H, int64_t Sq, int64_t Sk, int64_t D, float scale,
                                        int64_t block_q, int64_t block_k) {
    clk_status s = validate_attention("attention", dtype, N, H, Sq, Sk, D);
    if (s != CLK_OK) return s;
    if (block_q <= 0 || block_k <= 0)
        return fail(CLK_INVALID_ARGUMENT, "attention: block_q and block_k must be positive");
    if (N * H * Sq == 0) return ok();
    if (!q || !k || !v || !bias || !out)
        return fail(CLK_INVALID_ARGUMENT, "attention: null operand pointer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(bias) || !aligned16(out))
        return fail(CLK_INVALID_ARGUMENT, "attention: q, k, v, bias, out must be 16-byte aligned");
    if (dtype == CLK_BF16)
        dispatch_fwd<BF16>(stream, D, q, k, v, bias, kmask, out, lse, (int)N, (int)H, (int)Sq,
                           (int)Sk, scale);
    else
        dispatch_fwd<F16>(stream, D, q, k, v, bias, kmask, out, lse, (int)N, (int)H, (int)Sq,
                          (int)Sk, scale);
    return check_launch("attention");
}
