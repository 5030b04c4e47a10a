// Flash attention forward with a per-head pair bias and a per-row key mask, for gfx950.
// Replaces VoltaMma (cuda/volta_mma_attn.cu:70-351) and VoltaWmma (cuda/volta_wmma_attn.cu:
// 47-311) with one kernel for f16 and bf16 on MFMA 16x16x32 with float32 accumulation.
//
// Work split: a block of 4 waves owns (query tile of 64*QT rows, head h, row n); each wave owns
// 16*QT queries and streams the keys in tiles of 64 through LDS (K row-major, V row-major, both
// double-staged through registers so the next tile's global loads overlap this tile's math).
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

template <typename TR, int D, int QT>
__global__ __launch_bounds__(256) void attn_fwd_kernel(
    const typename TR::elem* __restrict__ q, const typename TR::elem* __restrict__ k,
    const typename TR::elem* __restrict__ v, const typename TR::elem* __restrict__ bias,
    const uint8_t* __restrict__ kmask, typename TR::elem* __restrict__ out,
    float* __restrict__ lse, int H, int Sq, int Sk, float scale, int vec_ok) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    using G = AttnGeom<D>;
    constexpr int BQ = 4 * 16 * QT;
    constexpr int BK = G::BK;

    __shared__ __attribute__((aligned(16))) E k_lds[BK * G::KLD];
    __shared__ __attribute__((aligned(16))) E v_lds[BK * G::VLD];

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

    zero_v_padding<E, D>(v_lds);
    const float masked_logit = masked_logit_for_row(mp, Sk);

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

    float m_run[QT], l_run[QT];
    f32x4 acc[QT][G::DT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        m_run[qt] = -INFINITY;
        l_run[qt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) acc[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    TileStager<E, D> stage;
    const int ntiles = (Sk + BK - 1) / BK;
    if (ntiles > 0) stage.load(kp, vp, 0, Sk);
    for (int kt = 0; kt < ntiles; ++kt) {
        const int k0 = kt * BK;
        __syncthreads();
        stage.store(k_lds, v_lds);
        __syncthreads();
        if (kt + 1 < ntiles) stage.load(kp, vp, k0 + BK, Sk);

        // Bias (as float) and key validity for the lane's keys k0 + 32c + 8g + j.
        float bv[QT][2][8];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const int brow = min(qbase + qt * 16 + r16, Sq - 1);
#pragma unroll
            for (int c = 0; c < 2; ++c)
                load_bias8<TR>(bp + (size_t)brow * Sk, k0 + 32 * c + 8 * g, Sk, vec_ok,
                               bv[qt][c]);
        }
        unsigned valid[2];
        bool all_valid = true;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            valid[c] = key_valid8(mp, k0 + 32 * c + 8 * g, Sk, vec_ok);
            all_valid = all_valid && valid[c] == 0xffu && (k0 + 32 * c + 8 * g + 8 <= Sk);
        }
        const bool need_mask = !__all(all_valid);

        // S^T = K . Q^T for the four 16-key sub-tiles (chunk c = t/2, half t%2).
        f32x4 s[QT][4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int key = perm_key(t, r16);
#pragma unroll
            for (int ks = 0; ks < G::KS; ++ks) {
                const V8 kf = lds_row_operand<V8, D>(k_lds, key, G::KLD, ks, g);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
                    s[qt][t] = TR::mfma(kf, qf[qt][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f}
                                                               : s[qt][t]);
            }
        }

        // A operand V^T (rows = head dims, k-slots = the chunk's keys in lane order).
        V8 vf[G::DT][2];
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
            for (int c = 0; c < 2; ++c) vf[dt][c] = lds_tr_operand<V8>(v_lds, G::VLD, c, dt, r16, g);

#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            float x[2][8];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[c][j] = s[qt][2 * c][j] * scale + bv[qt][c][j];
                    x[c][4 + j] = s[qt][2 * c + 1][j] * scale + bv[qt][c][4 + j];
                }
            if (need_mask) {
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int key = k0 + 32 * c + 8 * g + j;
                        x[c][j] = key >= Sk ? -INFINITY
                                            : (((valid[c] >> j) & 1u) ? x[c][j] : masked_logit);
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

template <typename TR, int D>
void launch_fwd(hipStream_t st, const void* q, const void* k, const void* v, const void* bias,
                const uint8_t* kmask, void* out, float* lse, int N, int H, int Sq, int Sk,
                float scale) {
    using E = typename TR::elem;
    const int vec_ok = (Sk % 8 == 0) ? 1 : 0;
    KernelTimer timer("attn_fwd", st);
    if (Sq <= 64) {
        dim3 grid(ceil_div(Sq, 64), H, N);
        attn_fwd_kernel<TR, D, 1><<<grid, 256, 0, st>>>(
            (const E*)q, (const E*)k, (const E*)v, (const E*)bias, kmask, (E*)out, lse, H, Sq,
            Sk, scale, vec_ok);
    } else {
        dim3 grid(ceil_div(Sq, 128), H, N);
        attn_fwd_kernel<TR, D, 2><<<grid, 256, 0, st>>>(
            (const E*)q, (const E*)k, (const E*)v, (const E*)bias, kmask, (E*)out, lse, H, Sq,
            Sk, scale, vec_ok);
    }
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
