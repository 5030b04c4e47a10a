// Attention backward for gfx950 (no reference counterpart: the reference is forward-only). It is
// the gradient of attention_fwd.hip's math with the caller's additive-mask convention, so dS
// reaches masked keys too:
//   D_i = rowsum(dO * O);  P = exp(logit - lse);  dS = P * (dO.V^T - D_i)
//   dQ = scale * dS.K;  dK = scale * dS^T.Q;  dV = P^T.dO;  dBias[h] = sum over rows n of dS[n,h]
//
// Deterministic, without floating-point atomics. Four launches on the caller's stream:
//   1. attn_bwd_dot   D_i per query row (16-byte loads of O and dO).
//   2. attn_bwd_dq    "row owner": a block owns (64 queries, head h, a chunk of NB rows n, a key
//                     range of up to 64*KT keys). For each n it recomputes S^T = K.Q^T and
//                     dP^T = V.dO^T per 64-key tile (keys permuted as in the forward, so dS^T is
//                     directly the B operand of dQ^T = K^T.dS^T with K^T read by the LDS
//                     transpose), accumulates dQ in registers across the key tiles, and
//                     accumulates dBias for all its (query, key) pairs in registers across the
//                     chunk's rows. dBias partials go to workspace [chunk][H][Sq][Sk] (or straight
//                     to dbias when there is one chunk); dQ partials per key range likewise.
//   3. attn_bwd_dkv   "column owner": a block owns (64 keys, head h, row n) and streams the
//                     queries in 64-row tiles through LDS (Q, dO, the bias tile, lse, D). Per
//                     tile it computes S = Q.K^T and dP = dO.V^T with the queries permuted so P
//                     and dS are directly the B operands of dV^T = dO^T.P and dK^T = Q^T.dS.
//   4. fixed-order sums of the dBias (and, for Sk > 512, dQ) partials.
// P is recomputed in 2 and 3 from the saved lse; it is never stored.
#include "attention_common.hpp"

#include <algorithm>
#include <type_traits>

namespace clk {
namespace {

// How a row-owner block's rows are masked, and the chunk code a row step runs.
constexpr int kRowsClean = 0, kRowsEmpty = 1, kRowsMixed = 2;
constexpr int kChunksClean = 0, kChunksSelect = 1, kChunksEmpty = 2;


// D_i = rowsum(dO * O) for every query row (rows in the operands' order; with NSHD the
// [N, S, H] order, written to di in the [N, H, S] order).
template <typename TR, int D, bool NSHD>
__global__ __launch_bounds__(256) void attn_bwd_dot(const typename TR::elem* __restrict__ out,
                                                    const typename TR::elem* __restrict__ dout,
                                                    float* __restrict__ di, int64_t rows, int H,
                                                    int Sq) {
    constexpr int LPR = D / 8;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = gid / LPR;
    const int part = (int)(gid % LPR);
    float s = 0.f;
    if (row < rows) {
        float o[8], d[8];
        unpack8<TR>(ld16(out + row * D + part * 8), o);
        unpack8<TR>(ld16(dout + row * D + part * 8), d);
#pragma unroll
        for (int j = 0; j < 8; ++j) s += o[j] * d[j];
    }
    s = group_sum<LPR>(s);
    if (row < rows && part == 0) {
        int64_t at = row;
        if constexpr (NSHD) {  // row = (n*Sq + q)*H + h
            const int64_t hh = row % H, nq = row / H;
            at = (nq / Sq * H + hh) * Sq + nq % Sq;
        }
        di[at] = s;
    }
}

template <typename TR, int D, int KT, bool NSHD>
__global__ __launch_bounds__(256) void attn_bwd_dq(
    const typename TR::elem* __restrict__ q, const typename TR::elem* __restrict__ k,
    const typename TR::elem* __restrict__ v, const typename TR::elem* __restrict__ bias,
    const uint8_t* __restrict__ kmask, const typename TR::elem* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ di,
    typename TR::elem* __restrict__ dq, float* __restrict__ dq_part,
    float* __restrict__ dbias_dst, int N, int H, int Sq, int Sk, int NB, int nranges,
    float scale, int vec_ok) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    using G = AttnGeom<D>;
    constexpr int LD = G::VLD;

    __shared__ __attribute__((aligned(16))) E k_lds[64 * LD];
    __shared__ __attribute__((aligned(16))) E v_lds[64 * LD];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int q0 = blockIdx.x * 64, h = blockIdx.y;
    const int chunk = blockIdx.z / nranges, range = blockIdx.z % nranges;
    const int kbeg = range * 64 * KT;
    const int kend = min(Sk, kbeg + 64 * KT);
    const int ktiles = (kend - kbeg + 63) / 64;
    const int n0 = chunk * NB, n1 = min(N, n0 + NB);
    const int qrow = q0 + wave * 16 + r16;
    const bool qin = qrow < Sq;
    const int brow = min(qrow, Sq - 1);

    zero_v_padding<E, D>(k_lds);
    zero_v_padding<E, D>(v_lds);

    f32x4 dbias_acc[KT][4];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int t = 0; t < 4; ++t) dbias_acc[kt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    RowTileStager<E, D, 2> stage;
    E* const dst[2] = {k_lds, v_lds};
    const int lds_ld[2] = {LD, LD};
    using HR = HeadRows<D, NSHD>;
    auto load_tile = [&](int n, int kstart) {
        const size_t base = HR::at(n, h, 0, Sk, H);
        const E* src[2] = {k + base, v + base};
        stage.load(src, kstart, kend, HR::ld(H));
    };
    if (n0 < n1) load_tile(n0, kbeg);

    for (int n = n0; n < n1; ++n) {
        const size_t nh = (size_t)n * H + h;
        V8 qf[G::KS], dof[G::KS];
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            const int d0 = ks * 32 + g * 8;
            u32x4 rq = {0u, 0u, 0u, 0u}, rd = {0u, 0u, 0u, 0u};
            if (qin && d0 < D) {
                rq = ld16(q + HR::at(n, h, qrow, Sq, H) + d0);
                rd = ld16(dout + HR::at(n, h, qrow, Sq, H) + d0);
            }
            qf[ks] = bits_as<V8>(rq);
            dof[ks] = bits_as<V8>(rd);
        }
        const float lse2 = qin ? lse[nh * Sq + qrow] * kLog2e : INFINITY;
        const float di_q = qin ? di[nh * Sq + qrow] : 0.f;
        const uint8_t* mp = kmask ? kmask + (size_t)n * Sk : nullptr;
        const float masked_logit = masked_logit_for_row(mp, Sk);
        const E* brow_p = bias + ((size_t)h * Sq + brow) * Sk;

        f32x4 dq_acc[G::DT];
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) dq_acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
            // Keep the scheduler from interleaving tiles: the accumulators are the live state.
            __builtin_amdgcn_sched_barrier(0);
            if (kt < ktiles) {
                const int k0 = kbeg + 64 * kt;
                __syncthreads();
                stage.store(dst, lds_ld);
                __syncthreads();
                if (kt + 1 < ktiles) load_tile(n, k0 + 64);
                else if (n + 1 < n1) load_tile(n + 1, kbeg);

                float bv[2][8];
                unsigned valid[2];
                bool all_valid = true;
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const int kk = k0 + 32 * c + 8 * g;
                    load_bias8<TR>(brow_p, kk, Sk, vec_ok, bv[c]);
                    valid[c] = key_valid8(mp, kk, Sk, vec_ok);
                    all_valid = all_valid && valid[c] == 0xffu && kk + 8 <= Sk;
                }
                const bool need_mask = !__all(all_valid);

                f32x4 s[4], dp[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int key = perm_key(t, r16);
#pragma unroll
                    for (int ks = 0; ks < G::KS; ++ks) {
                        const V8 ka = lds_row_operand<V8, D>(k_lds, key, LD, ks, g);
                        const V8 va = lds_row_operand<V8, D>(v_lds, key, LD, ks, g);
                        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                        s[t] = TR::mfma(ka, qf[ks], ks == 0 ? z : s[t]);
                        dp[t] = TR::mfma(va, dof[ks], ks == 0 ? z : dp[t]);
                    }
                }

                V8 dsf[2];
                f32x4 ds4[4];
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int t = 2 * c + (j >> 2), i = j & 3;
                        float x = s[t][i] * scale + bv[c][j];
                        if (need_mask) {
                            const int key = k0 + 32 * c + 8 * g + j;
                            x = key >= Sk ? -INFINITY : (((valid[c] >> j) & 1u) ? x : masked_logit);
                        }
                        const float p = fast_exp2(fmaf(x, kLog2e, -lse2));
                        const float ds = p * (dp[t][i] - di_q);
                        ds4[t][i] = ds;
                        dsf[c][j] = TR::from_f(ds);
                    }
#pragma unroll
                for (int t = 0; t < 4; ++t) dbias_acc[kt][t] += ds4[t];
#pragma unroll
                for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
                    for (int c = 0; c < 2; ++c)
                        dq_acc[dt] = TR::mfma(lds_tr_operand<V8>(k_lds, LD, c, dt, r16, g), dsf[c],
                                              dq_acc[dt]);
            }
        }

        if (qin) {
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
                const int d = 16 * dt + 4 * g;
                if (d < D) {
                    if (nranges == 1) {
                        store4<TR>(dq + HR::at(n, h, qrow, Sq, H) + d, dq_acc[dt] * scale);
                    } else {  // range's partial, in dq's layout
                        float* o = dq_part + (size_t)range * N * H * Sq * D +
                                   HR::at(n, h, qrow, Sq, H) + d;
                        *reinterpret_cast<f32x4*>(o) = dq_acc[dt] * scale;
                    }
                }
            }
        }
    }

    if (!qin) return;
    float* drow = dbias_dst + (((size_t)chunk * H + h) * Sq + qrow) * Sk;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        if (kt < ktiles) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int kb = kbeg + 64 * kt + 32 * c + 8 * g;
                const f32x4 lo = dbias_acc[kt][2 * c], hi = dbias_acc[kt][2 * c + 1];
                if (vec_ok && kb + 8 <= Sk) {
                    *reinterpret_cast<f32x4*>(drow + kb) = lo;
                    *reinterpret_cast<f32x4*>(drow + kb + 4) = hi;
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (kb + j < Sk) drow[kb + j] = lo[j];
                        if (kb + 4 + j < Sk) drow[kb + 4 + j] = hi[j];
                    }
                }
            }
        }
    }
}

template <typename TR, int D, bool NSHD>
__global__ __launch_bounds__(256) void attn_bwd_dkv(
    const typename TR::elem* __restrict__ q, const typename TR::elem* __restrict__ k,
    const typename TR::elem* __restrict__ v, const typename TR::elem* __restrict__ bias,
    const uint8_t* __restrict__ kmask, const typename TR::elem* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ di,
    typename TR::elem* __restrict__ dk, typename TR::elem* __restrict__ dv, int H, int Sq, int Sk,
    float scale, int vec_ok) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    using G = AttnGeom<D>;
    constexpr int LD = G::VLD;
    constexpr int BLD = 64 + 8;

    __shared__ __attribute__((aligned(16))) E q_lds[64 * LD];
    __shared__ __attribute__((aligned(16))) E do_lds[64 * LD];
    __shared__ __attribute__((aligned(16))) E b_lds[64 * BLD];
    __shared__ __attribute__((aligned(16))) float lse_lds[64];
    __shared__ __attribute__((aligned(16))) float di_lds[64];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int k0 = blockIdx.x * 64, h = blockIdx.y, n = blockIdx.z;
    const size_t nh = (size_t)n * H + h;
    using HR = HeadRows<D, NSHD>;
    const int key = k0 + wave * 16 + r16;
    const bool kin = key < Sk;

    V8 kf[G::KS], vf[G::KS];
#pragma unroll
    for (int ks = 0; ks < G::KS; ++ks) {
        const int d0 = ks * 32 + g * 8;
        u32x4 rk = {0u, 0u, 0u, 0u}, rv = {0u, 0u, 0u, 0u};
        if (kin && d0 < D) {
            rk = ld16(k + HR::at(n, h, key, Sk, H) + d0);
            rv = ld16(v + HR::at(n, h, key, Sk, H) + d0);
        }
        kf[ks] = bits_as<V8>(rk);
        vf[ks] = bits_as<V8>(rv);
    }
    const uint8_t* mp = kmask ? kmask + (size_t)n * Sk : nullptr;
    const float masked_logit = masked_logit_for_row(mp, Sk);
    const bool present = kin && (mp == nullptr || mp[key] != 0);
    const float absent_logit = kin ? masked_logit : -INFINITY;

    zero_v_padding<E, D>(q_lds);
    zero_v_padding<E, D>(do_lds);

    f32x4 dk_acc[G::DT], dv_acc[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt) {
        dk_acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        dv_acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    RowTileStager<E, D, 2> stage;
    E* const dst[2] = {q_lds, do_lds};
    const int lds_ld[2] = {LD, LD};
    const E* src[2] = {q + HR::at(n, h, 0, Sq, H), dout + HR::at(n, h, 0, Sq, H)};

    // Bias tile [64 queries][64 keys]: two 16-byte chunks per thread.
    u32x4 breg[2];
    const E* bhead = bias + (size_t)h * Sq * Sk;
    auto load_bias_tile = [&](int qs) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int ch = threadIdx.x + 256 * i;
            const int row = ch >> 3, c8 = (ch & 7) * 8;
            const int gq = qs + row, gk = k0 + c8;
            breg[i] = u32x4{0u, 0u, 0u, 0u};
            if (gq < Sq) {
                const E* p = bhead + (size_t)gq * Sk + gk;
                if (vec_ok && gk + 8 <= Sk) {
                    breg[i] = ld16(p);
                } else {
                    E e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) e[j] = (gk + j < Sk) ? p[j] : E(0.f);
                    __builtin_memcpy(&breg[i], e, 16);
                }
            }
        }
    };

    const int qtiles = (Sq + 63) / 64;
    if (qtiles > 0) {
        stage.load(src, 0, Sq, HR::ld(H));
        load_bias_tile(0);
    }
    for (int qt = 0; qt < qtiles; ++qt) {
        const int qs = qt * 64;
        __syncthreads();
        stage.store(dst, lds_ld);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int ch = threadIdx.x + 256 * i;
            *reinterpret_cast<u32x4*>(b_lds + (ch >> 3) * BLD + (ch & 7) * 8) = breg[i];
        }
        if (threadIdx.x < 64) {
            const int gq = qs + threadIdx.x;
            lse_lds[threadIdx.x] = gq < Sq ? lse[nh * Sq + gq] * kLog2e : INFINITY;
            di_lds[threadIdx.x] = gq < Sq ? di[nh * Sq + gq] : 0.f;
        }
        __syncthreads();
        if (qt + 1 < qtiles) {
            stage.load(src, qs + 64, Sq, HR::ld(H));
            load_bias_tile(qs + 64);
        }

        f32x4 s[4], dp[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int qr = perm_key(t, r16);
#pragma unroll
            for (int ks = 0; ks < G::KS; ++ks) {
                const V8 qa = lds_row_operand<V8, D>(q_lds, qr, LD, ks, g);
                const V8 da = lds_row_operand<V8, D>(do_lds, qr, LD, ks, g);
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                s[t] = TR::mfma(qa, kf[ks], ks == 0 ? z : s[t]);
                dp[t] = TR::mfma(da, vf[ks], ks == 0 ? z : dp[t]);
            }
        }

        V8 pf[2], dsf[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            float bvals[8], l8[8], d8[8];
            unpack8<TR>(__builtin_bit_cast(u32x4, lds_tr_operand<V8>(b_lds, BLD, c, wave, r16, g)),
                        bvals);
            const f32x4* lp = reinterpret_cast<const f32x4*>(lse_lds + 32 * c + 8 * g);
            const f32x4* dp4 = reinterpret_cast<const f32x4*>(di_lds + 32 * c + 8 * g);
            const f32x4 la = lp[0], lb = lp[1], da4 = dp4[0], db4 = dp4[1];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                l8[j] = la[j];
                l8[4 + j] = lb[j];
                d8[j] = da4[j];
                d8[4 + j] = db4[j];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int t = 2 * c + (j >> 2), i = j & 3;
                const float x = present ? s[t][i] * scale + bvals[j] : absent_logit;
                const float p = fast_exp2(fmaf(x, kLog2e, -l8[j]));
                const float ds = p * (dp[t][i] - d8[j]);
                pf[c][j] = TR::from_f(p);
                dsf[c][j] = TR::from_f(ds);
            }
        }
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                dv_acc[dt] = TR::mfma(lds_tr_operand<V8>(do_lds, LD, c, dt, r16, g), pf[c],
                                      dv_acc[dt]);
                dk_acc[dt] = TR::mfma(lds_tr_operand<V8>(q_lds, LD, c, dt, r16, g), dsf[c],
                                      dk_acc[dt]);
            }
    }

    if (!kin) return;
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt) {
        const int d = 16 * dt + 4 * g;
        if (d < D) {
            store4<TR>(dk + HR::at(n, h, key, Sk, H) + d, dk_acc[dt] * scale);
            store4<TR>(dv + HR::at(n, h, key, Sk, H) + d, dv_acc[dt]);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Head dims up to 32: a prep launch, a row-owner dQ + dBias launch and a column-owner dK/dV
// launch whose operands all arrive by direct global->LDS loads into static double buffers.
// ---------------------------------------------------------------------------------------------

// Bit j set when byte j of the eight is nonzero.
__device__ __forceinline__ unsigned nonzero_bits8(u32x2 w) {
    unsigned bits = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        bits |= (((w[0] >> (8 * j)) & 0xffu) != 0u ? 1u : 0u) << j;
        bits |= (((w[1] >> (8 * j)) & 0xffu) != 0u ? 1u : 0u) << (4 + j);
    }
    return bits;
}

// Mask bytes of keys kk .. kk+7 of one mask row (0 past Sk; all present without a mask). VEC:
// one 8-byte load (Sk % 8 == 0, 8-byte aligned rows), the address clamped into the row.
template <bool VEC>
__device__ __forceinline__ u32x2 mask_bytes8(const uint8_t* mrow, int kk, int Sk) {
    if (!mrow) return u32x2{~0u, ~0u};
    if constexpr (VEC) {
        return *reinterpret_cast<const u32x2*>(mrow + min(kk, Sk - 8));
    } else {
        uint8_t b[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) b[j] = kk + j < Sk ? mrow[kk + j] : uint8_t(0);
        u32x2 w;
        __builtin_memcpy(&w, b, 8);
        return w;
    }
}

// Tile t (of H * tiles_q * tiles_k) of bias [H][Sq][Sk] -> bias_t [H][Sk][SqP] (SqP = Sq rounded
// up to 64, padding zero), through the 64 x 64 LDS tile `tile`, by threads tid, tid + nthreads,
// ... of the block. Returns after the stores are issued; the caller synchronises before `tile`
// is used again.
template <typename TR>
__device__ void transpose_bias_tile(const typename TR::elem* __restrict__ bias,
                                    typename TR::elem* __restrict__ bias_t,
                                    typename TR::elem (*tile)[72], int t, int Sq, int Sk,
                                    int SqP, int tiles_q, int tiles_k, int tid, int nthreads) {
    using E = typename TR::elem;
    const int tk = t % tiles_k;
    t /= tiles_k;
    const int tq = t % tiles_q, h = t / tiles_q;
    const int q0 = tq * 64, k0 = tk * 64;
    // Loads: 16-byte pieces of 8 keys of one query row when the piece lies inside the row and
    // the rows are 16-byte aligned; element loads otherwise.
    const bool vec = Sk % 8 == 0;
    for (int ch = tid; ch < 512; ch += nthreads) {
        const int r = ch >> 3, c8 = (ch & 7) * 8;  // r: query, c8: first key
        const int qq = q0 + r, kk = k0 + c8;
        E e[8];
        if (vec && qq < Sq && kk + 8 <= Sk) {
            const u32x4 raw = ld16(bias + ((size_t)h * Sq + qq) * Sk + kk);
            __builtin_memcpy(e, &raw, 16);
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                e[j] = (qq < Sq && kk + j < Sk) ? bias[((size_t)h * Sq + qq) * Sk + kk + j]
                                                : E(0.f);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) tile[c8 + j][r] = e[j];
    }
    __syncthreads();
    // Stores: 16-byte pieces of 8 queries of one key row (SqP % 8 == 0 keeps them aligned).
    for (int ch = tid; ch < 512; ch += nthreads) {
        const int r = ch >> 3, c8 = (ch & 7) * 8;  // r: key, c8: first query
        const int kk = k0 + r, qq = q0 + c8;
        if (kk < Sk && qq < SqP)
            st16(bias_t + ((size_t)h * Sk + kk) * SqP + qq,
                 *reinterpret_cast<const u32x4*>(&tile[r][c8]));
    }
}

// One wave's share of a direct-to-LDS tile fill: wave instructions m = w, w + WSTRIDE, ... of a
// tile of ROWS rows of D columns (rows `ld` elements apart, from row r0 of the resource) into a
// swizzled LDS tile, as stage_rows; w is wave-uniform (a scalar), so the instruction count and
// the LDS addresses are scalar too.
template <int D, int ROWS, int WSTRIDE>
__device__ __forceinline__ void stage_rows_wave(Rsrc r, int r0, int ld, char* lds, int w,
                                                int lane) {
    using T = SwzTile<D>;
    constexpr int INSTR = ROWS * T::PL / 64;
    static_assert(ROWS * T::PL % 64 == 0, "tile must be whole wave instructions");
#pragma unroll
    for (int i = 0; i < (INSTR + WSTRIDE - 1) / WSTRIDE; ++i) {
        const int m = w + i * WSTRIDE;
        if (INSTR % WSTRIDE != 0 && m >= INSTR) break;
        const int slot = m * 64 + lane;
        const int row = slot / T::PL;
        const int piece = (slot % T::PL) ^ T::swz(row);
        const int voff = piece < T::P ? (row * ld + piece * 8) * 2 : kPastEnd;
        buf_dma16(r, voff, r0 * ld * 2, lds + m * 64 * 16);
    }
}

// Row owner. A block of 8 waves owns (64 queries, head h, rows n0..n1, key range [kbeg, kend)
// of up to 128*KCW keys). Wave w = 4*qg + kq owns queries 32*qg + 0..31 (two 16-query
// sub-tiles) and the 32-key chunks j = 4*i + kq, i < KCW, of the range. The bias of those
// (query, key) pairs stays in registers for the whole block, and so does their dBias sum over
// the block's rows. Per row n the K/V rows of the range and the Q/dO/O rows of the block's
// queries sit in LDS (row n+1's are loaded directly into the other buffer meanwhile); per chunk
// the wave computes S^T = K.Q^T and dP^T - D = V.dO^T - D (D_i = rowsum(dO*O) enters as the
// accumulator input), dS, and dQ^T += K^T.dS^T. The four key-quarter waves of a query group
// then add their dQ partials through LDS in a fixed order. Also writes lse*log2(e) and -D_i
// per query for the column-owner pass.
template <typename TR, int D, int KCW, bool VEC, int QG, int QTW, bool NSHD>
__global__ __launch_bounds__(256 * QG) void attn_bwd_dq2(
    const typename TR::elem* __restrict__ q, const typename TR::elem* __restrict__ k,
    const typename TR::elem* __restrict__ v, const typename TR::elem* __restrict__ bias,
    const uint8_t* __restrict__ kmask, const typename TR::elem* __restrict__ out,
    const typename TR::elem* __restrict__ dout, const float* __restrict__ lse,
    float* __restrict__ row_logit, unsigned long long* __restrict__ mbits,
    float* __restrict__ lse2_out,
    float* __restrict__ ndi_out, typename TR::elem* __restrict__ dq,
    float* __restrict__ dq_part, float* __restrict__ dbias_dst, int N, int H, int Sq, int Sk,
    int NB, int nranges, float scale, LogitForm lf, typename TR::elem* __restrict__ bias_t,
    int SqP, int tiles_q, int tiles_k) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    using T = SwzTile<D>;
    static_assert(D <= 32, "row-owner kernel holds one 32-dim k-slot group");
    constexpr int KQ = 4, BQ = 16 * QTW * QG, DT = AttnGeom<D>::DT;
    constexpr int NWV = KQ * QG, NT = 64 * NWV;  // waves, threads
    constexpr int RK = KQ * KCW * 32;
    constexpr int KVB = RK * T::ROWB;
    constexpr int QB = BQ * T::ROWB;

    __shared__ __attribute__((aligned(16))) char kv0[2 * KVB];
    __shared__ __attribute__((aligned(16))) char kv1[2 * KVB];
    // Per-row extras staged with Q/dO/O when VEC: lse of the block's 64 queries (256 bytes),
    // then the row's presence words of the key range (RK/64 64-bit words; one wave of 4-byte
    // loads, 256 bytes).
    static_assert(RK % 64 == 0 && RK / 32 <= 64, "presence words of a key range: one wave");
    constexpr int XB = VEC ? 512 : 0;
    __shared__ __attribute__((aligned(16))) char qd0[3 * QB + XB];
    __shared__ __attribute__((aligned(16))) char qd1[3 * QB + XB];
    __shared__ __attribute__((aligned(16))) char xch_raw[NWV * QTW * DT * 64 * 16];
    f32x4* const xch = reinterpret_cast<f32x4*>(xch_raw);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int qg = wave >> 2, kq = wave & 3;
    // The wave index as a scalar: per-wave choices below are scalar branches.
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    // 1-D grid of (query tile, head, key range, row chunk) work items, query tile fastest,
    // placed so that the query tiles that stream the same K/V rows share an XCD's L2.
    const int qtiles = (Sq + BQ - 1) / BQ;
    const int item = xcd_contiguous(blockIdx.x, gridDim.x);
    const int q0 = (item % qtiles) * BQ, h = (item / qtiles) % H;
    const int zr = item / (qtiles * H);
    const int range = zr % nranges, chunk = zr / nranges;
    const int kbeg = range * RK, kend = min(Sk, kbeg + RK);
    const int n0 = chunk * NB, n1 = min(N, n0 + NB);
    int qrow[QTW];
#pragma unroll
    for (int qt = 0; qt < QTW; ++qt) qrow[qt] = q0 + 16 * QTW * qg + 16 * qt + r16;

    // Resident bias in the logit form's units (bias * lf.bscale, float32), laid out as the
    // accumulator input of S^T: chunk i, sub-tile qt, half t -> keys kbeg + 32j + 8g + 4t + 0..3
    // of query qrow[qt] (j = i*KQ + kq). The S^T product then yields the logit up to the factor
    // lf.cexp, and no per-row instruction touches the bias.
    f32x4 bacc[KCW][QTW][2];
#pragma unroll
    for (int i = 0; i < KCW; ++i)
#pragma unroll
        for (int qt = 0; qt < QTW; ++qt) {
            const int kk = kbeg + 32 * (i * KQ + kq) + 8 * g;
            const E* brow = bias + ((size_t)h * Sq + min(qrow[qt], Sq - 1)) * Sk;
            float b[8];
            if constexpr (VEC) {
                unpack8<TR>(ld16(brow + min(kk, Sk - 8)), b);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) b[j] = kk + j < Sk ? TR::to_f(brow[kk + j]) : 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) bacc[i][qt][j >> 2][j & 3] = lf.bias_units(b[j]);
        }

    // Keys absent from every row of the block, or past Sk: bit 8i + j of the lane's keys
    // kbeg + 32(i*KQ + kq) + 8g + j (the rows' presence is ORed in below). Their resident bias
    // becomes an infinity of the sign of lf.cexp's inverse (-inf for a positive scale), so
    // S^T * lf.cexp is -inf there and P is 0 without any per-score instruction.
    unsigned cabs = 0;
#pragma unroll
    for (int i = 0; i < KCW; ++i) {
        const int lim = Sk - (kbeg + 32 * (i * KQ + kq) + 8 * g);
        cabs |= (lim >= 8 ? 0u : lim <= 0 ? 0xffu : (0xffu << lim) & 0xffu) << (8 * i);
    }

    // The two halves of the 16 x 32 identity [I | 0], [0 | I] as MFMA A operands: with dS^T as
    // the B operand, the product adds dS of keys 16t + 0..15 (rows) of every query (column) to
    // the accumulator, so the dBias sums run on the matrix core.
    V8 eye[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) eye[t][j] = TR::from_f(8 * g + j == r16 + 16 * t ? 1.f : 0.f);
    // dBias of chunk i, sub-tile qt, half t: keys kbeg + 32j + 16t + 4g + 0..3 of query qrow[qt].
    f32x4 dbias[KCW][QTW][2];
#pragma unroll
    for (int i = 0; i < KCW; ++i)
#pragma unroll
        for (int qt = 0; qt < QTW; ++qt)
#pragma unroll
            for (int t = 0; t < 2; ++t) dbias[i][qt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Row n's operands into (kv, qd) by direct-to-LDS loads, in three parts issued between the
    // chunks of the row before (so the vector memory path drains while the block computes):
    // part 0 the K rows of the key range, part 1 the V rows (both over all waves), part 2 the
    // Q and O rows (first half of the waves), the dO rows and the per-row extras (second half).
    auto stage_part = [&](int part, int n, char* kv, char* qd) __attribute__((always_inline)) {
        using HR = HeadRows<D, NSHD>;
        const int ld = HR::ld(H);
        if (part < 2) {
            const Rsrc r = buffer_rsrc((part == 0 ? k : v) + HR::at(n, h, 0, Sk, H),
                                       HR::bytes(Sk, H));
            stage_rows_wave<D, RK, NWV>(r, kbeg, ld, kv + part * KVB, wv, lane);
            return;
        }
        const size_t qo = HR::at(n, h, 0, Sq, H);
        const uint32_t qb = HR::bytes(Sq, H);
        constexpr int HW = NWV / 2;
        if (wv < HW) {
            stage_rows_wave<D, BQ, HW>(buffer_rsrc(q + qo, qb), q0, ld, qd, wv, lane);
            stage_rows_wave<D, BQ, HW>(buffer_rsrc(out + qo, qb), q0, ld, qd + 2 * QB, wv, lane);
        } else {
            stage_rows_wave<D, BQ, HW>(buffer_rsrc(dout + qo, qb), q0, ld, qd + QB, wv - HW,
                                       lane);
            if constexpr (VEC) {
                // Queries past Sq and keys past Sk read zeros. Mask rows are 8-byte aligned.
                char* ex = qd + 3 * QB;
                const size_t nh = (size_t)n * H + h;
                if (wv == HW)
                    buf_dma4(buffer_rsrc(lse + nh * Sq, (uint32_t)Sq * 4), lane * 4, q0 * 4, ex);
                // Words kbeg/64 .. of the row's presence bits (kbeg % 64 == 0); words past the
                // row read zeros.
                const int words = (Sk + 63) >> 6;
                if (kmask && wv == HW + 1)
                    buf_dma4(buffer_rsrc(mbits + (size_t)n * words, (uint32_t)words * 8),
                             lane * 4, (kbeg >> 6) * 8, ex + 256);
            }
        }
    };
    // Per-row values kept in registers one row ahead when they are not staged (not VEC), raw:
    // anything computed from them right after the load would wait for the row's direct-to-LDS
    // loads too.
    float lse_nx[VEC ? 1 : QTW], ml_nx = kMaskedLogit;
    u32x2 mask_nx[VEC ? 1 : KCW];
    auto prefetch = [&](int n) {
        if constexpr (!VEC) {
            const size_t nh = (size_t)n * H + h;
#pragma unroll
            for (int qt = 0; qt < QTW; ++qt) lse_nx[qt] = lse[nh * Sq + min(qrow[qt], Sq - 1)];
            const uint8_t* mrow = kmask ? kmask + (size_t)n * Sk : nullptr;
#pragma unroll
            for (int i = 0; i < KCW; ++i)
                mask_nx[i] = mask_bytes8<VEC>(mrow, kbeg + 32 * (i * KQ + kq) + 8 * g, Sk);
        }
        ml_nx = kmask ? row_logit[n] : kMaskedLogit;
    };

    // dQ of the last row (this wave's slice), stored at the start of the next step by the waves
    // kq < QTW * DT: sub-tile dqt, head dims dd .. dd+3 of query qrow[dqt], at element offset
    // dq_off of the (n, h) slice, by the lanes with dq_ok.
    const int dqt = min(kq / DT, QTW - 1), dd = 16 * (kq % DT) + 4 * g;
    const bool dq_ok = qrow[dqt] < Sq && dd < D;
    const int dq_off = qrow[dqt] * HeadRows<D, NSHD>::ld(H) + dd;
    f32x4 pend_dq = {0.f, 0.f, 0.f, 0.f};
    auto flush_dq = [&](int pn) __attribute__((always_inline)) {
        if (pn < 0 || wv % KQ >= QTW * DT || !dq_ok) return;
        using HR = HeadRows<D, NSHD>;
        const size_t at = HR::at(pn, h, 0, Sq, H);
        if (nranges == 1) {
            const Rsrc r = buffer_rsrc(dq + at, HR::bytes(Sq, H));
            E e[4] = {TR::from_f(pend_dq[0]), TR::from_f(pend_dq[1]), TR::from_f(pend_dq[2]),
                      TR::from_f(pend_dq[3])};
            u32x2 w;
            __builtin_memcpy(&w, e, 8);
            __builtin_amdgcn_raw_buffer_store_b64(w, r, dq_off * 2, 0, 0);
        } else {  // range's partial, in dq's layout
            const Rsrc r = buffer_rsrc(dq_part + (size_t)range * N * H * Sq * D + at,
                                       HR::bytes(Sq, H) * 2);
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, pend_dq), r,
                                                   dq_off * 4, 0, 0);
        }
    };
    // lse2_out / ndi_out: stored by the lanes g == 0 of the waves kq == 0 of key range 0.
    int ls_off[QTW];
#pragma unroll
    for (int qt = 0; qt < QTW; ++qt)
        ls_off[qt] = range == 0 && g == 0 && qrow[qt] < Sq ? qrow[qt] * 4 : kPastEnd;

    // One row step; `rows_tag` says how the block's rows are masked (kRowsClean, kRowsEmpty,
    // kRowsMixed, below).
    auto step = [&](int n, const char* kvc, const char* qdc, char* kvn, char* qdn,
                    auto rows_tag) __attribute__((always_inline)) {
        constexpr int ROWS = decltype(rows_tag)::value;
        const size_t nh = (size_t)n * H + h;
        const bool more = n + 1 < n1;  // block-uniform: stage row n+1 during this step
        async_wait();
        __syncthreads();  // row n in (kvc, qdc); every wave is done with row n-1
        float lse2c[QTW];
        const float mlc = ml_nx;
        // Presence bits of this wave's keys: chunk i in bits 8i .. 8i+7 (one register).
        unsigned vbits = 0;
        if constexpr (VEC) {
            const char* ex = qdc + 3 * QB;
#pragma unroll
            for (int qt = 0; qt < QTW; ++qt) {
                // Read in every lane (queries past Sq read the staged zeros), then selected.
                const float l = reinterpret_cast<const float*>(ex)[16 * QTW * qg + 16 * qt + r16];
                lse2c[qt] = qrow[qt] < Sq ? l * kLog2e : INFINITY;
            }
            if (kmask) {
                // Chunk i's 32 keys start at bit rel % 64 of staged word rel / 64 (rel = key
                // offset in the range, a multiple of 32); the lane's 8 keys are bits 8g .. 8g+7
                // of that. The word's address is the same in every lane (an LDS broadcast).
                const unsigned long long* wd =
                    reinterpret_cast<const unsigned long long*>(ex + 256);
#pragma unroll
                for (int i = 0; i < KCW; ++i) {
                    const int rel = 32 * (i * KQ + kq);
                    const unsigned w32 = (unsigned)(wd[rel >> 6] >> (rel & 32));
                    vbits |= ((w32 >> (8 * g)) & 0xffu) << (8 * i);
                }
            } else {
                vbits = 0xffffffu;
            }
        } else {
#pragma unroll
            for (int qt = 0; qt < QTW; ++qt)
                lse2c[qt] = qrow[qt] < Sq ? lse_nx[qt] * kLog2e : INFINITY;
#pragma unroll
            for (int i = 0; i < KCW; ++i) vbits |= nonzero_bits8(mask_nx[i]) << (8 * i);
        }

        V8 qf[QTW], dof[QTW];
        float di[QTW];
#pragma unroll
        for (int qt = 0; qt < QTW; ++qt) {
            const int row = 16 * QTW * qg + 16 * qt + r16;
            qf[qt] = swz_row_operand<V8, D>(qdc, row, 0, g);
            if (lf.qzero) qf[qt] = V8{};
            dof[qt] = swz_row_operand<V8, D>(qdc + QB, row, 0, g);
            const V8 of = swz_row_operand<V8, D>(qdc + 2 * QB, row, 0, g);
            // Packed pair dot products: the element products are exact in float32.
            u32x4 dw, ow;
            __builtin_memcpy(&dw, &dof[qt], 16);
            __builtin_memcpy(&ow, &of, 16);
            float part = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) part = dot2<TR>(dw[j], ow[j], part);
            di[qt] = xgroup_sum(part);
        }
        if (wv % KQ == 0) {
            const Rsrc rl = buffer_rsrc(lse2_out + nh * Sq, (uint32_t)Sq * 4);
            const Rsrc rn = buffer_rsrc(ndi_out + nh * Sq, (uint32_t)Sq * 4);
#pragma unroll
            for (int qt = 0; qt < QTW; ++qt) {
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lse2c[qt]), rl, ls_off[qt],
                                                      0, 0);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(-di[qt]), rn, ls_off[qt],
                                                      0, 0);
            }
        }
        // The stores of this row and the last go out before row n+1's loads are issued, so the
        // next barrier's wait for those loads finds them long written.
        flush_dq(n > n0 ? n - 1 : -1);

        f32x4 ndi4[QTW];
#pragma unroll
        for (int qt = 0; qt < QTW; ++qt) ndi4[qt] = f32x4{-di[qt], -di[qt], -di[qt], -di[qt]};
        f32x4 dqa[QTW][DT];
#pragma unroll
        for (int qt = 0; qt < QTW; ++qt)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) dqa[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};

        // The wave's 32-key chunks: S^T and dP^T - D by MFMA, P, dS, the dBias sums, and
        // dQ^T += K^T.dS^T. CHUNKS: kChunksClean (every key present, or absent from every row of
        // the block: resident bias -inf, so P = 0 there without any per-score instruction),
        // kChunksSelect (absent keys take the row's masked logit by per-score selects, in the
        // chunks that have one), kChunksEmpty (a row without any present key: every logit is the
        // masked logit 0, so P = exp2(-lse*log2e) for every key and no S is needed). Each
        // version's chunks are straight-line code apart from kChunksSelect's test: a branch
        // between the MFMAs and the exponentials of a chunk, or between chunks, keeps the
        // scheduler from overlapping them.
        auto chunks = [&](auto chunks_tag) __attribute__((always_inline)) {
            constexpr int CHUNKS = decltype(chunks_tag)::value;
            // An absent key's log2(P): its row's masked logit, in the same units.
            float mx[QTW];
#pragma unroll
            for (int qt = 0; qt < QTW; ++qt) mx[qt] = fmaf(mlc, kLog2e, -lse2c[qt]);
            float pe[QTW];  // kChunksEmpty: the one P of the row's queries
            if constexpr (CHUNKS == kChunksEmpty) {
#pragma unroll
                for (int qt = 0; qt < QTW; ++qt) pe[qt] = fast_exp2(mx[qt]);
            }
#pragma unroll
            for (int i = 0; i < KCW; ++i) {
                const int c0 = 32 * (i * KQ + kq);  // chunk's first key, relative to kbeg
                V8 kf[2], vf[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int row = c0 + 8 * (r16 >> 2) + 4 * t + (r16 & 3);
                    if constexpr (CHUNKS != kChunksEmpty)
                        kf[t] = swz_row_operand<V8, D>(kvc, row, 0, g);
                    vf[t] = swz_row_operand<V8, D>(kvc + KVB, row, 0, g);
                }
                f32x4 s[QTW][2], dp[QTW][2];
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int qt = 0; qt < QTW; ++qt) {
                        if constexpr (CHUNKS != kChunksEmpty)
                            s[qt][t] = TR::mfma(kf[t], qf[qt], bacc[i][qt][t]);
                        dp[qt][t] = TR::mfma(vf[t], dof[qt], ndi4[qt]);
                    }
                // Row n+1's loads, a third after each chunk's first MFMAs.
                if (more) {
#pragma unroll
                    for (int part = i * 3 / KCW; part < (i + 1) * 3 / KCW; ++part)
                        stage_part(part, n + 1, kvn, qdn);
                    if (i == KCW - 1) prefetch(n + 1);
                }
                // The chunk's VALU work (exponentials, dS, the dBias sums) runs at a raised wave
                // priority until its dQ MFMAs are issued: the other wave on the SIMD then gets
                // the issue slots while this one waits on its S and dP MFMAs.
                __builtin_amdgcn_s_setprio(1);
                // x = log2(P) = logit * log2(e) - lse * log2(e), one FMA per score.
                float x[QTW][8];
                if constexpr (CHUNKS != kChunksEmpty) {
#pragma unroll
                    for (int qt = 0; qt < QTW; ++qt)
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            x[qt][j] = fmaf(s[qt][j >> 2][j & 3], lf.cexp, -lse2c[qt]);
                }
                if constexpr (CHUNKS == kChunksSelect) {
                    // The selects, for a chunk with a key absent in this row but present in
                    // another row of the block, or in a row with no present key (wave-uniform).
                    // Bit j of `valid` spread over a word (0 or ~0) selects x or mx bitwise. Keys
                    // past Sk have no valid bit: in a row with a present key their P is 0; in a
                    // row without one, P = exp2(-lse2) as for the absent keys in range, which is
                    // harmless: their K rows are staged as zeros and their dBias is never stored.
                    const unsigned valid = (vbits >> (8 * i)) & 0xffu;
                    if (mlc == 0.f || __any((valid | ((cabs >> (8 * i)) & 0xffu)) != 0xffu)) {
                        // Opaque to speculation: nothing of it is hoisted onto the unmasked path.
                        asm volatile("");
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const int sel = __builtin_amdgcn_sbfe((int)valid, j, 1);
#pragma unroll
                            for (int qt = 0; qt < QTW; ++qt)
                                x[qt][j] = __int_as_float((sel & __float_as_int(x[qt][j])) |
                                                          (~sel & __float_as_int(mx[qt])));
                        }
                    }
                }
                V8 dsf[QTW];
#pragma unroll
                for (int qt = 0; qt < QTW; ++qt)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        // (Keys past Sk get pe too in kChunksEmpty, harmless as above.)
                        const float p = CHUNKS == kChunksEmpty ? pe[qt] : fast_exp2(x[qt][j]);
                        dsf[qt][j] = TR::from_f(p * dp[qt][j >> 2][j & 3]);
                    }
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const V8 kt = swz_tr_operand<V8, D>(kvc, c0, dt, r16, g);
#pragma unroll
                    for (int qt = 0; qt < QTW; ++qt)
                        dqa[qt][dt] = TR::mfma(kt, dsf[qt], dqa[qt][dt]);
                }
#pragma unroll
                for (int qt = 0; qt < QTW; ++qt)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
                        dbias[i][qt][t] = TR::mfma(eye[t], dsf[qt], dbias[i][qt][t]);
                __builtin_amdgcn_s_setprio(0);
            }
        };
        if constexpr (ROWS == kRowsMixed) {
            chunks(std::integral_constant<int, kChunksSelect>{});
        } else if constexpr (ROWS == kRowsEmpty) {
            if (mlc == 0.f)  // block-uniform: the row has no present key
                chunks(std::integral_constant<int, kChunksEmpty>{});
            else
                chunks(std::integral_constant<int, kChunksClean>{});
        } else {
            chunks(std::integral_constant<int, kChunksClean>{});
        }

#pragma unroll
        for (int qt = 0; qt < QTW; ++qt)
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                xch[((wave * QTW + qt) * DT + dt) * 64 + lane] = dqa[qt][dt];
        lds_barrier();  // the exchange is LDS only
        if (kq < QTW * DT) {
            const int qt = kq / DT, dt = kq % DT;
            f32x4 acc = xch[(((qg * 4) * QTW + qt) * DT + dt) * 64 + lane];
#pragma unroll
            for (int w = 1; w < 4; ++w)
                acc += xch[(((qg * 4 + w) * QTW + qt) * DT + dt) * 64 + lane];
            pend_dq = acc * scale;
        }
    };

    // How the block's rows are masked (set below when a mask is given): kRowsClean (every key
    // is present in all rows or in none), kRowsEmpty (that, apart from rows with no present key),
    // kRowsMixed (some key present in some rows with a present key and absent in others).
    int block_rows = kRowsClean;

    // Work of the column-owner pass that would otherwise take a kernel of its own: the
    // transposed bias (one 64 x 64 tile per block, through the dQ exchange buffer, which is
    // idle until the first row ends) and the logit of the absent keys of this block's rows
    // (-1e9, or 0 when a row has no present key; every block covering the rows writes the same
    // values).
    {
        const int ttiles = H * tiles_q * tiles_k;
        for (int t = blockIdx.x; t < ttiles; t += gridDim.x) {
            static_assert(sizeof(xch_raw) >= 64 * 72 * sizeof(E), "transpose tile fits");
            transpose_bias_tile<TR>(bias, bias_t, reinterpret_cast<E(*)[72]>(xch_raw), t, Sq, Sk,
                                    SqP, tiles_q, tiles_k, threadIdx.x, NT);
            __syncthreads();
        }
        if (kmask) {
            // Also each row's presence bits, 64 keys per word (bit j of word i: key 64i + j is
            // present), read by the row steps in place of the mask bytes (VEC); and, lane w
            // holding word kbeg/64 + w of the key range, their OR and AND over this wave's rows.
            const int words = (Sk + 63) >> 6;
            unsigned long long seen = 0ull, always = ~0ull;
            bool empty_row = false;
            for (int nr = n0 + wave; nr < n1; nr += NWV) {
                const uint8_t* m = kmask + (size_t)nr * Sk;
                bool any = false;
                if constexpr (VEC) {
                    unsigned long long mine = 0ull;  // this lane's word of the row
                    for (int i = 0; i < words; ++i) {
                        const int kk = 64 * i + lane;
                        const unsigned long long b = __ballot(kk < Sk && m[kk] != 0);
                        any |= b != 0ull;
                        if (lane == 0) mbits[(size_t)nr * words + i] = b;
                        if (lane == i - (kbeg >> 6)) mine = b;
                    }
                    if (any) {  // rows with a present key only
                        seen |= mine;
                        always &= mine;
                    }
                } else {
                    for (int i = lane; i < Sk; i += 64) any |= m[i] != 0;
                    any = __any(any);
                }
                empty_row |= !any;
                if (lane == 0) row_logit[nr] = any ? kMaskedLogit : 0.f;
            }
            if constexpr (VEC) {
                // The waves' words combined through the second Q/dO/O buffer (idle until the
                // first row step stages row n0 + 1): the keys present in no row of the block
                // (their bias becomes -inf), whether every key of the range is present in all
                // rows that have a present key or in none of them, and whether a row has none.
                constexpr int NWD = RK / 64;
                unsigned long long* orw = reinterpret_cast<unsigned long long*>(qd1);
                unsigned long long* andw = orw + NWV * NWD;
                int* emptyw = reinterpret_cast<int*>(andw + NWV * NWD);
                static_assert(sizeof(qd1) >= 2 * NWV * NWD * 8 + NWV * 4, "presence words fit");
                if (lane < NWD) {
                    orw[wave * NWD + lane] = seen;
                    andw[wave * NWD + lane] = always;
                }
                if (lane == 0) emptyw[wave] = empty_row ? 1 : 0;
                __syncthreads();
#pragma unroll
                for (int i = 0; i < KCW; ++i) {
                    const int rel = 32 * (i * KQ + kq);
                    unsigned long long w = 0ull;
#pragma unroll
                    for (int ww = 0; ww < NWV; ++ww) w |= orw[ww * NWD + (rel >> 6)];
                    const unsigned bits = (unsigned)(w >> ((rel & 32) + 8 * g)) & 0xffu;
                    cabs |= (~bits & 0xffu) << (8 * i);
                }
                bool mixed = false;
                if (lane < NWD) {
                    unsigned long long o = 0ull, a = ~0ull;
#pragma unroll
                    for (int ww = 0; ww < NWV; ++ww) {
                        o |= orw[ww * NWD + lane];
                        a &= andw[ww * NWD + lane];
                    }
                    const int lim = kend - (kbeg + 64 * lane);  // keys of the word in range
                    const unsigned long long inr = lim >= 64 ? ~0ull : lim <= 0 ? 0ull
                                                                      : (1ull << lim) - 1ull;
                    mixed = ((o ^ a) & inr) != 0ull;
                }
                bool empty = false;
#pragma unroll
                for (int ww = 0; ww < NWV; ++ww) empty |= emptyw[ww] != 0;
                block_rows = __any(mixed) ? kRowsMixed : empty ? kRowsEmpty : kRowsClean;
            } else {
                block_rows = kRowsMixed;
            }
            __syncthreads();  // this block's prefetches read them; the combined words are read
        }
    }
    const float absent_bias = lf.cexp > 0.f ? -INFINITY : INFINITY;
#pragma unroll
    for (int i = 0; i < KCW; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int sel = __builtin_amdgcn_sbfe((int)cabs, 8 * i + j, 1);
#pragma unroll
            for (int qt = 0; qt < QTW; ++qt) {
                const float b = bacc[i][qt][j >> 2][j & 3];
                bacc[i][qt][j >> 2][j & 3] =
                    __int_as_float((~sel & __float_as_int(b)) | (sel & __float_as_int(absent_bias)));
            }
        }

    if (n0 < n1) {
#pragma unroll
        for (int part = 0; part < 3; ++part) stage_part(part, n0, kv0, qd0);
        prefetch(n0);
    }
    auto rows = [&](auto masked_tag) __attribute__((always_inline)) {
        for (int n = n0; n < n1; n += 2) {
            step(n, kv0, qd0, kv1, qd1, masked_tag);
            if (n + 1 < n1) step(n + 1, kv1, qd1, kv0, qd0, masked_tag);
        }
    };
    if (block_rows == kRowsMixed)
        rows(std::integral_constant<int, kRowsMixed>{});
    else if (block_rows == kRowsEmpty)
        rows(std::integral_constant<int, kRowsEmpty>{});
    else
        rows(std::integral_constant<int, kRowsClean>{});
    flush_dq(n1 > n0 ? n1 - 1 : -1);

#pragma unroll
    for (int i = 0; i < KCW; ++i) {
        if (kbeg + 32 * (i * KQ + kq) >= kend) continue;
#pragma unroll
        for (int qt = 0; qt < QTW; ++qt) {
            if (qrow[qt] >= Sq) continue;
            float* drow = dbias_dst + (((size_t)chunk * H + h) * Sq + qrow[qt]) * Sk;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int kk = kbeg + 32 * (i * KQ + kq) + 16 * t + 4 * g;
                if (VEC) {
                    // kk % 4 == Sk % 4 == 0, so kk < Sk means kk + 4 <= Sk
                    if (kk < Sk) *reinterpret_cast<f32x4*>(drow + kk) = dbias[i][qt][t];
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (kk + j < Sk) drow[kk + j] = dbias[i][qt][t][j];
                }
            }
        }
    }
}

// out[i] = part[i] + part[count4 + i] + ... over nparts slices of count4 16-byte vectors, added
// in slice order 0, 1, 2, ... with four slices in flight; block blk of nblk, NT threads a block.
__device__ __forceinline__ void sum_slices(const f32x4* __restrict__ part, size_t count4,
                                           int nparts, f32x4* __restrict__ out, int blk, int nblk,
                                           int tid, int NT) {
    for (size_t i = (size_t)blk * NT + tid; i < count4; i += (size_t)nblk * NT) {
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
        int p = 0;
        for (; p + 4 <= nparts; p += 4) {
            const f32x4 v0 = part[(size_t)p * count4 + i];
            const f32x4 v1 = part[(size_t)(p + 1) * count4 + i];
            const f32x4 v2 = part[(size_t)(p + 2) * count4 + i];
            const f32x4 v3 = part[(size_t)(p + 3) * count4 + i];
            a += v0;
            a += v1;
            a += v2;
            a += v3;
        }
        for (; p < nparts; ++p) a += part[(size_t)p * count4 + i];
        out[i] = a;
    }
}

// Column owner. A block of NW waves owns (16*KSUB*NW keys, head h, row n); wave w owns keys
// k0 + 16*KSUB*w + 0..16*KSUB-1 with K and V held as MFMA B operands. The queries stream in
// 64-row tiles: Q, dO, the transposed bias tile and lse*log2(e), -D_i arrive by direct
// global->LDS loads into the other buffer while the current tile is computed (one barrier per
// tile). Per 32-query chunk: S = Q.K^T and dP - D = dO.V^T with the queries permuted so that P
// and dS are directly the B operands of dV^T += dO^T.P and dK^T += Q^T.dS.
template <typename TR, int D, int KSUB, int NW, bool VEC, bool NSHD>
__global__ __launch_bounds__(64 * NW) void attn_bwd_dkv2(
    const typename TR::elem* __restrict__ q, const typename TR::elem* __restrict__ k,
    const typename TR::elem* __restrict__ v, const typename TR::elem* __restrict__ bias_t,
    const uint8_t* __restrict__ kmask, const typename TR::elem* __restrict__ dout,
    const float* __restrict__ lse2, const float* __restrict__ ndi,
    const float* __restrict__ row_logit, typename TR::elem* __restrict__ dk,
    typename TR::elem* __restrict__ dv, int H, int Sq, int Sk, int SqP, float scale,
    int main_blocks, const f32x4* __restrict__ dbias_part, f32x4* __restrict__ dbias,
    size_t dbias_count4, int dbias_parts) {
    using V8 = typename TR::vec8;
    using T = SwzTile<D>;
    static_assert(D <= 32, "column-owner kernel holds one 32-dim k-slot group");
    if ((int)blockIdx.x >= main_blocks) {
        // Blocks past the work items sum the row-owner pass's dBias slices (written by the
        // kernel before this one): they start as the work items run out, in the grid's tail.
        sum_slices(dbias_part, dbias_count4, dbias_parts, dbias, (int)blockIdx.x - main_blocks,
                   (int)gridDim.x - main_blocks, threadIdx.x, 64 * NW);
        return;
    }
    constexpr int DT = AttnGeom<D>::DT;
    constexpr int KW = 16 * KSUB, KB = NW * KW, NT = 64 * NW;
    constexpr int QB = 64 * T::ROWB;
    constexpr int BTB = KB * 128;  // bias^T tile: KB key rows of 64 queries

    __shared__ __attribute__((aligned(16))) char qd0[2 * QB];
    __shared__ __attribute__((aligned(16))) char qd1[2 * QB];
    __shared__ __attribute__((aligned(16))) char bt0[BTB];
    __shared__ __attribute__((aligned(16))) char bt1[BTB];
    __shared__ __attribute__((aligned(16))) float st0[128];
    __shared__ __attribute__((aligned(16))) float st1[128];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    // 1-D grid of (key block, head, row) work items, key block fastest, placed so that the key
    // blocks of one (row, head) -- which stream the same Q and dO rows -- share an XCD's L2.
    const int kblocks = (Sk + KB - 1) / KB;
    const int item = xcd_contiguous(blockIdx.x, main_blocks);
    const int k0 = (item % kblocks) * KB, h = (item / kblocks) % H, n = item / (kblocks * H);
    const size_t nh = (size_t)n * H + h;
    using HR = HeadRows<D, NSHD>;
    const int kw0 = k0 + wave * KW;

    // In a row with a present key an absent key's P is 0, so its dK and dV are 0: its lane (one
    // key per lane column of every product) computes without selects and stores zeros. Only a
    // row without any present key needs the masked logit in place of the logit.
    const float ml = kmask ? row_logit[n] : kMaskedLogit;
    V8 kf[KSUB], vf[KSUB];
    bool present[KSUB], none_present = true;
    float absent_logit[KSUB];
#pragma unroll
    for (int s = 0; s < KSUB; ++s) {
        const int key = kw0 + 16 * s + r16;
        const bool kin = key < Sk;
        u32x4 rk = {0u, 0u, 0u, 0u}, rv = {0u, 0u, 0u, 0u};
        if (kin && 8 * g < D) {
            rk = ld16(k + HR::at(n, h, key, Sk, H) + 8 * g);
            rv = ld16(v + HR::at(n, h, key, Sk, H) + 8 * g);
        }
        kf[s] = bits_as<V8>(rk);
        vf[s] = bits_as<V8>(rv);
        present[s] = kin && (kmask == nullptr || kmask[(size_t)n * Sk + key] != 0);
        absent_logit[s] = kin ? ml : -INFINITY;
        none_present = none_present && !__any(present[s]);
    }
    // Wave-uniform: every key of the wave is past Sk, or absent in a row with a present key.
    const bool active = kw0 < Sk && !(ml != 0.f && none_present);

    f32x4 dka[KSUB][DT], dva[KSUB][DT];
#pragma unroll
    for (int s = 0; s < KSUB; ++s)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            dka[s][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
            dva[s][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }

    const uint32_t qbytes = HR::bytes(Sq, H);
    const Rsrc rq = buffer_rsrc(q + HR::at(n, h, 0, Sq, H), qbytes);
    const Rsrc rdo = buffer_rsrc(dout + HR::at(n, h, 0, Sq, H), qbytes);
    // The block's transposed-bias rows (keys k0 .. k0+KB-1 that exist) and the two per-query
    // vectors of (n, h).
    const Rsrc rbt = buffer_rsrc(bias_t + ((size_t)h * Sk + k0) * SqP,
                                 (uint32_t)(min(KB, Sk - k0) * SqP * 2));
    const Rsrc rl = buffer_rsrc(lse2 + nh * Sq, (uint32_t)Sq * 4);
    const Rsrc rn = buffer_rsrc(ndi + nh * Sq, (uint32_t)Sq * 4);
    auto stage = [&](int qs, char* qd, char* bt, float* st) {
        stage_head_rows<D, 64, NT, NSHD>(rq, qs, H, qd);
        stage_head_rows<D, 64, NT, NSHD>(rdo, qs, H, qd + QB);
        // bias^T rows k0 .. k0+KB-1, eight 16-byte pieces of 8 queries each, piece p of row r
        // at position p ^ (r & 7). Keys past Sk read zeros; SqP is a multiple of 64, so a tile
        // never runs past its row.
#pragma unroll
        for (int b = wave * 64; b < KB * 8; b += NT) {
            const int slot = b + lane;
            const int row = slot >> 3, piece = (slot & 7) ^ (row & 7);
            buf_dma16(rbt, (row * SqP + 8 * piece) * 2, qs * 2, bt + b * 16);
        }
        if (wave == 0) {  // queries past Sq read zeros
            buf_dma4(rl, lane * 4, qs * 4, reinterpret_cast<char*>(st));
            buf_dma4(rn, lane * 4, qs * 4, reinterpret_cast<char*>(st + 64));
        }
    };

    // EMPTY: the row has no present key, so every logit in range is the masked logit 0 and no
    // S is needed. Otherwise absent keys' lanes compute without selects (and store zeros).
    // Either version is straight-line code.
    auto compute = [&](const char* qd, const char* bt, const float* st, auto empty_tag)
                       __attribute__((always_inline)) {
        constexpr bool EMPTY = decltype(empty_tag)::value;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            V8 qa[2], da[2];
            f32x4 l4[2], n4[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int row = 32 * c + 8 * (r16 >> 2) + 4 * t + (r16 & 3);
                qa[t] = swz_row_operand<V8, D>(qd, row, 0, g);
                da[t] = swz_row_operand<V8, D>(qd + QB, row, 0, g);
                l4[t] = *reinterpret_cast<const f32x4*>(st + 32 * c + 8 * g + 4 * t);
                n4[t] = *reinterpret_cast<const f32x4*>(st + 64 + 32 * c + 8 * g + 4 * t);
            }
            V8 doT[DT], qT[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                doT[dt] = swz_tr_operand<V8, D>(qd + QB, 32 * c, dt, r16, g);
                qT[dt] = swz_tr_operand<V8, D>(qd, 32 * c, dt, r16, g);
            }
#pragma unroll
            for (int s = 0; s < KSUB; ++s) {
                f32x4 S[2], dP[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    if constexpr (!EMPTY) S[t] = TR::mfma(qa[t], kf[s], f32x4{0.f, 0.f, 0.f, 0.f});
                    dP[t] = TR::mfma(da[t], vf[s], n4[t]);
                }
                float x[8];
                if constexpr (EMPTY) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) x[j] = absent_logit[s];
                } else {
                    const int row = wave * KW + 16 * s + r16;
                    float b[8];
                    unpack8<TR>(*reinterpret_cast<const u32x4*>(
                                    bt + row * 128 + 16 * ((4 * c + g) ^ (row & 7))),
                                b);
#pragma unroll
                    for (int j = 0; j < 8; ++j) x[j] = fmaf(S[j >> 2][j & 3], scale, b[j]);
                }
                V8 pf, dsf;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int t = j >> 2, e = j & 3;
                    const float p = fast_exp2(fmaf(x[j], kLog2e, -l4[t][e]));
                    const float ds = p * dP[t][e];
                    pf[j] = TR::from_f(p);
                    dsf[j] = TR::from_f(ds);
                }
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    dva[s][dt] = TR::mfma(doT[dt], pf, dva[s][dt]);
                    dka[s][dt] = TR::mfma(qT[dt], dsf, dka[s][dt]);
                }
            }
        }
    };

    const int ntq = (Sq + 63) / 64;
    if (ntq > 0) stage(0, qd0, bt0, st0);
    auto tiles = [&](auto empty_tag) __attribute__((always_inline)) {
        for (int it = 0; it < ntq; it += 2) {
            async_wait();
            __syncthreads();
            if (it + 1 < ntq) stage(64 * (it + 1), qd1, bt1, st1);
            if (active) compute(qd0, bt0, st0, empty_tag);
            if (it + 1 < ntq) {
                async_wait();
                __syncthreads();
                if (it + 2 < ntq) stage(64 * (it + 2), qd0, bt0, st0);
                if (active) compute(qd1, bt1, st1, empty_tag);
            }
        }
    };
    if (ml == 0.f)  // block-uniform: the row has no present key
        tiles(std::true_type{});
    else
        tiles(std::false_type{});

#pragma unroll
    for (int s = 0; s < KSUB; ++s) {
        const int key = kw0 + 16 * s + r16;
        if (key >= Sk) continue;
        const bool zero = !present[s] && ml != 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int d = 16 * dt + 4 * g;
            if (d < D) {
                const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                store4<TR>(dk + HR::at(n, h, key, Sk, H) + d, zero ? z : dka[s][dt] * scale);
                store4<TR>(dv + HR::at(n, h, key, Sk, H) + d, zero ? z : dva[s][dt]);
            }
        }
    }
}

// out[i] = sum over p = 0..nparts-1 (in order) of part[p*count + i]; nparts = 0 writes zeros.
__global__ __launch_bounds__(256) void sum_partials_f32(const float* __restrict__ part,
                                                        size_t count, int nparts,
                                                        float* __restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count;
         i += (size_t)gridDim.x * 256) {
        float a = 0.f;
        for (int p = 0; p < nparts; ++p) a += part[(size_t)p * count + i];
        out[i] = a;
    }
}

// The same sum four elements at a time (count4 = count / 4, 16-byte aligned arrays).
__global__ __launch_bounds__(256) void sum_partials_f32x4(const f32x4* __restrict__ part,
                                                          size_t count4, int nparts,
                                                          f32x4* __restrict__ out) {
    sum_slices(part, count4, nparts, out, blockIdx.x, gridDim.x, threadIdx.x, 256);
}

template <typename TR>
__global__ __launch_bounds__(256) void sum_partials_cast(const float* __restrict__ part,
                                                         size_t count, int nparts,
                                                         typename TR::elem* __restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < count;
         i += (size_t)gridDim.x * 256) {
        float a = 0.f;
        for (int p = 0; p < nparts; ++p) a += part[(size_t)p * count + i];
        out[i] = TR::from_f(a);
    }
}

int grid_for(size_t count) {
    const size_t b = (count + 255) / 256;
    return (int)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

// Work decomposition of the backward pass; a pure function of the sizes, so the workspace size
// and the launches always agree and the reduction order is fixed. Head dims up to 32 take the
// prep / dq2 / dkv2 path (v2); D = 64 takes dot / dq / dkv.
constexpr int kTargetBlocks = 256;  // one row-owner block per CU of an MI355X
// Row-owner block shape for head dim D: QG query groups of four waves, each wave QTW 16-query
// sub-tiles (BQ = 16*QG*QTW queries per block). Two groups of two sub-tiles (8 waves, two per
// SIMD, 255 VGPRs at D = 32): three groups of one sub-tile (12 waves, three per SIMD, 161
// VGPRs) measured only 1 us faster at N_res = 384, with a third more LDS reads per MFMA, and its
// 48-query tiles leave an eighth of the work empty at Sq = 256.
template <int D>
struct DqShape {
    static constexpr int QG = 2, QTW = 2;
    static constexpr int BQ = 16 * QG * QTW;
};
inline int dq_block_queries(int64_t) { return DqShape<32>::BQ; }

struct BwdPlan {
    bool v2 = false;
    int KT = 0, KCW = 0, KSUB = 0, KNW = 0, nranges = 0, NB = 0, nchunks = 0, SqP = 0;
    size_t off_di = 0, off_bt = 0, off_rowl = 0, off_mbits = 0, off_lse2 = 0, off_ndi = 0,
           off_dbias = 0,
           off_dq = 0, bytes = 0;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Whether the column-owner kernel's extra blocks sum the dBias slices of count elements (v2, more
// than one slice, slices of whole 16-byte vectors) instead of a kernel of their own.
bool dbias_folded(const BwdPlan& p, size_t count) {
    return p.v2 && p.nchunks > 1 && count % 4 == 0;
}

BwdPlan plan_bwd(int64_t N, int64_t H, int64_t Sq, int64_t Sk, int64_t D) {
    BwdPlan p;
    p.v2 = D <= 32;
    int64_t range_keys;
    int64_t qtiles;
    if (p.v2) {
        const int64_t chunks32 = (Sk + 31) / 32;
        const int64_t kcw = (chunks32 + 3) / 4;
        p.KCW = (int)(kcw < 1 ? 1 : kcw > 3 ? 3 : kcw);
        range_keys = 128 * (int64_t)p.KCW;
        // dK/dV blocks: 16*KSUB keys per wave, KNW waves, 128 keys per block. At 32 keys per
        // wave (168 VGPRs, three waves per SIMD) three 4-wave blocks share a CU, so one block's
        // first loads overlap the others' work: measured 14-19% faster than one 8- or 12-wave
        // block of 256 or 384 keys per CU (Sk = 256, 384).
        if (Sk <= 128) {
            p.KSUB = 1;
            p.KNW = 8;
        } else {
            p.KSUB = 2;
            p.KNW = 4;
        }
        p.SqP = (int)((Sq + 63) / 64 * 64);
        qtiles = (Sq + dq_block_queries(D) - 1) / dq_block_queries(D);
    } else {
        const int64_t ktiles = (Sk + 63) / 64;
        p.KT = ktiles <= 2 ? 2 : ktiles <= 4 ? 4 : ktiles <= 6 ? 6 : 8;
        range_keys = 64 * (int64_t)p.KT;
        qtiles = (Sq + 63) / 64;
    }
    p.nranges = (int)((Sk + range_keys - 1) / range_keys);
    const int64_t base = qtiles * H * (p.nranges > 0 ? p.nranges : 1);
    const int64_t target = p.v2 ? kTargetBlocks : 512;
    int64_t chunks = base > 0 ? (p.v2 ? target / base : (target + base - 1) / base) : 1;
    if (chunks > N) chunks = N;
    if (chunks < 1) chunks = 1;
    p.NB = (int)((N + chunks - 1) / chunks);
    if (p.NB < 1) p.NB = 1;
    p.nchunks = (int)((N + p.NB - 1) / p.NB);
    const size_t rows = (size_t)(N * H * Sq);
    size_t off = 0;
    if (p.v2) {
        p.off_bt = off;
        off += align256((size_t)(H * Sk) * p.SqP * 2);
        p.off_rowl = off;
        off += align256((size_t)N * sizeof(float));
        p.off_mbits = off;  // 64-bit presence words of each mask row
        off += align256((size_t)N * ((Sk + 63) / 64) * 8);
        p.off_lse2 = off;
        off += align256(rows * sizeof(float));
        p.off_ndi = off;
        off += align256(rows * sizeof(float));
    } else {
        p.off_di = off;
        off += align256(rows * sizeof(float));
    }
    p.off_dbias = off;
    if (p.nchunks > 1) off += align256((size_t)p.nchunks * H * Sq * Sk * sizeof(float));
    p.off_dq = off;
    if (p.nranges > 1) off += align256((size_t)p.nranges * rows * D * sizeof(float));
    p.bytes = off;
    return p;
}

template <typename TR, int D, int KT, bool NSHD>
void launch_dq(hipStream_t st, dim3 grid, const void* q, const void* k, const void* v,
               const void* bias, const uint8_t* kmask, const void* dout, const float* lse,
               const float* di, void* dq, float* dq_part, float* dbias_dst, int N, int H, int Sq,
               int Sk, int NB, int nranges, float scale, int vec_ok) {
    using E = typename TR::elem;
    KernelTimer timer("attn_bwd_dq", st);
    attn_bwd_dq<TR, D, KT, NSHD><<<grid, 256, 0, st>>>(
        (const E*)q, (const E*)k, (const E*)v, (const E*)bias, kmask, (const E*)dout, lse, di,
        (E*)dq, dq_part, dbias_dst, N, H, Sq, Sk, NB, nranges, scale, vec_ok);
}

// The partial sums (dBias over row chunks, dQ over key ranges) in fixed order.
template <typename TR>
void finish_partials(hipStream_t st, const BwdPlan& p, float* dbias_part, float* dq_part,
                     float* dbias, void* dq, size_t dbias_count, size_t dq_count) {
    using E = typename TR::elem;
    if (p.nchunks > 1 && !dbias_folded(p, dbias_count)) {
        KernelTimer timer("attn_bwd_dbias_sum", st);
        if (dbias_count % 4 == 0)  // partial arrays are then 16-byte aligned
            sum_partials_f32x4<<<grid_for(dbias_count / 4), 256, 0, st>>>(
                reinterpret_cast<const f32x4*>(dbias_part), dbias_count / 4, p.nchunks,
                reinterpret_cast<f32x4*>(dbias));
        else
            sum_partials_f32<<<grid_for(dbias_count), 256, 0, st>>>(dbias_part, dbias_count,
                                                                    p.nchunks, dbias);
    }
    if (p.nranges > 1) {
        KernelTimer timer("attn_bwd_dq_sum", st);
        sum_partials_cast<TR><<<grid_for(dq_count), 256, 0, st>>>(dq_part, dq_count, p.nranges,
                                                                  (E*)dq);
    }
}

template <typename TR, int D, bool NSHD>
void run_bwd_v1(hipStream_t st, const BwdPlan& p, const void* q, const void* k, const void* v,
                const void* bias, const uint8_t* kmask, const void* out, const void* dout,
                const float* lse, void* dq, void* dk, void* dv, float* dbias, char* ws, int N,
                int H, int Sq, int Sk, float scale) {
    using E = typename TR::elem;
    const int vec_ok = (Sk % 8 == 0) ? 1 : 0;
    float* di = reinterpret_cast<float*>(ws + p.off_di);
    float* dbias_part = reinterpret_cast<float*>(ws + p.off_dbias);
    float* dq_part = reinterpret_cast<float*>(ws + p.off_dq);
    const int64_t rows = (int64_t)N * H * Sq;

    {
        const int64_t threads = rows * (D / 8);
        KernelTimer timer("attn_bwd_dot", st);
        attn_bwd_dot<TR, D, NSHD><<<(int)((threads + 255) / 256), 256, 0, st>>>(
            (const E*)out, (const E*)dout, di, rows, H, Sq);
    }
    {
        dim3 grid(ceil_div(Sq, 64), H, p.nchunks * p.nranges);
        float* dbias_dst = p.nchunks > 1 ? dbias_part : dbias;
        switch (p.KT) {
#define CLK_KT(KTV)                                                                              \
    case KTV:                                                                                    \
        launch_dq<TR, D, KTV, NSHD>(st, grid, q, k, v, bias, kmask, dout, lse, di, dq, dq_part,  \
                              dbias_dst, N, H, Sq, Sk, p.NB, p.nranges, scale, vec_ok);          \
        break;
            CLK_KT(2) CLK_KT(4) CLK_KT(6) CLK_KT(8)
#undef CLK_KT
        }
    }
    {
        dim3 grid(ceil_div(Sk, 64), H, N);
        KernelTimer timer("attn_bwd_dkv", st);
        attn_bwd_dkv<TR, D, NSHD><<<grid, 256, 0, st>>>((const E*)q, (const E*)k, (const E*)v,
                                                  (const E*)bias, kmask, (const E*)dout, lse, di,
                                                  (E*)dk, (E*)dv, H, Sq, Sk, scale, vec_ok);
    }
    finish_partials<TR>(st, p, dbias_part, dq_part, dbias, dq, (size_t)H * Sq * Sk,
                        (size_t)rows * D);
}

template <typename TR, int D, int KCW, bool VEC, bool NSHD>
void launch_dq2(hipStream_t st, const BwdPlan& p, const void* q, const void* k, const void* v,
                const void* bias, const uint8_t* kmask, const void* out, const void* dout,
                const float* lse, float* rowl, unsigned long long* mbits, float* lse2, float* ndi,
                void* dq, float* dq_part, float* dbias_dst, void* bias_t, int N, int H, int Sq,
                int Sk, float scale) {
    using E = typename TR::elem;
    using S = DqShape<D>;
    const dim3 grid(ceil_div(Sq, S::BQ) * H * p.nchunks * p.nranges);
    KernelTimer timer("attn_bwd_dq", st);
    attn_bwd_dq2<TR, D, KCW, VEC, S::QG, S::QTW, NSHD><<<grid, 64 * 4 * S::QG, 0, st>>>(
        (const E*)q, (const E*)k, (const E*)v, (const E*)bias, kmask, (const E*)out,
        (const E*)dout, lse, rowl, mbits, lse2, ndi, (E*)dq, dq_part, dbias_dst, N, H, Sq, Sk, p.NB,
        p.nranges, scale, LogitForm::make(scale), (E*)bias_t, p.SqP, ceil_div(p.SqP, 64),
        ceil_div(Sk, 64));
}

template <typename TR, int D, int KSUB, int NW, bool VEC, bool NSHD>
void launch_dkv2(hipStream_t st, const BwdPlan& p, const void* q, const void* k, const void* v,
                 const void* bias_t, const uint8_t* kmask, const void* dout, const float* lse2,
                 const float* ndi, const float* rowl, void* dk, void* dv, const float* dbias_part,
                 float* dbias, int N, int H, int Sq, int Sk, float scale) {
    using E = typename TR::elem;
    const int main_blocks = ceil_div(Sk, 16 * KSUB * NW) * H * N;
    // The dBias slices are summed by extra blocks of this grid when they are 16-byte vectors.
    const size_t count = (size_t)H * Sq * Sk;
    const size_t per_block = 64 * NW, vecs = count / 4;
    const int extra =
        dbias_folded(p, count) ? (int)std::min<size_t>((vecs + per_block - 1) / per_block, 2048) : 0;
    KernelTimer timer("attn_bwd_dkv", st);
    attn_bwd_dkv2<TR, D, KSUB, NW, VEC, NSHD><<<dim3(main_blocks + extra), 64 * NW, 0, st>>>(
        (const E*)q, (const E*)k, (const E*)v, (const E*)bias_t, kmask, (const E*)dout, lse2,
        ndi, rowl, (E*)dk, (E*)dv, H, Sq, Sk, p.SqP, scale, main_blocks,
        reinterpret_cast<const f32x4*>(dbias_part), reinterpret_cast<f32x4*>(dbias), vecs,
        p.nchunks);
}

template <typename TR, int D, bool VEC, bool NSHD>
void run_bwd_v2(hipStream_t st, const BwdPlan& p, const void* q, const void* k, const void* v,
                const void* bias, const uint8_t* kmask, const void* out, const void* dout,
                const float* lse, void* dq, void* dk, void* dv, float* dbias, char* ws, int N,
                int H, int Sq, int Sk, float scale) {
    using E = typename TR::elem;
    E* bias_t = reinterpret_cast<E*>(ws + p.off_bt);
    float* rowl = reinterpret_cast<float*>(ws + p.off_rowl);
    unsigned long long* mbits = reinterpret_cast<unsigned long long*>(ws + p.off_mbits);
    float* lse2 = reinterpret_cast<float*>(ws + p.off_lse2);
    float* ndi = reinterpret_cast<float*>(ws + p.off_ndi);
    float* dbias_part = reinterpret_cast<float*>(ws + p.off_dbias);
    float* dq_part = reinterpret_cast<float*>(ws + p.off_dq);
    float* dbias_dst = p.nchunks > 1 ? dbias_part : dbias;
    switch (p.KCW) {
#define CLK_KCW(V)                                                                               \
    case V:                                                                                      \
        launch_dq2<TR, D, V, VEC, NSHD>(st, p, q, k, v, bias, kmask, out, dout, lse, rowl,       \
                                        mbits, lse2, ndi, dq, dq_part, dbias_dst, bias_t, N, H,  \
                                        Sq, Sk, scale);                                          \
        break;
        CLK_KCW(1) CLK_KCW(2) CLK_KCW(3)
#undef CLK_KCW
    }
    switch (p.KSUB * 100 + p.KNW) {
#define CLK_KSUB(V, W)                                                                           \
    case V * 100 + W:                                                                            \
        launch_dkv2<TR, D, V, W, VEC, NSHD>(st, p, q, k, v, bias_t, kmask, dout, lse2, ndi,      \
                                            rowl, dk, dv, dbias_part, dbias, N, H, Sq, Sk,       \
                                            scale);                                              \
        break;
        CLK_KSUB(1, 8) CLK_KSUB(2, 4)
#undef CLK_KSUB
    }
    finish_partials<TR>(st, p, dbias_part, dq_part, dbias, dq, (size_t)H * Sq * Sk,
                        (size_t)N * H * Sq * D);
}

template <typename TR, int D, bool NSHD>
void run_bwd(hipStream_t st, const BwdPlan& p, const void* q, const void* k, const void* v,
             const void* bias, const uint8_t* kmask, const void* out, const void* dout,
             const float* lse, void* dq, void* dk, void* dv, float* dbias, char* ws, int N,
             int H, int Sq, int Sk, float scale) {
    if constexpr (D <= 32) {
        const bool vec = Sk % 8 == 0 && (reinterpret_cast<uintptr_t>(kmask) & 7u) == 0;
        if (vec)
            run_bwd_v2<TR, D, true, NSHD>(st, p, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv,
                                          dbias, ws, N, H, Sq, Sk, scale);
        else
            run_bwd_v2<TR, D, false, NSHD>(st, p, q, k, v, bias, kmask, out, dout, lse, dq, dk,
                                           dv, dbias, ws, N, H, Sq, Sk, scale);
    } else {
        run_bwd_v1<TR, D, NSHD>(st, p, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv, dbias,
                                ws, N, H, Sq, Sk, scale);
    }
}

// Sizes with an empty axis: write the zeros that the gradient formulas give (fill kernels, so
// the call stays graph-capturable) -- dbias when N = 0, dq when Sk = 0, dk and dv when Sq = 0.
template <typename TR>
void zero_grads(hipStream_t st, int64_t N, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                void* dq, void* dk, void* dv, float* dbias) {
    using E = typename TR::elem;
    const size_t nb = (size_t)(H * Sq * Sk), nq = (size_t)(N * H * Sq * D),
                 nk = (size_t)(N * H * Sk * D);
    if (nb) sum_partials_f32<<<grid_for(nb), 256, 0, st>>>(nullptr, nb, 0, dbias);
    if (nq) sum_partials_cast<TR><<<grid_for(nq), 256, 0, st>>>(nullptr, nq, 0, (E*)dq);
    if (nk) {
        sum_partials_cast<TR><<<grid_for(nk), 256, 0, st>>>(nullptr, nk, 0, (E*)dk);
        sum_partials_cast<TR><<<grid_for(nk), 256, 0, st>>>(nullptr, nk, 0, (E*)dv);
    }
}

template <typename TR>
void dispatch_bwd(hipStream_t st, int64_t D, const BwdPlan& p, const void* q, const void* k,
                  const void* v, const void* bias, const uint8_t* kmask, const void* out,
                  const void* dout, const float* lse, void* dq, void* dk, void* dv,
                  float* dbias, char* ws, int N, int H, int Sq, int Sk, float scale,
                  bool nshd = false) {
    switch (D) {
#define CLK_D(DV)                                                                               \
    case DV:                                                                                    \
        if (nshd)                                                                               \
            run_bwd<TR, DV, true>(st, p, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv,      \
                                  dbias, ws, N, H, Sq, Sk, scale);                              \
        else                                                                                    \
            run_bwd<TR, DV, false>(st, p, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv,     \
                                   dbias, ws, N, H, Sq, Sk, scale);                             \
        break;
        CLK_D(8) CLK_D(16) CLK_D(32) CLK_D(64)
#undef CLK_D
    }
}

}  // namespace
}  // namespace clk

using namespace clk;

extern "C" size_t clk_attention_bwd_workspace_size(int64_t N, int64_t H, int64_t Sq, int64_t Sk,
                                                   int64_t D) {
    if (N < 0 || H < 0 || Sq < 0 || Sk < 0 || D <= 0) return 0;
    return plan_bwd(N, H, Sq, Sk, D).bytes;
}

namespace {

// The backward entries share this body: nshd selects AlphaFold's [N, S, H, D] layout for q, k, v,
// out, dout, dq, dk and dv (lse stays [N, H, Sq]).
clk_status attention_bwd_entry(const char* who, hipStream_t stream, clk_dtype dtype,
                               const void* q, const void* k, const void* v, const void* bias,
                               const uint8_t* kmask, const void* out, const void* dout,
                               const float* lse, void* dq, void* dk, void* dv, float* dbias,
                               void* workspace, size_t workspace_bytes, int64_t N, int64_t H,
                               int64_t Sq, int64_t Sk, int64_t D, float scale, bool nshd) {
    clk_status s = validate_attention(who, dtype, N, H, Sq, Sk, D);
    if (s != CLK_OK) return s;
    // [N, S, H, D]: byte offsets within the rows of one (n, h) are 32-bit.
    if (nshd && (Sq > Sk ? Sq : Sk) * H * D * 2 >= ((int64_t)1 << 31))
        return fail(CLK_INVALID_ARGUMENT, "%s: S*H*D too large for the [N,S,H,D] layout", who);
    const BwdPlan p = plan_bwd(N, H, Sq, Sk, D);
    if (workspace_bytes < p.bytes)
        return fail(CLK_INVALID_ARGUMENT, "%s: workspace %zu bytes, needs %zu", who,
                    workspace_bytes, p.bytes);
    if (N == 0 || H == 0 || Sq == 0 || Sk == 0) {
        const bool need_b = H * Sq * Sk > 0, need_q = N * H * Sq > 0, need_k = N * H * Sk > 0;
        if ((need_b && !dbias) || (need_q && !dq) || (need_k && (!dk || !dv)))
            return fail(CLK_INVALID_ARGUMENT, "%s: null gradient pointer", who);
        if (dtype == CLK_BF16) zero_grads<BF16>(stream, N, H, Sq, Sk, D, dq, dk, dv, dbias);
        else zero_grads<F16>(stream, N, H, Sq, Sk, D, dq, dk, dv, dbias);
        return check_launch(who);
    }
    if (!q || !k || !v || !bias || !out || !dout || !lse || !dq || !dk || !dv || !dbias ||
        !workspace)
        return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(bias) || !aligned16(out) ||
        !aligned16(dout) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv) ||
        !aligned16(dbias) || !aligned16(lse) || (reinterpret_cast<uintptr_t>(workspace) & 255u))
        return fail(CLK_INVALID_ARGUMENT,
                    "%s: operands must be 16-byte and workspace 256-byte aligned", who);
    char* ws = static_cast<char*>(workspace);
    if (dtype == CLK_BF16)
        dispatch_bwd<BF16>(stream, D, p, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv, dbias,
                           ws, (int)N, (int)H, (int)Sq, (int)Sk, scale, nshd);
    else
        dispatch_bwd<F16>(stream, D, p, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv, dbias,
                          ws, (int)N, (int)H, (int)Sq, (int)Sk, scale, nshd);
    return check_launch(who);
}

}  // namespace

extern "C" clk_status clk_attention_bwd(hipStream_t stream, clk_dtype dtype, const void* q,
                                        const void* k, const void* v, const void* bias,
                                        const uint8_t* kmask, const void* out, const void* dout,
                                        const float* lse, void* dq, void* dk, void* dv,
                                        float* dbias, void* workspace, size_t workspace_bytes,
                                        int64_t N, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                                        float scale) {
    return attention_bwd_entry("attention_bwd", stream, dtype, q, k, v, bias, kmask, out, dout,
                               lse, dq, dk, dv, dbias, workspace, workspace_bytes, N, H, Sq, Sk,
                               D, scale, false);
}

extern "C" clk_status clk_attention_bwd_nshd(hipStream_t stream, clk_dtype dtype, const void* q,
                                             const void* k, const void* v, const void* bias,
                                             const uint8_t* kmask, const void* out,
                                             const void* dout, const float* lse, void* dq,
                                             void* dk, void* dv, float* dbias, void* workspace,
                                             size_t workspace_bytes, int64_t N, int64_t H,
                                             int64_t Sq, int64_t Sk, int64_t D, float scale) {
    return attention_bwd_entry("attention_bwd_nshd", stream, dtype, q, k, v, bias, kmask, out,
                               dout, lse, dq, dk, dv, dbias, workspace, workspace_bytes, N, H, Sq,
                               Sk, D, scale, true);
}
