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

namespace clk {
namespace {

template <typename TR, int D>
__global__ __launch_bounds__(256) void attn_bwd_dot(const typename TR::elem* __restrict__ out,
                                                    const typename TR::elem* __restrict__ dout,
                                                    float* __restrict__ di, int64_t rows) {
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
#pragma unroll
    for (int off = 1; off < LPR; off <<= 1) s += __shfl_xor(s, off);
    if (row < rows && part == 0) di[row] = s;
}

template <typename TR, int D, int KT>
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
    auto load_tile = [&](int n, int kstart) {
        const size_t base = ((size_t)n * H + h) * Sk * D;
        const E* src[2] = {k + base, v + base};
        stage.load(src, kstart, kend);
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
                rq = ld16(q + (nh * Sq + qrow) * D + d0);
                rd = ld16(dout + (nh * Sq + qrow) * D + d0);
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
                        store4<TR>(dq + (nh * Sq + qrow) * D + d, dq_acc[dt] * scale);
                    } else {
                        float* o = dq_part + (((size_t)range * N + n) * H + h) * Sq * D +
                                   (size_t)qrow * D + d;
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

template <typename TR, int D>
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
    const int key = k0 + wave * 16 + r16;
    const bool kin = key < Sk;

    V8 kf[G::KS], vf[G::KS];
#pragma unroll
    for (int ks = 0; ks < G::KS; ++ks) {
        const int d0 = ks * 32 + g * 8;
        u32x4 rk = {0u, 0u, 0u, 0u}, rv = {0u, 0u, 0u, 0u};
        if (kin && d0 < D) {
            rk = ld16(k + (nh * Sk + key) * D + d0);
            rv = ld16(v + (nh * Sk + key) * D + d0);
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
    const E* src[2] = {q + nh * Sq * D, dout + nh * Sq * D};

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
        stage.load(src, 0, Sq);
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
            stage.load(src, qs + 64, Sq);
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
            store4<TR>(dk + (nh * Sk + key) * D + d, dk_acc[dt] * scale);
            store4<TR>(dv + (nh * Sk + key) * D + d, dv_acc[dt]);
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
// and the launches always agree and the reduction order is fixed.
struct BwdPlan {
    int KT = 0, nranges = 0, NB = 0, nchunks = 0;
    size_t off_di = 0, off_dbias = 0, off_dq = 0, bytes = 0;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

BwdPlan plan_bwd(int64_t N, int64_t H, int64_t Sq, int64_t Sk, int64_t D) {
    BwdPlan p;
    const int64_t ktiles = (Sk + 63) / 64;
    p.KT = ktiles <= 2 ? 2 : ktiles <= 4 ? 4 : ktiles <= 6 ? 6 : 8;
    p.nranges = (int)((ktiles + p.KT - 1) / p.KT);
    const int64_t qtiles = (Sq + 63) / 64;
    const int64_t base = qtiles * H * (p.nranges > 0 ? p.nranges : 1);
    int64_t chunks = base > 0 ? (512 + base - 1) / base : 1;
    if (chunks > N) chunks = N;
    if (chunks < 1) chunks = 1;
    p.NB = (int)((N + chunks - 1) / chunks);
    if (p.NB < 1) p.NB = 1;
    p.nchunks = (int)((N + p.NB - 1) / p.NB);
    size_t off = 0;
    p.off_di = off;
    off += align256((size_t)(N * H * Sq) * sizeof(float));
    p.off_dbias = off;
    if (p.nchunks > 1) off += align256((size_t)p.nchunks * H * Sq * Sk * sizeof(float));
    p.off_dq = off;
    if (p.nranges > 1) off += align256((size_t)p.nranges * N * H * Sq * D * sizeof(float));
    p.bytes = off;
    return p;
}

template <typename TR, int D, int KT>
void launch_dq(hipStream_t st, dim3 grid, const void* q, const void* k, const void* v,
               const void* bias, const uint8_t* kmask, const void* dout, const float* lse,
               const float* di, void* dq, float* dq_part, float* dbias_dst, int N, int H, int Sq,
               int Sk, int NB, int nranges, float scale, int vec_ok) {
    using E = typename TR::elem;
    KernelTimer timer("attn_bwd_dq", st);
    attn_bwd_dq<TR, D, KT><<<grid, 256, 0, st>>>(
        (const E*)q, (const E*)k, (const E*)v, (const E*)bias, kmask, (const E*)dout, lse, di,
        (E*)dq, dq_part, dbias_dst, N, H, Sq, Sk, NB, nranges, scale, vec_ok);
}

template <typename TR, int D>
void run_bwd(hipStream_t st, const BwdPlan& p, const void* q, const void* k, const void* v,
             const void* bias, const uint8_t* kmask, const void* out, const void* dout,
             const float* lse, void* dq, void* dk, void* dv, float* dbias, char* ws, int N,
             int H, int Sq, int Sk, float scale) {
    using E = typename TR::elem;
    const int vec_ok = (Sk % 8 == 0) ? 1 : 0;
    float* di = reinterpret_cast<float*>(ws + p.off_di);
    float* dbias_part = reinterpret_cast<float*>(ws + p.off_dbias);
    float* dq_part = reinterpret_cast<float*>(ws + p.off_dq);
    const int64_t rows = (int64_t)N * H * Sq;
    const size_t dbias_count = (size_t)H * Sq * Sk;

    {
        const int64_t threads = rows * (D / 8);
        KernelTimer timer("attn_bwd_dot", st);
        attn_bwd_dot<TR, D><<<(int)((threads + 255) / 256), 256, 0, st>>>(
            (const E*)out, (const E*)dout, di, rows);
    }
    {
        dim3 grid(ceil_div(Sq, 64), H, p.nchunks * p.nranges);
        float* dbias_dst = p.nchunks > 1 ? dbias_part : dbias;
        switch (p.KT) {
#define CLK_KT(KTV)                                                                              \
    case KTV:                                                                                    \
        launch_dq<TR, D, KTV>(st, grid, q, k, v, bias, kmask, dout, lse, di, dq, dq_part,        \
                              dbias_dst, N, H, Sq, Sk, p.NB, p.nranges, scale, vec_ok);          \
        break;
            CLK_KT(2) CLK_KT(4) CLK_KT(6) CLK_KT(8)
#undef CLK_KT
        }
    }
    {
        dim3 grid(ceil_div(Sk, 64), H, N);
        KernelTimer timer("attn_bwd_dkv", st);
        attn_bwd_dkv<TR, D><<<grid, 256, 0, st>>>((const E*)q, (const E*)k, (const E*)v,
                                                  (const E*)bias, kmask, (const E*)dout, lse, di,
                                                  (E*)dk, (E*)dv, H, Sq, Sk, scale, vec_ok);
    }
    if (p.nchunks > 1) {
        KernelTimer timer("attn_bwd_dbias_sum", st);
        sum_partials_f32<<<grid_for(dbias_count), 256, 0, st>>>(dbias_part, dbias_count,
                                                                p.nchunks, dbias);
    }
    if (p.nranges > 1) {
        KernelTimer timer("attn_bwd_dq_sum", st);
        sum_partials_cast<TR><<<grid_for((size_t)rows * D), 256, 0, st>>>(
            dq_part, (size_t)rows * D, p.nranges, (E*)dq);
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
                  float* dbias, char* ws, int N, int H, int Sq, int Sk, float scale) {
    switch (D) {
#define CLK_D(DV)                                                                           \
    case DV:                                                                                \
        run_bwd<TR, DV>(st, p, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv, dbias, ws, \
                        N, H, Sq, Sk, scale);                                               \
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

extern "C" clk_status clk_attention_bwd(hipStream_t stream, clk_dtype dtype, const void* q,
                                        const void* k, const void* v, const void* bias,
                                        const uint8_t* kmask, const void* out, const void* dout,
                                        const float* lse, void* dq, void* dk, void* dv,
                                        float* dbias, void* workspace, size_t workspace_bytes,
                                        int64_t N, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                                        float scale) {
    clk_status s = validate_attention("attention_bwd", dtype, N, H, Sq, Sk, D);
    if (s != CLK_OK) return s;
    const BwdPlan p = plan_bwd(N, H, Sq, Sk, D);
    if (workspace_bytes < p.bytes)
        return fail(CLK_INVALID_ARGUMENT, "attention_bwd: workspace %zu bytes, needs %zu",
                    workspace_bytes, p.bytes);
    if (N == 0 || H == 0 || Sq == 0 || Sk == 0) {
        const bool need_b = H * Sq * Sk > 0, need_q = N * H * Sq > 0, need_k = N * H * Sk > 0;
        if ((need_b && !dbias) || (need_q && !dq) || (need_k && (!dk || !dv)))
            return fail(CLK_INVALID_ARGUMENT, "attention_bwd: null gradient pointer");
        if (dtype == CLK_BF16) zero_grads<BF16>(stream, N, H, Sq, Sk, D, dq, dk, dv, dbias);
        else zero_grads<F16>(stream, N, H, Sq, Sk, D, dq, dk, dv, dbias);
        return check_launch("attention_bwd");
    }
    if (!q || !k || !v || !bias || !out || !dout || !lse || !dq || !dk || !dv || !dbias ||
        !workspace)
        return fail(CLK_INVALID_ARGUMENT, "attention_bwd: null operand pointer");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(bias) || !aligned16(out) ||
        !aligned16(dout) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv) ||
        !aligned16(dbias) || !aligned16(lse) || (reinterpret_cast<uintptr_t>(workspace) & 255u))
        return fail(CLK_INVALID_ARGUMENT,
                    "attention_bwd: operands must be 16-byte and workspace 256-byte aligned");
    char* ws = static_cast<char*>(workspace);
    if (dtype == CLK_BF16)
        dispatch_bwd<BF16>(stream, D, p, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv, dbias,
                           ws, (int)N, (int)H, (int)Sq, (int)Sk, scale);
    else
        dispatch_bwd<F16>(stream, D, p, q, k, v, bias, kmask, out, dout, lse, dq, dk, dv, dbias,
                          ws, (int)N, (int)H, (int)Sq, (int)Sk, scale);
    return check_launch("attention_bwd");
}
