// Gated dual projection for gfx950:
//   out[m, n] = mask[m] * (x[m,:].wp[:,n] + bp[n]) * sigmoid(x[m,:].wg[:,n] + bg[n])
// gdp_kernel replaces VoltaGdp / VoltaGdpWmma (cuda/volta_ops.cu:109-265,
// cuda/volta_gdp_wmma.cu:16-140); ln_gdp_kernel fuses the LayerNorm in front of both gated
// branches of the triangle multiplication (one read of z for LN + two GDPs).
//
// Both compute out^T = W^T . x^T on MFMA 16x16x32: the weights are the A operand, read from LDS
// with ds_read_b64_tr_b16 (W stays row-major [K][N] in LDS, as in global memory), and x^T is the
// B operand, loaded straight from global memory as 16-byte row chunks. The output columns of
// each 32-column chunk are permuted across the two 16-row A tiles so that a lane's accumulators
// hold 8 consecutive output columns of one row: the epilogue (bias, sigmoid gate, row mask) ends
// in one 16-byte store per lane and chunk. At K = N = 128 the op is HBM-bound (about 170 flop/B
// against MI355X's ridge of about 315).
#include "common.hpp"

#include <mutex>

namespace clk {
namespace {

// A operand W^T for output-column chunk c (32 columns), half h, contraction rows kbase + 8g + 0..7.
// A-tile row r16 stands for output column 32c + 8*(r16/4) + 4h + r16%4, so the C tile's rows
// 4g'+i land in lane group g' as columns 32c + 8g' + 4h + i. For the transposed read, lane
// (r16, g) supplies row kbase + 8g + (r16>>2) (+4 for the upper four slots), columns
// 32c + 8*(r16&3) + 4h .. +3 (four consecutive output columns of one A-row group).
template <typename V8, typename E>
__device__ __forceinline__ V8 w_operand(const E* lds, int ld, int kbase, int c, int h, int r16,
                                        int g) {
    const E* lo = lds + (kbase + 8 * g + (r16 >> 2)) * ld + 32 * c + 8 * (r16 & 3) + 4 * h;
    return lds_tr8<V8>(lo, lo + 4 * ld);
}

__device__ __forceinline__ float sigmoid(float x) {
    return fast_rcp(1.f + fast_exp2(-x * kLog2e));
}

// Stages rows [0, KP) x columns [n0, n0 + BN) of a row-major [K, N] weight into LDS (row stride
// ld); rows past K and columns past N read as zero.
template <typename E>
__device__ void stage_weight(E* lds, int ld, const E* w, int K, int N, int KP, int n0, int BN,
                             int tid, int nthreads) {
    const int cpr = BN / 8;
    for (int i = tid; i < KP * cpr; i += nthreads) {
        const int k = i / cpr, c8 = (i % cpr) * 8;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (k < K && n0 + c8 < N) v = ld16(w + (size_t)k * N + n0 + c8);
        *reinterpret_cast<u32x4*>(lds + k * ld + c8) = v;
    }
}

// ---------------------------------------------------------------------------------------------
// GDP: a block owns BN output columns and walks row tiles of 4 waves x 16*RT rows. The weights of
// its columns sit in LDS, KP contraction rows at a time: all of K when K <= KP (staged once), else
// restaged per KP-row chunk inside each row tile (any K, as the reference's bounds-checked K loop,
// cuda/volta_ops.cu:143-183). XVEC: K % 8 == 0, so x rows are read as 16-byte chunks; otherwise
// element by element.
// ---------------------------------------------------------------------------------------------
template <typename TR, int BN, bool XVEC>
__global__ __launch_bounds__(256) void gdp_kernel(const typename TR::elem* __restrict__ x,
                                                  const typename TR::elem* __restrict__ wp,
                                                  const typename TR::elem* __restrict__ bp,
                                                  const typename TR::elem* __restrict__ wg,
                                                  const typename TR::elem* __restrict__ bg,
                                                  const typename TR::elem* __restrict__ mask,
                                                  typename TR::elem* __restrict__ out, int M,
                                                  int K, int N, int KP) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    constexpr int NT = BN / 16;   // 16-column A tiles
    constexpr int RT = 256 / BN;  // 16-row B tiles per wave
    constexpr int LD = BN + 8;
    extern __shared__ __attribute__((aligned(16))) char smem[];
    E* wp_lds = reinterpret_cast<E*>(smem);
    E* wg_lds = wp_lds + KP * LD;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.y * BN;

    const bool chunked = K > KP;  // block-uniform
    if (!chunked) {
        stage_weight(wp_lds, LD, wp, K, N, KP, n0, BN, threadIdx.x, 256);
        stage_weight(wg_lds, LD, wg, K, N, KP, n0, BN, threadIdx.x, 256);
    }

    // Biases of the lane's output columns n0 + 32c + 8g + j.
    float bpv[NT / 2][8], bgv[NT / 2][8];
#pragma unroll
    for (int c = 0; c < NT / 2; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int n = n0 + 32 * c + 8 * g + j;
            bpv[c][j] = n < N ? TR::to_f(bp[n]) : 0.f;
            bgv[c][j] = n < N ? TR::to_f(bg[n]) : 0.f;
        }
    __syncthreads();

    const int rows_per_iter = 4 * 16 * RT;
    for (int r0 = blockIdx.x * rows_per_iter; r0 < M; r0 += gridDim.x * rows_per_iter) {
        const int rbase = r0 + wave * 16 * RT;
        f32x4 ap[RT][NT], ag[RT][NT];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                ap[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
                ag[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        for (int kc = 0; kc < K; kc += KP) {
          if (chunked) {
            __syncthreads();  // every wave is done with the previous chunk
            stage_weight(wp_lds, LD, wp + (size_t)kc * N, K - kc, N, KP, n0, BN, threadIdx.x, 256);
            stage_weight(wg_lds, LD, wg + (size_t)kc * N, K - kc, N, KP, n0, BN, threadIdx.x, 256);
            __syncthreads();
          }
          for (int kb = 0; kb < KP; kb += 32) {
            V8 xf[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int row = rbase + 16 * rt + r16;
                const int k = kc + kb + 8 * g;
                if constexpr (XVEC) {
                    u32x4 raw = {0u, 0u, 0u, 0u};
                    if (row < M && k < K) raw = ld16(x + (size_t)row * K + k);
                    xf[rt] = bits_as<V8>(raw);
                } else {
                    typename TR::elem e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        e[j] = (row < M && k + j < K) ? x[(size_t)row * K + k + j]
                                                      : typename TR::elem(0.f);
                    __builtin_memcpy(&xf[rt], e, 16);
                }
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const V8 pa = w_operand<V8>(wp_lds, LD, kb, t >> 1, t & 1, r16, g);
                const V8 ga = w_operand<V8>(wg_lds, LD, kb, t >> 1, t & 1, r16, g);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    ap[rt][t] = TR::mfma(pa, xf[rt], ap[rt][t]);
                    ag[rt][t] = TR::mfma(ga, xf[rt], ag[rt][t]);
                }
            }
          }
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int row = rbase + 16 * rt + r16;
            if (row >= M) continue;
            const float mv = TR::to_f(mask[row]);
#pragma unroll
            for (int c = 0; c < NT / 2; ++c) {
                const int n = n0 + 32 * c + 8 * g;
                if (n >= N) continue;
                float o[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int t = 2 * c + (j >> 2), i = j & 3;
                    const float p = ap[rt][t][i] + bpv[c][j];
                    const float gt = ag[rt][t][i] + bgv[c][j];
                    o[j] = mv * p * sigmoid(gt);
                }
                st16(out + (size_t)row * N + n, pack8<TR>(o));
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// GDP for K <= 32*KS with K % 8 == 0 (the pair and MSA widths), 128 output columns per block:
// the operand layout of gdp_kernel, but a block stays resident over many 64-row tiles (the
// weight slab is staged once per block, not once per tile), each wave's x fragments of its next
// tile are in flight while the current tile is computed (two register sets, the row loop
// unrolled by two so that neither is ever copied), and the biases enter as the accumulators'
// starting values, read from LDS.
// ---------------------------------------------------------------------------------------------
template <typename TR, int KS>
__global__ __launch_bounds__(256) void gdp_stream_kernel(
    const typename TR::elem* __restrict__ x, const typename TR::elem* __restrict__ wp,
    const typename TR::elem* __restrict__ bp, const typename TR::elem* __restrict__ wg,
    const typename TR::elem* __restrict__ bg, const typename TR::elem* __restrict__ mask,
    typename TR::elem* __restrict__ out, int M, int K, int N) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    constexpr int BN = 128, NT = BN / 16, RT = 1, LD = BN + 8, KP = 32 * KS;
    constexpr int ROWS = 4 * 16 * RT;  // rows per block and tile
    __shared__ __attribute__((aligned(16))) E wp_lds[KP * LD];
    __shared__ __attribute__((aligned(16))) E wg_lds[KP * LD];
    __shared__ __attribute__((aligned(16))) float b_lds[2][BN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.y * BN;
    stage_weight(wp_lds, LD, wp, K, N, KP, n0, BN, tid, 256);
    stage_weight(wg_lds, LD, wg, K, N, KP, n0, BN, tid, 256);
    for (int i = tid; i < BN; i += 256) {
        const int n = n0 + i;
        b_lds[0][i] = n < N ? TR::to_f(bp[n]) : 0.f;
        b_lds[1][i] = n < N ? TR::to_f(bg[n]) : 0.f;
    }
    __syncthreads();

    using XF = V8[KS][RT];
    auto load = [&](int r0, XF& xf) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int row = r0 + wave * 16 * RT + 16 * rt + r16;
                const int k = 32 * ks + 8 * g;
                u32x4 raw = {0u, 0u, 0u, 0u};
                if (row < M && k < K) raw = ld16(x + (size_t)row * K + k);
                xf[ks][rt] = bits_as<V8>(raw);
            }
    };
    auto tile = [&](int r0, const XF& xf) {
        f32x4 ap[RT][NT], ag[RT][NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            // Accumulator row 4g+i of A tile t is output column 32(t/2) + 8g + 4(t%2) + i.
            const int col = 32 * (t >> 1) + 8 * g + 4 * (t & 1);
            const f32x4 bpi = *reinterpret_cast<const f32x4*>(&b_lds[0][col]);
            const f32x4 bgi = *reinterpret_cast<const f32x4*>(&b_lds[1][col]);
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                ap[rt][t] = bpi;
                ag[rt][t] = bgi;
            }
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const V8 pa = w_operand<V8>(wp_lds, LD, 32 * ks, t >> 1, t & 1, r16, g);
                const V8 ga = w_operand<V8>(wg_lds, LD, 32 * ks, t >> 1, t & 1, r16, g);
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    ap[rt][t] = TR::mfma(pa, xf[ks][rt], ap[rt][t]);
                    ag[rt][t] = TR::mfma(ga, xf[ks][rt], ag[rt][t]);
                }
            }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const int row = r0 + wave * 16 * RT + 16 * rt + r16;
            if (row >= M) continue;
            const float mv = TR::to_f(mask[row]);
#pragma unroll
            for (int c = 0; c < NT / 2; ++c) {
                const int n = n0 + 32 * c + 8 * g;
                if (n >= N) continue;
                float o[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int t = 2 * c + (j >> 2), i = j & 3;
                    o[j] = mv * ap[rt][t][i] * sigmoid(ag[rt][t][i]);
                }
                st16(out + (size_t)row * N + n, pack8<TR>(o));
            }
        }
    };

    const int stride = gridDim.x * ROWS;
    XF xa, xb;
    int r0 = blockIdx.x * ROWS;
    if (r0 < M) load(r0, xa);
    for (; r0 < M; r0 += 2 * stride) {
        if (r0 + stride < M) load(r0 + stride, xb);
        tile(r0, xa);
        if (r0 + stride >= M) break;
        if (r0 + 2 * stride < M) load(r0 + 2 * stride, xa);
        tile(r0 + stride, xb);
    }
}

// ---------------------------------------------------------------------------------------------
// LayerNorm + both gated branches (the two inputs of the triangle multiplication). A block has
// two kinds of waves. MFMA wave w of the N/16 owns the 32 output columns 32*cb + 0..31
// (cb = w % (N/32)) of branch w / (N/32) and holds the matching columns of that branch's
// projection and gate weights as MFMA A operands in registers for the whole kernel, with the LN
// affine folded in:
//   (xhat*gamma + beta).W + b = xhat.(diag(gamma) W) + (beta.W + b),
// the folded biases being the accumulators' starting values. Four LayerNorm waves stage 64-row
// tiles of z by direct buffer->LDS loads two tiles ahead and write xhat (in the input type) into
// a swizzled LDS tile. In step j the LayerNorm waves normalise tile j while the MFMA waves read
// tile j-1 as the B operand of out^T = W^T . xhat^T; one barrier per step. A-tile row r of column
// half h stands for output column 32cb + 8*(r/4) + 4h + r%4, so a lane's accumulators hold 8
// consecutive output columns of one row and the epilogue (bias, sigmoid gate, row mask) ends in
// one 16-byte piece per lane and 16-row sub-tile. Where LDS allows (LnGdpPlan::STAGED_OUT) the
// pieces go to an LDS staging tile and the next step stores whole rows with non-temporal
// stores (a wave's 32 columns are only half of a 128-byte line, and non-temporal stores of half
// lines are slower than cached ones; whole-line ones are 12-15% faster here); otherwise they
// are stored from registers. HBM traffic is one read of z and the mask and one write of a and b.
//
// The row statistics follow volta_ops.cu:40-52: one pass of sum and sum of squares in fp32,
// var = max(sum_sq/C - mean^2, 0). With bf16/f16 inputs the pair products are exact in fp32, so
// this loses accuracy only for rows whose mean is large against their spread (|mean|/std beyond
// about 10^3).
// ---------------------------------------------------------------------------------------------

// Weights and biases of the two branches, passed by value: w = {wpa, wga, wpb, wgb}, same for b.
template <typename E>
struct LnGdpWeights {
    const E* w[4];
    const E* b[4];
};

constexpr int kLnGdpRows = 64;  // rows per tile

// LDS plan of ln_gdp_kernel<C, N, NB, CM>. PER_CU blocks share a CU (one 12-wave block at
// C = N = 128). Each projected tile goes out through an LDS staging buffer (two, rows padded by
// 16 bytes) when both still fit PER_CU blocks: one store instruction then writes whole output
// rows (row-major: a position's N channels; CM: a channel's 64 positions of the tile), which lets
// the stores stream past the caches (non-temporal).
template <int C, int N, int NB, bool CM = false>
struct LnGdpPlan {
    static constexpr int R = kLnGdpRows;
    static constexpr int TILE = R * C * 2;                // a z or normalised tile
    static constexpr int OSTR = (CM ? 2 * R : 2 * N) + 16;  // staged output row stride (bytes)
    static constexpr int OBB = NB * (CM ? N : R) * OSTR;    // one staging buffer, every branch
    static constexpr int PER_CU = NB == 2 ? 128 / N : (C == 128 ? 1 : 2);
    static constexpr int BASE = 5 * TILE + 2 * R * 4;  // five tiles and two row-mask vectors
    static constexpr bool STAGED_OUT = PER_CU * (BASE + 2 * OBB) <= 160 * 1024;
};

template <int PL>
struct LnGdpGeom {
    // XOR swizzle of 16-byte pieces within a row: the largest power-of-two group that divides PL.
    static constexpr int SWZ = (PL % 16 == 0) ? 15 : (PL % 8 == 0) ? 7 : 3;
    // LayerNorm lanes per row: PL rounded up to a power of two (C = 96 leaves 4 lanes idle).
    static constexpr int LPR = PL <= 4 ? 4 : PL <= 8 ? 8 : 16;
};

// N 16-byte LDS reads at addr + i * STRIDE and the wait for them, as one asm statement.
template <int N, int STRIDE>
__device__ __forceinline__ void lds_rows(uint32_t addr, u32x4 (&r)[N]) {
    static_assert((N == 1 || N == 2 || N == 4) && (N - 1) * STRIDE < 65536, "ds offset field");
    if constexpr (N == 1) {
        asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r[0]) : "v"(addr)
                     : "memory");
    } else if constexpr (N == 2) {
        asm volatile(
            "ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:%3\n\ts_waitcnt lgkmcnt(0)"
            : "=&v"(r[0]), "=&v"(r[1])
            : "v"(addr), "i"(STRIDE)
            : "memory");
    } else {
        asm volatile(
            "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:%5\n\t"
            "ds_read_b128 %2, %4 offset:%6\n\tds_read_b128 %3, %4 offset:%7\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
            : "v"(addr), "i"(STRIDE), "i"(2 * STRIDE), "i"(3 * STRIDE)
            : "memory");
    }
}

// CM = false: a and b are [M, N] row-major (the pair layout). CM = true: a and b are channel-
// major [N, M] (a[n][m]), the operand layout of the triangle-multiplication contraction; the MFMA
// operands swap roles (out = xhat . W') so that a lane's accumulators hold four consecutive rows
// of one output column (16 consecutive rows per lane after the four sub-tiles), staged as a
// [channel][64 rows] tile when LDS allows and stored as whole 128-byte lines of the channels'
// planes, else as two 16-byte pieces per lane and column. CM needs M % 64 == 0.
// LN = false, NB = 1: the plain gated dual projection of one branch (x = z as it is; the four
// staging waves only move z into the swizzled tile, and gamma, beta are not read).
// Block: NB*N/32 MFMA waves, then 4 LayerNorm (staging) waves.
template <typename TR, int C, int N, bool CM, bool LN = true, int NB = 2>
__global__ __launch_bounds__(64 * NB * N / 32 + 256) void ln_gdp_kernel(
    const typename TR::elem* __restrict__ z, const float* __restrict__ gamma,
    const float* __restrict__ beta, LnGdpWeights<typename TR::elem> wb,
    const typename TR::elem* __restrict__ mask, typename TR::elem* __restrict__ outa,
    typename TR::elem* __restrict__ outb, int M, float eps) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    constexpr int NWM = NB * N / 32;     // MFMA waves
    constexpr int NTL = 256;             // LayerNorm threads (4 waves)
    constexpr int KS = C / 32;
    constexpr int R = kLnGdpRows, SUB = R / 16;
    constexpr int PL = C / 8;
    using GM = LnGdpGeom<PL>;
    constexpr int LPR = GM::LPR, RPP = NTL / LPR, PASSES = (R + RPP - 1) / RPP;
    constexpr int ZB = R * C * 2;
    constexpr int DPW = (R * PL + NTL - 1) / NTL;  // 16-byte loads per LayerNorm lane and tile
    constexpr int ZBP = DPW * NTL * 16;
    using PLAN = LnGdpPlan<C, N, NB, CM>;
    constexpr bool OST = PLAN::STAGED_OUT;
    constexpr int OSTR = PLAN::OSTR;

    // Three z tiles (normalised, landing, in flight), two normalised tiles and their row masks.
    __shared__ __attribute__((aligned(16))) char z0[ZBP];
    __shared__ __attribute__((aligned(16))) char z1[ZBP];
    __shared__ __attribute__((aligned(16))) char z2[ZBP];
    __shared__ __attribute__((aligned(16))) char xh0[ZB];
    __shared__ __attribute__((aligned(16))) char xh1[ZB];
    __shared__ float mk0[R];
    __shared__ float mk1[R];
    // Projected tiles on their way out (OST): written in step j to ob[j % 2], stored in step j+1.
    __shared__ __attribute__((aligned(16))) char ob0[OST ? PLAN::OBB : 16];
    __shared__ __attribute__((aligned(16))) char ob1[OST ? PLAN::OBB : 16];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const bool mfma_wave = wave < NWM;
    const int br = wave / (N / 32), cb = wave % (N / 32);
    E* const out = br == 0 ? outa : outb;

    // MFMA waves: resident A operands W'^T and the folded biases.
    V8 wa[2][2][KS];
    f32x4 binit[2][2];
    if (mfma_wave) {
#pragma unroll
        for (int mat = 0; mat < 2; ++mat) {
            const E* W = wb.w[2 * br + mat];
            const float fold = mat == 1 ? -kLog2e : 1.f;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int col = 32 * cb + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
                float part = 0.f;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int k = 32 * ks + 8 * g + j;
                        const float v = TR::to_f(W[(size_t)k * N + col]);
                        wa[mat][h][ks][j] = TR::from_f((LN ? gamma[k] : 1.f) * v * fold);
                        if constexpr (LN) part = fmaf(beta[k], v, part);
                    }
                const float bcol = (xgroup_sum(part) + TR::to_f(wb.b[2 * br + mat][col])) * fold;
                if constexpr (CM) {
                    binit[mat][h] = f32x4{bcol, bcol, bcol, bcol};
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) binit[mat][h][i] = __shfl(bcol, 4 * g + i);
                }
            }
        }
    }

    const int G = gridDim.x;
    const int ntiles = (M + R - 1) / R;
    const int mine = (ntiles - (int)blockIdx.x + G - 1) / G;  // tiles of this block, in turn
    auto tile_of = [&](int j) { return (int)blockIdx.x + j * G; };

    // ---- LayerNorm waves: stage z, normalise into xh, row mask into mk ----
    const int lt = tid - NWM * 64, lw = wave - NWM;
    const int lr = lt % LPR;
    // XOR swizzle of a row's 16-byte pieces. The MFMA waves' 16-lane reads touch rows
    // 16*sub + 0..15 (row-major outputs) or 16*a + 4*sub + b, a, b < 4 (channel-major): the
    // swizzle takes distinct values on either set.
    auto swz = [](int row) {
        return (CM ? (((row >> 4) & 3) << 2) | (row & 3) : row) & GM::SWZ;
    };
    auto stage = [&](int j, char* zb) {
        const int t = tile_of(j);
        const int rows = j < mine ? min(R, M - t * R) : 0;
        const Rsrc rz = buffer_rsrc(rows > 0 ? z + (size_t)t * R * C : z, (uint32_t)rows * C * 2);
#pragma unroll
        for (int k = 0; k < DPW; ++k) {
            const int b = lw * 64 + k * NTL;
            buf_dma16(rz, (b + lane) * 16, 0, zb + b * 16);
        }
    };
    auto load_mask = [&](int j, uint32_t (&mv)[PASSES]) {
        const uint16_t* m16 = reinterpret_cast<const uint16_t*>(mask);
        const int t = tile_of(j);
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int64_t r = (int64_t)t * R + p * RPP + lt / LPR;
            mv[p] = m16[r < M ? r : M - 1];
        }
    };
    auto normalise = [&](const char* zc, char* xh, float* mrow, const uint32_t (&mc)[PASSES]) {
        // The whole tile slice in one asm statement with its wait: the compiler sees no LDS load
        // here, so it adds no wait for the direct-to-LDS loads still in flight into other buffers.
        u32x4 raw[PASSES];
        lds_rows<PASSES, RPP * C * 2>(lds_addr(zc + (lt / LPR) * C * 2 + (lr < PL ? lr : 0) * 16),
                                      raw);
        if constexpr (!LN) {
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                const int row = p * RPP + lt / LPR;
                if (lr < PL)
                    *reinterpret_cast<u32x4*>(xh + row * PL * 16 + 16 * (lr ^ swz(row))) = raw[p];
                if (lr == 0) mrow[row] = TR::to_f(__builtin_bit_cast(E, (uint16_t)mc[p]));
            }
            return;
        }
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int row = p * RPP + lt / LPR;
            // Sum and sum of squares in one pass, as pair dot products on the packed inputs.
            float sum = 0.f, sq = 0.f;
            if (lr < PL) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    sum = dot2<TR>(raw[p][q], kOnePair<TR>, sum);
                    sq = dot2<TR>(raw[p][q], raw[p][q], sq);
                }
            }
            sum = group_sum<LPR>(sum);
            sq = group_sum<LPR>(sq);
            const float mean = sum * (1.f / C);
            const float var = fmaxf(fmaf(sq, 1.f / C, -mean * mean), 0.f);
            const float rstd = __builtin_amdgcn_rsqf(var + eps);
            const float shift = -mean * rstd;
            if (lr < PL) {
                float v[8], x[8];
                unpack8<TR>(raw[p], v);
#pragma unroll
                for (int q = 0; q < 8; ++q) x[q] = fmaf(v[q], rstd, shift);
                *reinterpret_cast<u32x4*>(xh + row * PL * 16 + 16 * (lr ^ swz(row))) =
                    pack8<TR>(x);
            }
            if (lr == 0) mrow[row] = TR::to_f(__builtin_bit_cast(E, (uint16_t)mc[p]));
        }
    };

    // ---- MFMA waves: the gated projections of a normalised tile, stores one step later ----
    u32x4 pend[SUB] = {};
    u32x2 pendc[SUB][2] = {};
    Rsrc pend_out = buffer_rsrc(out, 0);
    // CM: the pending tile's first row in channel 0's plane (null before the first tile). The
    // planes span M*N*2 bytes, past a buffer offset's 32 bits for large M, so the channel-major
    // stores take 64-bit addresses.
    E* pend_plane = nullptr;
    auto out_rsrc = [&](int t) {
        const int rows = min(R, M - t * R);
        return buffer_rsrc(out + (size_t)t * R * N, (uint32_t)rows * N * 2);
    };
    auto flush = [&]() {
        if constexpr (CM) {
            // Rows 16g .. 16g+15 of one column: two 16-byte pieces per lane, which with the
            // other three lane groups fill the column's 128-byte line of the tile.
            if (pend_plane == nullptr) return;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int col = 32 * cb + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
                E* const at = pend_plane + (size_t)col * M + 16 * g;
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const u32x2 a = pendc[2 * half][h], b = pendc[2 * half + 1][h];
                    __builtin_nontemporal_store(u32x4{a[0], a[1], b[0], b[1]},
                                                reinterpret_cast<u32x4*>(at + 8 * half));
                }
            }
        } else {
#pragma unroll
            for (int sub = 0; sub < SUB; ++sub)
                buf_st16(pend_out, ((16 * sub + r16) * N + 32 * cb + 8 * g) * 2, 0, pend[sub]);
        }
    };
    // OST: the branch's N/32 waves store its staged tile as whole rows (four instructions each).
    auto flush_staged = [&](const char* ob) {
        if constexpr (CM) {
            // 64 consecutive 16-byte pieces per instruction: eight channels' 128-byte lines.
            if (pend_plane == nullptr) return;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int f = (i * (N / 32) + cb) * 64 + lane;
                const int ch = f >> 3, piece = f & 7;
                __builtin_nontemporal_store(
                    *reinterpret_cast<const u32x4*>(ob + (br * N + ch) * OSTR + piece * 16),
                    reinterpret_cast<u32x4*>(pend_plane + (size_t)ch * M + piece * 8));
            }
        } else {
            store_staged_rows<R, N, OSTR, N / 32>(pend_out, ob + br * R * OSTR, cb, lane);
        }
    };
    auto project = [&](int t, const char* xh, const float* mrow, char* ob) {
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub) {
            // CM: A row r16 of sub-tile sub is tile row 16*(r16/4) + 4*sub + r16%4, so the C rows
            // 4g+i of the four sub-tiles are the 16 consecutive rows 16g .. 16g+15.
            const int xrow = CM ? 16 * (r16 >> 2) + 4 * sub + (r16 & 3) : 16 * sub + r16;
            f32x4 acc[2][2];
#pragma unroll
            for (int mat = 0; mat < 2; ++mat)
#pragma unroll
                for (int h = 0; h < 2; ++h) acc[mat][h] = binit[mat][h];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const V8 xb = *reinterpret_cast<const V8*>(
                    xh + xrow * PL * 16 + 16 * ((4 * ks + g) ^ swz(xrow)));
#pragma unroll
                for (int mat = 0; mat < 2; ++mat)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        acc[mat][h] = CM ? TR::mfma(xb, wa[mat][h][ks], acc[mat][h])
                                         : TR::mfma(wa[mat][h][ks], xb, acc[mat][h]);
            }
            if constexpr (CM) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    E e[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        e[i] = TR::from_f(mrow[16 * g + 4 * sub + i] * acc[0][h][i] *
                                          fast_rcp(1.f + fast_exp2(acc[1][h][i])));
                    __builtin_memcpy(&pendc[sub][h], e, 8);
                }
            } else {
                const float m = mrow[xrow];
                float o[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const int h = q >> 2, i = q & 3;
                    o[q] = m * acc[0][h][i] * fast_rcp(1.f + fast_exp2(acc[1][h][i]));
                }
                if constexpr (OST)
                    *reinterpret_cast<u32x4*>(ob + (br * R + 16 * sub + r16) * OSTR +
                                              (32 * cb + 8 * g) * 2) = pack8<TR>(o);
                else
                    pend[sub] = pack8<TR>(o);
            }
        }
        if constexpr (CM) {
            if constexpr (OST) {
                // Rows 16g .. 16g+15 of the lane's two columns, as two 16-byte pieces each.
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int col = 32 * cb + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
                    char* const at = ob + (br * N + col) * OSTR + 32 * g;
#pragma unroll
                    for (int half = 0; half < 2; ++half) {
                        const u32x2 a = pendc[2 * half][h], b = pendc[2 * half + 1][h];
                        *reinterpret_cast<u32x4*>(at + 16 * half) = u32x4{a[0], a[1], b[0], b[1]};
                    }
                }
            }
            pend_plane = out + (size_t)t * R;
        } else {
            pend_out = out_rsrc(t);
        }
    };

    // Step j: the LayerNorm waves normalise tile j (and start loading tile j + 2) while the MFMA
    // waves project tile j - 1; one barrier per step. The two roles run separate loops with the
    // same number of barriers, so neither holds the other's registers.
    if (mfma_wave) {
        auto mstep = [&](int j, const char* xr, const float* mr, char* obw, const char* obr) {
            lds_barrier();
            if constexpr (OST) flush_staged(obr);
            else flush();
            if (j >= 1) project(tile_of(j - 1), xr, mr, obw);
        };
        for (int j = 0; j <= mine; j += 2) {
            mstep(j, xh1, mk1, ob0, ob1);
            if (j + 1 > mine) break;
            mstep(j + 1, xh0, mk0, ob1, ob0);
        }
        if constexpr (OST) {
            lds_barrier();  // every wave's part of the last tile is staged (the LayerNorm waves
                            // take this barrier too)
            flush_staged(mine % 2 ? ob1 : ob0);
        } else {
            flush();
        }
    } else {
        uint32_t ma[PASSES], mb[PASSES];
        load_mask(0, ma);
        stage(0, z0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        stage(1, z1);
        auto lstep = [&](int j, const char* zc, char* zn, char* xw, float* mw,
                         uint32_t (&mc)[PASSES], uint32_t (&mn)[PASSES]) {
            vm_wait<DPW>();  // this wave's part of tile j, loaded two steps ago
            lds_barrier();
            if (j < mine) {
                load_mask(j + 1, mn);  // before the tile loads: waiting for it never waits for them
                stage(j + 2, zn);
                normalise(zc, xw, mw, mc);
            }
        };
        for (int j = 0; j <= mine; j += 6) {
            lstep(j, z0, z2, xh0, mk0, ma, mb);
            if (j + 1 > mine) break;
            lstep(j + 1, z1, z0, xh1, mk1, mb, ma);
            if (j + 2 > mine) break;
            lstep(j + 2, z2, z1, xh0, mk0, ma, mb);
            if (j + 3 > mine) break;
            lstep(j + 3, z0, z2, xh1, mk1, mb, ma);
            if (j + 4 > mine) break;
            lstep(j + 4, z1, z0, xh0, mk0, ma, mb);
            if (j + 5 > mine) break;
            lstep(j + 5, z2, z1, xh1, mk1, mb, ma);
        }
        if constexpr (OST) lds_barrier();  // the MFMA waves' last one, before their last stores
    }
    async_wait();  // no direct-to-LDS load may still be in flight when the workgroup ends
}

template <typename F>
void allow_lds(F* kern, size_t bytes) {
    // One attribute call per kernel instantiation (thread-safe, process lifetime).
    static std::once_flag once;
    std::call_once(once, [&] {
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    });
}

constexpr size_t kMaxLds = 160 * 1024;

int row_blocks(int64_t M, int rows_per_block, int cap) {
    const int64_t b = (M + rows_per_block - 1) / rows_per_block;
    return (int)(b < cap ? (b > 0 ? b : 1) : cap);
}

constexpr int kGdpMaxKP = 512;  // contraction rows of the weights staged at a time

template <typename TR, int BN, bool XVEC>
clk_status launch_gdp(hipStream_t st, const void* x, const void* wp, const void* bp,
                      const void* wg, const void* bg, const void* mask, void* out, int M, int K,
                      int N) {
    using E = typename TR::elem;
    const int KP = min((K + 31) / 32 * 32, kGdpMaxKP);
    const size_t lds = (size_t)2 * KP * (BN + 8) * sizeof(E);
    static_assert((size_t)2 * kGdpMaxKP * (64 + 8) * 2 <= kMaxLds, "64-column weight slab fits");
    if (lds > kMaxLds) return fail(CLK_INTERNAL, "gated_dual_proj: K=%d weight slab too large", K);
    allow_lds(gdp_kernel<TR, BN, XVEC>, kMaxLds);
    dim3 grid(row_blocks(M, 256, 2048), (N + BN - 1) / BN);
    KernelTimer timer("gdp", st);
    gdp_kernel<TR, BN, XVEC><<<grid, 256, lds, st>>>((const E*)x, (const E*)wp, (const E*)bp,
                                                      (const E*)wg, (const E*)bg, (const E*)mask,
                                                      (E*)out, M, K, N, KP);
    return check_launch("gated_dual_proj");
}

// The plain gated dual projection through the LN + GDP kernel without its LayerNorm: one branch,
// each wave's 32 output columns of both weights resident in registers, x shared through LDS.
template <typename TR, int K, int N>
clk_status launch_gdp_resident(hipStream_t st, const void* x, const void* wp, const void* bp,
                               const void* wg, const void* bg, const void* mask, void* out,
                               int M) {
    using E = typename TR::elem;
    LnGdpWeights<E> wb;
    wb.w[0] = (const E*)wp;
    wb.w[1] = (const E*)wg;
    wb.b[0] = (const E*)bp;
    wb.b[1] = (const E*)bg;
    wb.w[2] = wb.w[3] = nullptr;  // one branch: the second pair is never read
    wb.b[2] = wb.b[3] = nullptr;
    // Resident blocks per CU: the five 64-row LDS tiles take 80 KB at K = 128 (one block), 40 KB
    // at K = 64 (two).
    const int ntiles = (M + kLnGdpRows - 1) / kLnGdpRows;
    const int per_cu = LnGdpPlan<K, N, 1>::PER_CU;
    const int grid = ntiles < 256 * per_cu ? ntiles : 256 * per_cu;
    KernelTimer timer("gdp", st);
    ln_gdp_kernel<TR, K, N, false, false, 1><<<grid, 2 * N + 256, 0, st>>>(
        (const E*)x, nullptr, nullptr, wb, (const E*)mask, (E*)out, nullptr, M, 0.f);
    return check_launch("gated_dual_proj");
}

template <typename TR, int KS>
clk_status launch_gdp_stream(hipStream_t st, const void* x, const void* wp, const void* bp,
                             const void* wg, const void* bg, const void* mask, void* out, int M,
                             int K, int N) {
    using E = typename TR::elem;
    // Two resident blocks per CU (the 128-column slab of both weights takes 70 KB of LDS at
    // K = 128), each walking row tiles of 64.
    dim3 grid(row_blocks(M, 64, 2 * 256), (N + 127) / 128);
    KernelTimer timer("gdp", st);
    gdp_stream_kernel<TR, KS><<<grid, 256, 0, st>>>((const E*)x, (const E*)wp, (const E*)bp,
                                                     (const E*)wg, (const E*)bg, (const E*)mask,
                                                     (E*)out, M, K, N);
    return check_launch("gated_dual_proj");
}

template <typename TR>
clk_status dispatch_gdp(hipStream_t st, const void* x, const void* wp, const void* bp,
                        const void* wg, const void* bg, const void* mask, void* out, int M, int K,
                        int N) {
    const int KP = (K + 31) / 32 * 32;
#define CLK_GDPR(KK, NN)                                                                           \
    if (K == KK && N == NN)                                                                        \
        return launch_gdp_resident<TR, KK, NN>(st, x, wp, bp, wg, bg, mask, out, M);
    CLK_GDPR(128, 128) CLK_GDPR(128, 64) CLK_GDPR(64, 128) CLK_GDPR(64, 64)
#undef CLK_GDPR
    if (K % 8 == 0 && N >= 64 && K <= 128) {
        if (KP <= 64) return launch_gdp_stream<TR, 2>(st, x, wp, bp, wg, bg, mask, out, M, K, N);
        return launch_gdp_stream<TR, 4>(st, x, wp, bp, wg, bg, mask, out, M, K, N);
    }
    if (K % 8)
        return launch_gdp<TR, 64, false>(st, x, wp, bp, wg, bg, mask, out, M, K, N);
    if (N >= 128 && KP <= 256)
        return launch_gdp<TR, 128, true>(st, x, wp, bp, wg, bg, mask, out, M, K, N);
    return launch_gdp<TR, 64, true>(st, x, wp, bp, wg, bg, mask, out, M, K, N);
}

template <typename TR, int C, int N, bool CM = false>
clk_status launch_ln_gdp(hipStream_t st, const void* z, const float* gamma, const float* beta,
                         const LnGdpWeights<typename TR::elem>& wb, const void* mask, void* a,
                         void* b, int M, float eps) {
    using E = typename TR::elem;
    // One 12-wave block per CU at N = C = 128 (its five 16 KB LDS tiles take half the CU's LDS,
    // its registers three waves per SIMD); narrower N runs more, smaller blocks per CU.
    const int ntiles = (M + kLnGdpRows - 1) / kLnGdpRows;
    const int per_cu = LnGdpPlan<C, N, 2>::PER_CU;
    const int grid = ntiles < 256 * per_cu ? ntiles : 256 * per_cu;
    KernelTimer timer("ln_gdp", st);
    ln_gdp_kernel<TR, C, N, CM><<<grid, 4 * N + 256, 0, st>>>((const E*)z, gamma, beta, wb,
                                                     (const E*)mask, (E*)a, (E*)b, M, eps);
    return check_launch("ln_gated_dual_proj");
}

template <typename TR>
clk_status dispatch_ln_gdp(hipStream_t st, const void* z, const float* gamma, const float* beta,
                           const void* const* w, const void* const* bias, const void* mask,
                           void* a, void* b, int M, int C, int N, float eps) {
    using E = typename TR::elem;
    LnGdpWeights<E> wb;
    for (int i = 0; i < 4; ++i) {
        wb.w[i] = static_cast<const E*>(w[i]);
        wb.b[i] = static_cast<const E*>(bias[i]);
    }
#define CLK_LNGDP(CC, NN)                                                                   \
    if (C == (CC) && N == (NN))                                                             \
        return launch_ln_gdp<TR, CC, NN>(st, z, gamma, beta, wb, mask, a, b, M, eps);
    CLK_LNGDP(128, 128) CLK_LNGDP(128, 64) CLK_LNGDP(64, 128) CLK_LNGDP(64, 64)
    CLK_LNGDP(128, 32) CLK_LNGDP(32, 128) CLK_LNGDP(96, 96) CLK_LNGDP(64, 32) CLK_LNGDP(32, 64)
    CLK_LNGDP(32, 32) CLK_LNGDP(96, 128) CLK_LNGDP(128, 96) CLK_LNGDP(96, 64) CLK_LNGDP(64, 96)
    CLK_LNGDP(96, 32) CLK_LNGDP(32, 96)
#undef CLK_LNGDP
    return fail(CLK_INVALID_ARGUMENT, "ln_gated_dual_proj: C=%d, N=%d not supported", C, N);
}

}  // namespace

// LayerNorm + both gated branches with channel-major outputs a, b [N][M], for the triangle-
// multiplication contraction. Arguments checked by the caller; M % 64 == 0.
clk_status ln_gdp_channel_major(hipStream_t st, clk_dtype dtype, const void* z,
                                const float* gamma, const float* beta, const void* const* w,
                                const void* const* bias, const void* mask, void* a, void* b, int M,
                                int C, int N, float eps) {
    auto run = [&](auto tr) -> clk_status {
        using TR = decltype(tr);
        using E = typename TR::elem;
        LnGdpWeights<E> wb;
        for (int i = 0; i < 4; ++i) {
            wb.w[i] = static_cast<const E*>(w[i]);
            wb.b[i] = static_cast<const E*>(bias[i]);
        }
        if (C == 128 && N == 128)
            return launch_ln_gdp<TR, 128, 128, true>(st, z, gamma, beta, wb, mask, a, b, M, eps);
        if (C == 64 && N == 64)
            return launch_ln_gdp<TR, 64, 64, true>(st, z, gamma, beta, wb, mask, a, b, M, eps);
        return fail(CLK_INVALID_ARGUMENT, "ln_gdp_channel_major: C=%d, N=%d not supported", C, N);
    };
    return dtype == CLK_BF16 ? run(BF16{}) : run(F16{});
}

}  // namespace clk

using namespace clk;

extern "C" clk_status clk_gated_dual_proj(hipStream_t stream, clk_dtype dtype, const void* x,
                                          const void* wp, const void* bp, const void* wg,
                                          const void* bg, const void* mask, void* out, int64_t M,
                                          int64_t K, int64_t N) {
    const char* who = "gated_dual_proj";
    if (dtype != CLK_F16 && dtype != CLK_BF16)
        return fail(CLK_INVALID_ARGUMENT, "%s: dtype %s not supported (f16, bf16)", who,
                    dtype_name(dtype));
    if (M < 0 || K <= 0 || N <= 0) return fail(CLK_INVALID_ARGUMENT, "%s: bad dims", who);
    // Same divisibility rule as the reference for N (cuda/volta_ops.cu:234-236); any K, as the
    // reference's bounds-checked K loop.
    if (N % 8) return fail(CLK_INVALID_ARGUMENT, "%s: N must be a multiple of 8", who);
    if (M > INT32_MAX || K > INT32_MAX || N > (1 << 20))
        return fail(CLK_INVALID_ARGUMENT, "%s: dims too large", who);
    if (M == 0) return ok();
    if (!x || !wp || !bp || !wg || !bg || !mask || !out)
        return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    if (!aligned16(x) || !aligned16(wp) || !aligned16(wg) || !aligned16(out))
        return fail(CLK_INVALID_ARGUMENT, "%s: x, wp, wg, out must be 16-byte aligned", who);
    if (dtype == CLK_BF16)
        return dispatch_gdp<BF16>(stream, x, wp, bp, wg, bg, mask, out, (int)M, (int)K, (int)N);
    return dispatch_gdp<F16>(stream, x, wp, bp, wg, bg, mask, out, (int)M, (int)K, (int)N);
}

extern "C" clk_status clk_ln_gated_dual_proj(hipStream_t stream, clk_dtype dtype, const void* z,
                                             const float* ln_scale, const float* ln_offset,
                                             const void* wpa, const void* bpa, const void* wga,
                                             const void* bga, const void* wpb, const void* bpb,
                                             const void* wgb, const void* bgb, const void* mask,
                                             void* a, void* b, int64_t M, int64_t C, int64_t N,
                                             float eps) {
    const char* who = "ln_gated_dual_proj";
    if (dtype != CLK_F16 && dtype != CLK_BF16)
        return fail(CLK_INVALID_ARGUMENT, "%s: dtype %s not supported (f16, bf16)", who,
                    dtype_name(dtype));
    if (M < 0 || C % 32 || N % 32 || C < 32 || N < 32 || C > 128 || N > 128)
        return fail(CLK_INVALID_ARGUMENT,
                    "%s: C and N must be multiples of 32 in [32, 128] (C=%lld, N=%lld)", who,
                    (long long)C, (long long)N);
    if (M > INT32_MAX) return fail(CLK_INVALID_ARGUMENT, "%s: M too large", who);
    if (M == 0) return ok();
    const void* w[4] = {wpa, wga, wpb, wgb};
    const void* bias[4] = {bpa, bga, bpb, bgb};
    for (int i = 0; i < 4; ++i)
        if (!w[i] || !bias[i]) return fail(CLK_INVALID_ARGUMENT, "%s: null weight", who);
    if (!z || !ln_scale || !ln_offset || !mask || !a || !b)
        return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    if (!aligned16(z) || !aligned16(a) || !aligned16(b))
        return fail(CLK_INVALID_ARGUMENT, "%s: z, a, b must be 16-byte aligned", who);
    if (dtype == CLK_BF16)
        return dispatch_ln_gdp<BF16>(stream, z, ln_scale, ln_offset, w, bias, mask, a, b, (int)M,
                                     (int)C, (int)N, eps);
    return dispatch_ln_gdp<F16>(stream, z, ln_scale, ln_offset, w, bias, mask, a, b, (int)M,
                                (int)C, (int)N, eps);
}
