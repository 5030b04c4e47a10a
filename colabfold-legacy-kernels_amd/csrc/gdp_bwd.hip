// Backward of the gated dual projection (new; the reference is forward-only,
// cuda/volta_ops.cu:97-208):
//   out = mask * p * s,  p = x.wp + bp,  s = sigmoid(x.wg + bg)
//   dp = dout * mask * s,  dg = dout * mask * p * s * (1 - s)
//   dx = dp.wp^T + dg.wg^T,  dwp = x^T.dp,  dwg = x^T.dg,  dbp = sum_m dp,  dbg = sum_m dg
// Four kernels (three at K = N), deterministic (no float atomics):
//   gdp_bwd_grad  recomputes p and the gate on MFMA (weights resident as in the forward) and
//                 writes dpg = [dp | dg] (M x 2N, input dtype) and per-block column sums of dp, dg;
//                 at K = N it also computes dx from the tile it holds;
//   gdp_bwd_dx    dx = dpg . [wp | wg]^T, the transposed weights resident as MFMA A operands;
//   gdp_bwd_dw    per-block partials of x^T . dpg over a contiguous range of rows, both operands
//                 read transposed from LDS (ds_read_b64_tr_b16);
//   gdp_bwd_sum   adds the partials in block order into dwp, dwg, dbp, dbg (float32).
// Layout: x [M,K], wp, wg [K,N], bp, bg [N], mask [M], dout, [M,N], dx [M,K]; K, N in {64, 128}.
// The attention output gate's backward (further below) is the same computation with o in the
// role of p and one weight matrix: its own grad kernel, then gdp_bwd_dx, _dw and _sum with
// NMAT = 1.
#include "common.hpp"

namespace clk {
namespace {

constexpr int kBwdRows = 64;  // rows per tile
// Most rows of one backward call: row and tile indices are 32-bit, and so is the tiles' row
// count rounded up to whole tiles.
constexpr int64_t kMaxBwdM = ((int64_t)1 << 31) - kBwdRows;

// Rows of a [rows, W] 2-byte tile in LDS, 16-byte pieces XOR-swizzled by row % 8 (W >= 128): the
// operand reads of 16 rows and the transposed reads of 4 rows x 32 bytes hit distinct banks.
template <int W>
struct SwzRows {
    static constexpr int PL = W / 8;
    static_assert(PL >= 8, "at least 8 pieces per row");
    __device__ static int piece_at(int row, int piece) { return row * PL + (piece ^ (row & 7)); }
    __device__ static int byte_at(int row, int col) {
        return piece_at(row, col >> 3) * 16 + (col & 7) * 2;
    }
};

// Stages rows [r0, r0 + R) of a [M, W] matrix (the resource covers the valid rows; the rest read
// zeros) into a swizzled LDS tile: every lane issues exactly DP loads. SRC_W > W: the W columns
// are a slice of rows SRC_W elements long.
template <int W, int R, int NT, int SRC_W = W>
__device__ __forceinline__ void stage_swz(Rsrc rsrc, char* lds, int wave, int lane) {
    using S = SwzRows<W>;
    constexpr int SLOTS = R * S::PL, DP = SLOTS / NT;
    static_assert(DP * NT == SLOTS, "whole load rounds");
#pragma unroll
    for (int k = 0; k < DP; ++k) {
        const int b = k * NT + wave * 64, slot = b + lane;
        const int row = slot / S::PL, piece = (slot % S::PL) ^ (row & 7);
        buf_dma16(rsrc, (row * SRC_W + piece * 8) * 2, 0, lds + b * 16);
    }
}

// ---------------------------------------------------------------------------------------------
// dp, dg: wave w of the N/32 waves owns columns 32w..32w+31 of p and of the gate; per 64-row tile
// x arrives by buffer->LDS loads two tiles ahead and dout, mask of the next tile are loaded into
// registers. A lane's accumulators hold 8 consecutive columns of one row, the layout of its
// 16-byte dout vector and of its two 16-byte stores into dpg.
// FDX (K == N): dx of the tile as well, so that dpg is not read back for it. The tile's
// [dp | dg] rows go into LDS in the dx kernel's swizzled layout, and after a second barrier wave
// w computes dx columns 32w..32w+31 = [dp | dg] . wcat^T's rows, held as A operands in registers
// as in the dx kernel (with one wave per SIMD the registers allow it); dx is stored (or added to,
// with accumulate) through a resource per tile.
// ---------------------------------------------------------------------------------------------
template <typename TR, int K, int N, bool FDX = false>
__global__ __launch_bounds__(2 * N) void gdp_bwd_grad_kernel(
    const typename TR::elem* __restrict__ x, const typename TR::elem* __restrict__ wp,
    const typename TR::elem* __restrict__ bp, const typename TR::elem* __restrict__ wg,
    const typename TR::elem* __restrict__ bg, const typename TR::elem* __restrict__ mask,
    const typename TR::elem* __restrict__ dout, typename TR::elem* __restrict__ dpg,
    float* __restrict__ dbpart, int M, typename TR::elem* __restrict__ dx = nullptr,
    int accumulate = 0) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    using S = SwzRows<K < 128 ? 128 : K>;  // K = 64 rows use a 128-wide tile (upper half zero)
    constexpr int KT = K < 128 ? 128 : K;
    constexpr int NT = 2 * N, KS = K / 32, R = kBwdRows, SUB = R / 16;
    constexpr int XB = R * KT * 2;
    constexpr int DPW = R * S::PL / NT;

    static_assert(!FDX || K == N, "the fused dx takes one wave per 32 dx columns: K == N");
    constexpr int W2 = 2 * N, KS2 = W2 / 32;
    using S2 = SwzRows<W2>;

    __shared__ __attribute__((aligned(16))) char x0[XB];
    __shared__ __attribute__((aligned(16))) char x1[XB];
    __shared__ __attribute__((aligned(16))) char x2[XB];
    __shared__ __attribute__((aligned(16))) char tg[FDX ? R * W2 * 2 : 16];  // [dp | dg] tile

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;

    // FDX: wcat^T's rows k = 32w + 8(r16/4) + 4h + r16%4 (8 consecutive n' per 16-byte load).
    V8 wd[FDX ? 2 : 1][FDX ? KS2 : 1];
    if constexpr (FDX) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = 32 * wave + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
#pragma unroll
            for (int ks = 0; ks < KS2; ++ks) {
                const int n = 32 * ks + 8 * g;
                wd[h][ks] = bits_as<V8>(ld16(n < N ? wp + k * N + n : wg + k * N + (n - N)));
            }
        }
    }

    V8 wa[2][2][KS];
    f32x4 binit[2][2];
#pragma unroll
    for (int mat = 0; mat < 2; ++mat) {
        const E* W = mat == 0 ? wp : wg;
        const float fold = mat == 1 ? -kLog2e : 1.f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int col = 32 * wave + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    wa[mat][h][ks][j] = TR::from_f(fold * TR::to_f(W[(32 * ks + 8 * g + j) * N + col]));
            const E* b = mat == 0 ? bp : bg;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                binit[mat][h][i] = fold * TR::to_f(b[32 * wave + 8 * g + 4 * h + i]);
        }
    }

    const int ntiles = (M + R - 1) / R;
    const int col0 = 32 * wave + 8 * g;
    auto rows_of = [&](int t) { return t < ntiles ? min(R, M - t * R) : 0; };
    auto stage = [&](int t, char* xb) {
        const int rows = rows_of(t);
        const Rsrc rx = buffer_rsrc(rows > 0 ? x + (size_t)t * R * K : x, (uint32_t)rows * K * 2);
        if constexpr (K == KT) {
            stage_swz<KT, R, NT>(rx, xb, wave, lane);
        } else {
            // K = 64: pieces 8..15 of each 128-wide row read past the row and are zero-filled by
            // pointing them past the resource.
#pragma unroll
            for (int k = 0; k < DPW; ++k) {
                const int b = k * NT + wave * 64, slot = b + lane;
                const int row = slot / S::PL, piece = (slot % S::PL) ^ (row & 7);
                buf_dma16(rx, piece < K / 8 ? (row * K + piece * 8) * 2 : kPastEnd, 0,
                          xb + b * 16);
            }
        }
    };
    auto load_rows = [&](int t, u32x4 (&dv)[SUB], uint32_t (&mv)[SUB]) {
        const uint16_t* m16 = reinterpret_cast<const uint16_t*>(mask);
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub) {
            const int row = min(t * R + 16 * sub + r16, M - 1);
            dv[sub] = ld16(dout + (size_t)row * N + col0);
            mv[sub] = m16[row];
        }
    };
    auto out_rsrc = [&](int t) {
        const int rows = rows_of(t);
        return buffer_rsrc(rows > 0 ? dpg + (size_t)t * R * 2 * N : dpg,
                           (uint32_t)rows * 2 * N * 2);
    };
    float cs[2][8];  // column sums of dp, dg over this block's rows
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int j = 0; j < 8; ++j) cs[q][j] = 0.f;
    u32x4 res[2][SUB] = {};
    auto store = [&](Rsrc ro) {
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub)
#pragma unroll
            for (int q = 0; q < 2; ++q)
                buf_st16(ro, ((16 * sub + r16) * 2 * N + q * N + col0) * 2, 0, res[q][sub]);
    };

    const int G = gridDim.x;
    u32x4 da[SUB], db[SUB];
    uint32_t ma[SUB], mb[SUB];
    auto tile = [&](int t, const char* xc, char* xn, const u32x4 (&dc)[SUB],
                    const uint32_t (&mc)[SUB], u32x4 (&dn)[SUB], uint32_t (&mn)[SUB]) {
        vm_wait<4 * SUB + DPW>();
        lds_barrier();  // x tile t in xc; every wave is done reading xn
        if (t + G < ntiles) load_rows(t + G, dn, mn);
        stage(t + 2 * G, xn);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const int rows = rows_of(t);
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub) {
            const int xrow = 16 * sub + r16;
            f32x4 acc[2][2];
#pragma unroll
            for (int mat = 0; mat < 2; ++mat)
#pragma unroll
                for (int h = 0; h < 2; ++h) acc[mat][h] = binit[mat][h];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const V8 xv = *reinterpret_cast<const V8*>(xc + S::piece_at(xrow, 4 * ks + g) * 16);
#pragma unroll
                for (int mat = 0; mat < 2; ++mat)
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        acc[mat][h] = TR::mfma(wa[mat][h][ks], xv, acc[mat][h]);
            }
            float d[8], dp[8], dg[8];
            unpack8<TR>(dc[sub], d);
            // Rows past M contribute nothing to the column sums.
            const float m = xrow < rows ? TR::to_f(__builtin_bit_cast(E, (uint16_t)mc[sub])) : 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int h = j >> 2, i = j & 3;
                const float sg = fast_rcp(1.f + fast_exp2(acc[1][h][i]));
                const float dm = d[j] * m;
                dp[j] = dm * sg;
                dg[j] = dp[j] * acc[0][h][i] * (1.f - sg);
                cs[0][j] += dp[j];
                cs[1][j] += dg[j];
            }
            res[0][sub] = pack8<TR>(dp);
            res[1][sub] = pack8<TR>(dg);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        store(out_rsrc(t));
        if constexpr (FDX) {
            // tg is free: every wave finished reading the previous tile's before this tile's
            // first barrier.
#pragma unroll
            for (int sub = 0; sub < SUB; ++sub)
#pragma unroll
                for (int q = 0; q < 2; ++q)
                    *reinterpret_cast<u32x4*>(
                        tg + S2::piece_at(16 * sub + r16, (q * N + col0) / 8) * 16) = res[q][sub];
            lds_barrier();
            const Rsrc rdx = buffer_rsrc(rows > 0 ? dx + (size_t)t * R * K : dx,
                                         (uint32_t)rows * K * 2);
#pragma unroll
            for (int sub = 0; sub < SUB; ++sub) {
                const int xrow = 16 * sub + r16;
                f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
                for (int ks = 0; ks < KS2; ++ks) {
                    const V8 v = *reinterpret_cast<const V8*>(tg + S2::piece_at(xrow, 4 * ks + g) * 16);
#pragma unroll
                    for (int h = 0; h < 2; ++h) acc[h] = TR::mfma(wd[h][ks], v, acc[h]);
                }
                float o[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = acc[j >> 2][j & 3];
                if (accumulate && xrow < rows) {
                    float prev[8];
                    unpack8<TR>(ld16(dx + ((size_t)t * R + xrow) * K + col0), prev);
#pragma unroll
                    for (int j = 0; j < 8; ++j) o[j] += prev[j];
                }
                buf_st16(rdx, (xrow * K + col0) * 2, 0, pack8<TR>(o));
            }
        }
    };

    int t = blockIdx.x;
    const Rsrc none = out_rsrc(ntiles);
    load_rows(t, da, ma);
    stage(t, x0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    store(none);
    stage(t + G, x1);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    store(none);
    for (; t < ntiles; t += 6 * G) {
        tile(t, x0, x2, da, ma, db, mb);
        if (t + G >= ntiles) break;
        tile(t + G, x1, x0, db, mb, da, ma);
        if (t + 2 * G >= ntiles) break;
        tile(t + 2 * G, x2, x1, da, ma, db, mb);
        if (t + 3 * G >= ntiles) break;
        tile(t + 3 * G, x0, x2, db, mb, da, ma);
        if (t + 4 * G >= ntiles) break;
        tile(t + 4 * G, x1, x0, da, ma, db, mb);
        if (t + 5 * G >= ntiles) break;
        tile(t + 5 * G, x2, x1, db, mb, da, ma);
    }
    // Column sums: the 16 lanes of a lane group hold the same 8 columns of different rows.
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int j = 0; j < 8; ++j) cs[q][j] = group_sum<16>(cs[q][j]);
    if (r16 == 0) {
        float* o = dbpart + (size_t)blockIdx.x * 2 * N;
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int j = 0; j < 8; ++j) o[q * N + col0 + j] = cs[q][j];
    }
    async_wait();
}

// ---------------------------------------------------------------------------------------------
// The attention output gate's backward (attention_gate.hip: out[m, c] = o'[m, c] * s[m, c],
// s = sigmoid(x.wg + bg), o'[m, h*D + d] = o[n, h, s, d] for m = n*Sq + s):
//   do = dout * s (written in o's [N, H, Sq, D] layout, the attention backward's dout),
//   dgl = dout * o' * s * (1 - s) ([M, N] into the workspace, for dx, dwg and dbg).
// The grad kernel of the gated dual projection with o' in the role of the projection p and one
// weight matrix: wave w of the N/32 waves owns gate columns 32w..32w+31 (8 consecutive columns
// per lane: 8 consecutive d of one head, D % 8 == 0), x tiles arrive by buffer->LDS loads two
// tiles ahead, and the dout and o vectors of the next tile are loaded into registers (of the
// current tile, at its start, when K = N = 256: a second set would not fit 256 registers).
// ---------------------------------------------------------------------------------------------
template <typename TR, int K, int N>
__global__ __launch_bounds__(2 * N) void gate_bwd_grad_kernel(
    const typename TR::elem* __restrict__ o, const typename TR::elem* __restrict__ x,
    const typename TR::elem* __restrict__ wg, const typename TR::elem* __restrict__ bg,
    const typename TR::elem* __restrict__ dout, typename TR::elem* __restrict__ dov,
    typename TR::elem* __restrict__ dgl, float* __restrict__ dbpart, int M, int H, int Sq,
    int D) {
    using V8 = typename TR::vec8;
    using S = SwzRows<K < 128 ? 128 : K>;  // K = 64 rows use a 128-wide tile (upper half zero)
    constexpr int KT = K < 128 ? 128 : K;
    constexpr int NT = 2 * N, KS = K / 32, R = kBwdRows, SUB = R / 16;
    constexpr int XB = R * KT * 2;
    constexpr int DPW = R * S::PL / NT;
    constexpr bool PREF = K < 256 || N < 256;  // dout, o of the next tile in registers

    __shared__ __attribute__((aligned(16))) char x0[XB];
    __shared__ __attribute__((aligned(16))) char x1[XB];
    __shared__ __attribute__((aligned(16))) char x2[XB];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;

    // Resident A operands -log2(e) * wg^T and the matching bias, as in the forward gate.
    V8 wa[2][KS];
    f32x4 binit[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int col = 32 * wave + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                wa[h][ks][j] = TR::from_f(-kLog2e * TR::to_f(wg[(32 * ks + 8 * g + j) * N + col]));
#pragma unroll
        for (int i = 0; i < 4; ++i)
            binit[h][i] = -kLog2e * TR::to_f(bg[32 * wave + 8 * g + 4 * h + i]);
    }

    const int ntiles = (M + R - 1) / R;
    const int col0 = 32 * wave + 8 * g;
    const int hd = col0 / D, d0 = col0 - hd * D;  // the lane's head and first d
    auto rows_of = [&](int t) { return t < ntiles ? min(R, M - t * R) : 0; };
    // Element offset of (row m, column col0) in o's [N, H, Sq, D] layout.
    auto o_at = [&](int m) {
        const int n = m / Sq, sq = m - n * Sq;
        return (((size_t)n * H + hd) * Sq + sq) * D + d0;
    };
    auto stage = [&](int t, char* xb) {
        const int rows = rows_of(t);
        const Rsrc rx = buffer_rsrc(rows > 0 ? x + (size_t)t * R * K : x, (uint32_t)rows * K * 2);
        if constexpr (K == KT) {
            stage_swz<KT, R, NT>(rx, xb, wave, lane);
        } else {
#pragma unroll
            for (int k = 0; k < DPW; ++k) {
                const int b = k * NT + wave * 64, slot = b + lane;
                const int row = slot / S::PL, piece = (slot % S::PL) ^ (row & 7);
                buf_dma16(rx, piece < K / 8 ? (row * K + piece * 8) * 2 : kPastEnd, 0,
                          xb + b * 16);
            }
        }
    };
    // dout and o of a tile's rows (rows past M read row M - 1 and are never stored).
    auto load_rows = [&](int t, u32x4 (&dv)[SUB], u32x4 (&ov)[SUB]) {
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub) {
            const int row = min(t * R + 16 * sub + r16, M - 1);
            dv[sub] = ld16(dout + (size_t)row * N + col0);
            ov[sub] = ld16(o + o_at(row));
        }
    };
    auto out_rsrc = [&](int t) {
        const int rows = rows_of(t);
        return buffer_rsrc(rows > 0 ? dgl + (size_t)t * R * N : dgl, (uint32_t)rows * N * 2);
    };
    float cs[8];  // column sums of dgl over this block's rows
#pragma unroll
    for (int j = 0; j < 8; ++j) cs[j] = 0.f;
    // do of tile t through a resource based at its first row's sample n0 (element n0*H*Sq*D of
    // do), covering at most 2^30 - 16 bytes from there: the tile's rows lie in samples n0 and
    // n0 + 1 (Sq >= 64) or within 3 * 64 rows of n0's first (Sq < 64), so with Sq*H*D*4 < 2^30
    // bytes every offset fits. Rows past M get an offset past its end and are dropped, so every
    // tile issues the same 2 * SUB stores (two per sub-tile, as soon as it is computed), the
    // count the waits below assume.
    struct DoTile {
        Rsrc r;
        int n0;  // the sample the resource starts at
    };
    auto do_tile = [&](int t) {
        const int rows = rows_of(t);
        if (rows == 0) return DoTile{buffer_rsrc(dov, 0), 0};
        const int n0 = (t * R) / Sq;
        const size_t base = (size_t)n0 * H * Sq * D;
        const size_t left = ((size_t)M * N - base) * 2;
        const size_t cap = (size_t)kPastEnd - 16;
        return DoTile{buffer_rsrc(dov + base, (uint32_t)(left < cap ? left : cap)), n0};
    };
    // Byte offset of (row m, column col0) from sample n0's first element (32-bit: bounded above).
    auto do_at = [&](int m, int n0) {
        const int n = m / Sq, sq = m - n * Sq;
        return ((((n - n0) * H + hd) * Sq + sq) * D + d0) * 2;
    };
    auto store_sub = [&](Rsrc rd, const DoTile& dt, int t, int rows, int sub, u32x4 vg,
                         u32x4 vo) {
        const int xrow = 16 * sub + r16;
        buf_st16(rd, (xrow * N + col0) * 2, 0, vg);
        buf_st16(dt.r, xrow < rows ? do_at(t * R + xrow, dt.n0) : kPastEnd, 0, vo);
    };

    const int G = gridDim.x;
    u32x4 da[SUB], db[SUB], oa[SUB], ob[SUB];
    auto tile = [&](int t, const char* xc, char* xn, u32x4 (&dc)[SUB], u32x4 (&oc)[SUB],
                    u32x4 (&dn)[SUB], u32x4 (&on)[SUB]) {
        vm_wait<4 * SUB + DPW>();
        lds_barrier();  // x tile t in xc; every wave is done reading xn
        if constexpr (PREF) {
            if (t + G < ntiles) load_rows(t + G, dn, on);
        } else {
            load_rows(t, dc, oc);
        }
        stage(t + 2 * G, xn);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const int rows = rows_of(t);
        const Rsrc rd = out_rsrc(t);
        const DoTile dt = do_tile(t);
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub) {
            const int xrow = 16 * sub + r16;
            f32x4 acc[2] = {binit[0], binit[1]};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const V8 xv = *reinterpret_cast<const V8*>(xc + S::piece_at(xrow, 4 * ks + g) * 16);
#pragma unroll
                for (int h = 0; h < 2; ++h) acc[h] = TR::mfma(wa[h][ks], xv, acc[h]);
            }
            float d[8], ov[8], dov8[8], dg[8];
            unpack8<TR>(dc[sub], d);
            unpack8<TR>(oc[sub], ov);
            // Rows past M contribute nothing to the column sums.
            const float live = xrow < rows ? 1.f : 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float sg = fast_rcp(1.f + fast_exp2(acc[j >> 2][j & 3]));
                dov8[j] = d[j] * sg;
                dg[j] = dov8[j] * ov[j] * (1.f - sg);
                cs[j] += live * dg[j];
            }
            store_sub(rd, dt, t, rows, sub, pack8<TR>(dg), pack8<TR>(dov8));
        }
    };

    int t = blockIdx.x;
    if constexpr (PREF) load_rows(t, da, oa);
    stage(t, x0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    // Stores of no rows (all dropped): the per-tile count of memory operations the waits assume.
    const u32x4 zero = {0u, 0u, 0u, 0u};
    const Rsrc none = out_rsrc(ntiles);
    const DoTile no_do = do_tile(ntiles);
#pragma unroll
    for (int sub = 0; sub < SUB; ++sub) store_sub(none, no_do, ntiles, 0, sub, zero, zero);
    stage(t + G, x1);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int sub = 0; sub < SUB; ++sub) store_sub(none, no_do, ntiles, 0, sub, zero, zero);
    // Without PREF every tile uses the one register set (da, oa).
    u32x4 (&dB)[SUB] = PREF ? db : da;
    u32x4 (&oB)[SUB] = PREF ? ob : oa;
    for (; t < ntiles; t += 6 * G) {
        tile(t, x0, x2, da, oa, dB, oB);
        if (t + G >= ntiles) break;
        tile(t + G, x1, x0, dB, oB, da, oa);
        if (t + 2 * G >= ntiles) break;
        tile(t + 2 * G, x2, x1, da, oa, dB, oB);
        if (t + 3 * G >= ntiles) break;
        tile(t + 3 * G, x0, x2, dB, oB, da, oa);
        if (t + 4 * G >= ntiles) break;
        tile(t + 4 * G, x1, x0, da, oa, dB, oB);
        if (t + 5 * G >= ntiles) break;
        tile(t + 5 * G, x2, x1, dB, oB, da, oa);
    }
    // Column sums: the 16 lanes of a lane group hold the same 8 columns of different rows.
#pragma unroll
    for (int j = 0; j < 8; ++j) cs[j] = group_sum<16>(cs[j]);
    if (r16 == 0) {
        float* out = dbpart + (size_t)blockIdx.x * N;
#pragma unroll
        for (int j = 0; j < 8; ++j) out[col0 + j] = cs[j];
    }
    async_wait();
}

// ---------------------------------------------------------------------------------------------
// dx = dpg . wcat with wcat[n'][k] = n' < N ? wp[k][n'] : wg[k][n' - N]: wave w of the K/32
// waves owns dx columns 32w..32w+31 and holds wcat^T's matching rows (16-byte loads of wp, wg
// rows) as A operands; dpg rows arrive two tiles ahead. NMAT = 1: one weight matrix, wp
// (dpg [M, N], the attention gate's backward).
// ---------------------------------------------------------------------------------------------
template <typename TR, int K, int N, int NMAT = 2>
__global__ __launch_bounds__(2 * K) void gdp_bwd_dx_kernel(
    const typename TR::elem* __restrict__ dpg, const typename TR::elem* __restrict__ wp,
    const typename TR::elem* __restrict__ wg, typename TR::elem* __restrict__ dx, int M,
    int accumulate) {
    using V8 = typename TR::vec8;
    constexpr int W2 = NMAT * N;
    using S = SwzRows<W2>;
    constexpr int NT = 2 * K, KS = W2 / 32, R = kBwdRows, SUB = R / 16;
    constexpr int TB = R * W2 * 2;
    constexpr int DPW = R * S::PL / NT;
    static_assert(DPW * NT == R * S::PL, "whole load rounds");

    __shared__ __attribute__((aligned(16))) char t0[TB];
    __shared__ __attribute__((aligned(16))) char t1[TB];
    __shared__ __attribute__((aligned(16))) char t2[TB];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;

    V8 wa[2][KS];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int k = 32 * wave + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int n = 32 * ks + 8 * g;  // 8 consecutive n' of one matrix row
            wa[h][ks] = bits_as<V8>(ld16(n < N ? wp + k * N + n : wg + k * N + (n - N)));
        }
    }

    const int ntiles = (M + R - 1) / R;
    const int col0 = 32 * wave + 8 * g;
    auto rows_of = [&](int t) { return t < ntiles ? min(R, M - t * R) : 0; };
    auto stage = [&](int t, char* tb) {
        const int rows = rows_of(t);
        const Rsrc r = buffer_rsrc(rows > 0 ? dpg + (size_t)t * R * W2 : dpg,
                                   (uint32_t)rows * W2 * 2);
        stage_swz<W2, R, NT>(r, tb, wave, lane);
    };
    auto out_rsrc = [&](int t) {
        const int rows = rows_of(t);
        return buffer_rsrc(rows > 0 ? dx + (size_t)t * R * K : dx, (uint32_t)rows * K * 2);
    };
    u32x4 res[SUB] = {};
    auto store = [&](Rsrc ro) {
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub)
            buf_st16(ro, ((16 * sub + r16) * K + col0) * 2, 0, res[sub]);
    };

    const int G = gridDim.x;
    auto tile = [&](int t, const char* tc, char* tn) {
        vm_wait<2 * SUB + DPW>();
        lds_barrier();
        stage(t + 2 * G, tn);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const int rows = rows_of(t);
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub) {
            const int xrow = 16 * sub + r16;
            f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const V8 v = *reinterpret_cast<const V8*>(tc + S::piece_at(xrow, 4 * ks + g) * 16);
#pragma unroll
                for (int h = 0; h < 2; ++h) acc[h] = TR::mfma(wa[h][ks], v, acc[h]);
            }
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = acc[j >> 2][j & 3];
            if (accumulate && xrow < rows) {
                float prev[8];
                unpack8<TR>(ld16(dx + ((size_t)t * R + xrow) * K + col0), prev);
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] += prev[j];
            }
            res[sub] = pack8<TR>(o);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        store(out_rsrc(t));
    };

    int t = blockIdx.x;
    const Rsrc none = out_rsrc(ntiles);
    stage(t, t0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    store(none);
    stage(t + G, t1);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    store(none);
    for (; t < ntiles; t += 3 * G) {
        tile(t, t0, t2);
        if (t + G >= ntiles) break;
        tile(t + G, t1, t0);
        if (t + 2 * G >= ntiles) break;
        tile(t + 2 * G, t2, t1);
    }
    async_wait();
}

// ---------------------------------------------------------------------------------------------
// Partials of x^T . dpg: block b sums rows [b*RB, (b+1)*RB). 8 waves: wave (wk, wn) owns dw^T
// rows n' = 128wn + 16nt + (0..15) and columns k = 32wk + 16kt + (0..15) -- accumulators with
// A = dpg^T (transposed read of the dpg tile) and B = x^T (transposed read of the x tile), so a
// lane's accumulator holds four consecutive k of one n' and the partial is written [2N][K].
// NMAT = 1: dpg has N columns ([N][K] partials). NSPLIT = 2: the n' range is split between
// blockIdx.y = 0 and 1, each block staging and accumulating its half of the dpg columns (a
// [2N x K] partial over 8 waves would not fit their registers at 2N = K = 256).
// ---------------------------------------------------------------------------------------------
template <typename TR, int K, int N, int NMAT = 2, int NSPLIT = 1>
__global__ __launch_bounds__(512) void gdp_bwd_dw_kernel(const typename TR::elem* __restrict__ x,
                                                         const typename TR::elem* __restrict__ dpg,
                                                         float* __restrict__ part, int M,
                                                         int tiles_per_block) {
    using V8 = typename TR::vec8;
    constexpr int W2 = NMAT * N, WB = W2 / NSPLIT, KT = K < 128 ? 128 : K;
    using SX = SwzRows<KT>;
    using SG = SwzRows<WB>;
    constexpr int NT = 512, R = kBwdRows;
    constexpr int XB = R * KT * 2, GB = R * WB * 2;
    constexpr int DPX = R * SX::PL / NT, DPG = R * SG::PL / NT;
    constexpr int WK = K / 32;                 // waves along k (32 k each)
    constexpr int WN = 8 / WK;                 // waves along n'
    constexpr int NTL = WB / (16 * WN);        // 16-wide n' tiles per wave
    static_assert(WK * WN == 8 && NTL * 16 * WN == WB, "eight waves cover [WB x K]");

    // Separate arrays per stage: the compiler then sees that a stage being read is not the one
    // being loaded.
    __shared__ __attribute__((aligned(16))) char x0[XB];
    __shared__ __attribute__((aligned(16))) char x1[XB];
    __shared__ __attribute__((aligned(16))) char x2[XB];
    __shared__ __attribute__((aligned(16))) char g0[GB];
    __shared__ __attribute__((aligned(16))) char g1[GB];
    __shared__ __attribute__((aligned(16))) char g2[GB];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int wk = wave % WK, wn = wave / WK;

    const int row0 = blockIdx.x * tiles_per_block * R;
    const int nt = tiles_per_block;
    const int n_off = NSPLIT > 1 ? (int)blockIdx.y * WB : 0;  // first dpg column of the block
    auto stage = [&](int i, char* xb, char* gb) {
        const int r0 = row0 + i * R;
        const int rows = i < nt ? max(0, min(R, M - r0)) : 0;
        const Rsrc rx = buffer_rsrc(rows > 0 ? x + (size_t)r0 * K : x, (uint32_t)rows * K * 2);
        const Rsrc rg = buffer_rsrc(rows > 0 ? dpg + (size_t)r0 * W2 + n_off : dpg,
                                    rows > 0 ? (uint32_t)(rows * W2 - n_off) * 2 : 0u);
        if constexpr (K == KT) {
            stage_swz<KT, R, NT>(rx, xb, wave, lane);
        } else {
#pragma unroll
            for (int k = 0; k < DPX; ++k) {
                const int b = k * NT + wave * 64, slot = b + lane;
                const int row = slot / SX::PL, piece = (slot % SX::PL) ^ (row & 7);
                buf_dma16(rx, piece < K / 8 ? (row * K + piece * 8) * 2 : kPastEnd, 0,
                          xb + b * 16);
            }
        }
        stage_swz<WB, R, NT, W2>(rg, gb, wave, lane);
    };

    f32x4 acc[NTL][2];
#pragma unroll
    for (int a = 0; a < NTL; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto step = [&](int i, const char* xc, const char* gc, char* xn, char* gn) {
        vm_wait<DPX + DPG>();
        lds_barrier();
        stage(i + 2, xn, gn);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        // The lane's row and column within each transposed read, made opaque here so that the
        // per-tile LDS addresses are formed in the step instead of being held in registers
        // across it.
        int lr = lane;
        asm volatile("" : "+v"(lr));
        const int tcol = 4 * (lr & 3), trow = 8 * (lr >> 4) + ((lr >> 2) & 3);
        // Transposed operand: lane (r16, g) gets column c0 + r16 of rows 8g + ms .. 8g + ms + 7
        // of a swizzled tile (two 4-row transposed reads).
        auto tr_operand = [&](const char* base, auto swz, int ms, int c0) {
            using SW = decltype(swz);
            const int rlo = ms + trow;
            return lds_tr8<V8>(base + SW::byte_at(rlo, c0 + tcol),
                               base + SW::byte_at(rlo + 4, c0 + tcol));
        };
#pragma unroll
        for (int ms = 0; ms < R; ms += 32) {
            V8 bx[2];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) bx[kt] = tr_operand(xc, SX{}, ms, 32 * wk + 16 * kt);
#pragma unroll
            for (int a = 0; a < NTL; ++a) {
                const V8 ag = tr_operand(gc, SG{}, ms, (NTL * wn + a) * 16);
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) acc[a][kt] = TR::mfma(ag, bx[kt], acc[a][kt]);
            }
        }
    };

    stage(0, x0, g0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    stage(1, x1, g1);
    for (int i = 0; i < nt; i += 3) {
        step(i, x0, g0, x2, g2);
        if (i + 1 >= nt) break;
        step(i + 1, x1, g1, x0, g0);
        if (i + 2 >= nt) break;
        step(i + 2, x2, g2, x1, g1);
    }
    // C lane (r16, g) of accumulator (a, kt): n' = n_off + (NTL*wn + a)*16 + 4g + q,
    // k = 32wk + 16kt + r16.
    float* pb = part + (size_t)blockIdx.x * (W2 * K + W2);
#pragma unroll
    for (int a = 0; a < NTL; ++a)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n_off + (NTL * wn + a) * 16 + 4 * g + q;
                pb[n * K + 32 * wk + 16 * kt + r16] = acc[a][kt][q];
            }
    async_wait();
}

// dwp, dwg [K][N] and dbp, dbg [N] from nb partials [nb][2N*K + 2N] ([2N][K] then [2N]) and the
// grad kernel's column sums [ng][2N]. A block owns 64 consecutive outputs: thread (c, s) adds the
// partials s, s + 16, s + 32, ... of four consecutive outputs (16-byte loads, eight in flight), and
// the 16 subtotals are then added in s order -- a fixed order, so the sums are reproducible.
// NMAT = 1: partials [nb][N*K + N] and column sums [ng][N], all into dwp and dbp.
template <int K, int N, int NMAT = 2>
__global__ __launch_bounds__(256) void gdp_bwd_sum_kernel(const float* __restrict__ part, int nb,
                                                          const float* __restrict__ dbpart, int ng,
                                                          float* __restrict__ dwp,
                                                          float* __restrict__ dwg,
                                                          float* __restrict__ dbp,
                                                          float* __restrict__ dbg) {
    constexpr int W2 = NMAT * N, PS = W2 * K + W2, NW = W2 * K;
    static_assert(NW % 64 == 0 && W2 % 64 == 0 && PS % 4 == 0, "whole 64-output blocks");
    __shared__ f32x4 sub[16][16];
    const int c = threadIdx.x % 16, s = threadIdx.x / 16;
    const int e0 = blockIdx.x * 64;  // first output of the block; [0, NW) weights, then biases
    const bool weights = e0 < NW;
    const float* src = weights ? part + e0 + 4 * c : dbpart + (e0 - NW) + 4 * c;
    const int stride = weights ? PS : W2, count = weights ? nb : ng;
    constexpr int kIn = 8;  // loads issued before their adds (in b order)
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
    for (int b0 = s; b0 < count; b0 += 16 * kIn) {
        f32x4 v[kIn];
#pragma unroll
        for (int i = 0; i < kIn; ++i) {
            const int b = b0 + 16 * i;
            v[i] = b < count ? *reinterpret_cast<const f32x4*>(src + (size_t)b * stride)
                             : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int i = 0; i < kIn; ++i) a += v[i];
    }
    sub[s][c] = a;
    __syncthreads();
    if (s != 0) return;
    f32x4 t = sub[0][c];
#pragma unroll
    for (int q = 1; q < 16; ++q) t += sub[q][c];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int e = e0 + 4 * c + q;
        if (weights) {
            const int n = e / K, k = e % K;
            if (n < N) dwp[k * N + n] = t[q];
            else dwg[k * N + (n - N)] = t[q];
        } else {
            const int n = e - NW;
            if (n < N) dbp[n] = t[q];
            else dbg[n - N] = t[q];
        }
    }
}

struct BwdGeom {
    int grad_blocks, dw_blocks, dw_tiles;
    size_t dpg_off, part_off, dbpart_off, total;
};

BwdGeom bwd_geom(int64_t M, int K, int N) {
    BwdGeom g;
    const int64_t ntiles = (M + kBwdRows - 1) / kBwdRows;
    const int per_cu = 128 / N;
    g.grad_blocks = (int)(ntiles < 256 * per_cu ? ntiles : 256 * per_cu);
    g.dw_blocks = (int)(ntiles < 256 ? ntiles : 256);
    g.dw_tiles = (int)((ntiles + g.dw_blocks - 1) / g.dw_blocks);
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    g.dpg_off = 0;
    g.part_off = up((size_t)M * 2 * N * 2);
    g.dbpart_off = g.part_off + up((size_t)g.dw_blocks * (2 * N * K + 2 * N) * 4);
    g.total = g.dbpart_off + up((size_t)g.grad_blocks * 2 * N * 4);
    return g;
}

template <typename TR, int K, int N>
clk_status run_gdp_bwd(hipStream_t st, const void* x, const void* wp, const void* bp,
                       const void* wg, const void* bg, const void* mask, const void* dout,
                       void* dx, float* dwp, float* dbp, float* dwg, float* dbg, char* ws, int M,
                       int accumulate) {
    using E = typename TR::elem;
    const BwdGeom gm = bwd_geom(M, K, N);
    E* dpg = reinterpret_cast<E*>(ws + gm.dpg_off);
    float* part = reinterpret_cast<float*>(ws + gm.part_off);
    float* dbpart = reinterpret_cast<float*>(ws + gm.dbpart_off);
    if constexpr (K == N) {
        // dx computed by the grad kernel from the tile it already holds.
        KernelTimer timer("gdp_bwd_grad", st);
        gdp_bwd_grad_kernel<TR, K, N, true><<<gm.grad_blocks, 2 * N, 0, st>>>(
            (const E*)x, (const E*)wp, (const E*)bp, (const E*)wg, (const E*)bg, (const E*)mask,
            (const E*)dout, dpg, dbpart, M, (E*)dx, accumulate);
    } else {
        {
            KernelTimer timer("gdp_bwd_grad", st);
            gdp_bwd_grad_kernel<TR, K, N><<<gm.grad_blocks, 2 * N, 0, st>>>(
                (const E*)x, (const E*)wp, (const E*)bp, (const E*)wg, (const E*)bg,
                (const E*)mask, (const E*)dout, dpg, dbpart, M);
        }
        const int ntiles = (M + kBwdRows - 1) / kBwdRows;
        const int per_cu = 128 / K;
        const int grid = ntiles < 256 * per_cu ? ntiles : 256 * per_cu;
        KernelTimer timer("gdp_bwd_dx", st);
        gdp_bwd_dx_kernel<TR, K, N><<<grid, 2 * K, 0, st>>>(dpg, (const E*)wp, (const E*)wg,
                                                           (E*)dx, M, accumulate);
    }
    {
        KernelTimer timer("gdp_bwd_dw", st);
        gdp_bwd_dw_kernel<TR, K, N><<<gm.dw_blocks, 512, 0, st>>>((const E*)x, dpg, part, M,
                                                                  gm.dw_tiles);
    }
    {
        constexpr int count = 2 * N * K + 2 * N;
        KernelTimer timer("gdp_bwd_sum", st);
        gdp_bwd_sum_kernel<K, N><<<count / 64, 256, 0, st>>>(
            part, gm.dw_blocks, dbpart, gm.grad_blocks, dwp, dwg, dbp, dbg);
    }
    return check_launch("gated_dual_proj_bwd");
}

// M = 0: the weight and bias gradients are sums over no rows, i.e. zero. The sum kernel with no
// partials writes exactly that (a fill kernel, so the call stays graph-capturable).
clk_status zero_gdp_bwd(hipStream_t st, float* dwp, float* dbp, float* dwg, float* dbg, int K,
                        int N) {
#define CLK_GDPZ(KK, NN)                                                                       \
    if (K == (KK) && N == (NN)) {                                                              \
        constexpr int count = 2 * NN * KK + 2 * NN;                                            \
        gdp_bwd_sum_kernel<KK, NN><<<count / 64, 256, 0, st>>>(nullptr, 0, nullptr, 0, dwp,     \
                                                               dwg, dbp, dbg);                 \
        return check_launch("gated_dual_proj_bwd");                                             \
    }
    CLK_GDPZ(128, 128) CLK_GDPZ(64, 64) CLK_GDPZ(128, 64) CLK_GDPZ(64, 128)
#undef CLK_GDPZ
    return fail(CLK_INVALID_ARGUMENT, "gated_dual_proj_bwd: K=%d, N=%d not supported", K, N);
}

template <typename TR>
clk_status dispatch_gdp_bwd(hipStream_t st, const void* x, const void* wp, const void* bp,
                            const void* wg, const void* bg, const void* mask, const void* dout,
                            void* dx, float* dwp, float* dbp, float* dwg, float* dbg, char* ws,
                            int M, int K, int N, int accumulate) {
#define CLK_GDPB(KK, NN)                                                                   \
    if (K == (KK) && N == (NN))                                                            \
        return run_gdp_bwd<TR, KK, NN>(st, x, wp, bp, wg, bg, mask, dout, dx, dwp, dbp, dwg, \
                                       dbg, ws, M, accumulate);
    CLK_GDPB(128, 128) CLK_GDPB(64, 64) CLK_GDPB(128, 64) CLK_GDPB(64, 128)
#undef CLK_GDPB
    return fail(CLK_INVALID_ARGUMENT, "gated_dual_proj_bwd: K=%d, N=%d not supported", K, N);
}

// ---- The attention output gate's backward: the grad kernel above, then the dx, dw and sum
// kernels with one weight matrix (K = C input channels, N = H*D gate columns). ----

// Halves of the gate columns per dw block: one, except at C = H*D = 256, where a block's
// [256 x 256] partial would not fit its eight waves' registers (and three stages of both 64-row
// tiles would not fit the LDS).
constexpr int gate_dw_split(int C, int HD) { return C == 256 && HD == 256 ? 2 : 1; }
// Blocks per CU of a kernel holding three staged 64-row tiles of `width` 2-byte columns.
constexpr int three_stage_per_cu(int width) {
    const int b = 160 * 1024 / (3 * kBwdRows * width * 2);
    return b < 1 ? 1 : (b > 4 ? 4 : b);
}

struct GateBwdGeom {
    int grad_blocks, dx_blocks, dw_blocks, dw_tiles;
    size_t dgl_off, part_off, dbpart_off, total;
};

GateBwdGeom gate_bwd_geom(int64_t M, int C, int HD) {
    GateBwdGeom g;
    const int64_t ntiles = (M + kBwdRows - 1) / kBwdRows;
    auto cap = [&](int64_t blocks) { return (int)(ntiles < blocks ? ntiles : blocks); };
    g.grad_blocks = cap(256 * three_stage_per_cu(C < 128 ? 128 : C));
    g.dx_blocks = cap(256 * three_stage_per_cu(HD));
    const int cap_dw = 256 / gate_dw_split(C, HD);
    g.dw_blocks = (int)(ntiles < cap_dw ? ntiles : cap_dw);
    g.dw_tiles = g.dw_blocks > 0 ? (int)((ntiles + g.dw_blocks - 1) / g.dw_blocks) : 0;
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    g.dgl_off = 0;
    g.part_off = up((size_t)M * HD * 2);
    g.dbpart_off = g.part_off + up((size_t)g.dw_blocks * (HD * C + HD) * 4);
    g.total = g.dbpart_off + up((size_t)g.grad_blocks * HD * 4);
    return g;
}

template <typename TR, int C, int HD>
clk_status run_gate_bwd(hipStream_t st, const void* o, const void* x, const void* wg,
                        const void* bg, const void* dout, void* dov, void* dx, float* dwg,
                        float* dbg, char* ws, int M, int H, int Sq, int D, int accumulate) {
    using E = typename TR::elem;
    const GateBwdGeom gm = gate_bwd_geom(M, C, HD);
    E* dgl = reinterpret_cast<E*>(ws + gm.dgl_off);
    float* part = reinterpret_cast<float*>(ws + gm.part_off);
    float* dbpart = reinterpret_cast<float*>(ws + gm.dbpart_off);
    {
        KernelTimer timer("gate_bwd_grad", st);
        gate_bwd_grad_kernel<TR, C, HD><<<gm.grad_blocks, 2 * HD, 0, st>>>(
            (const E*)o, (const E*)x, (const E*)wg, (const E*)bg, (const E*)dout, (E*)dov, dgl,
            dbpart, M, H, Sq, D);
    }
    {
        KernelTimer timer("gate_bwd_dx", st);
        gdp_bwd_dx_kernel<TR, C, HD, 1><<<gm.dx_blocks, 2 * C, 0, st>>>(
            dgl, (const E*)wg, (const E*)wg, (E*)dx, M, accumulate);
    }
    {
        KernelTimer timer("gate_bwd_dw", st);
        constexpr int split = gate_dw_split(C, HD);
        gdp_bwd_dw_kernel<TR, C, HD, 1, split><<<dim3(gm.dw_blocks, split), 512, 0, st>>>(
            (const E*)x, dgl, part, M, gm.dw_tiles);
    }
    {
        constexpr int count = HD * C + HD;
        KernelTimer timer("gate_bwd_sum", st);
        gdp_bwd_sum_kernel<C, HD, 1><<<count / 64, 256, 0, st>>>(
            part, gm.dw_blocks, dbpart, gm.grad_blocks, dwg, nullptr, dbg, nullptr);
    }
    return check_launch("attention_gate_bwd");
}

#define CLK_GATE_SHAPES(X) \
    X(64, 64) X(64, 128) X(64, 256) X(128, 64) X(128, 128) X(128, 256) X(256, 64) X(256, 128) \
    X(256, 256)

// M = 0: zero weight and bias gradients (the sum kernel with no partials, a fill kernel).
clk_status zero_gate_bwd(hipStream_t st, float* dwg, float* dbg, int C, int HD) {
#define CLK_GATEZ(CC, NN)                                                                 \
    if (C == (CC) && HD == (NN)) {                                                        \
        gdp_bwd_sum_kernel<CC, NN, 1><<<(NN * CC + NN) / 64, 256, 0, st>>>(nullptr, 0,     \
                                                                         nullptr, 0, dwg,  \
                                                                         nullptr, dbg,     \
                                                                         nullptr);         \
        return check_launch("attention_gate_bwd");                                        \
    }
    CLK_GATE_SHAPES(CLK_GATEZ)
#undef CLK_GATEZ
    return fail(CLK_INVALID_ARGUMENT, "attention_gate_bwd: C=%d, H*D=%d not supported", C, HD);
}

template <typename TR>
clk_status dispatch_gate_bwd(hipStream_t st, const void* o, const void* x, const void* wg,
                             const void* bg, const void* dout, void* dov, void* dx, float* dwg,
                             float* dbg, char* ws, int M, int H, int Sq, int D, int C,
                             int accumulate) {
    const int HD = H * D;
#define CLK_GATEB(CC, NN)                                                                  \
    if (C == (CC) && HD == (NN))                                                           \
        return run_gate_bwd<TR, CC, NN>(st, o, x, wg, bg, dout, dov, dx, dwg, dbg, ws, M, H, \
                                        Sq, D, accumulate);
    CLK_GATE_SHAPES(CLK_GATEB)
#undef CLK_GATEB
    return fail(CLK_INVALID_ARGUMENT, "attention_gate_bwd: C=%d, H*D=%d not supported", C, HD);
}

}  // namespace
}  // namespace clk

using namespace clk;

extern "C" size_t clk_gated_dual_proj_bwd_workspace_size(int64_t M, int64_t K, int64_t N) {
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    return bwd_geom(M, (int)K, (int)N).total;
}

extern "C" clk_status clk_gated_dual_proj_bwd(hipStream_t stream, clk_dtype dtype, const void* x,
                                              const void* wp, const void* bp, const void* wg,
                                              const void* bg, const void* mask, const void* dout,
                                              void* dx, float* dwp, float* dbp, float* dwg,
                                              float* dbg, void* workspace, size_t workspace_bytes,
                                              int64_t M, int64_t K, int64_t N, int accumulate_dx) {
    const char* who = "gated_dual_proj_bwd";
    if (dtype != CLK_F16 && dtype != CLK_BF16)
        return fail(CLK_INVALID_ARGUMENT, "%s: dtype %s not supported (f16, bf16)", who,
                    dtype_name(dtype));
    if (M < 0 || (K != 64 && K != 128) || (N != 64 && N != 128))
        return fail(CLK_INVALID_ARGUMENT, "%s: K and N must be 64 or 128 (K=%lld, N=%lld)", who,
                    (long long)K, (long long)N);
    if (M > kMaxBwdM)
        return fail(CLK_INVALID_ARGUMENT, "%s: M=%lld too large (at most 2^31 - 64 rows)", who,
                    (long long)M);
    if (M == 0) {
        if (!dwp || !dbp || !dwg || !dbg)
            return fail(CLK_INVALID_ARGUMENT, "%s: null gradient pointer", who);
        return zero_gdp_bwd(stream, dwp, dbp, dwg, dbg, (int)K, (int)N);
    }
    if (!x || !wp || !bp || !wg || !bg || !mask || !dout || !dx || !dwp || !dbp || !dwg || !dbg ||
        !workspace)
        return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    if (!aligned16(x) || !aligned16(dout) || !aligned16(dx) || !aligned16(wp) || !aligned16(wg) ||
        !aligned16(workspace))
        return fail(CLK_INVALID_ARGUMENT, "%s: x, wp, wg, dout, dx, workspace must be 16-byte "
                    "aligned", who);
    const size_t need = bwd_geom(M, (int)K, (int)N).total;
    if (workspace_bytes < need)
        return fail(CLK_INVALID_ARGUMENT, "%s: workspace of %zu bytes, %zu needed", who,
                    workspace_bytes, need);
    char* ws = static_cast<char*>(workspace);
    if (dtype == CLK_BF16)
        return dispatch_gdp_bwd<BF16>(stream, x, wp, bp, wg, bg, mask, dout, dx, dwp, dbp, dwg,
                                      dbg, ws, (int)M, (int)K, (int)N, accumulate_dx);
    return dispatch_gdp_bwd<F16>(stream, x, wp, bp, wg, bg, mask, dout, dx, dwp, dbp, dwg, dbg,
                                 ws, (int)M, (int)K, (int)N, accumulate_dx);
}

extern "C" size_t clk_attention_gate_bwd_workspace_size(int64_t N, int64_t H, int64_t Sq,
                                                        int64_t D, int64_t C) {
    if (N <= 0 || H <= 0 || Sq <= 0 || D <= 0 || C <= 0) return 0;
    return gate_bwd_geom(N * Sq, (int)C, (int)(H * D)).total;
}

extern "C" clk_status clk_attention_gate_bwd(hipStream_t stream, clk_dtype dtype, const void* o,
                                             const void* x, const void* wg, const void* bg,
                                             const void* dout, void* d_o, void* dx, float* dwg,
                                             float* dbg, void* workspace, size_t workspace_bytes,
                                             int64_t N, int64_t H, int64_t Sq, int64_t D,
                                             int64_t C, int accumulate_dx) {
    const char* who = "attention_gate_bwd";
    if (dtype != CLK_F16 && dtype != CLK_BF16)
        return fail(CLK_INVALID_ARGUMENT, "%s: dtype %s not supported (f16, bf16)", who,
                    dtype_name(dtype));
    if (N < 0 || Sq < 0 || H <= 0 || D <= 0 || D % 8 != 0)
        return fail(CLK_INVALID_ARGUMENT,
                    "%s: need N, Sq >= 0, H > 0 and D a positive multiple of 8 (N=%lld, H=%lld, "
                    "Sq=%lld, D=%lld)", who, (long long)N, (long long)H, (long long)Sq,
                    (long long)D);
    const int64_t HD = H * D;
    if ((C != 64 && C != 128 && C != 256) || (HD != 64 && HD != 128 && HD != 256))
        return fail(CLK_INVALID_ARGUMENT, "%s: C and H*D must each be 64, 128 or 256 (C=%lld, "
                    "H*D=%lld)", who, (long long)C, (long long)HD);
    const int64_t M = N * Sq;
    if (M > kMaxBwdM)
        return fail(CLK_INVALID_ARGUMENT, "%s: N*Sq=%lld rows too many (at most 2^31 - 64)", who,
                    (long long)M);
    if (Sq * HD * 4 >= ((int64_t)1 << 30))
        return fail(CLK_INVALID_ARGUMENT, "%s: Sq=%lld too long (Sq*H*D*4 must stay under 2^30)",
                    who, (long long)Sq);
    if (!dwg || !dbg) return fail(CLK_INVALID_ARGUMENT, "%s: null gradient pointer", who);
    if (M == 0) return zero_gate_bwd(stream, dwg, dbg, (int)C, (int)HD);
    if (!o || !x || !wg || !bg || !dout || !d_o || !dx || !workspace)
        return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    if (!aligned16(o) || !aligned16(x) || !aligned16(wg) || !aligned16(dout) ||
        !aligned16(d_o) || !aligned16(dx) || !aligned16(workspace))
        return fail(CLK_INVALID_ARGUMENT, "%s: o, x, wg, dout, d_o, dx, workspace must be "
                    "16-byte aligned", who);
    const size_t need = gate_bwd_geom(M, (int)C, (int)HD).total;
    if (workspace_bytes < need)
        return fail(CLK_INVALID_ARGUMENT, "%s: workspace of %zu bytes, %zu needed", who,
                    workspace_bytes, need);
    char* ws = static_cast<char*>(workspace);
    if (dtype == CLK_BF16)
        return dispatch_gate_bwd<BF16>(stream, o, x, wg, bg, dout, d_o, dx, dwg, dbg, ws, (int)M,
                                       (int)H, (int)Sq, (int)D, (int)C, accumulate_dx);
    return dispatch_gate_bwd<F16>(stream, o, x, wg, bg, dout, d_o, dx, dwg, dbg, ws, (int)M,
                                  (int)H, (int)Sq, (int)D, (int)C, accumulate_dx);
}
