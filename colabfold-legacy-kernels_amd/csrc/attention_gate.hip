// Gated attention output for gfx950:
//   out[n, s, h*D + d] = o[n, h, s, d] * sigmoid(x[n, s, :] . wg[:, h*D + d] + bg[h*D + d])
// the gating that AlphaFold's Attention module applies to the attention-weighted values before
// the output projection (ColabFold's MSA row/column and triangle attention; the reference
// library leaves it to the caller's jnp code). One pass: the gate GEMM on MFMA, the sigmoid, the
// product with o, and the [N,H,S,D] -> [N,S,H*D] transpose that the output projection reads.
//
// Layout: o [N,H,Sq,D]; x [N,Sq,C] (the attention's query-side input); wg [C, H*D] row-major;
// bg [H*D]; out [N,Sq,H*D]. All of one 2-byte dtype. HBM traffic is one read of x and o and one
// write of out: at C = H*D = 256 about 13 flop/B, far below the MFMA ridge, so the op is
// HBM-bound.
//
// Wave w of the HD/32 waves of a block owns the gate columns 32w + 0..31 and holds their weights
// as MFMA A operands (W^T) in registers for the whole kernel, pre-multiplied by -log2(e) so the
// accumulator is the argument of exp2 in 1/(1 + exp2(.)). A-tile row r of half h stands for
// column 32w + 8*(r/4) + 4h + r%4, so a lane's accumulators hold 8 consecutive columns of one
// query row: 8 consecutive d of one head, read from o and written to out as 16-byte vectors.
// The block walks 64-query tiles of one (n, query block); x rows reach a swizzled LDS tile by
// direct buffer->LDS loads two tiles ahead, and the o vectors of the next tile are loaded into
// registers while the current one is computed.
#include "common.hpp"

namespace clk {
namespace {

constexpr int kGateRows = 64;  // query rows per tile

template <typename TR, int C, int HD>
__global__ __launch_bounds__(2 * HD) void attn_gate_kernel(
    const typename TR::elem* __restrict__ o, const typename TR::elem* __restrict__ x,
    const typename TR::elem* __restrict__ wg, const typename TR::elem* __restrict__ bg,
    typename TR::elem* __restrict__ out, int H, int Sq, int D, int ntiles, int qblocks) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    constexpr int NW = HD / 32, NT = 64 * NW;
    constexpr int KS = C / 32;
    constexpr int R = kGateRows, SUB = R / 16;
    constexpr int PL = C / 8;  // 16-byte pieces per x row
    // XOR swizzle of the pieces within a row: the largest power-of-two group dividing PL.
    constexpr int SWZ = (PL % 16 == 0) ? 15 : (PL % 8 == 0) ? 7 : 3;
    constexpr int DPW = (R * PL + NT - 1) / NT;  // 16-byte loads per lane and tile
    constexpr int XB = DPW * NT * 16;           // tile bytes, padded to whole load rounds

    // Three x tiles: the one being read and the next two in flight.
    __shared__ __attribute__((aligned(16))) char x0[XB];
    __shared__ __attribute__((aligned(16))) char x1[XB];
    __shared__ __attribute__((aligned(16))) char x2[XB];
    // The gated tile on its way out, rows padded by 16 bytes: written at the end of a tile (after
    // a barrier: every wave has stored the last one), stored as whole rows in the next.
    constexpr int OSTR = 2 * HD + 16;
    __shared__ __attribute__((aligned(16))) char ob[R * OSTR];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;

    // Resident A operands -log2(e) * wg^T and the matching bias.
    V8 wa[2][KS];
    f32x4 binit[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int col = 32 * wave + 8 * (r16 >> 2) + 4 * h + (r16 & 3);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                wa[h][ks][j] = TR::from_f(-kLog2e * TR::to_f(wg[(32 * ks + 8 * g + j) * HD + col]));
        // C lane (r16, g) holds the columns 32w + 8g + 4h + i.
#pragma unroll
        for (int i = 0; i < 4; ++i)
            binit[h][i] = -kLog2e * TR::to_f(bg[32 * wave + 8 * g + 4 * h + i]);
    }

    // The lane's 8 columns are d0..d0+7 of head hh.
    const int col0 = 32 * wave + 8 * g;
    const int hh = col0 / D, d0 = col0 % D;

    auto rows_of = [&](int t, int& n, int& s0) {
        n = t / qblocks;
        s0 = (t - n * qblocks) * R;
        return t < ntiles ? min(R, Sq - s0) : 0;
    };
    // Every tile issues the same vector memory operations in every wave: SUB = 4 stores (rows past
    // the tile fall outside the store resource and are dropped), the o loads and DPW direct-to-
    // LDS loads (pieces past the tile's rows read zeros; tiles past the end use an empty
    // resource).
    auto stage = [&](int t, char* xb) {
        int n, s0;
        const int rows = rows_of(t, n, s0);
        const Rsrc rx = buffer_rsrc(rows > 0 ? x + ((size_t)n * Sq + s0) * C : x,
                                    (uint32_t)rows * C * 2);
#pragma unroll
        for (int k = 0; k < DPW; ++k) {
            const int b = wave * 64 + k * NT;
            const int slot = b + lane, row = slot / PL;
            const int piece = (slot % PL) ^ (row & SWZ);
            // Non-temporal: every row of x is read once (MSA row attention's gate: 4.63-4.66
            // against 4.39-4.40 TB/s).
            buf_dma16_nt(rx, row < R ? (row * C + piece * 8) * 2 : kPastEnd, 0, xb + b * 16);
        }
    };
    auto load_o = [&](int t, u32x4 (&ov)[SUB]) {
        int n, s0;
        rows_of(t, n, s0);
        const E* ob = o + (((size_t)n * H + hh) * Sq) * D + d0;
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub) {
            const int s = min(s0 + 16 * sub + r16, Sq - 1);
            ov[sub] = ld16(ob + (size_t)s * D);
        }
    };
    auto out_rsrc = [&](int t) {
        int n, s0;
        const int rows = rows_of(t, n, s0);
        return buffer_rsrc(rows > 0 ? out + ((size_t)n * Sq + s0) * HD : out,
                           (uint32_t)rows * HD * 2);
    };
    // The staged tile as whole rows: four store instructions per wave, as many as the SUB
    // stores the wait counts assume.
    static_assert(SUB == 4, "four stores per wave and tile");
    auto store = [&](Rsrc ro) { store_staged_rows<R, HD, OSTR, NW>(ro, ob, wave, lane); };

    const int G = gridDim.x;
    u32x4 ov0[SUB], ov1[SUB];  // the o vectors of alternate tiles
    Rsrc pend_out = out_rsrc(ntiles);  // the staged tile's rows (none before the first)

    // Tile t is read from xc; tile t + 2G goes into xn, which held tile t - G. Issued after xc's
    // loads: at least the stores of tile t - 2G, the o loads of tile t and the loads of tile
    // t + G. The o vectors of tile t are in oc (loaded during tile t - G, before the x loads of
    // tile t + G, so waiting for them never waits for those); tile t + G's go into on.
    auto tile = [&](int t, const char* xc, char* xn, const u32x4 (&oc)[SUB], u32x4 (&on)[SUB]) {
        vm_wait<2 * SUB + DPW>();
        lds_barrier();  // x tile t in xc, tile t - G staged; every wave is done reading xn
        store(pend_out);
        if (t + G < ntiles) load_o(t + G, on);
        stage(t + 2 * G, xn);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        u32x4 res[SUB];
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub) {
            const int xrow = 16 * sub + r16;
            f32x4 acc[2] = {binit[0], binit[1]};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const V8 xv = *reinterpret_cast<const V8*>(
                    xc + (xrow * PL + ((4 * ks + g) ^ (xrow & SWZ))) * 16);
#pragma unroll
                for (int h = 0; h < 2; ++h) acc[h] = TR::mfma(wa[h][ks], xv, acc[h]);
            }
            float ov[8], r[8];
            unpack8<TR>(oc[sub], ov);
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] = ov[j] * fast_rcp(1.f + fast_exp2(acc[j >> 2][j & 3]));
            res[sub] = pack8<TR>(r);
        }
        lds_barrier();  // every wave has read the staged tile t - G
#pragma unroll
        for (int sub = 0; sub < SUB; ++sub)
            *reinterpret_cast<u32x4*>(ob + (16 * sub + r16) * OSTR + col0 * 2) = res[sub];
        pend_out = out_rsrc(t);
    };

    // Prologue: two tiles in flight, each followed by a batch of (empty) stores, so that the
    // first two waits count as every later one does.
    int t = blockIdx.x;
    const Rsrc none = out_rsrc(ntiles);
    load_o(t, ov0);
    stage(t, x0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    store(none);
    stage(t + G, x1);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    store(none);
    // Three x buffers and two o register sets: the pattern repeats every six tiles.
    for (; t < ntiles; t += 6 * G) {
        tile(t, x0, x2, ov0, ov1);
        if (t + G >= ntiles) break;
        tile(t + G, x1, x0, ov1, ov0);
        if (t + 2 * G >= ntiles) break;
        tile(t + 2 * G, x2, x1, ov0, ov1);
        if (t + 3 * G >= ntiles) break;
        tile(t + 3 * G, x0, x2, ov1, ov0);
        if (t + 4 * G >= ntiles) break;
        tile(t + 4 * G, x1, x0, ov0, ov1);
        if (t + 5 * G >= ntiles) break;
        tile(t + 5 * G, x2, x1, ov1, ov0);
    }
    lds_barrier();  // the last tile is staged
    store(pend_out);
    async_wait();  // no direct-to-LDS load may still be in flight when the workgroup ends
}

template <typename TR, int C, int HD>
clk_status launch_gate(hipStream_t st, const void* o, const void* x, const void* wg,
                       const void* bg, void* out, int N, int H, int Sq, int D) {
    using E = typename TR::elem;
    const int qblocks = (Sq + kGateRows - 1) / kGateRows;
    const int ntiles = N * qblocks;
    // Registers hold two waves per SIMD at HD = 256 (one 8-wave block per CU); narrower blocks
    // run several per CU.
    const int per_cu = 256 / HD;
    const int grid = ntiles < 256 * per_cu ? ntiles : 256 * per_cu;
    KernelTimer timer("attn_gate", st);
    attn_gate_kernel<TR, C, HD><<<grid, 2 * HD, 0, st>>>(
        (const E*)o, (const E*)x, (const E*)wg, (const E*)bg, (E*)out, H, Sq, D, ntiles, qblocks);
    return check_launch("attention_gate");
}

template <typename TR>
clk_status dispatch_gate(hipStream_t st, const void* o, const void* x, const void* wg,
                         const void* bg, void* out, int N, int H, int Sq, int D, int C) {
    const int HD = H * D;
#define CLK_GATE(CC, HH) \
    if (C == (CC) && HD == (HH)) return launch_gate<TR, CC, HH>(st, o, x, wg, bg, out, N, H, Sq, D);
    CLK_GATE(256, 256) CLK_GATE(256, 128) CLK_GATE(256, 64)
    CLK_GATE(128, 256) CLK_GATE(128, 128) CLK_GATE(128, 64)
    CLK_GATE(64, 256) CLK_GATE(64, 128) CLK_GATE(64, 64)
#undef CLK_GATE
    return fail(CLK_INVALID_ARGUMENT, "attention_gate: C=%d, H*D=%d not supported", C, HD);
}

}  // namespace
}  // namespace clk

using namespace clk;

extern "C" clk_status clk_attention_gate(hipStream_t stream, clk_dtype dtype, const void* o,
                                         const void* x, const void* wg, const void* bg, void* out,
                                         int64_t N, int64_t H, int64_t Sq, int64_t D, int64_t C) {
    const char* who = "attention_gate";
    if (dtype != CLK_F16 && dtype != CLK_BF16)
        return fail(CLK_INVALID_ARGUMENT, "%s: dtype %s not supported (f16, bf16)", who,
                    dtype_name(dtype));
    if (N < 0 || H <= 0 || Sq < 0 || D <= 0 || C <= 0)
        return fail(CLK_INVALID_ARGUMENT, "%s: bad dims", who);
    if (D % 8) return fail(CLK_INVALID_ARGUMENT, "%s: D=%lld is not a multiple of 8", who,
                           (long long)D);
    const int64_t HD = H * D;
    if ((C != 64 && C != 128 && C != 256) || (HD != 64 && HD != 128 && HD != 256))
        return fail(CLK_INVALID_ARGUMENT,
                    "%s: C and H*D must each be 64, 128 or 256 (C=%lld, H*D=%lld)", who,
                    (long long)C, (long long)HD);
    if (N * Sq > INT32_MAX || N * ((Sq + kGateRows - 1) / kGateRows) > INT32_MAX / 2)
        return fail(CLK_INVALID_ARGUMENT, "%s: N*Sq too large", who);
    if (N == 0 || Sq == 0) return ok();
    if (!o || !x || !wg || !bg || !out)
        return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    if (!aligned16(o) || !aligned16(x) || !aligned16(out))
        return fail(CLK_INVALID_ARGUMENT, "%s: o, x, out must be 16-byte aligned", who);
    if (dtype == CLK_BF16)
        return dispatch_gate<BF16>(stream, o, x, wg, bg, out, (int)N, (int)H, (int)Sq, (int)D,
                                   (int)C);
    return dispatch_gate<F16>(stream, o, x, wg, bg, out, (int)N, (int)H, (int)Sq, (int)D,
                              (int)C);
}
