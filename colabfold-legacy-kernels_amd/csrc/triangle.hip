// Triangle multiplication for gfx950: the channel-batched contraction at the centre of
// AlphaFold's TriangleMultiplication (the step that consumes the a and b the gated dual
// projection writes; the reference library stops at the projection, cuda/volta_ops.cu:97):
//   outgoing  x[i,j,c] = sum_k a[i,k,c] b[j,k,c]        incoming  x[i,j,c] = sum_k a[k,i,c] b[k,j,c]
// Per channel both are a plain N x N x N product once a and b are stored channel-major (the
// layout the fused LayerNorm + gated projection writes for this consumer, plane c row-major
// over the pair index): outgoing X_c = A_c . B_c^T with the contraction index last in both
// (A_c[i][k] = a[i,k,c]); incoming X_c = A_c^T . B_c with it first (A_c[k][i] = a[k,i,c]).
//
// tri_einsum_kernel: one 256 x 256 output tile of one channel per block of 8 waves (2 x 4 wave
// tiles of 128 i x 64 j, 32 MFMA 16x16x32 accumulators each). The operands reach LDS in
// 64-wide k slices by direct buffer->LDS loads, two stages (the next slice loads while the
// current one is multiplied). Contraction index last: 256 rows of 128 bytes per operand (whole
// cache lines: 32-wide slices read half lines, 5% slower), each 16-byte piece XOR-swizzled by
// row % 8 so the sixteen rows an operand read touches fall in distinct banks. Contraction index
// first: 64 rows of 512 bytes, read with ds_read_b64_tr_b16 (a transposed 4 x 16 block per
// 16-lane group), pieces swizzled by 2 * (row % 4). Per slice a block moves 64 KB from L2 for
// 8.4 MFLOP (128 flop/B). Tiles of one channel run on one XCD, whose L2 then serves both
// operands.
#include "common.hpp"

namespace clk {
namespace {

constexpr int kTriTile = 256;  // output tile edge
constexpr int kTriK = 32;      // contraction depth of one half slice (two per stage)

// The twelve 16-byte fragments of one half slice (four B rows, eight A rows, 16-row blocks STRIDE
// bytes apart) read from LDS and waited for in one asm statement: the loop picks its stage at
// run time, and a read the compiler can see would have to wait for every direct-to-LDS load in
// flight. All outputs are complete when the statement ends, so no register is read before its
// data has arrived; the "memory" clobber keeps the statement behind the barrier that publishes
// the stage.
template <int STRIDE, typename V8>
__device__ __forceinline__ void read_fragments_s(uint32_t ba, uint32_t bb, V8 (&fb)[4],
                                                 V8 (&fa)[8]) {
    asm volatile(
        "ds_read_b128 %0, %13\n\t"
        "ds_read_b128 %1, %13 offset:%14\n\t"
        "ds_read_b128 %2, %13 offset:%15\n\t"
        "ds_read_b128 %3, %13 offset:%16\n\t"
        "ds_read_b128 %4, %12\n\t"
        "ds_read_b128 %5, %12 offset:%14\n\t"
        "ds_read_b128 %6, %12 offset:%15\n\t"
        "ds_read_b128 %7, %12 offset:%16\n\t"
        "ds_read_b128 %8, %12 offset:%17\n\t"
        "ds_read_b128 %9, %12 offset:%18\n\t"
        "ds_read_b128 %10, %12 offset:%19\n\t"
        "ds_read_b128 %11, %12 offset:%20\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(fb[0]), "=&v"(fb[1]), "=&v"(fb[2]), "=&v"(fb[3]), "=&v"(fa[0]), "=&v"(fa[1]),
          "=&v"(fa[2]), "=&v"(fa[3]), "=&v"(fa[4]), "=&v"(fa[5]), "=&v"(fa[6]), "=&v"(fa[7])
        : "v"(ba), "v"(bb), "i"(STRIDE), "i"(2 * STRIDE), "i"(3 * STRIDE), "i"(4 * STRIDE),
          "i"(5 * STRIDE), "i"(6 * STRIDE), "i"(7 * STRIDE)
        : "memory");
}

// The 24 transposed fragment reads of one TN slice (A: 8 fragments, B: 4, each two
// ds_read_b64_tr_b16 of rows 8g+j and 8g+4+j, 2 KB apart) and their wait, as one asm statement.
__device__ __forceinline__ void read_tr_fragments(const uint32_t (&ad)[12], i16x4 (&r)[24]) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %24\n\tds_read_b64_tr_b16 %1, %24 offset:2048\n\t"
        "ds_read_b64_tr_b16 %2, %25\n\tds_read_b64_tr_b16 %3, %25 offset:2048\n\t"
        "ds_read_b64_tr_b16 %4, %26\n\tds_read_b64_tr_b16 %5, %26 offset:2048\n\t"
        "ds_read_b64_tr_b16 %6, %27\n\tds_read_b64_tr_b16 %7, %27 offset:2048\n\t"
        "ds_read_b64_tr_b16 %8, %28\n\tds_read_b64_tr_b16 %9, %28 offset:2048\n\t"
        "ds_read_b64_tr_b16 %10, %29\n\tds_read_b64_tr_b16 %11, %29 offset:2048\n\t"
        "ds_read_b64_tr_b16 %12, %30\n\tds_read_b64_tr_b16 %13, %30 offset:2048\n\t"
        "ds_read_b64_tr_b16 %14, %31\n\tds_read_b64_tr_b16 %15, %31 offset:2048\n\t"
        "ds_read_b64_tr_b16 %16, %32\n\tds_read_b64_tr_b16 %17, %32 offset:2048\n\t"
        "ds_read_b64_tr_b16 %18, %33\n\tds_read_b64_tr_b16 %19, %33 offset:2048\n\t"
        "ds_read_b64_tr_b16 %20, %34\n\tds_read_b64_tr_b16 %21, %34 offset:2048\n\t"
        "ds_read_b64_tr_b16 %22, %35\n\tds_read_b64_tr_b16 %23, %35 offset:2048\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]),
          "=&v"(r[6]), "=&v"(r[7]), "=&v"(r[8]), "=&v"(r[9]), "=&v"(r[10]), "=&v"(r[11]),
          "=&v"(r[12]), "=&v"(r[13]), "=&v"(r[14]), "=&v"(r[15]), "=&v"(r[16]), "=&v"(r[17]),
          "=&v"(r[18]), "=&v"(r[19]), "=&v"(r[20]), "=&v"(r[21]), "=&v"(r[22]), "=&v"(r[23])
        : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5]), "v"(ad[6]),
          "v"(ad[7]), "v"(ad[8]), "v"(ad[9]), "v"(ad[10]), "v"(ad[11])
        : "memory");
}

// TN = false: X[c] = A[c] . B[c]^T for A, B, X [C][N][N] row-major (the contraction index
// last). TN = true: X[c] = A[c]^T . B[c] (the contraction index first, A[c][k][i], B[c][k][j]):
// a slice is 32 rows k of A (B) x the tile's 256 columns i (j), and the fragments are read
// transposed with ds_read_b64_tr_b16, so the incoming direction needs no plane transposes.
// N must be a multiple of 8.
template <typename TR, bool TN>
__global__ __launch_bounds__(512) void tri_einsum_kernel(const typename TR::elem* __restrict__ A,
                                                         const typename TR::elem* __restrict__ B,
                                                         typename TR::elem* __restrict__ X, int N,
                                                         int T, int ntiles) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    constexpr int BT = kTriTile, KC = 2 * kTriK;
    constexpr int NSTG = 2;  // two stages of 64 k
    constexpr int PR = KC / 8;             // 16-byte pieces per row slice
    constexpr int SLICE = BT * PR * 16;    // bytes of one operand slice
    constexpr int NT = 512, DPW = 2 * BT * PR / NT;  // loads per lane and slice (A and B)
    static_assert(BT * PR % NT == 0, "whole load rounds");

    constexpr int STAGE = 2 * SLICE;
    __shared__ __attribute__((aligned(16))) char smem[NSTG * STAGE];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int wi = wave >> 2, wj = wave & 3;  // wave tile: rows 128*wi.., columns 64*wj..

    const int w = xcd_contiguous(blockIdx.x, ntiles);
    const int c = w / (T * T), ti = (w / T) % T, tj = w % T;
    const int i0 = ti * BT, j0 = tj * BT;
    const size_t plane = (size_t)N * N;
    const E* Ac = A + c * plane;
    const E* Bc = B + c * plane;
    // NT: rows of the tile past N read zeros (the resource ends with the channel's plane).
    // TN: the resources cover the whole plane; rows k past N read zeros, columns past N are
    // given an out-of-range offset.
    const Rsrc ra = TN ? buffer_rsrc(Ac, (uint32_t)(plane * 2))
                       : buffer_rsrc(Ac + (size_t)i0 * N, (uint32_t)((size_t)min(BT, N - i0) * N * 2));
    const Rsrc rb = TN ? buffer_rsrc(Bc, (uint32_t)(plane * 2))
                       : buffer_rsrc(Bc + (size_t)j0 * N, (uint32_t)((size_t)min(BT, N - j0) * N * 2));
    const Rsrc none = buffer_rsrc(A, 0);
    const int nk = (N + KC - 1) / KC;

    // Slice kk of both operands into buffer st: A rows at st, B rows at st + SLICE. Piece q of
    // LDS row r holds the row's 16-byte piece q ^ (r % 8); pieces past N read zeros.
    // TN: LDS row r (k = kk*64 + r) holds the tile's 256 columns as 32 pieces; slot q holds
    // piece q ^ 2*(r % 4), so that the four rows of a transposed read fall in distinct banks.
    auto stage = [&](int kk, char* st) {
        const bool live = kk < nk;
#pragma unroll
        for (int k = 0; k < DPW; ++k) {
            const int op = k / (DPW / 2);  // 0: A, 1: B
            const int b = (k % (DPW / 2)) * NT + wave * 64;
            const int slot = b + lane;
            int voff;
            if constexpr (TN) {
                const int row = slot / (BT / 8), piece = (slot % (BT / 8)) ^ (2 * (row & 3));
                const int col = (op ? j0 : i0) + piece * 8;
                voff = col < N ? ((kk * KC + row) * N + col) * 2 : kPastEnd;
            } else {
                const int row = slot / PR;
                const int piece = (slot % PR) ^ (row & 7);
                const int kcol = kk * KC + piece * 8;
                voff = kcol < N ? (row * N + kcol) * 2 : kPastEnd;
            }
            buf_dma16(live ? (op ? rb : ra) : none, voff, 0, st + op * SLICE + b * 16);
        }
    };

    f32x4 acc[4][8];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Operand reads (NT). Lane (r16, g) reads k 32h + 8g .. +7 (piece 4h + g) of row 16t + r16 of
    // its wave's rows; the swizzle term row % 8 is the same for every t, so one address per half
    // h serves all tiles of a slice with an immediate offset of 2 KB per 16 rows.
    const uint32_t lds0 = lds_addr(smem);
    uint32_t rda2[2], rdb2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t rd = (uint32_t)(r16 * PR + ((4 * h + g) ^ (r16 & 7))) * 16;
        rda2[h] = rd + 128 * wi * PR * 16;
        rdb2[h] = rd + SLICE + 64 * wj * PR * 16;
    }
    // TN: fragment f (it = 0..7 of A, then jt = 0..3 of B) is column block m0 = 128wi + 16it
    // (64wj + 16jt); lane 4j + t reads row 8g + j (and + 4), columns m0 + 4t .. + 3.
    uint32_t trd[12];
    if constexpr (TN) {
        const int j = r16 >> 2, t = r16 & 3, row = 8 * g + j;
#pragma unroll
        for (int f = 0; f < 12; ++f) {
            const int m0 = f < 8 ? 128 * wi + 16 * f : 64 * wj + 16 * (f - 8);
            const int piece = ((m0 + 4 * t) >> 3) ^ (2 * j);
            trd[f] = (f < 8 ? 0 : SLICE) + row * (BT * 2) + piece * 16 + 8 * (t & 1);
        }
    }

    // X^T tile products: the A operand is B (rows j), the B operand is A (rows i), so a lane's
    // accumulator holds four consecutive j of one i. Two stages of 64 k: slice kk + 1 loads
    // while slice kk is multiplied, as two halves of 32 k. The loop body is not unrolled (copies of it cost the register allocator more than
    // the 256 VGPRs a lane has), so the stage is picked at run time and the fragments are read
    // by asm statements.
    stage(0, smem);
    for (int kk = 0; kk < nk; ++kk) {
        const int cur = kk & 1;
        vm_wait<0>();
        lds_barrier();  // slice kk in stage cur; every wave is done reading the other stage
        stage(kk + 1, smem + (cur ^ 1) * STAGE);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            V8 fb[4], fa[8];
            if constexpr (TN) {
                // Rows 32h .. 32h+31 of the slice.
                uint32_t ad[12];
#pragma unroll
                for (int f = 0; f < 12; ++f) ad[f] = lds0 + cur * STAGE + trd[f] + h * 32 * BT * 2;
                i16x4 r[24];
                read_tr_fragments(ad, r);
#pragma unroll
                for (int f = 0; f < 12; ++f) {
                    const i16x4 lo = r[2 * f], hi = r[2 * f + 1];
                    typedef short i16x8 __attribute__((ext_vector_type(8)));
                    const i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                    if (f < 8) fa[f] = __builtin_bit_cast(V8, v);
                    else fb[f - 8] = __builtin_bit_cast(V8, v);
                }
            } else {
                read_fragments_s<16 * PR * 16>(lds0 + cur * STAGE + rda2[h],
                                               lds0 + cur * STAGE + rdb2[h], fb, fa);
            }
#pragma unroll
            for (int it = 0; it < 8; ++it)
#pragma unroll
                for (int jt = 0; jt < 4; ++jt) acc[jt][it] = TR::mfma(fb[jt], fa[it], acc[jt][it]);
        }
    }

    // Lane (r16, g) of accumulator (jt, it) holds X[i][j..j+3] for i = i0 + 128wi + 16it + r16,
    // j = j0 + 64wj + 16jt + 4g. The tile goes out through LDS (the two stages, 128 KB, are free
    // once every wave's last loads have landed and its last reads are done): bf16 rows of 512
    // bytes, 16-byte pieces XOR-swizzled by row % 32, then stored by the whole block as rows of
    // whole cache lines (an 8-byte store per lane and accumulator writes a quarter line).
    // Rows past N fall outside the resource; columns past N (whole pieces, N being a multiple
    // of 8) are skipped.
    static_assert(BT * BT * 2 <= NSTG * STAGE, "the output tile fits the stages");
    async_wait();
    lds_barrier();
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int il = 128 * wi + 16 * it + r16, piece = 8 * wj + 2 * jt + (g >> 1);
            E e[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) e[q] = TR::from_f(acc[jt][it][q]);
            u32x2 v;
            __builtin_memcpy(&v, e, 8);
            *reinterpret_cast<u32x2*>(smem + (il * 32 + (piece ^ (il & 31))) * 16 + 8 * (g & 1)) =
                v;
        }
    lds_barrier();
    const Rsrc rx = buffer_rsrc(X + c * plane + (size_t)i0 * N,
                                (uint32_t)((size_t)min(BT, N - i0) * N * 2));
#pragma unroll
    for (int k = 0; k < BT * BT / 8 / NT; ++k) {
        const int f = k * NT + tid, row = f >> 5, piece = f & 31;
        const u32x4 v = *reinterpret_cast<const u32x4*>(smem + (row * 32 + (piece ^ (row & 31))) * 16);
        if (j0 + 8 * piece < N) buf_st16_nt(rx, (row * N + j0 + 8 * piece) * 2, 0, v);
    }
}

// ---------------------------------------------------------------------------------------------
// Output stage of the triangle multiplication (AlphaFold's centre LayerNorm, output projection
// and output gate), one pass over the contraction result x and the input z:
//   out[p, o] = (LN_c(x[:, p]) . w_out[:, o] + b_out[o]) * sigmoid(LN_in(z[p, :]) . w_g[:, o] + b_g[o])
// x is channel-major [C][M] (as the contraction writes it), z and out are [M][C] (M = N*N
// positions, C channels, both LayerNorms over C). As in the fused LayerNorm + gated projection,
// the LN affines fold into the weights and biases, the gate carries -log2(e), and each wave holds
// its 32 output columns of both matrices as MFMA A operands. A block walks 64-position tiles:
// x's [C][64] slab and z's [64][C] rows arrive by direct buffer->LDS loads two tiles ahead; four
// waves normalise the x slab (lane = position, 32 channels per lane group, reduced across the
// four groups) and four the z rows, both into swizzled [64][C] tiles that feed the MFMAs.
// ---------------------------------------------------------------------------------------------
template <typename E>
struct TriOutParams {
    const E* x;
    const E* z;
    const float* gin;    // LN_in scale [C]
    const float* bin;    // LN_in offset [C]
    const float* gc;     // LN_c scale [C]
    const float* bc;     // LN_c offset [C]
    const E* wout;       // [C][C]
    const E* bout;       // [C]
    const E* wg;         // [C][C]
    const E* bg;         // [C]
    E* out;
    int M;
    float eps;
};

template <typename TR, int C>
__global__ __launch_bounds__(512) void tri_out_kernel(TriOutParams<typename TR::elem> pr) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    constexpr int NT = 512, KS = C / 32, R = 64, SUB = R / 16, PL = C / 8;
    constexpr int NCG = C / 32, NSPLIT = 8 / NCG, SUBW = SUB / NSPLIT;  // column groups, subs
    static_assert(NSPLIT * NCG == 8 && SUBW * NSPLIT == SUB, "eight waves");
    constexpr int SWZ = 15 & (PL - 1);
    constexpr int LPR = PL;  // z LayerNorm: lanes per row (8 channels each)
    constexpr int CPG = C / 4;  // x LayerNorm: channels per lane group
    static_assert(LPR == 8 || LPR == 16, "C = 64 or 128");
    constexpr int ZB = R * C * 2;
    constexpr int DPZ = R * PL / NT;           // z loads per lane and tile
    constexpr int XSLOTS = C * (R / 8);        // 16-byte pieces of the x slab
    constexpr int DPX = XSLOTS / NT;           // x loads per lane and tile
    static_assert(DPZ * NT == R * PL && DPX * NT == XSLOTS, "whole load rounds");
    // x slab in LDS: channel row c holds 128 bytes; every 8 rows (one wave's load) are followed
    // by 16 bytes of padding, so the four lane groups of a LayerNorm read hit distinct banks.
    constexpr int XB = XSLOTS * 16 + (XSLOTS / 64) * 16;

    __shared__ __attribute__((aligned(16))) char z0[ZB];
    __shared__ __attribute__((aligned(16))) char z1[ZB];
    __shared__ __attribute__((aligned(16))) char z2[ZB];
    __shared__ __attribute__((aligned(16))) char x0[XB];
    __shared__ __attribute__((aligned(16))) char x1[XB];
    __shared__ __attribute__((aligned(16))) char x2[XB];
    __shared__ __attribute__((aligned(16))) char xh1[ZB];  // LN_c(x), [64][C] swizzled
    __shared__ __attribute__((aligned(16))) char xh2[ZB];  // LN_in(z), [64][C] swizzled
    // The projected tile on its way out, rows padded by 16 bytes: written after the tile's
    // second barrier, stored by every wave as whole rows after the next tile's first.
    constexpr int OSTR = 2 * C + 16;
    constexpr int NST = C / 64;  // 64-piece store instructions per wave and tile
    __shared__ __attribute__((aligned(16))) char ob[R * OSTR];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int cb = wave % NCG, sh = wave / NCG;
    const int M = pr.M;

    // Resident A operands: mat 0 = diag(gc) w_out, mat 1 = -log2(e) diag(gin) w_g, and the folded
    // biases (bc . w_out + b_out, -log2(e) (bin . w_g + b_g)) in C-tile layout.
    V8 wa[2][2][KS];
    f32x4 binit[2][2];
#pragma unroll
    for (int mat = 0; mat < 2; ++mat) {
        const E* W = mat == 0 ? pr.wout : pr.wg;
        const float* gam = mat == 0 ? pr.gc : pr.gin;
        const float* bet = mat == 0 ? pr.bc : pr.bin;
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
                    const float v = TR::to_f(W[k * C + col]);
                    wa[mat][h][ks][j] = TR::from_f(gam[k] * v * fold);
                    part = fmaf(bet[k], v, part);
                }
            const E* bias = mat == 0 ? pr.bout : pr.bg;
            const float bcol = (xgroup_sum(part) + TR::to_f(bias[col])) * fold;
#pragma unroll
            for (int i = 0; i < 4; ++i) binit[mat][h][i] = __shfl(bcol, 4 * g + i);
        }
    }

    const int ntiles = M / R;
    // Every tile issues DPX + DPZ direct-to-LDS loads and NST stores in every wave (tiles past
    // the end load from empty resources; the first store batch goes to an empty resource).
    // One x load of a wave covers eight channels: its resource starts at the first of them, so
    // offsets stay below 8*M*2 bytes whatever C*M is.
    auto stage = [&](int t, char* xb, char* zb) {
        const bool live = t < ntiles;
        const Rsrc rz = buffer_rsrc(live ? pr.z + (size_t)t * R * C : pr.z,
                                    live ? (uint32_t)(R * C * 2) : 0u);
#pragma unroll
        for (int k = 0; k < DPX; ++k) {
            const int b = k * NT + wave * 64, c0 = b / (R / 8);
            const Rsrc rx = buffer_rsrc(live ? pr.x + (size_t)c0 * M + (size_t)t * R : pr.x,
                                        live ? (uint32_t)(7u * (uint32_t)M * 2u + R * 2) : 0u);
            const uint32_t c = lane / (R / 8), q = lane % (R / 8);
            buf_dma16(rx, (int)((c * (uint32_t)M + q * 8) * 2u), 0, xb + b * 16 + (b / 64) * 16);
        }
#pragma unroll
        for (int k = 0; k < DPZ; ++k) {
            const int b = k * NT + wave * 64;
            buf_dma16(rz, (b + lane) * 16, 0, zb + b * 16);
        }
    };
    // The staged tile's output rows (an empty resource before the first tile), stored as whole
    // rows by all eight waves (NST instructions each).
    Rsrc pend_out = buffer_rsrc(pr.out, 0);
    auto flush = [&]() { store_staged_rows<R, C, OSTR, 8>(pend_out, ob, wave, lane); };

    auto tile = [&](int t, const char* xc, const char* zc, char* xn, char* zn) {
        vm_wait<NST + DPX + DPZ>();
        lds_barrier();  // tile t in xc, zc; every wave is done with xh1, xh2 of the last tile
        flush();
        if (wave < 4) {
            // LN_c over the x slab: lane (r16, g) of wave w takes position 16w + r16, channels
            // CPG*g .. CPG*g + CPG-1; the four lane groups of a position combine by permlane
            // swaps.
            const int p = 16 * wave + r16;
            // Channel pairs packed two to a register (the values stay in the input type).
            uint32_t vp[CPG / 2];
            auto val = [&](int j) {
                const uint32_t w2 = vp[j >> 1];
                return TR::to_f(__builtin_bit_cast(E, (uint16_t)((j & 1) ? w2 >> 16 : w2)));
            };
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < CPG; j += 2) {
                const char* at = xc + (CPG * g + j) * (R * 2) + ((CPG * g + j) / 8) * 16 + p * 2;
                const uint32_t lo = *reinterpret_cast<const uint16_t*>(at);
                const uint32_t hi = *reinterpret_cast<const uint16_t*>(at + R * 2);
                vp[j >> 1] = lo | (hi << 16);
                sum += val(j) + val(j + 1);
            }
            const float mean = xgroup_sum(sum) * (1.f / C);
            float m2 = 0.f;
#pragma unroll
            for (int j = 0; j < CPG; ++j) {
                const float d = val(j) - mean;
                m2 = fmaf(d, d, m2);
            }
            const float rstd = rsqrtf(xgroup_sum(m2) * (1.f / C) + pr.eps);
#pragma unroll
            for (int q = 0; q < CPG / 8; ++q) {
                float xo[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) xo[j] = (val(8 * q + j) - mean) * rstd;
                const int piece = (CPG / 8) * g + q;
                *reinterpret_cast<u32x4*>(xh1 + p * PL * 16 + 16 * (piece ^ (p & SWZ))) =
                    pack8<TR>(xo);
            }
        } else {
            // LN_in over the z rows: LPR lanes per row, 8 channels each.
            const int lt = tid - 256, lr = lt % LPR;
            constexpr int RPP = 256 / LPR;
#pragma unroll
            for (int pass = 0; pass < R / RPP; ++pass) {
                const int row = pass * RPP + lt / LPR;
                float v[8];
                unpack8<TR>(*reinterpret_cast<const u32x4*>(zc + row * C * 2 + lr * 16), v);
                float sum = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) sum += v[j];
                const float mean = group_sum<LPR>(sum) * (1.f / C);
                float m2 = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float d = v[j] - mean;
                    m2 = fmaf(d, d, m2);
                }
                const float rstd = rsqrtf(group_sum<LPR>(m2) * (1.f / C) + pr.eps);
                float xo[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) xo[j] = (v[j] - mean) * rstd;
                *reinterpret_cast<u32x4*>(xh2 + row * PL * 16 + 16 * (lr ^ (row & SWZ))) =
                    pack8<TR>(xo);
            }
        }
        lds_barrier();  // xh1, xh2 of tile t ready; xn, zn are free
        stage(t + 2 * gridDim.x, xn, zn);
        pend_out = buffer_rsrc(pr.out + (size_t)t * R * C, R * C * 2);
#pragma unroll
        for (int s = 0; s < SUBW; ++s) {
            const int xrow = 16 * (sh * SUBW + s) + r16;
            f32x4 acc[2][2];
#pragma unroll
            for (int mat = 0; mat < 2; ++mat)
#pragma unroll
                for (int h = 0; h < 2; ++h) acc[mat][h] = binit[mat][h];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int off = xrow * PL * 16 + 16 * ((4 * ks + g) ^ (xrow & SWZ));
                const V8 b1 = *reinterpret_cast<const V8*>(xh1 + off);
                const V8 b2 = *reinterpret_cast<const V8*>(xh2 + off);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    acc[0][h] = TR::mfma(wa[0][h][ks], b1, acc[0][h]);
                    acc[1][h] = TR::mfma(wa[1][h][ks], b2, acc[1][h]);
                }
            }
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int h = j >> 2, i = j & 3;
                o[j] = acc[0][h][i] * fast_rcp(1.f + fast_exp2(acc[1][h][i]));
            }
            *reinterpret_cast<u32x4*>(ob + xrow * OSTR + (32 * cb + 8 * g) * 2) = pack8<TR>(o);
        }
    };

    const int G = gridDim.x;
    int t = blockIdx.x;
    stage(t, x0, z0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    flush();
    stage(t + G, x1, z1);
    for (; t < ntiles; t += 3 * G) {
        tile(t, x0, z0, x2, z2);
        if (t + G >= ntiles) break;
        tile(t + G, x1, z1, x0, z0);
        if (t + 2 * G >= ntiles) break;
        tile(t + 2 * G, x2, z2, x1, z1);
    }
    lds_barrier();  // the last tile is staged
    flush();
    async_wait();  // no direct-to-LDS load may still be in flight when the workgroup ends
}

template <typename TR, bool TN = false>
clk_status launch_einsum(hipStream_t st, const void* a, const void* b, void* x, int C, int N) {
    using E = typename TR::elem;
    const int T = (N + kTriTile - 1) / kTriTile;
    const int ntiles = C * T * T;
    KernelTimer timer("tri_einsum", st);
    tri_einsum_kernel<TR, TN><<<ntiles, 512, 0, st>>>((const E*)a, (const E*)b, (E*)x, N, T,
                                                       ntiles);
    return check_launch("triangle_einsum");
}

// Positions of an [N, N] grid of U-units (u units per position) copied to or from an [NP, NP]
// grid (NP >= N): TO_PADDED fills the positions past N with zeros; otherwise only the N x N
// positions are written back.
template <typename U, bool TO_PADDED>
__global__ __launch_bounds__(256) void pad_pairs(const U* __restrict__ src, U* __restrict__ dst,
                                                 int N, int NP, int u) {
    const int S = TO_PADDED ? NP : N;  // grid edge of the destination
    const size_t total = (size_t)S * S * u;
    for (size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * 256) {
        const size_t pos = idx / u;
        const int e = (int)(idx % u), i = (int)(pos / S), j = (int)(pos % S);
        if constexpr (TO_PADDED) {
            dst[idx] = (i < N && j < N) ? src[((size_t)i * N + j) * u + e] : U{};
        } else {
            dst[idx] = src[((size_t)i * NP + j) * u + e];
        }
    }
}

template <typename U, bool TO_PADDED>
clk_status launch_pad(hipStream_t st, const void* src, void* dst, int N, int NP, int u) {
    const int S = TO_PADDED ? NP : N;
    const size_t total = (size_t)S * S * u;
    const size_t blocks = (total + 255) / 256;
    pad_pairs<U, TO_PADDED><<<(int)(blocks < 4096 ? blocks : 4096), 256, 0, st>>>(
        static_cast<const U*>(src), static_cast<U*>(dst), N, NP, u);
    return check_launch("triangle_multiply (padding)");
}

template <typename TR, int C>
clk_status launch_tri_out(hipStream_t st, const TriOutParams<typename TR::elem>& pr) {
    const int ntiles = pr.M / 64;
    const int grid = ntiles < 256 ? ntiles : 256;
    KernelTimer timer("tri_out", st);
    tri_out_kernel<TR, C><<<grid, 512, 0, st>>>(pr);
    return check_launch("triangle_multiply (output)");
}

}  // namespace

clk_status ln_gdp_channel_major(hipStream_t st, clk_dtype dtype, const void* z,
                                const float* gamma, const float* beta, const void* const* w,
                                const void* const* bias, const void* mask, void* a, void* b, int M,
                                int C, int N, float eps);

}  // namespace clk

using namespace clk;

extern "C" clk_status clk_triangle_einsum(hipStream_t stream, clk_dtype dtype, const void* a,
                                          const void* b, void* x, int64_t C, int64_t N) {
    const char* who = "triangle_einsum";
    if (dtype != CLK_F16 && dtype != CLK_BF16)
        return fail(CLK_INVALID_ARGUMENT, "%s: dtype %s not supported (f16, bf16)", who,
                    dtype_name(dtype));
    if (C < 0 || N < 0) return fail(CLK_INVALID_ARGUMENT, "%s: bad dims", who);
    if (N % 8) return fail(CLK_INVALID_ARGUMENT, "%s: N=%lld is not a multiple of 8", who,
                           (long long)N);
    if (N > 16384 || C * ((N + kTriTile - 1) / kTriTile) * ((N + kTriTile - 1) / kTriTile) >
                         INT32_MAX)
        return fail(CLK_INVALID_ARGUMENT, "%s: dims too large", who);
    if (C == 0 || N == 0) return ok();
    if (!a || !b || !x) return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    if (!aligned16(a) || !aligned16(b) || !aligned16(x))
        return fail(CLK_INVALID_ARGUMENT, "%s: a, b, x must be 16-byte aligned", who);
    if (dtype == CLK_BF16) return launch_einsum<BF16>(stream, a, b, x, (int)C, (int)N);
    return launch_einsum<F16>(stream, a, b, x, (int)C, (int)N);
}

namespace {
// N rounded up to a multiple of 8: a ragged N runs the module on a zero-padded grid.
int64_t padded_n(int64_t N) { return (N + 7) / 8 * 8; }
size_t round256(size_t v) { return (v + 255) / 256 * 256; }
// Workspace layout: left, right, x channel-major [C][NP][NP]; for a ragged N also the padded z,
// mask and output.
struct TriWorkspace {
    size_t planes, zp, mp, outp, total;
};
TriWorkspace tri_workspace(int64_t N, int64_t C) {
    const int64_t NP = padded_n(N);
    const size_t plane_set = (size_t)C * NP * NP * 2;
    TriWorkspace w;
    w.planes = 0;
    w.zp = round256(3 * plane_set);
    w.mp = w.zp + (N % 8 ? round256(plane_set) : 0);
    w.outp = w.mp + (N % 8 ? round256((size_t)NP * NP * 2) : 0);
    w.total = w.outp + (N % 8 ? plane_set : 0);
    return w;
}
}  // namespace

extern "C" size_t clk_triangle_multiply_workspace_size(int64_t N, int64_t C) {
    if (N <= 0 || C <= 0) return 0;
    return tri_workspace(N, C).total;
}

extern "C" clk_status clk_triangle_multiply(hipStream_t stream, clk_dtype dtype, const void* z,
                                            const void* mask, const float* const* ln,
                                            const void* const* w, const void* const* b, void* out,
                                            void* workspace, size_t workspace_bytes, int64_t N,
                                            int64_t C, int outgoing, float eps) {
    const char* who = "triangle_multiply";
    if (dtype != CLK_F16 && dtype != CLK_BF16)
        return fail(CLK_INVALID_ARGUMENT, "%s: dtype %s not supported (f16, bf16)", who,
                    dtype_name(dtype));
    if (N < 0 || (C != 64 && C != 128))
        return fail(CLK_INVALID_ARGUMENT, "%s: C must be 64 or 128 (C=%lld)", who, (long long)C);
    // The contraction's limit (its transposed operands span one channel plane per resource).
    if (padded_n(N) > 16384)
        return fail(CLK_INVALID_ARGUMENT, "%s: N=%lld too large (at most 16384)", who,
                    (long long)N);
    if (N == 0) return ok();
    if (!z || !mask || !ln || !w || !b || !out || !workspace)
        return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    for (int i = 0; i < 4; ++i)
        if (!ln[i]) return fail(CLK_INVALID_ARGUMENT, "%s: null LayerNorm parameter", who);
    for (int i = 0; i < 6; ++i)
        if (!w[i] || !b[i]) return fail(CLK_INVALID_ARGUMENT, "%s: null weight or bias", who);
    if (!aligned16(z) || !aligned16(out) || !aligned16(workspace))
        return fail(CLK_INVALID_ARGUMENT, "%s: z, out, workspace must be 16-byte aligned", who);
    const size_t need = clk_triangle_multiply_workspace_size(N, C);
    if (workspace_bytes < need)
        return fail(CLK_INVALID_ARGUMENT, "%s: workspace of %zu bytes, %zu needed", who,
                    workspace_bytes, need);
    // A ragged N runs on a zero-padded NP x NP grid (mask 0 there, so the padded positions
    // contribute nothing to the contraction) and copies the N x N outputs back.
    const TriWorkspace lay = tri_workspace(N, C);
    char* const ws = static_cast<char*>(workspace);
    const bool ragged = N % 8 != 0;
    const int64_t NP = padded_n(N);
    if (ragged) {
        clk_status ps = launch_pad<u32x4, true>(stream, z, ws + lay.zp, (int)N, (int)NP,
                                                (int)C * 2 / 16);
        if (ps == CLK_OK)
            ps = launch_pad<uint16_t, true>(stream, mask, ws + lay.mp, (int)N, (int)NP, 1);
        if (ps != CLK_OK) return ps;
        z = ws + lay.zp;
        mask = ws + lay.mp;
    }
    void* const out_final = out;
    if (ragged) out = ws + lay.outp;
    const int64_t N0 = N;  // the caller's grid edge
    N = NP;
    const int M = (int)(N * N), n = (int)N, c = (int)C;
    const size_t plane_set = (size_t)C * M * 2;
    char* wa = ws + lay.planes;
    char* wb = wa + plane_set;
    char* wx = wb + plane_set;
    // 1. LN_in(z) and the four projections -> left (wa), right (wb), channel-major [C][N][N].
    const void* proj_w[4] = {w[0], w[2], w[1], w[3]};  // left proj, left gate, right proj, right gate
    const void* proj_b[4] = {b[0], b[2], b[1], b[3]};
    clk_status s = ln_gdp_channel_major(stream, dtype, z, ln[0], ln[1], proj_w, proj_b, mask, wa,
                                        wb, M, c, c, eps);
    if (s != CLK_OK) return s;
    // 2. The contraction: outgoing x[c] = left[c] . right[c]^T; incoming x[c] = right[c]^T .
    //    left[c] (x[i,j] = sum_k left[k,j] right[k,i]), the contraction index first, read
    //    transposed from LDS.
    void* X = wx;
    s = outgoing ? clk_triangle_einsum(stream, dtype, wa, wb, X, C, N)
                 : (dtype == CLK_BF16 ? launch_einsum<BF16, true>(stream, wb, wa, X, c, n)
                                      : launch_einsum<F16, true>(stream, wb, wa, X, c, n));
    if (s != CLK_OK) return s;
    // 3. LN_c(x), output projection, output gate from LN_in(z).
    auto finish = [&](auto tr) -> clk_status {
        using TR = decltype(tr);
        using E = typename TR::elem;
        TriOutParams<E> pr;
        pr.x = static_cast<const E*>(X);
        pr.z = static_cast<const E*>(z);
        pr.gin = ln[0];
        pr.bin = ln[1];
        pr.gc = ln[2];
        pr.bc = ln[3];
        pr.wout = static_cast<const E*>(w[4]);
        pr.bout = static_cast<const E*>(b[4]);
        pr.wg = static_cast<const E*>(w[5]);
        pr.bg = static_cast<const E*>(b[5]);
        pr.out = static_cast<E*>(out);
        pr.M = M;
        pr.eps = eps;
        return c == 128 ? launch_tri_out<TR, 128>(stream, pr) : launch_tri_out<TR, 64>(stream, pr);
    };
    s = dtype == CLK_BF16 ? finish(BF16{}) : finish(F16{});
    if (s != CLK_OK || !ragged) return s;
    return launch_pad<u32x4, false>(stream, out, out_final, (int)N0, (int)NP, (int)C * 2 / 16);
}
