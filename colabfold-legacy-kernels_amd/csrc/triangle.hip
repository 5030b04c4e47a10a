// Triangle multiplication for gfx950: the channel-batched contraction at the centre of
// AlphaFold's TriangleMultiplication (the step that consumes the a and b the gated dual
// projection writes; the reference library stops at the projection, cuda/volta_ops.cu:97):
//   outgoing  x[i,j,c] = sum_k a[i,k,c] b[j,k,c]        incoming  x[i,j,c] = sum_k a[k,i,c] b[k,j,c]
// Per channel both are a plain N x N x N product X_c = A_c . B_c^T once a and b are stored
// channel-major with the contraction index last (A_c[i][k] = a[i,k,c] outgoing, a[k,i,c]
// incoming) -- the layout the fused LayerNorm + gated projection writes for this consumer.
//
// tri_einsum_kernel: one 256 x 256 output tile of one channel per block of 8 waves (2 x 4 wave
// tiles of 128 i x 64 j, 32 MFMA 16x16x32 accumulators each). Rows of A_c and B_c reach LDS in
// 32-wide k slices by direct buffer->LDS loads, three slices in flight; each 16-byte piece of a
// row is XOR-swizzled by (row / 4) % 4 so the sixteen rows an operand read touches fall in
// distinct banks. Per slice a block moves 32 KB from L2 for 4.2 MFLOP (128 flop/B). Tiles of
// one channel run on one XCD, whose L2 then serves A_c and B_c to all of them.
#include "common.hpp"

namespace clk {
namespace {

constexpr int kTriTile = 256;  // output tile edge
constexpr int kTriK = 32;      // contraction slice per stage

// X[c] = A[c] . B[c]^T for A, B, X [C][N][N] row-major. N must be a multiple of 8.
template <typename TR>
__global__ __launch_bounds__(512) void tri_einsum_kernel(const typename TR::elem* __restrict__ A,
                                                         const typename TR::elem* __restrict__ B,
                                                         typename TR::elem* __restrict__ X, int N,
                                                         int T, int ntiles) {
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    constexpr int BT = kTriTile, KC = kTriK;
    constexpr int PR = KC / 8;             // 16-byte pieces per row slice
    constexpr int SLICE = BT * PR * 16;    // bytes of one operand slice
    constexpr int NT = 512, DPW = 2 * BT * PR / NT;  // loads per lane and slice (A and B)
    static_assert(BT * PR % NT == 0, "whole load rounds");

    // Three stages of (A slice, B slice).
    constexpr int STAGE = 2 * SLICE;
    __shared__ __attribute__((aligned(16))) char smem[3 * STAGE];

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
    // Rows of the tile past N read zeros (the resource ends with the channel's plane).
    const Rsrc ra = buffer_rsrc(Ac + (size_t)i0 * N, (uint32_t)((size_t)min(BT, N - i0) * N * 2));
    const Rsrc rb = buffer_rsrc(Bc + (size_t)j0 * N, (uint32_t)((size_t)min(BT, N - j0) * N * 2));
    const Rsrc none = buffer_rsrc(A, 0);
    const int nk = (N + KC - 1) / KC;

    // Slice kk of both operands into buffer st: A rows at st, B rows at st + SLICE. Piece q of
    // LDS row r holds the row's 16-byte piece q ^ ((r >> 2) & 3); pieces past N read zeros.
    auto stage = [&](int kk, char* st) {
        const bool live = kk < nk;
#pragma unroll
        for (int k = 0; k < DPW; ++k) {
            const int op = k / (DPW / 2);  // 0: A, 1: B
            const int b = (k % (DPW / 2)) * NT + wave * 64;
            const int slot = b + lane, row = slot / PR;
            const int piece = (slot % PR) ^ ((row >> 2) & (PR - 1));
            const int kcol = kk * KC + piece * 8;
            const int voff = kcol < N ? (row * N + kcol) * 2 : kPastEnd;
            buf_dma16(live ? (op ? rb : ra) : none, voff, 0, st + op * SLICE + b * 16);
        }
    };

    f32x4 acc[4][8];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Operand reads. Lane (r16, g) reads k 8g..8g+7 of row 16t + r16 of its wave's rows; the
    // swizzle term (row / 4) % 4 is the same for every t, so one address serves all tiles of a
    // slice with an immediate offset of 1 KB per 16 rows.
    const uint32_t lds0 = lds_addr(smem);
    const uint32_t rd = (uint32_t)(r16 * PR + (g ^ ((r16 >> 2) & (PR - 1)))) * 16;
    const uint32_t rda = rd + 128 * wi * PR * 16, rdb = rd + SLICE + 64 * wj * PR * 16;

    stage(0, smem);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    stage(1, smem + STAGE);

    // X^T tile products: the A operand is B (rows j), the B operand is A (rows i), so a lane's
    // accumulator holds four consecutive j of one i. The loop body is not unrolled (copies of it
    // cost the register allocator more than the 256 VGPRs a lane has), so the stage buffers are
    // picked at run time and the fragment reads are explicit LDS instructions with explicit
    // waits: the compiler cannot then tie them to the direct-to-LDS loads in flight.
    for (int kk = 0; kk < nk; ++kk) {
        const int cur = kk % 3, nxt = (kk + 2) % 3;
        vm_wait<DPW>();
        lds_barrier();  // slice kk in stage cur; every wave is done reading stage nxt
        stage(kk + 2, smem + nxt * STAGE);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        const uint32_t ba = lds0 + cur * STAGE + rda, bb = lds0 + cur * STAGE + rdb;
        V8 fb0 = lds_read16<V8, 0>(bb), fb1 = lds_read16<V8, 1024>(bb);
        V8 fb2 = lds_read16<V8, 2048>(bb), fb3 = lds_read16<V8, 3072>(bb);
        V8 fa[8];
        fa[0] = lds_read16<V8, 0>(ba);
        fa[1] = lds_read16<V8, 1024>(ba);
        fa[2] = lds_read16<V8, 2048>(ba);
        fa[3] = lds_read16<V8, 3072>(ba);
        fa[4] = lds_read16<V8, 4096>(ba);
        fa[5] = lds_read16<V8, 5120>(ba);
        fa[6] = lds_read16<V8, 6144>(ba);
        fa[7] = lds_read16<V8, 7168>(ba);
        // LDS reads complete in order: fragment fa[it] is in once at most 7 - it remain.
        lds_wait<7>(fb0, fb1, fb2, fb3, fa[0]);
        auto step = [&](int it, const V8& x) {
            acc[0][it] = TR::mfma(fb0, x, acc[0][it]);
            acc[1][it] = TR::mfma(fb1, x, acc[1][it]);
            acc[2][it] = TR::mfma(fb2, x, acc[2][it]);
            acc[3][it] = TR::mfma(fb3, x, acc[3][it]);
        };
        step(0, fa[0]);
        lds_wait<6>(fa[1]);
        step(1, fa[1]);
        lds_wait<5>(fa[2]);
        step(2, fa[2]);
        lds_wait<4>(fa[3]);
        step(3, fa[3]);
        lds_wait<3>(fa[4]);
        step(4, fa[4]);
        lds_wait<2>(fa[5]);
        step(5, fa[5]);
        lds_wait<1>(fa[6]);
        step(6, fa[6]);
        lds_wait<0>(fa[7]);
        step(7, fa[7]);
    }

    // Lane (r16, g) of accumulator (jt, it) holds X[i][j..j+3] for i = i0 + 128wi + 16it + r16,
    // j = j0 + 64wj + 16jt + 4g: one 8-byte store each. Rows past N fall outside the resource;
    // columns past N (whole groups of four, N being a multiple of 8) are skipped.
    const Rsrc rx = buffer_rsrc(X + c * plane + (size_t)i0 * N,
                                (uint32_t)((size_t)min(BT, N - i0) * N * 2));
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
        const int jl = 64 * wj + 16 * jt + 4 * g;
        if (j0 + jl >= N) continue;
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int il = 128 * wi + 16 * it + r16;
            E e[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) e[q] = TR::from_f(acc[jt][it][q]);
            u32x2 v;
            __builtin_memcpy(&v, e, 8);
            __builtin_amdgcn_raw_buffer_store_b64(v, rx, (il * N + j0 + jl) * 2, 0, 0);
        }
    }
    async_wait();  // no direct-to-LDS load may still be in flight when the workgroup ends
}

template <typename TR>
clk_status launch_einsum(hipStream_t st, const void* a, const void* b, void* x, int C, int N) {
    using E = typename TR::elem;
    const int T = (N + kTriTile - 1) / kTriTile;
    const int ntiles = C * T * T;
    KernelTimer timer("tri_einsum", st);
    tri_einsum_kernel<TR><<<ntiles, 512, 0, st>>>((const E*)a, (const E*)b, (E*)x, N, T, ntiles);
    return check_launch("triangle_einsum");
}

}  // namespace
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
