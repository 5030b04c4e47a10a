// LayerNorm over the last axis for gfx950: forward (replaces VoltaLayerNorm,
// cuda/volta_ops.cu:28-95) and backward (new).
//
// Layout: x, y, dy, dx [M, C] of bf16, f16 or f32; scale, offset [C] float32.
// Each row is owned by LPR consecutive lanes; lane s of a row holds NV 16-byte vectors at
// columns ((v*LPR + s)*VEC ... +VEC), so a wave's loads are contiguous 16-byte chunks. The row
// stays in registers: the statistics are a per-lane two-pass mean/M2 merged across the LPR lanes
// with Chan's pairwise (Welford) update, then y is formed from the same registers -- one read and
// one write of HBM per element (the reference reads x twice, volta_ops.cu:40-45 and :55-58).
// HBM-bound: forward moves M*C*(b_in + b_out) bytes, backward M*C*(2*b_in + b_out).
#include "common.hpp"

namespace clk {
namespace {
// Streaming 16-byte load that does not keep its line in the caches (each row is read once):
// measured 4-8% faster for the backward and the pair-bias projection, which only read rows;
// 15% slower for the forward, whose stores are non-temporal already.
__device__ __forceinline__ u32x4 ld16_nt(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

constexpr int kThreads = 256;
// Row blocking, chosen by measurement on [512*512, 128] bf16 (each block owns a contiguous run
// of rows; the forward is fastest with one round of 16 rows per block, the backward with eight
// rounds of two rows per lane, which also keeps its partial column sums few).
constexpr int kFwdRowsPerLane = 1, kFwdRounds = 1;
constexpr int kBwdRowsPerLane = 2, kBwdRounds = 8;

template <typename TR>
struct Vec {
    static constexpr int N = 16 / sizeof(typename TR::elem);
};

template <typename TR>
__device__ __forceinline__ void unpack(u32x4 raw, float* out) {
    using E = typename TR::elem;
    constexpr int N = Vec<TR>::N;
    E e[N];
    __builtin_memcpy(e, &raw, 16);
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = TR::to_f(e[i]);
}

template <typename TR>
__device__ __forceinline__ u32x4 pack(const float* in) {
    using E = typename TR::elem;
    constexpr int N = Vec<TR>::N;
    E e[N];
#pragma unroll
    for (int i = 0; i < N; ++i) e[i] = TR::from_f(in[i]);
    u32x4 raw;
    __builtin_memcpy(&raw, e, 16);
    return raw;
}

// Chan's merge of (mean, M2) over the LPR lanes of a row, each lane starting from `count`
// elements. Every step combines the pair symmetrically (the pair's order only flips the sign of
// d), so every lane of the row ends with bit-identical values.
template <int LPR>
__device__ __forceinline__ void merge_stats(float& mean, float& m2, float count) {
    if constexpr (LPR >= 2) {
        merge_stats<LPR / 2>(mean, m2, count);
        const u32x2 pm = lane_pair<LPR / 2>(mean), p2 = lane_pair<LPR / 2>(m2);
        const float a = __uint_as_float(pm[0]), b = __uint_as_float(pm[1]);
        const float d = b - a;
        mean = (a + b) * 0.5f;
        m2 = (__uint_as_float(p2[0]) + __uint_as_float(p2[1])) + d * d * (count * (LPR / 4.f));
    }
}

template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
    return group_sum<LPR>(v);
}

// Stores of results that nothing in the kernel reads again: non-temporal, so they stream to HBM
// without displacing inputs still to be read from the caches.
__device__ __forceinline__ void st16_stream(void* p, u32x4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// Forward. A lane group of LPR lanes owns a row; each lane handles RB rows per round (rows
// row0 + r*stride), issuing all RB*NV 16-byte loads before any arithmetic so that RB loads per
// lane are in flight.
template <typename TR, int LPR, int NV, int RB>
__global__ __launch_bounds__(kThreads) void ln_fwd_kernel(const void* __restrict__ xv,
                                                          const float* __restrict__ scale,
                                                          const float* __restrict__ offset,
                                                          void* __restrict__ yv, int M,
                                                          int rows_per_block, float eps) {
    using E = typename TR::elem;
    constexpr int VEC = Vec<TR>::N;
    constexpr int C = LPR * NV * VEC;
    constexpr int ROWS = kThreads / LPR;
    const E* x = static_cast<const E*>(xv);
    E* y = static_cast<E*>(yv);
    const int s = threadIdx.x % LPR;
    const int slot = threadIdx.x / LPR;
    const int stride = gridDim.x * ROWS;

    float g[NV][VEC], b[NV][VEC];
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            const int c = (v * LPR + s) * VEC + i;
            g[v][i] = scale[c];
            b[v][i] = offset[c];
        }

    // Block b owns the contiguous rows [b*rpb, (b+1)*rpb): consecutive blocks stream
    // consecutive memory, which spreads the traffic over the HBM channels best.
    const int rpb = rows_per_block;
    const int rend = min(M, (blockIdx.x + 1) * rpb);
    (void)stride;
    for (int row0 = blockIdx.x * rpb + slot; row0 < rend; row0 += RB * ROWS) {
        u32x4 raw[RB][NV];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int row = row0 + r * ROWS;
#pragma unroll
            for (int v = 0; v < NV; ++v)
                raw[r][v] = row < rend ? ld16(x + (size_t)row * C + (v * LPR + s) * VEC)
                                       : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            // Rows past the block's range run on zeros (every lane of a group takes part in the
            // reductions) and store nothing.
            const int row = row0 + r * ROWS;
            float xs[NV][VEC];
#pragma unroll
            for (int v = 0; v < NV; ++v) unpack<TR>(raw[r][v], xs[v]);
            float sum = 0.f;
#pragma unroll
            for (int v = 0; v < NV; ++v)
#pragma unroll
                for (int i = 0; i < VEC; ++i) sum += xs[v][i];
            float mean = sum * (1.f / (NV * VEC));
            float m2 = 0.f;
#pragma unroll
            for (int v = 0; v < NV; ++v)
#pragma unroll
                for (int i = 0; i < VEC; ++i) {
                    const float d = xs[v][i] - mean;
                    m2 += d * d;
                }
            merge_stats<LPR>(mean, m2, (float)(NV * VEC));
            const float rstd = rsqrtf(m2 * (1.f / C) + eps);
            if (row < rend) {
                E* yr = y + (size_t)row * C;
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    float o[VEC];
#pragma unroll
                    for (int i = 0; i < VEC; ++i)
                        o[i] = (xs[v][i] - mean) * rstd * g[v][i] + b[v][i];
                    st16_stream(yr + (v * LPR + s) * VEC, pack<TR>(o));
                }
            }
        }
    }
}

// Streaming copy with the LayerNorm kernels' access pattern (16-byte loads, four per lane in
// flight before the stores, non-temporal stores): the HBM rate this library can reach with its
// own code, against which the LayerNorm and projection kernels are measured.
// Block b copies the contiguous 16-byte vectors [b*kCopyChunk, (b+1)*kCopyChunk) (32 KiB), four
// per thread in flight per round.
constexpr int kCopyChunk = 2048;
__global__ __launch_bounds__(kThreads) void stream_copy_kernel(const u32x4* __restrict__ src,
                                                               u32x4* __restrict__ dst,
                                                               size_t n16) {
    constexpr int RB = 4;
    const size_t beg = (size_t)blockIdx.x * kCopyChunk;
    const size_t end = beg + kCopyChunk < n16 ? beg + kCopyChunk : n16;
    for (size_t i0 = beg + threadIdx.x; i0 < end; i0 += RB * kThreads) {
        u32x4 v[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const size_t i = i0 + r * kThreads;
            v[r] = i < end ? src[i] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const size_t i = i0 + r * kThreads;
            if (i < end) st16_stream(dst + i, v[r]);
        }
    }
}

// One wave per row, any C: two passes over the row from global memory.
template <typename TR>
__global__ __launch_bounds__(kThreads) void ln_fwd_generic(const void* __restrict__ xv,
                                                           const float* __restrict__ scale,
                                                           const float* __restrict__ offset,
                                                           void* __restrict__ yv, int M, int C,
                                                           float eps) {
    using E = typename TR::elem;
    const E* x = static_cast<const E*>(xv);
    E* y = static_cast<E*>(yv);
    const int lane = threadIdx.x % 64;
    const int waves = kThreads / 64;
    for (int row = blockIdx.x * waves + threadIdx.x / 64; row < M; row += gridDim.x * waves) {
        const E* xr = x + (size_t)row * C;
        float sum = 0.f;
        for (int c = lane; c < C; c += 64) sum += TR::to_f(xr[c]);
        sum = row_sum<64>(sum);
        const float mean = sum / C;
        float m2 = 0.f;
        for (int c = lane; c < C; c += 64) {
            const float d = TR::to_f(xr[c]) - mean;
            m2 += d * d;
        }
        m2 = row_sum<64>(m2);
        const float rstd = rsqrtf(m2 / C + eps);
        E* yr = y + (size_t)row * C;
        for (int c = lane; c < C; c += 64)
            yr[c] = TR::from_f((TR::to_f(xr[c]) - mean) * rstd * scale[c] + offset[c]);
    }
}

// Backward. Per row: dx = r*(g - mean(g) - xhat*mean(g*xhat)), g = scale*dy. Column sums of
// dy*xhat and dy accumulate per lane over the rows the lane visits, then over the block's row
// slots in a fixed order, into the block-major partials part[block][which*C + c] (16-byte
// stores); ln_colsum_blocks adds each column's blocks in a fixed order.
template <typename TR, int LPR, int NV, int RB>
__global__ __launch_bounds__(kThreads) void ln_bwd_kernel(const void* __restrict__ xv,
                                                          const float* __restrict__ scale,
                                                          const void* __restrict__ dyv,
                                                          void* __restrict__ dxv,
                                                          float* __restrict__ part, int M,
                                                          int rows_per_block, float eps) {
    using E = typename TR::elem;
    constexpr int VEC = Vec<TR>::N;
    constexpr int C = LPR * NV * VEC;
    constexpr int ROWS = kThreads / LPR;
    const E* x = static_cast<const E*>(xv);
    const E* dy = static_cast<const E*>(dyv);
    E* dx = static_cast<E*>(dxv);
    const int s = threadIdx.x % LPR;
    const int slot = threadIdx.x / LPR;
    // Block b owns the contiguous rows [b*rows_per_block, (b+1)*rows_per_block).
    const int rend = min(M, (blockIdx.x + 1) * rows_per_block);

    float g[NV][VEC], acc_g[NV][VEC], acc_b[NV][VEC];
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            g[v][i] = scale[(v * LPR + s) * VEC + i];
            acc_g[v][i] = 0.f;
            acc_b[v][i] = 0.f;
        }

    // RB rows per lane per round, all their loads issued before any arithmetic. Rows past M run
    // on zeros (every lane of a group takes part in the reductions), add zero to the column
    // sums and store nothing.
    for (int row0 = blockIdx.x * rows_per_block + slot; row0 < rend; row0 += RB * ROWS) {
        u32x4 rx[RB][NV], rd[RB][NV];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int row = row0 + r * ROWS;
            const size_t base = (size_t)row * C;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                rx[r][v] = u32x4{0u, 0u, 0u, 0u};
                rd[r][v] = u32x4{0u, 0u, 0u, 0u};
                if (row < rend) {
                    rx[r][v] = ld16_nt(x + base + (v * LPR + s) * VEC);
                    rd[r][v] = ld16_nt(dy + base + (v * LPR + s) * VEC);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int row = row0 + r * ROWS;
            const size_t base = (size_t)row * C;
            float xs[NV][VEC], ds[NV][VEC];
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                unpack<TR>(rx[r][v], xs[v]);
                unpack<TR>(rd[r][v], ds[v]);
            }
            float sum = 0.f;
#pragma unroll
            for (int v = 0; v < NV; ++v)
#pragma unroll
                for (int i = 0; i < VEC; ++i) sum += xs[v][i];
            float mean = sum * (1.f / (NV * VEC));
            float m2 = 0.f;
#pragma unroll
            for (int v = 0; v < NV; ++v)
#pragma unroll
                for (int i = 0; i < VEC; ++i) {
                    const float d = xs[v][i] - mean;
                    m2 += d * d;
                }
            merge_stats<LPR>(mean, m2, (float)(NV * VEC));
            const float rstd = rsqrtf(m2 * (1.f / C) + eps);
            float sg = 0.f, sgx = 0.f;
#pragma unroll
            for (int v = 0; v < NV; ++v)
#pragma unroll
                for (int i = 0; i < VEC; ++i) {
                    const float xh = (xs[v][i] - mean) * rstd;
                    const float gg = g[v][i] * ds[v][i];
                    xs[v][i] = xh;
                    sg += gg;
                    sgx += gg * xh;
                    acc_g[v][i] += ds[v][i] * xh;
                    acc_b[v][i] += ds[v][i];
                }
            sg = row_sum<LPR>(sg) * (1.f / C);
            sgx = row_sum<LPR>(sgx) * (1.f / C);
            if (row < rend) {
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    float o[VEC];
#pragma unroll
                    for (int i = 0; i < VEC; ++i)
                        o[i] = rstd * (g[v][i] * ds[v][i] - sg - xs[v][i] * sgx);
                    st16_stream(dx + base + (v * LPR + s) * VEC, pack<TR>(o));
                }
            }
        }
    }

    // Fixed-order reduction over the ROWS row slots of this block.
    __shared__ __attribute__((aligned(16))) float red[ROWS][2][C];
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            const int c = (v * LPR + s) * VEC + i;
            red[slot][0][c] = acc_g[v][i];
            red[slot][1][c] = acc_b[v][i];
        }
    __syncthreads();
    // Block-major partials part[block][t], t = which*C + c, as 16-byte vectors of four
    // consecutive sums (one 2*C*4-byte row per block: no partial-line writes). Vector u of the
    // row sums the ROWS slots in G groups of SPG slots each, then the groups in order.
    constexpr int T4 = C / 2;  // 16-byte vectors in a block's row of 2*C sums
    constexpr int G = kThreads >= 2 * T4 ? kThreads / T4 : 1;
    constexpr int SPG = (ROWS + G - 1) / G;
    const f32x4* red4 = reinterpret_cast<const f32x4*>(&red[0][0][0]);
    f32x4* out4 = reinterpret_cast<f32x4*>(part + (size_t)blockIdx.x * 2 * C);
    if constexpr (G == 1) {
        for (int u = threadIdx.x; u < T4; u += kThreads) {
            f32x4 a = red4[u];
            for (int r = 1; r < ROWS; ++r) a += red4[r * T4 + u];
            out4[u] = a;
        }
    } else {
        __shared__ f32x4 grp[G][T4];
        const int u = threadIdx.x % T4, gi = threadIdx.x / T4;
        if (gi < G) {
            f32x4 a = {0.f, 0.f, 0.f, 0.f};
            for (int r = gi * SPG; r < min(ROWS, (gi + 1) * SPG); ++r) a += red4[r * T4 + u];
            grp[gi][u] = a;
        }
        __syncthreads();
        if (threadIdx.x < T4) {
            f32x4 a = grp[0][threadIdx.x];
#pragma unroll
            for (int i = 1; i < G; ++i) a += grp[i][threadIdx.x];
            out4[threadIdx.x] = a;
        }
    }
}

template <typename TR>
__global__ __launch_bounds__(kThreads) void ln_bwd_generic(const void* __restrict__ xv,
                                                           const float* __restrict__ scale,
                                                           const void* __restrict__ dyv,
                                                           void* __restrict__ dxv,
                                                           float* __restrict__ part, int M, int C,
                                                           float eps) {
    using E = typename TR::elem;
    const E* x = static_cast<const E*>(xv);
    const E* dy = static_cast<const E*>(dyv);
    E* dx = static_cast<E*>(dxv);
    const int lane = threadIdx.x % 64;
    const int wave = threadIdx.x / 64;
    constexpr int waves = kThreads / 64;
    // Per-wave column partials live in part as scratch rows [block][wave][2][C] -> reduced below.
    float* wpart = part + ((size_t)blockIdx.x * (waves + 1) + 1 + wave) * 2 * C;
    for (int c = lane; c < C; c += 64) {
        wpart[c] = 0.f;
        wpart[C + c] = 0.f;
    }
    for (int row = blockIdx.x * waves + wave; row < M; row += gridDim.x * waves) {
        const size_t base = (size_t)row * C;
        float sum = 0.f;
        for (int c = lane; c < C; c += 64) sum += TR::to_f(x[base + c]);
        const float mean = row_sum<64>(sum) / C;
        float m2 = 0.f;
        for (int c = lane; c < C; c += 64) {
            const float d = TR::to_f(x[base + c]) - mean;
            m2 += d * d;
        }
        const float rstd = rsqrtf(row_sum<64>(m2) / C + eps);
        float sg = 0.f, sgx = 0.f;
        for (int c = lane; c < C; c += 64) {
            const float xh = (TR::to_f(x[base + c]) - mean) * rstd;
            const float d = TR::to_f(dy[base + c]);
            sg += scale[c] * d;
            sgx += scale[c] * d * xh;
            wpart[c] += d * xh;
            wpart[C + c] += d;
        }
        sg = row_sum<64>(sg) / C;
        sgx = row_sum<64>(sgx) / C;
        for (int c = lane; c < C; c += 64) {
            const float xh = (TR::to_f(x[base + c]) - mean) * rstd;
            const float d = TR::to_f(dy[base + c]);
            dx[base + c] = TR::from_f(rstd * (scale[c] * d - sg - xh * sgx));
        }
    }
    __syncthreads();
    float* bpart = part + (size_t)blockIdx.x * (waves + 1) * 2 * C;
    for (int t = threadIdx.x; t < 2 * C; t += kThreads) {
        float a = 0.f;
        for (int w = 0; w < waves; ++w)
            a += part[((size_t)blockIdx.x * (waves + 1) + 1 + w) * 2 * C + t];
        bpart[t] = a;
    }
}

// out[which][c] = sum over the partial rows b of part[b*stride + which*C + c], in a fixed order:
// 64 row groups (b = sp, sp+64, ...) each summed with sixteen interleaved accumulators, so that a
// thousand partial rows are one round of loads in flight per thread, then the groups are added
// in order. 16 columns per 1024-thread block.
constexpr int kColsumCols = 16;
__global__ __launch_bounds__(1024) void ln_colsum(const float* __restrict__ part, size_t stride,
                                                  int nblocks, int C, float* __restrict__ dscale,
                                                  float* __restrict__ doffset) {
    constexpr int kCols = kColsumCols, kSplit = 64, kAcc = 16;
    __shared__ float red[kSplit][kCols];
    const int cl = threadIdx.x % kCols, sp = threadIdx.x / kCols;
    const int t = blockIdx.x * kCols + cl;  // over 2*C outputs
    float acc[kAcc];
#pragma unroll
    for (int i = 0; i < kAcc; ++i) acc[i] = 0.f;
    if (t < 2 * C) {
        int b = sp;
        for (; b + (kAcc - 1) * kSplit < nblocks; b += kAcc * kSplit) {
#pragma unroll
            for (int i = 0; i < kAcc; ++i) acc[i] += part[(size_t)(b + i * kSplit) * stride + t];
        }
#pragma unroll
        for (int i = 0; i < kAcc - 1; ++i)
            if (b + i * kSplit < nblocks) acc[i] += part[(size_t)(b + i * kSplit) * stride + t];
    }
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < kAcc; ++i) a += acc[i];
    red[sp][cl] = a;
    __syncthreads();
    if (sp == 0 && t < 2 * C) {
        float r = 0.f;
        for (int i = 0; i < kSplit; ++i) r += red[i][cl];
        if (t < C) dscale[t] = r;
        else doffset[t - C] = r;
    }
}

// The fast backward's column sums: out[t] = sum over the nblocks partial rows b of
// part[b*2*C + t] (block-major, 16-byte aligned), four columns t = 4u .. 4u+3 per block of 256
// threads: thread i adds rows i, i+256, ... in order (all its loads issued first), each wave
// reduces its 64 lanes by a fixed butterfly (group_sum), and the four waves' sums are added in
// order. Deterministic.
__global__ __launch_bounds__(256) void ln_colsum_blocks(const float* __restrict__ part,
                                                        int nblocks, int C,
                                                        float* __restrict__ dscale,
                                                        float* __restrict__ doffset) {
    constexpr int kIn = 8;  // loads in flight per thread (2048 partial rows in one round)
    // Column groups placed XCD-contiguously: the eight groups of one 128-byte line of every
    // partial row then run on one XCD, whose L2 fetches the line once (the identity order put
    // them on eight XCDs, each fetching it: 8.4 MB read for 1 MB of partials at C = 128).
    const int u = xcd_contiguous(blockIdx.x, gridDim.x);
    const f32x4* p4 = reinterpret_cast<const f32x4*>(part) + u;
    const size_t rs = (size_t)C / 2;  // 16-byte vectors per partial row
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
    for (int b0 = threadIdx.x; b0 < nblocks; b0 += 256 * kIn) {
        f32x4 v[kIn];
#pragma unroll
        for (int i = 0; i < kIn; ++i) {
            const int b = b0 + 256 * i;
            v[i] = b < nblocks ? p4[(size_t)b * rs] : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int i = 0; i < kIn; ++i) a += v[i];
    }
    __shared__ f32x4 wsum[4];
    f32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = group_sum<64>(a[j]);
    if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = w;
    __syncthreads();
    if (threadIdx.x < 4) {
        const float v = ((wsum[0][threadIdx.x] + wsum[1][threadIdx.x]) + wsum[2][threadIdx.x]) +
                        wsum[3][threadIdx.x];
        const int t = 4 * u + (int)threadIdx.x;
        if (t < C) dscale[t] = v;
        else doffset[t - C] = v;
    }
}

// (LPR, NV) for a row of C elements of VEC per 16-byte vector; {0,0} when no fast kernel fits.
struct RowShape {
    int lpr, nv;
};
// Lanes per row: a power of two from 4 to 64 dividing the row's vector count, and at most half
// of it when there are eight vectors or more, so that a lane holds two vectors: at C = 128 bf16,
// 8 lanes of two vectors measured 5.9 TB/s forward (the streaming copy's rate at that size)
// against 5.0 with 16 lanes of one (shorter lane reductions, two loads in flight per lane).
RowShape row_shape(int64_t C, int vec) {
    if (C <= 0 || C % vec != 0) return {0, 0};
    const int64_t nvec = C / vec;
    const int64_t cap = nvec >= 8 ? nvec / 2 : nvec;
    int lpr = 1;
    while (lpr < 64 && lpr * 2 <= cap && nvec % (lpr * 2) == 0) lpr *= 2;
    const int64_t nv = nvec / lpr;
    if (lpr < 4 || nv > 4) return {0, 0};
    return {lpr, (int)nv};
}

constexpr int kMaxBwdBlocks = 1024;

int fwd_blocks(int64_t M, int rows_per_block) {
    const int64_t b = (M + rows_per_block - 1) / rows_per_block;
    return (int)(b < 4096 ? b : 4096);
}
// Rows per block of the fast backward: kBwdRounds times the block's row slots (rounds of
// kBwdRowsPerLane rows per lane cover it in kBwdRounds / kBwdRowsPerLane), and few enough blocks that the partial column sums stay within the generic
// path's workspace (kMaxBwdBlocks * 5 partial rows).
int fast_bwd_rows_per_block(int64_t M, int lpr) {
    const int64_t round = kThreads / lpr;
    int64_t rpb = round * kBwdRounds;
    const int64_t cap_blocks = (int64_t)kMaxBwdBlocks * (kThreads / 64 + 1);
    while ((M + rpb - 1) / rpb > cap_blocks) rpb += round;
    return (int)rpb;
}

int bwd_blocks(int64_t M, int rows_per_block) {
    const int64_t b = (M + rows_per_block - 1) / rows_per_block;
    return (int)(b < kMaxBwdBlocks ? b : kMaxBwdBlocks);
}

// ---------------------------------------------------------------------------------------------
// Pair-bias projection (AlphaFold's triangle-attention / MSA-row-attention bias, the step before
// the attention kernels): bias[h, m] = sum_c LN(z)[m, c] * w[c, h], i.e. LN(z).w transposed to
// [H, M] = [H, Sq, Sk], the layout the attention bias argument takes. One pass over z, with LN
// folded into the projection:
//   LN(z).w = rstd * (z.w' - mean * sum_c w'[c]) + offset.w,   w' = diag(scale) w,
// so a row needs only its raw values: the sum and sum of squares (one pass, as the reference's
// LayerNorm, volta_ops.cu:40-52) and the H dot products z.w' are pair dot products (v_dot2) on
// the packed 16-bit inputs, with w' rounded to the input type like the MFMA operands of the fused
// LN + GDP. The LPR lanes of a row reduce them with DPP; lane h < H of the row stores head h.
// HBM-bound on the read of z (M*C*b_in bytes in, M*H*b_out out).
// ---------------------------------------------------------------------------------------------
template <typename TR, int LPR, int NV, int H>
__global__ __launch_bounds__(kThreads) void ln_bias_kernel(const void* __restrict__ xv,
                                                           const float* __restrict__ scale,
                                                           const float* __restrict__ offset,
                                                           const void* __restrict__ wv,
                                                           void* __restrict__ biasv, int M,
                                                           float eps) {
    using E = typename TR::elem;
    constexpr int VEC = Vec<TR>::N;
    static_assert(VEC == 8, "16-bit inputs: four pairs per 16-byte vector");
    constexpr int C = LPR * NV * VEC;
    constexpr int ROWS = kThreads / LPR;
    static_assert(H <= LPR, "one storing lane per head");
    const E* x = static_cast<const E*>(xv);
    const E* w = static_cast<const E*>(wv);
    E* bias = static_cast<E*>(biasv);
    const int s = threadIdx.x % LPR;
    const int slot = threadIdx.x / LPR;

    // w' for this lane's channels as packed pairs, its column sums and offset . w, both reduced
    // over the row's lanes (the column sums from the rounded w' the dot products use).
    uint32_t wp[NV][4][H];
    float csum[H], hb[H];
#pragma unroll
    for (int h = 0; h < H; ++h) csum[h] = hb[h] = 0.f;
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int h = 0; h < H; ++h) {
                E pr[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int c = (v * LPR + s) * VEC + 2 * q + e;
                    const float wch = TR::to_f(w[c * H + h]);
                    pr[e] = TR::from_f(scale[c] * wch);
                    csum[h] += TR::to_f(pr[e]);
                    hb[h] = fmaf(offset[c], wch, hb[h]);
                }
                __builtin_memcpy(&wp[v][q][h], pr, 4);
            }
#pragma unroll
    for (int h = 0; h < H; ++h) {
        csum[h] = row_sum<LPR>(csum[h]);
        hb[h] = row_sum<LPR>(hb[h]);
    }

    // A row group takes RPI consecutive rows per iteration: RPI loads in flight per lane, and
    // lane h stores head h of those rows as one RPI*2-byte piece.
    constexpr int RPI = 4;
    const int64_t stride = (int64_t)gridDim.x * ROWS * RPI;
    for (int64_t r0 = ((int64_t)blockIdx.x * ROWS + slot) * RPI; r0 < M; r0 += stride) {
        u32x4 raw[RPI][NV];
#pragma unroll
        for (int r = 0; r < RPI; ++r)
#pragma unroll
            for (int v = 0; v < NV; ++v)
                raw[r][v] = r0 + r < M ? ld16_nt(x + (r0 + r) * C + (v * LPR + s) * VEC) : u32x4{};
        E out[RPI];
#pragma unroll
        for (int r = 0; r < RPI; ++r) {
            float sum = 0.f, sq = 0.f, d[H];
#pragma unroll
            for (int h = 0; h < H; ++h) d[h] = 0.f;
#pragma unroll
            for (int v = 0; v < NV; ++v)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    sum = dot2<TR>(raw[r][v][q], kOnePair<TR>, sum);
                    sq = dot2<TR>(raw[r][v][q], raw[r][v][q], sq);
#pragma unroll
                    for (int h = 0; h < H; ++h) d[h] = dot2<TR>(raw[r][v][q], wp[v][q][h], d[h]);
                }
            const float mean = row_sum<LPR>(sum) * (1.f / C);
            const float var = fmaxf(fmaf(row_sum<LPR>(sq), 1.f / C, -mean * mean), 0.f);
            const float rstd = __builtin_amdgcn_rsqf(var + eps);
            float mine = 0.f;
#pragma unroll
            for (int h = 0; h < H; ++h) {
                const float val = fmaf(rstd, fmaf(-mean, csum[h], row_sum<LPR>(d[h])), hb[h]);
                if (s == h) mine = val;
            }
            out[r] = TR::from_f(mine);
        }
        if (s < H) {
            E* dst = bias + (size_t)s * M + r0;
            if (r0 + RPI <= M && (M % RPI) == 0 && (reinterpret_cast<uintptr_t>(bias) & 7) == 0) {
                uint64_t piece;
                __builtin_memcpy(&piece, out, 8);
                *reinterpret_cast<uint64_t*>(dst) = piece;
            } else {
#pragma unroll
                for (int r = 0; r < RPI; ++r)
                    if (r0 + r < M) dst[r] = out[r];
            }
        }
    }
}

template <typename TR, int LPR, int NV, int H>
void launch_bias(hipStream_t st, const void* x, const float* sc, const float* of, const void* w,
                 void* bias, int M, float eps) {
    // Four rows per row group and iteration; 1024 blocks (four per CU) measured faster than
    // one block per row group (each wave then prepares w' for only four rows).
    const int64_t groups = ((int64_t)M + 3) / 4, per = kThreads / LPR;
    const int grid = (int)std::min<int64_t>((groups + per - 1) / per, 1024);
    KernelTimer timer("ln_bias", st);
    ln_bias_kernel<TR, LPR, NV, H><<<grid, kThreads, 0, st>>>(x, sc, of, w, bias, M, eps);
}

template <typename TR, int H>
bool dispatch_bias_h(hipStream_t st, const void* x, const float* sc, const float* of,
                     const void* w, void* bias, int M, int C, float eps) {
    RowShape rs = row_shape(C, Vec<TR>::N);
    if (rs.lpr < H && rs.nv % 2 == 0) {  // one storing lane per head: twice the lanes
        rs.lpr *= 2;
        rs.nv /= 2;
    }
#define CLK_LNB_CASE(L, V)                                              \
    if constexpr (H <= (L))                                             \
        if (rs.lpr == (L) && rs.nv == (V)) {                            \
            launch_bias<TR, L, V, H>(st, x, sc, of, w, bias, M, eps);   \
            return true;                                                \
        }
    CLK_LNB_CASE(4, 1) CLK_LNB_CASE(4, 2) CLK_LNB_CASE(8, 1) CLK_LNB_CASE(8, 2)
    CLK_LNB_CASE(16, 1) CLK_LNB_CASE(16, 2) CLK_LNB_CASE(32, 1) CLK_LNB_CASE(32, 2)
#undef CLK_LNB_CASE
    return false;
}

template <typename TR>
bool dispatch_bias(hipStream_t st, const void* x, const float* sc, const float* of, const void* w,
                   void* bias, int M, int C, int H, float eps) {
    switch (H) {
        case 1: return dispatch_bias_h<TR, 1>(st, x, sc, of, w, bias, M, C, eps);
        case 2: return dispatch_bias_h<TR, 2>(st, x, sc, of, w, bias, M, C, eps);
        case 4: return dispatch_bias_h<TR, 4>(st, x, sc, of, w, bias, M, C, eps);
        case 8: return dispatch_bias_h<TR, 8>(st, x, sc, of, w, bias, M, C, eps);
        default: return false;
    }
}

template <typename TR, int LPR, int NV>
void launch_fwd(hipStream_t st, const void* x, const float* sc, const float* of, void* y, int M,
                float eps) {
    constexpr int RB = kFwdRowsPerLane;
    constexpr int ROWS = kThreads / LPR;
    const int rpb = ROWS * RB * kFwdRounds;
    const int grid = ceil_div(M, rpb);
    KernelTimer timer("ln_fwd", st);
    ln_fwd_kernel<TR, LPR, NV, RB><<<grid, kThreads, 0, st>>>(x, sc, of, y, M, rpb, eps);
}

template <typename TR>
bool dispatch_fwd(hipStream_t st, const void* x, const float* sc, const float* of, void* y,
                  int M, int C, float eps) {
    const RowShape rs = row_shape(C, Vec<TR>::N);
#define CLK_LN_CASE(L, V)                                        \
    if (rs.lpr == (L) && rs.nv == (V)) {                         \
        launch_fwd<TR, L, V>(st, x, sc, of, y, M, eps);          \
        return true;                                             \
    }
#define CLK_LN_ROW(L) CLK_LN_CASE(L, 1) CLK_LN_CASE(L, 2) CLK_LN_CASE(L, 3) CLK_LN_CASE(L, 4)
    CLK_LN_ROW(4) CLK_LN_ROW(8) CLK_LN_ROW(16) CLK_LN_ROW(32) CLK_LN_ROW(64)
#undef CLK_LN_ROW
#undef CLK_LN_CASE
    const int grid = fwd_blocks(M, kThreads / 64);
    KernelTimer timer("ln_fwd", st);
    ln_fwd_generic<TR><<<grid, kThreads, 0, st>>>(x, sc, of, y, M, C, eps);
    return false;
}

template <typename TR, int LPR, int NV>
void launch_bwd(hipStream_t st, const void* x, const float* sc, const void* dy, void* dx,
                float* part, int M, float eps) {
    constexpr int RB = kBwdRowsPerLane;
    const int rpb = fast_bwd_rows_per_block(M, LPR);
    const int grid = ceil_div(M, rpb);
    KernelTimer timer("ln_bwd", st);
    ln_bwd_kernel<TR, LPR, NV, RB><<<grid, kThreads, 0, st>>>(x, sc, dy, dx, part, M, rpb, eps);
}

// Returns the number of partial rows written and their stride (floats); stride 0: the fast
// kernel's column-major runs (part[t][block]).
template <typename TR>
void dispatch_bwd(hipStream_t st, const void* x, const float* sc, const void* dy, void* dx,
                  float* part, int M, int C, float eps, int* nblocks, size_t* stride) {
    const RowShape rs = row_shape(C, Vec<TR>::N);
#define CLK_LN_CASE(L, V)                                          \
    if (rs.lpr == (L) && rs.nv == (V)) {                           \
        launch_bwd<TR, L, V>(st, x, sc, dy, dx, part, M, eps);     \
        *nblocks = ceil_div(M, fast_bwd_rows_per_block(M, L));     \
        *stride = 0; /* column-major runs */                       \
        return;                                                    \
    }
#define CLK_LN_ROW(L) CLK_LN_CASE(L, 1) CLK_LN_CASE(L, 2) CLK_LN_CASE(L, 3) CLK_LN_CASE(L, 4)
    CLK_LN_ROW(4) CLK_LN_ROW(8) CLK_LN_ROW(16) CLK_LN_ROW(32) CLK_LN_ROW(64)
#undef CLK_LN_ROW
#undef CLK_LN_CASE
    const int grid = bwd_blocks(M, kThreads / 64);
    KernelTimer timer("ln_bwd", st);
    ln_bwd_generic<TR><<<grid, kThreads, 0, st>>>(x, sc, dy, dx, part, M, C, eps);
    *nblocks = grid;
    *stride = (size_t)(kThreads / 64 + 1) * 2 * C;
}

size_t bwd_workspace(int64_t M, int64_t C) {
    // Generic path needs (waves + 1) * 2 * C floats per block; the fast path 2 * C.
    const int64_t blocks = bwd_blocks(M, kThreads / 64);
    return (size_t)blocks * (kThreads / 64 + 1) * 2 * C * sizeof(float);
}

clk_status validate(const char* who, clk_dtype dtype, const void* x, const float* scale,
                    const void* y, int64_t M, int64_t C) {
    if (dtype != CLK_F16 && dtype != CLK_BF16 && dtype != CLK_F32)
        return fail(CLK_INVALID_ARGUMENT, "%s: dtype %s not supported (f16, bf16, f32)", who,
                    dtype_name(dtype));
    if (M < 0 || C <= 0) return fail(CLK_INVALID_ARGUMENT, "%s: x must be [M,C] with C > 0", who);
    if (M > INT32_MAX || C > (1 << 20) || M * C > ((int64_t)1 << 40))
        return fail(CLK_INVALID_ARGUMENT, "%s: [M,C] = [%lld,%lld] too large", who,
                    (long long)M, (long long)C);
    if (M > 0 && (!x || !scale || !y))
        return fail(CLK_INVALID_ARGUMENT, "%s: null pointer", who);
    if (M > 0 && (!aligned16(x) || !aligned16(y)))
        return fail(CLK_INVALID_ARGUMENT, "%s: x and y must be 16-byte aligned", who);
    return CLK_OK;
}

}  // namespace
}  // namespace clk

using namespace clk;

extern "C" clk_status clk_stream_copy(hipStream_t stream, const void* src, void* dst,
                                      size_t bytes) {
    if (bytes == 0) return ok();
    if (!src || !dst || !aligned16(src) || !aligned16(dst) || bytes % 16)
        return fail(CLK_INVALID_ARGUMENT,
                    "stream_copy: src and dst must be 16-byte aligned, bytes a multiple of 16");
    const size_t n16 = bytes / 16;
    const size_t blocks = (n16 + kCopyChunk - 1) / kCopyChunk;
    if (blocks >= ((size_t)1 << 31))
        return fail(CLK_INVALID_ARGUMENT, "stream_copy: %zu bytes too large", bytes);
    const int grid = (int)blocks;
    KernelTimer timer("stream_copy", stream);
    stream_copy_kernel<<<grid, kThreads, 0, stream>>>(static_cast<const u32x4*>(src),
                                                      static_cast<u32x4*>(dst), n16);
    return check_launch("stream_copy");
}

extern "C" clk_status clk_layer_norm_fwd(hipStream_t stream, clk_dtype dtype, const void* x,
                                         const float* scale, const float* offset, void* y,
                                         int64_t M, int64_t C, float eps) {
    clk_status s = validate("layer_norm", dtype, x, scale, y, M, C);
    if (s != CLK_OK) return s;
    if (M > 0 && !offset) return fail(CLK_INVALID_ARGUMENT, "layer_norm: null offset");
    if (M == 0) return ok();
    switch (dtype) {
        case CLK_BF16: dispatch_fwd<BF16>(stream, x, scale, offset, y, (int)M, (int)C, eps); break;
        case CLK_F16: dispatch_fwd<F16>(stream, x, scale, offset, y, (int)M, (int)C, eps); break;
        default: dispatch_fwd<F32>(stream, x, scale, offset, y, (int)M, (int)C, eps); break;
    }
    return check_launch("layer_norm");
}

extern "C" size_t clk_layer_norm_bwd_workspace_size(int64_t M, int64_t C) {
    if (M <= 0 || C <= 0) return 0;
    return bwd_workspace(M, C);
}

extern "C" clk_status clk_layer_norm_bwd(hipStream_t stream, clk_dtype dtype, const void* x,
                                         const float* scale, const void* dy, void* dx,
                                         float* dscale, float* doffset, void* workspace,
                                         size_t workspace_bytes, int64_t M, int64_t C,
                                         float eps) {
    clk_status s = validate("layer_norm_bwd", dtype, x, scale, dx, M, C);
    if (s != CLK_OK) return s;
    if (M > 0 && (!dy || !dscale || !doffset || !workspace))
        return fail(CLK_INVALID_ARGUMENT, "layer_norm_bwd: null pointer");
    if (M > 0 && (!aligned16(dy) || !aligned16(workspace)))
        return fail(CLK_INVALID_ARGUMENT,
                    "layer_norm_bwd: dy and workspace must be 16-byte aligned");
    const size_t need = clk_layer_norm_bwd_workspace_size(M, C);
    if (workspace_bytes < need)
        return fail(CLK_INVALID_ARGUMENT, "layer_norm_bwd: workspace %zu bytes, needs %zu",
                    workspace_bytes, need);
    if (M == 0) {
        if (!dscale || !doffset) return fail(CLK_INVALID_ARGUMENT, "layer_norm_bwd: null pointer");
        // No rows: the column sums are zero (a fill kernel, so the call stays graph-capturable).
        ln_colsum<<<ceil_div(2 * C, kColsumCols), 1024, 0, stream>>>(nullptr, 0, 0, (int)C,
                                                                     dscale, doffset);
        return check_launch("layer_norm_bwd");
    }
    float* part = static_cast<float*>(workspace);
    int nblocks = 0;
    size_t stride = 0;
    switch (dtype) {
        case CLK_BF16:
            dispatch_bwd<BF16>(stream, x, scale, dy, dx, part, (int)M, (int)C, eps, &nblocks,
                               &stride);
            break;
        case CLK_F16:
            dispatch_bwd<F16>(stream, x, scale, dy, dx, part, (int)M, (int)C, eps, &nblocks,
                              &stride);
            break;
        default:
            dispatch_bwd<F32>(stream, x, scale, dy, dx, part, (int)M, (int)C, eps, &nblocks,
                              &stride);
            break;
    }
    KernelTimer timer("ln_bwd_colsum", stream);
    if (stride == 0)  // the fast kernel's block-major rows (C % 4 == 0: 16-byte vectors)
        ln_colsum_blocks<<<(int)(2 * C / 4), 256, 0, stream>>>(part, nblocks, (int)C, dscale,
                                                              doffset);
    else
        ln_colsum<<<ceil_div(2 * C, kColsumCols), 1024, 0, stream>>>(part, stride, nblocks,
                                                                     (int)C, dscale, doffset);
    return check_launch("layer_norm_bwd");
}

extern "C" clk_status clk_ln_pair_bias(hipStream_t stream, clk_dtype dtype, const void* z,
                                       const float* scale, const float* offset, const void* w,
                                       void* bias, int64_t M, int64_t C, int64_t H, float eps) {
    const char* who = "ln_pair_bias";
    if (dtype != CLK_F16 && dtype != CLK_BF16)
        return fail(CLK_INVALID_ARGUMENT, "%s: dtype %s not supported (f16, bf16)", who,
                    dtype_name(dtype));
    if (M < 0 || M > INT32_MAX || (H != 1 && H != 2 && H != 4 && H != 8))
        return fail(CLK_INVALID_ARGUMENT, "%s: M=%lld, H=%lld (H must be 1, 2, 4 or 8)", who,
                    (long long)M, (long long)H);
    if (C != 64 && C != 128 && C != 256)
        return fail(CLK_INVALID_ARGUMENT, "%s: C=%lld (64, 128 or 256)", who, (long long)C);
    if (M == 0) return ok();
    if (!z || !scale || !offset || !w || !bias)
        return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    if (!aligned16(z)) return fail(CLK_INVALID_ARGUMENT, "%s: z must be 16-byte aligned", who);
    const bool done = dtype == CLK_BF16
                          ? dispatch_bias<BF16>(stream, z, scale, offset, w, bias, (int)M,
                                                (int)C, (int)H, eps)
                          : dispatch_bias<F16>(stream, z, scale, offset, w, bias, (int)M,
                                               (int)C, (int)H, eps);
    if (!done) return fail(CLK_INVALID_ARGUMENT, "%s: C=%lld not supported", who, (long long)C);
    return check_launch(who);
}
