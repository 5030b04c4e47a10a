// Pieces shared by the attention forward and backward kernels: tile geometry, global->LDS tile
// staging, MFMA operand reads from LDS, bias/mask loads and host-side validation.
#pragma once

#include <cmath>

#include "common.hpp"

namespace clk {

// Geometry for head dim D: 64-key (or 64-query) tiles; KS contraction steps of 32 head dims for
// the products that contract over D; DT 16-row tiles of head dims for the products that output
// head dims. LDS rows are padded by 8 elements (16 bytes) to spread banks.
template <int D>
struct AttnGeom {
    static_assert(D == 8 || D == 16 || D == 32 || D == 64, "head dim 8, 16, 32 or 64");
    static constexpr int BK = 64;
    static constexpr int KS = (D + 31) / 32;
    static constexpr int DT = (D + 15) / 16;
    static constexpr int DV = DT * 16;
    static constexpr int KLD = D + 8;
    static constexpr int VLD = DV + 8;
};

// Row of the 16-row operand tile t (0..3) of a 64-row tile that lane row r16 supplies. Inside
// each 32-row chunk c = t/2 the rows are permuted so that the C tile of the product holds rows
// 32c + 8*(l/16) + 0..7 in lane l: half t%2 covers +0..3, the other +4..7.
// True when some byte of the eight is zero (an absent key).
__device__ __forceinline__ bool has_zero_byte(u32x2 w) {
    const unsigned a = (w[0] - 0x01010101u) & ~w[0] & 0x80808080u;
    const unsigned b = (w[1] - 0x01010101u) & ~w[1] & 0x80808080u;
    return (a | b) != 0u;
}

__device__ __forceinline__ int perm_key(int t, int r16) {
    return 32 * (t >> 1) + 8 * (r16 >> 2) + 4 * (t & 1) + (r16 & 3);
}

// 8-slot MFMA operand from a row-major LDS tile: row `row`, head dims 32*ks + 8*g + 0..7
// (zero beyond D).
template <typename V8, int D, typename E>
__device__ __forceinline__ V8 lds_row_operand(const E* lds, int row, int ld, int ks, int g) {
    const int d0 = ks * 32 + g * 8;
    u32x4 raw = {0u, 0u, 0u, 0u};
    if (d0 < D) raw = *reinterpret_cast<const u32x4*>(lds + row * ld + d0);
    return bits_as<V8>(raw);
}

// 8-slot MFMA operand of the transposed tile: lane (r16, g) gets column 16*dt + r16 of rows
// 32c + 8g + 0..7 of a row-major LDS tile (two ds_read_b64_tr_b16).
template <typename V8, typename E>
__device__ __forceinline__ V8 lds_tr_operand(const E* lds, int ld, int c, int dt, int r16,
                                             int g) {
    const E* lo = lds + (32 * c + 8 * g + (r16 >> 2)) * ld + 16 * dt + 4 * (r16 & 3);
    return lds_tr8<V8>(lo, lo + 4 * ld);
}

// Stages a 64-row x D tile of one or two [S, D] operands: 16-byte global loads into registers
// (rows past S read as zero), then 16-byte LDS stores.
template <typename E, int D, int NOPS>
struct RowTileStager {
    static constexpr int CPR = D / 8;
    static constexpr int CHUNKS = 64 * CPR;
    static constexpr int CPT = (CHUNKS + 255) / 256;
    u32x4 r[NOPS][CPT];

    // Rows row0 .. row0+63 of each src (rows gld elements apart; rows past S read zeros).
    __device__ __forceinline__ void load(const E* const* src, int row0, int S, int gld = D) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int ch = threadIdx.x + 256 * i;
            const int row = ch / CPR, c8 = (ch % CPR) * 8;
            const bool in = ch < CHUNKS && row0 + row < S;
#pragma unroll
            for (int o = 0; o < NOPS; ++o) {
                r[o][i] = u32x4{0u, 0u, 0u, 0u};
                if (in) r[o][i] = ld16(src[o] + (size_t)(row0 + row) * gld + c8);
            }
        }
    }
    __device__ __forceinline__ void store(E* const* dst, const int* ld) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int ch = threadIdx.x + 256 * i;
            if (ch < CHUNKS) {
                const int row = ch / CPR, c8 = (ch % CPR) * 8;
#pragma unroll
                for (int o = 0; o < NOPS; ++o)
                    *reinterpret_cast<u32x4*>(dst[o] + row * ld[o] + c8) = r[o][i];
            }
        }
    }
};

// K and V key tiles for the forward pass.
template <typename E, int D>
struct TileStager {
    RowTileStager<E, D, 2> st;
    __device__ __forceinline__ void load(const E* kp, const E* vp, int k0, int Sk) {
        const E* src[2] = {kp, vp};
        st.load(src, k0, Sk);
    }
    __device__ __forceinline__ void store(E* k_lds, E* v_lds) {
        E* dst[2] = {k_lds, v_lds};
        const int ld[2] = {AttnGeom<D>::KLD, AttnGeom<D>::VLD};
        st.store(dst, ld);
    }
};

// Zero the LDS columns D..DV-1 of a V-like tile (only D = 8 has any); they feed output rows that
// are never stored, but must not hold NaN bit patterns from earlier kernels.
template <typename E, int D>
__device__ __forceinline__ void zero_v_padding(E* lds) {
    constexpr int DV = AttnGeom<D>::DV, VLD = AttnGeom<D>::VLD;
    if constexpr (DV > D) {
        for (int i = threadIdx.x; i < 64 * (DV - D); i += blockDim.x)
            lds[(i / (DV - D)) * VLD + D + i % (DV - D)] = E(0.f);
    }
}

// Eight bias values bias_row[kk .. kk+7] as float (zero past Sk).
template <typename TR>
__device__ __forceinline__ void load_bias8(const typename TR::elem* row, int kk, int Sk,
                                           int vec_ok, float* out) {
    using E = typename TR::elem;
    if (vec_ok && kk + 8 <= Sk) {
        E e[8];
        u32x4 raw = ld16(row + kk);
        __builtin_memcpy(e, &raw, 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = TR::to_f(e[j]);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = (kk + j < Sk) ? TR::to_f(row[kk + j]) : 0.f;
    }
}

// Bit j set when key kk + j exists (< Sk) and is present in the mask row (or there is no mask).
__device__ __forceinline__ unsigned key_valid8(const uint8_t* mrow, int kk, int Sk, int vec_ok) {
    unsigned bits = 0;
    if (mrow && vec_ok && kk + 8 <= Sk && ((reinterpret_cast<uintptr_t>(mrow + kk) & 7u) == 0)) {
        const u32x2 w = *reinterpret_cast<const u32x2*>(mrow + kk);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bits |= (((w[0] >> (8 * j)) & 0xffu) != 0u ? 1u : 0u) << j;
            bits |= (((w[1] >> (8 * j)) & 0xffu) != 0u ? 1u : 0u) << (4 + j);
        }
        return bits;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const bool in = kk + j < Sk;
        const bool present = in && (mrow == nullptr || mrow[kk + j] != 0);
        bits |= (present ? 1u : 0u) << j;
    }
    return bits;
}

// Logit given to masked keys of one mask row: -1e9, or 0 when the row has no present key (the
// softmax is uniform either way; 0 keeps the running max and the logsumexp exact in float32).
// Must be reached by every thread of the block.
__device__ __forceinline__ float masked_logit_for_row(const uint8_t* mrow, int Sk) {
    int any = 0;
    if (mrow) {
        for (int i = threadIdx.x; i < Sk; i += blockDim.x) any |= mrow[i] != 0;
    }
    any = __syncthreads_or(any);
    return (mrow && !any) ? 0.f : kMaskedLogit;
}

// ---------------------------------------------------------------------------------------------
// Swizzled LDS tiles filled with direct global->LDS loads (global_load_lds_dwordx4: lane i of a
// wave instruction writes 16 bytes at the instruction's LDS base + 16*i).
//
// A tile row holds PL 16-byte pieces (PL = DV/8 >= 2; pieces past D/8 are zero padding used by
// the transposed reads of D = 8). Logical piece p of row r sits in physical slot p ^ swz(r),
// swz(r) = (r >> 3) & (PL - 1): the row reads of a 16-key operand (keys 8j + 0..3) and the 4x16
// transposed reads then touch distinct bank groups.
// ---------------------------------------------------------------------------------------------

template <int D>
struct SwzTile {
    static constexpr int DV = AttnGeom<D>::DV;
    static constexpr int PL = DV / 8;
    static constexpr int P = D / 8;
    static constexpr int ROWB = PL * 16;
    static __device__ __forceinline__ int swz(int row) { return (row >> 3) & (PL - 1); }
    static __device__ __forceinline__ int off(int row, int piece) {
        return row * ROWB + 16 * (piece ^ swz(row));
    }
};

// Issues async loads of rows [r0, r0 + ROWS) of a row-major [S, D] 2-byte slice (the resource
// covers its S rows, so rows past S read zeros, as do the padding pieces of D < 16) into a
// swizzled LDS tile. ROWS*PL must be a multiple of 64. Every thread of the block calls it;
// completion is awaited with async_wait() before a barrier.
template <int D, int ROWS, int NTHREADS>
__device__ __forceinline__ void stage_rows(Rsrc r, int r0, char* lds) {
    using T = SwzTile<D>;
    constexpr int SLOTS = ROWS * T::PL;
    static_assert(SLOTS % 64 == 0, "tile must be whole wave instructions");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int b = wave * 64; b < SLOTS; b += NTHREADS) {
        const int slot = b + lane;
        const int row = slot / T::PL;
        const int piece = (slot % T::PL) ^ T::swz(row);
        const int voff = piece < T::P ? (row * D + piece * 8) * 2 : kPastEnd;
        buf_dma16(r, voff, r0 * D * 2, lds + b * 16);
    }
}

// stage_rows for D-column rows that lie `ld` elements apart (a column block of a wider
// row-major matrix): row r of the resource starts at byte 2*r*ld. Rows past the resource read
// zeros. `tid` is the thread's index in the block (taken as an argument so that a caller can
// keep its offsets from being shared with, and kept live across, earlier code).
template <int D, int ROWS, int NTHREADS>
__device__ __forceinline__ void stage_rows_ld(Rsrc r, int r0, int ld, char* lds, int tid) {
    using T = SwzTile<D>;
    constexpr int SLOTS = ROWS * T::PL;
    static_assert(SLOTS % 64 == 0, "tile must be whole wave instructions");
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int i = 0; i < (SLOTS + NTHREADS - 1) / NTHREADS; ++i) {
        const int b = wave * 64 + i * NTHREADS;
        if (SLOTS % NTHREADS != 0 && b >= SLOTS) break;
        const int slot = b + lane;
        const int row = slot / T::PL;
        const int piece = (slot % T::PL) ^ T::swz(row);
        const int voff = piece < T::P ? (row * ld + piece * 8) * 2 : kPastEnd;
        buf_dma16(r, voff, r0 * ld * 2, lds + b * 16);
    }
}


// The rows of one (n, h) of an attention operand: [N, H, S, D] (rows D apart), or with NSHD
// AlphaFold's [N, S, H, D] (rows H*D apart, head h at column block h).
template <int D, bool NSHD>
struct HeadRows {
    // Element offset of row s of head h of batch row n.
    static __device__ __forceinline__ size_t at(int n, int h, int s, int S, int H) {
        return NSHD ? (((size_t)n * S + s) * H + h) * D : (((size_t)n * H + h) * S + s) * D;
    }
    static __device__ __forceinline__ int ld(int H) { return NSHD ? H * D : D; }
    // Bytes from row 0's start to row S-1's end: a buffer resource over exactly the S rows.
    static __device__ __forceinline__ uint32_t bytes(int S, int H) {
        if constexpr (NSHD) return S > 0 ? (uint32_t)(((size_t)(S - 1) * H * D + D) * 2) : 0u;
        else return (uint32_t)S * D * 2;
    }
};

// stage_rows over the rows of one (n, h) in either layout (`r` from HeadRows' offset and bytes).
template <int D, int ROWS, int NTHREADS, bool NSHD>
__device__ __forceinline__ void stage_head_rows(Rsrc r, int r0, int H, char* lds) {
    if constexpr (NSHD)
        stage_rows_ld<D, ROWS, NTHREADS>(r, r0, H * D, lds, threadIdx.x);
    else
        stage_rows<D, ROWS, NTHREADS>(r, r0, lds);
}

// Row operand from a swizzled tile: row `row`, head dims 32*ks + 8*g + 0..7 (zero beyond D).
template <typename V8, int D>
__device__ __forceinline__ V8 swz_row_operand(const char* lds, int row, int ks, int g) {
    const int piece = ks * 4 + g;
    u32x4 raw = {0u, 0u, 0u, 0u};
    if (piece * 8 < D) raw = *reinterpret_cast<const u32x4*>(lds + SwzTile<D>::off(row, piece));
    return bits_as<V8>(raw);
}

// Transposed operand from a swizzled tile: lane (r16, g) gets column 16*dt + r16 of rows
// rbase + 8g + 0..7 (rbase = 32*chunk).
template <typename V8, int D>
__device__ __forceinline__ V8 swz_tr_operand(const char* lds, int rbase, int dt, int r16, int g) {
    const int row = rbase + 8 * g + (r16 >> 2);
    const int col = 16 * dt + 4 * (r16 & 3);  // element column, a multiple of 4
    const int piece = col >> 3, inner = (col & 7) * 2;
    const char* lo = lds + SwzTile<D>::off(row, piece) + inner;
    const char* hi = lds + SwzTile<D>::off(row + 4, piece) + inner;
    return lds_tr8<V8>(lo, hi);
}

// swz_tr_operand for a split key order: lane (r16, g) gets column 16*dt + r16 of rows
// rbase + 4g + 0..3 and rbase + 16 + 4g + 0..3.
template <typename V8, int D>
__device__ __forceinline__ V8 swz_tr_operand_split(const char* lds, int rbase, int dt, int r16,
                                                   int g) {
    const int row = rbase + 4 * g + (r16 >> 2);
    const int col = 16 * dt + 4 * (r16 & 3);
    const int piece = col >> 3, inner = (col & 7) * 2;
    const char* lo = lds + SwzTile<D>::off(row, piece) + inner;
    const char* hi = lds + SwzTile<D>::off(row + 16, piece) + inner;
    return lds_tr8<V8>(lo, hi);
}

template <typename TR>
__device__ __forceinline__ void store4(typename TR::elem* p, f32x4 v) {
    using E = typename TR::elem;
    E e[4] = {TR::from_f(v[0]), TR::from_f(v[1]), TR::from_f(v[2]), TR::from_f(v[3])};
    u32x2 raw;
    __builtin_memcpy(&raw, e, 8);
    st8(p, raw);
}

// How the backward kernels form log2(P) with one FMA per score: the MFMA that computes q.k
// takes the bias, in "bias units", as its accumulator input, so its result r = q.k + bias*bscale
// and log2(e) * logit = cexp * r. For scale != 0: bscale = 1/scale, cexp = scale*log2(e). For a
// scale too small to invert (|scale| < 2^-100, including 0) the logit is the bias alone to
// float32 precision: Q is replaced by zeros, bscale = 1, cexp = log2(e). A bias whose scaled
// value exceeds 1e38 in magnitude saturates there (NaN stays NaN).
struct LogitForm {
    float bscale, cexp;
    int qzero;
    static LogitForm make(float scale) {
        if (fabsf(scale) < 0x1p-100f) return {1.f, kLog2e, 1};
        return {1.f / scale, scale * kLog2e, 0};
    }
    __device__ __forceinline__ float bias_units(float b) const {
        const float v = b * bscale;
        return fabsf(v) > 1e38f ? copysignf(1e38f, v) : v;
    }
};

// How the logits reach the softmax in the kernels that stream bias tiles through LDS (the
// forward and the dK/dV kernel). Plain: logit = fmaf(q.k, scale, bias) per score (bias unpacked
// to float32). Bias MFMA (when scale > 0): the accumulator of each 16x16 score tile starts as
// bias / scale, added by one more MFMA per 16x16 tile whose A
// operand is [hi*I | lo*I] (hi + lo = 1/scale as two values of the input type, each product
// with a bias value exact in float32) and whose B operand is the tile's bias, duplicated over
// the two halves of the contraction; the tile then holds logit / scale, and
// log2(e) * logit = cexp * S with cexp = scale * log2(e). No per-score instruction touches the bias. A bias of
// magnitude above 3.4e38 * scale overflows there (float32 cannot hold bias / scale).
struct BiasMfma {
    float hi, lo, bscale, cexp;
};

// The bias-MFMA constants for `scale`, when that form applies: scale > 0 with 1/scale finite
// and within the input type's range (hi + lo = 1/scale to about 16 bits).
template <typename TR>
bool bias_mfma_for(float scale, BiasMfma* bm) {
    using E = typename TR::elem;
    if (!(scale > 0.f) || !std::isfinite(scale)) return false;
    const float b = 1.f / scale;
    if (!std::isfinite(b) || b > 6.0e4f) return false;
    const float hi = (float)(E)b;
    *bm = {hi, (float)(E)(b - hi), b, scale * kLog2e};
    return true;
}

// Host-side shape/dtype validation shared by the forward and backward entry points. The
// reference checks only the rank of q (cuda/volta_mma_attn.cu:310-314); every size is checked
// here before any launch.
inline clk_status validate_attention(const char* who, clk_dtype dtype, int64_t N, int64_t H,
                                     int64_t Sq, int64_t Sk, int64_t D) {
    if (dtype != CLK_F16 && dtype != CLK_BF16)
        return fail(CLK_INVALID_ARGUMENT, "%s: dtype %s not supported (f16, bf16)", who,
                    dtype_name(dtype));
    if (N < 0 || H < 0 || Sq < 0 || Sk < 0)
        return fail(CLK_INVALID_ARGUMENT, "%s: negative dimension", who);
    if (D != 8 && D != 16 && D != 32 && D != 64)
        return fail(CLK_INVALID_ARGUMENT, "%s: unsupported head dim D=%lld (8, 16, 32, 64)", who,
                    (long long)D);
    if (N > 65535 || H > 65535 || Sq > (1 << 20) || Sk > (1 << 20))
        return fail(CLK_INVALID_ARGUMENT, "%s: dims [N=%lld,H=%lld,Sq=%lld,Sk=%lld] too large",
                    who, (long long)N, (long long)H, (long long)Sq, (long long)Sk);
    if (N * H * (Sq > Sk ? Sq : Sk) * D > ((int64_t)1 << 40) || H * Sq * Sk > ((int64_t)1 << 40))
        return fail(CLK_INVALID_ARGUMENT, "%s: tensor too large", who);
    if (N * H * (((Sq > Sk ? Sq : Sk) + 63) / 64) >= ((int64_t)1 << 31))  // 1-D grids of tiles
        return fail(CLK_INVALID_ARGUMENT, "%s: too many query or key tiles", who);
    return CLK_OK;
}

}  // namespace clk
