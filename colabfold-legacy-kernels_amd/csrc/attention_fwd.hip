// Flash attention forward with a per-head pair bias and a per-row key mask, for gfx950.
// Replaces VoltaMma (cuda/volta_mma_attn.cu:70-351) and VoltaWmma (cuda/volta_wmma_attn.cu:
// 47-311) with one kernel for f16 and bf16 on MFMA 16x16x32 with float32 accumulation.
//
// Work split: a block of 4 waves owns (query tile of 64*QT rows, head h, row n); each wave owns
// 16*QT queries and streams the keys in tiles of 64 through double-buffered LDS: tile kt+1 is
// fetched with direct global->LDS loads (and its bias rows into registers) while tile kt is
// computed, so each tile costs one barrier. Which tiles contain an absent key is worked out once
// per block from the mask row; the others skip the mask entirely.
//
// Per 64-key tile and 16-query sub-tile a wave computes S^T = K . Q^T with the keys of each
// 32-key chunk permuted so that lane l's accumulator holds keys 8*(l/16)+0..7 of the chunk for
// query l%16. Those eight values are exactly the B operand of O^T = V^T . P^T for that chunk, so
// P never leaves registers; V^T comes from LDS with ds_read_b64_tr_b16 (two 4x16 transposed
// reads per operand). O^T accumulates four consecutive head dims per lane, stored as 8 bytes.
//
// Numerics (volta_mma_attn.cu:137,174-272): logit = scale*(q.k) + bias in float32; a key with
// kmask == 0 gets the logit -1e9 (the float32 value of the caller's additive 1e9*(mask-1)), a
// key past Sk gets -inf; online softmax in the exp2 domain, whose running max moves only when a
// tile's max exceeds it by more than 2^8 in P (so P <= 256, and O and l are rescaled on few
// tiles); P rounded to the input type for the P.V product (as the reference rounds it to f16,
// :221: the relative rounding is the same at any magnitude); O = acc / max(l, 1e-30) (:265).
// A row whose keys are all masked gets the logit 0 for them instead: its softmax is the same
// (uniform over the Sk keys), but float32 cannot subtract a running max of -1e9 exactly (its
// rounding unit there is 128), which would scale P by up to 2^64.
// lse = m + log(l) (natural log) is written when requested, for the backward pass; for an
// all-masked row it is therefore ln(Sk), relative to the masked logit. Present-key logits are
// expected above -5e8 (half the masked logit, where the running max starts): a row whose
// present keys all lie below it has no weight, O = 0 and lse = +inf (zero gradients).
#include "attention_common.hpp"

#include <type_traits>

namespace clk {
namespace {

constexpr float kRescaleSlack = 8.f;  // log2 of the largest P before the running max moves
constexpr int kGateChannels = 128;    // gate channels (wg rows) per K/V buffer in the epilogue
constexpr int kPresWords = 256;       // most key tiles of the bias-patching forward (LDS words)
constexpr float kLn2 = 0.69314718055994531f;

// Cross-group max of two values at once (lanes l, l^16, l^32, l^48 share a query): the halves
// of a and b meet in one register, so the three lane swaps serve both.
__device__ __forceinline__ void xgroup_max2(float& a, float& b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                    false);
    // lanes 0..31: a's lanes l and l+32; lanes 32..63: b's lanes l-32 and l
    float c = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(c), false,
                                                    false);
    c = fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
    const auto u = __builtin_amdgcn_permlane32_swap(__float_as_uint(c), __float_as_uint(c), false,
                                                    false);
    a = __uint_as_float(u[0]);
    b = __uint_as_float(u[1]);
}

// Per-tile "some key absent or past Sk" flags of one mask row, as bits of a 64-bit word (tiles of
// 64 keys; tiles past the 64th always take the checked path), worked out by each wave on its
// own with ballots -- no LDS and no block barrier. Also returns the row's masked logit.
struct RowFlags {
    uint64_t bits;
    float masked_logit;
};
template <bool VEC>
__device__ __forceinline__ RowFlags row_flags(const uint8_t* mrow, int Sk) {
    const int lane = threadIdx.x & 63;
    const int ntiles = (Sk + 63) / 64;
    // The ragged last tile (tiles from the 64th on are always checked: no bit for them).
    uint64_t bits = (Sk % 64 && ntiles <= 64) ? 1ull << (ntiles - 1) : 0ull;
    bool any_present = false;
    if (mrow) {
        for (int base = 0; base < Sk; base += 512) {
            const int k = base + 8 * lane;
            bool absent = false, present = false;
            if constexpr (VEC) {
                // Sk % 8 == 0 and 8-byte aligned rows: whole 8-key groups.
                if (k < Sk) {
                    const u32x2 m = *reinterpret_cast<const u32x2*>(mrow + k);
                    present = (m[0] | m[1]) != 0u;
                    absent = has_zero_byte(m);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (k + j < Sk) {
                        const bool p = mrow[k + j] != 0;
                        present |= p;
                        absent |= !p;
                    }
            }
            const uint64_t ab = __ballot(absent);
            any_present |= __ballot(present) != 0ull;
#pragma unroll
            for (int t = 0; t < 8; ++t)
                if (base / 64 + t < 64 && ((ab >> (8 * t)) & 0xffull)) bits |= 1ull << (base / 64 + t);
        }
    }
    return {bits, (mrow && !any_present) ? 0.f : kMaskedLogit};
}

// Per-lane prefetch state of one key tile: the mask bytes of keys k0 + 32c + 8g + 0..7 (c = 0, 1)
// and, unless the bias tile travels through LDS (VEC), the bias of those keys for each of the
// lane's query rows. VEC (Sk % 8 == 0, 8-byte aligned mask rows): 8-byte mask loads whose address
// is clamped into the row (keys past Sk are forced to -inf anyway); otherwise element loads.
template <typename TR, int QT, bool VEC, bool BM = false>
struct TilePrefetch {
    u32x2 mask[2];
    u32x4 bias[VEC ? 1 : QT][2];
    __device__ __forceinline__ void load(const typename TR::elem* const* brow,
                                         const uint8_t* mrow, int k0, int g, int Sk) {
        using E = typename TR::elem;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int kk = k0 + 32 * c + 8 * g;
            if constexpr (VEC) {
                if constexpr (BM) {
                    // Keys k0 + 32c + 4g + 0..3 and k0 + 32c + 16 + 4g + 0..3 (the bias-MFMA
                    // key order), 4-byte loads clamped into the row.
                    const int k4 = k0 + 32 * c + 4 * g;
                    mask[c] = mrow ? u32x2{*reinterpret_cast<const unsigned*>(mrow + min(k4, Sk - 4)),
                                           *reinterpret_cast<const unsigned*>(
                                               mrow + min(k4 + 16, Sk - 4))}
                                   : u32x2{~0u, ~0u};
                } else {
                    mask[c] = mrow ? *reinterpret_cast<const u32x2*>(mrow + min(kk, Sk - 8))
                                   : u32x2{~0u, ~0u};
                }
            } else {
                uint8_t m[8];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    m[j] = kk + j < Sk ? (mrow ? mrow[kk + j] : uint8_t(1)) : uint8_t(0);
                __builtin_memcpy(&mask[c], m, 8);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) {
                    E e[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) e[j] = kk + j < Sk ? brow[qt][kk + j] : E(0.f);
                    __builtin_memcpy(&bias[qt][c], e, 16);
                }
            }
        }
    }
    // Bit j set when key k0 + 32c + 8g + j is present.
    __device__ __forceinline__ unsigned valid(int c) const {
        unsigned bits = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bits |= (((mask[c][0] >> (8 * j)) & 0xffu) != 0u ? 1u : 0u) << j;
            bits |= (((mask[c][1] >> (8 * j)) & 0xffu) != 0u ? 1u : 0u) << (4 + j);
        }
        return bits;
    }
};

// Operands of the output gate fused into the forward's epilogue:
//   gated[n, s, h*D + d] = O[n, h, s, d] * sigmoid(x[n, s, :] . wg[:, h*D + d] + bg[h*D + d])
// with x [N, Sq, C], wg [C, HD] row-major, bg [HD], gated [N, Sq, HD], HD = H*D, C % 32 == 0.
template <typename E>
struct GateArgs {
    const E* x;
    const E* wg;
    const E* bg;
    E* gated;
    int C, HD;
};

template <typename TR, int D, int QT, bool VEC, bool GATE, bool BM, bool NSHD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D <= 32 && VEC ? 3 : 1))) void attn_fwd_kernel(
    const typename TR::elem* __restrict__ q, const typename TR::elem* __restrict__ k,
    const typename TR::elem* __restrict__ v, const typename TR::elem* __restrict__ bias,
    const uint8_t* __restrict__ kmask, typename TR::elem* __restrict__ out,
    float* __restrict__ lse, int H, int Sq, int Sk, float scale,
    GateArgs<typename TR::elem> ga, BiasMfma bm, int grp) {
    static_assert(!BM || VEC, "the bias MFMA reads the bias tile from LDS");
    static_assert(!(NSHD && GATE), "the gated entry takes the [N, H, S, D] layout");
    using E = typename TR::elem;
    using V8 = typename TR::vec8;
    using G = AttnGeom<D>;
    using T = SwzTile<D>;
    // PATCH (the bias tile in LDS): a key tile with an absent key (or keys past Sk) has its bias
    // changed in LDS before use -- a large negative bias for an absent key (P = 0 after the
    // exponential once the row's max comes from a present key): the masked logit -1e9 in
    // bfloat16, float16's lowest value -65504 in float16 (the reference's own masked logit is
    // -1e4); 0 for every key in range in a row without any present key (whose Q^T is zero, so
    // every logit is that row's masked logit 0) -- and the scores need no per-key select, so the
    // tile's MFMAs and exponentials stay one straight-line block. (No larger magnitude: the
    // exponent's FMA against the running max leaves a rounding residue of about 2^-24 of the
    // logit, which must stay far below float32's exponent range.)
    constexpr bool PATCH = VEC;
    using PF = TilePrefetch<TR, QT, VEC, BM>;
    constexpr int BQ = 4 * 16 * QT;
    constexpr int BK = G::BK;
    constexpr int TILE = BK * T::ROWB;  // bytes of one K or V tile
    constexpr int BTILE = VEC ? BQ * 128 : 0;  // bias tile: BQ query rows of 64 keys

    // Two K/V buffers as separate LDS objects: the compiler then knows that reads of one do not
    // wait for the direct-to-LDS loads into the other.
    __shared__ __attribute__((aligned(16))) char kv0[2 * TILE + BTILE];  // K rows, V rows, bias
    __shared__ __attribute__((aligned(16))) char kv1[2 * TILE + BTILE];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    // 1-D grid of (query tile, head, row) work items, placed so that each XCD runs a contiguous
    // range of them. grp == 0: query tile fastest, then the head, then the row -- the blocks of
    // one (row, query tile) read the same gate rows of x and, in the [N, S, H, D] layout, the
    // same cache lines of q, k and v, and the query tiles of one (row, head) the same K and V.
    // grp > 0 (a bias too large to stay in an XCD's L2 over all heads): the head outermost, then
    // groups of grp rows, then the query tile, then the row within its group -- an XCD's resident
    // blocks then read one head's bias rows (the same for every row n) and the K and V of a few
    // rows, both of which stay in its L2.
    const int qtiles = (Sq + BQ - 1) / BQ;
    const int item = xcd_contiguous(blockIdx.x, gridDim.x);
    int q0, h, n;
    if (grp == 0) {
        q0 = (item % qtiles) * BQ;
        h = (item / qtiles) % H;
        n = item / (qtiles * H);
    } else {
        const int nrows = gridDim.x / (qtiles * H), per_head = qtiles * nrows;
        h = item / per_head;
        const int rem = item - h * per_head;
        const int gi = rem / (grp * qtiles), nb = gi * grp, gsz = min(grp, nrows - nb);
        q0 = (rem - gi * grp * qtiles) / gsz * BQ;
        n = nb + (rem - gi * grp * qtiles) % gsz;
    }
    const size_t nh = (size_t)n * H + h;
    // Rows of one (n, h) in q, k, v and out: [N, H, S, D] (rows D apart), or with NSHD
    // [N, S, H, D] (rows H*D apart, head h at column block h).
    const int ld = NSHD ? H * D : D;
    const E* qp = q + (NSHD ? ((size_t)n * Sq * H + h) * D : nh * Sq * D);
    const E* kp = k + (NSHD ? ((size_t)n * Sk * H + h) * D : nh * Sk * D);
    const E* vp = v + (NSHD ? ((size_t)n * Sk * H + h) * D : nh * Sk * D);
    E* const op = out ? out + (NSHD ? ((size_t)n * Sq * H + h) * D : nh * Sq * D) : nullptr;
    const E* bp = bias + (size_t)h * Sq * Sk;
    const uint8_t* mp = kmask ? kmask + (size_t)n * Sk : nullptr;
    const int qbase = q0 + wave * 16 * QT;
    const int ntiles = (Sk + BK - 1) / BK;

    // The Sk rows of (n, h): rows past Sk read zeros.
    const uint32_t kvbytes = NSHD ? (Sk > 0 ? (uint32_t)(((size_t)(Sk - 1) * ld + D) * 2) : 0u)
                                  : (uint32_t)Sk * D * 2;
    const Rsrc rk = buffer_rsrc(kp, kvbytes);
    const Rsrc rv = buffer_rsrc(vp, kvbytes);
    // The block's bias rows (queries q0 .. q0+BQ-1 that exist).
    const Rsrc rb = buffer_rsrc(bp + (size_t)q0 * Sk, (uint32_t)(min(BQ, Sq - q0) * Sk * 2));
    // Head h's D columns of the gate weight: row c (channel) starts HD elements after row c-1.
    const Rsrc rw = GATE ? buffer_rsrc(ga.wg + h * D, (uint32_t)((ga.C - 1) * ga.HD + D) * 2)
                         : rb;
    auto stage = [&](int k0, char* kv) {
        if constexpr (NSHD) {
            stage_rows_ld<D, BK, 256>(rk, k0, ld, kv, threadIdx.x);
            stage_rows_ld<D, BK, 256>(rv, k0, ld, kv + TILE, threadIdx.x);
        } else {
            stage_rows<D, BK, 256>(rk, k0, kv);
            stage_rows<D, BK, 256>(rv, k0, kv + TILE);
        }
        if constexpr (VEC) {
            // Bias rows q0 .. q0+BQ-1, keys k0 .. k0+63 as eight 16-byte pieces per row; piece
            // p of row r sits at position p ^ (r & 7), so a 16-row operand read is conflict-free.
            // Rows past Sq read zeros; keys past Sk (last tile) read whatever follows, and are
            // forced to -inf.
#pragma unroll
            for (int b = wave * 64; b < BQ * 8; b += 256) {
                const int slot = b + lane;
                const int row = slot >> 3, piece = (slot & 7) ^ (row & 7);
                buf_dma16(rb, (row * Sk + 8 * piece) * 2, k0 * 2, kv + 2 * TILE + b * 16);
            }
        }
    };
    // PATCH: this wave's mask bytes of its first two key tiles (t = wave, wave + 4; lane l:
    // key 64t + l), loaded before anything else so that the presence words below wait for them
    // alone.
    uint32_t mb[2] = {0u, 0u};
    if constexpr (PATCH) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int kk = (wave + 4 * i) * BK + lane;
            if (kk < Sk) mb[i] = mp ? mp[kk] : 1u;
        }
    }
    if (ntiles > 0) stage(0, kv0);

    // B operand Q^T: lane (query r16, group g) holds head dims 32*ks + 8*g + 0..7.
    V8 qf[QT][G::KS];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int row = qbase + qt * 16 + r16;
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            const int d0 = ks * 32 + g * 8;
            u32x4 raw = {0u, 0u, 0u, 0u};
            if (row < Sq && d0 < D) raw = ld16(qp + (size_t)row * ld + d0);
            qf[qt][ks] = bits_as<V8>(raw);
        }
    }

    // Bias rows of the lane's queries (clamped inside [0, Sq)), keys 32c + 8g + 0..7 per tile.
    const E* brow[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) brow[qt] = bp + (size_t)min(qbase + qt * 16 + r16, Sq - 1) * Sk;
    PF ca, cb;
    if (ntiles > 0) ca.load(brow, mp, 0, g, Sk);
    // The mask row's tile flags, with the Q and first-tile loads already in flight (PATCH
    // reads the same facts from the presence words instead).
    const RowFlags rf = PATCH ? RowFlags{0ull, kMaskedLogit} : row_flags<VEC>(mp, Sk);
    // PATCH: the row's presence bits, one 64-bit word per key tile (bit j: key 64t + j is
    // present and below Sk; the launch keeps ntiles <= kPresWords), and per wave 1 + the last
    // of its tiles that holds a present key (0 if none).
    __shared__ unsigned long long pres[PATCH ? kPresWords : 1];
    __shared__ int wave_last[PATCH ? 4 : 1];
    if constexpr (PATCH) {
        int last = 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int t = wave + 4 * i;
            if (t < ntiles) {
                const unsigned long long b = __ballot(mb[i] != 0u);
                if (b != 0ull) last = t + 1;
                if (lane == 0) pres[t] = b;
            }
        }
        for (int t = wave + 8; t < ntiles; t += 4) {
            const int kk = t * BK + lane;
            const unsigned long long b = __ballot(kk < Sk && (mp == nullptr || mp[kk] != 0));
            if (b != 0ull) last = t + 1;
            if (lane == 0) pres[t] = b;
        }
        if (lane == 0) wave_last[wave] = last;
    }
    // PATCH: a row without any present key: every logit is its masked logit 0, so Q^T = 0 and
    // the changed bias tiles hold 0 in range. Otherwise the key tiles after the row's last
    // present key (a padding tail) add P = 0 to O and l and are not run at all: after the row's
    // max is set their P underflows to 0.
    bool row_empty = false;
    int nrun = ntiles;  // key tiles the loop runs
    if constexpr (PATCH) {
        __syncthreads();  // the presence words and counts are visible
        const int last = max(max(wave_last[0], wave_last[1]), max(wave_last[2], wave_last[3]));
        row_empty = mp && last == 0;
        if (!row_empty) nrun = last;
        if (row_empty) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt)
#pragma unroll
                for (int ks = 0; ks < G::KS; ++ks) qf[qt][ks] = V8{};
        }
    }
    // PATCH: lane (row r16 of each sub-tile, group g) changes 16-byte pieces 4c + g (keys
    // k0 + 32c + 8g + 0..7) of its rows of tile kt's bias: all its pieces are read, changed and
    // written back in one round.
    auto patch = [&](const char* kvc, int kt) {
        char* const bt = const_cast<char*>(kvc) + 2 * TILE;
        const float fill_bias = std::is_same<TR, BF16>::value ? kMaskedLogit : -65504.f;
        const uint32_t neg = (uint32_t)__builtin_bit_cast(uint16_t, TR::from_f(fill_bias)) * 0x10001u;
        u32x4* at[2][QT];
        u32x4 v[2][QT];
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const int row = wave * 16 * QT + 16 * qt + r16;
                at[c][qt] = reinterpret_cast<u32x4*>(bt + row * 128 + 16 * ((4 * c + g) ^ (row & 7)));
                v[c][qt] = *at[c][qt];
            }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int kk = kt * BK + 32 * c + 8 * g;
            // A key past Sk gets the fill value in every row.
            const uint32_t fill = kk < Sk && row_empty ? 0u : neg;
            const uint32_t bits = reinterpret_cast<const uint32_t*>(pres)[2 * kt + c] >> (8 * g);
            // Dword i holds keys 2i, 2i+1 (low, high half): keep the bias of present keys.
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t keep = ((bits >> (2 * i)) & 1u ? 0xffffu : 0u) |
                                      ((bits >> (2 * i + 1)) & 1u ? 0xffff0000u : 0u);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
                    v[c][qt][i] = (v[c][qt][i] & keep) | (fill & ~keep);
            }
        }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) *at[c][qt] = v[c][qt];
    };
    // In the bias-MFMA form every score is in units of 1/scale of the logit (xs = scale*log2e
    // per unit); otherwise in logit units (xs = log2e).
    const float masked_logit = BM ? rf.masked_logit * bm.bscale : rf.masked_logit;
    const float xs = BM ? bm.cexp : kLog2e;
    // A operand [hi*I | lo*I] of the bias MFMA: lane (row r16, group g) holds columns
    // 8g .. 8g+7, so its one nonzero is element r16 % 8 when g % 2 == r16 / 8.
    V8 idn;
    if constexpr (BM) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            idn[j] = TR::from_f((j == (r16 & 7) && (g & 1) == (r16 >> 3)) ? (g < 2 ? bm.hi : bm.lo)
                                                                      : 0.f);
    }

    // Running max, and O^T plus one extra accumulator per sub-tile: the MFMA of an all-ones
    // A operand with P^T, i.e. the row sum of the (rounded) P that the P.V product uses.
    V8 ones;
#pragma unroll
    for (int j = 0; j < 8; ++j) ones[j] = TR::from_f(1.f);
    // The running max starts at half the masked logit: a tile whose keys are all absent (its
    // max the masked logit) then adds P = 0 exactly. Starting lower, the first such tile would
    // set the max, and P = exp2(x*xs - m*xs) of its keys would be the exponential of the FMA's
    // rounding residue (up to 2^6 at a logit of 1e9), which float16 cannot hold. In a row with
    // no present key every logit is the masked logit 0, the start.
    // Kept as nm = -m*xs, the exponent's offset itself: a tile's move test is one FMA, its
    // exponent FMAs take nm as it is, and lse = m*scale + ln(l) becomes -nm*ln2 + ln(l).
    float nm[QT];
    f32x4 acc[QT][G::DT], lsum[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        nm[qt] = -(0.5f * masked_logit) * xs;
        lsum[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) acc[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    auto tile = [&](int kt, const char* kvc, char* kvn, PF& cur, PF& nxt) {
        const int k0 = kt * BK;
        async_wait();
        __syncthreads();  // tile kt visible; every wave is done with the other buffer
        bool need_mask;
        if constexpr (PATCH) {
            const int rem = Sk - k0;  // keys of the tile below Sk
            const unsigned long long full = rem >= 64 ? ~0ull : (1ull << rem) - 1ull;
            need_mask = (rem < 64) || pres[kt] != full;
        } else {
            need_mask = kt >= 64 || ((rf.bits >> kt) & 1ull) != 0ull;
        }
        if (kt + 1 < nrun) {
            stage(k0 + BK, kvn);
            nxt.load(brow, mp, k0 + BK, g, Sk);
        } else if constexpr (GATE) {
            // The last key tile leaves the other buffer free: the wg rows of the first
            // kGateChannels gate channels go there now, ready for the epilogue.
            int t = threadIdx.x;
            asm volatile("" : "+v"(t));
            stage_rows_ld<D, kGateChannels, 256>(rw, 0, ga.HD, kvn, t);
        }
        // Each wave reads only its own rows of the bias tile: no barrier after the change.
        if (PATCH && need_mask) {
            patch(kvc, kt);
            // Nothing of the tile's work is interleaved with the change (registers).
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
        }
        V8 kf[4][G::KS];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int ks = 0; ks < G::KS; ++ks)
                kf[t][ks] = swz_row_operand<V8, D>(kvc, BM ? 16 * t + r16 : perm_key(t, r16), ks, g);
        V8 vf[G::DT][2];
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
            for (int c = 0; c < 2; ++c)
                vf[dt][c] = BM ? swz_tr_operand_split<V8, D>(kvc + TILE, 32 * c, dt, r16, g)
                               : swz_tr_operand<V8, D>(kvc + TILE, 32 * c, dt, r16, g);

        // S^T = K . Q^T for the four 16-key sub-tiles (chunk c = t/2, half t%2).
        f32x4 s[QT][4];
        if constexpr (BM) {
            // Bias / scale first. S^T tile t holds keys 16t + 0..15 of the key tile here, so
            // rows 8g' + j of the B operand (g' = g % 2, duplicated for the lo half) are keys
            // 16t + 8g' + 0..7 of the lane's query row: one 16-byte piece, 2t + g', of the
            // swizzled bias rows (piece p of row r at p ^ (r & 7)).
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const int row = wave * 16 * QT + 16 * qt + r16;
                const char* brow_l = kvc + 2 * TILE + row * 128;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const u32x4 raw = *reinterpret_cast<const u32x4*>(
                        brow_l + 16 * ((2 * t + (g & 1)) ^ (row & 7)));
                    s[qt][t] = TR::mfma(idn, bits_as<V8>(raw), f32x4{0.f, 0.f, 0.f, 0.f});
                }
            }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int ks = 0; ks < G::KS; ++ks)
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
                    s[qt][t] = TR::mfma(kf[t][ks], qf[qt][ks],
                                        (BM || ks > 0) ? s[qt][t] : f32x4{0.f, 0.f, 0.f, 0.f});

        float x[QT][2][8];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                if constexpr (BM) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        x[qt][c][j] = s[qt][2 * c][j];
                        x[qt][c][4 + j] = s[qt][2 * c + 1][j];
                    }
                    continue;
                }
                float bv[8];
                if constexpr (VEC) {
                    const int row = wave * 16 * QT + 16 * qt + r16;
                    unpack8<TR>(*reinterpret_cast<const u32x4*>(
                                    kvc + 2 * TILE + row * 128 + 16 * ((4 * c + g) ^ (row & 7))),
                                bv);
                } else {
                    unpack8<TR>(cur.bias[qt][c], bv);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[qt][c][j] = fmaf(s[qt][2 * c][j], scale, bv[j]);
                    x[qt][c][4 + j] = fmaf(s[qt][2 * c + 1][j], scale, bv[4 + j]);
                }
            }
        if (!PATCH && need_mask) {
            // One block for the whole tile, opaque to speculation: nothing of it is hoisted
            // into (or merged across sub-tiles onto) the unmasked path.
            asm volatile("");
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                // Slot j is key k0 + 32c + 8g + j, or in the bias-MFMA order
                // k0 + 32c + 4g + j (j < 4) and k0 + 32c + 12 + 4g + j (j >= 4): it is past Sk
                // when j (j + 12 for the upper four of that order) >= lim.
                const int lim = Sk - (k0 + 32 * c + (BM ? 4 : 8) * g);
                const unsigned valid = cur.valid(c);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        x[qt][c][j] = (BM && j >= 4 ? j + 12 : j) >= lim
                                          ? -INFINITY
                                          : (((valid >> j) & 1u) ? x[qt][c][j] : masked_logit);
            }
        }

        float mt[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            mt[qt] = x[qt][0][0];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int j = 0; j < 8; ++j) mt[qt] = fmaxf(mt[qt], x[qt][c][j]);
        }
        if constexpr (QT == 2) {
            xgroup_max2(mt[0], mt[1]);
        } else {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) mt[qt] = xgroup_max(mt[qt]);
        }
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            // Lazy rescaling: the running max moves only when the tile's max exceeds it by more
            // than kRescaleSlack (in log2 units), so P stays below 2^kRescaleSlack and most tiles
            // skip the rescale of O and l (a wave-uniform branch).
            const bool move = fmaf(mt[qt], xs, nm[qt]) > kRescaleSlack;
            if (__any(move)) {
                // Opaque to if-conversion: without it the compiler runs the rescale on every
                // tile (alpha = 1 when nothing moved gives the same values).
                asm volatile("");
                const float nm_new = move ? -mt[qt] * xs : nm[qt];
                const float alpha = fast_exp2(nm_new - nm[qt]);
                nm[qt] = nm_new;
                lsum[qt][0] *= alpha;  // only component 0 is read
#pragma unroll
                for (int dt = 0; dt < G::DT; ++dt) acc[qt][dt] *= alpha;
            }
            const float neg = nm[qt];
            V8 pf[2];
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int j = 0; j < 8; ++j) pf[c][j] = TR::from_f(fast_exp2(fmaf(x[qt][c][j], xs, neg)));
#pragma unroll
            for (int c = 0; c < 2; ++c) lsum[qt] = TR::mfma(ones, pf[c], lsum[qt]);
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
                for (int c = 0; c < 2; ++c) acc[qt][dt] = TR::mfma(vf[dt][c], pf[c], acc[qt][dt]);
        }
    };
    // PATCH, a row without any present key: every logit in range is the masked logit 0, so
    // P = 1 there (and 0 past Sk) with the running max at 0 -- the values the tiles above
    // compute for such a row -- and a tile needs only its V rows: no S, no exponential.
    auto tile_empty = [&](int kt, const char* kvc, char* kvn, PF& cur, PF& nxt) {
        const int k0 = kt * BK;
        async_wait();
        __syncthreads();  // tile kt visible; every wave is done with the other buffer
        if (kt + 1 < nrun) {
            stage(k0 + BK, kvn);
            nxt.load(brow, mp, k0 + BK, g, Sk);
        } else if constexpr (GATE) {
            int t = threadIdx.x;
            asm volatile("" : "+v"(t));
            stage_rows_ld<D, kGateChannels, 256>(rw, 0, ga.HD, kvn, t);
        }
        V8 vf[G::DT][2];
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
            for (int c = 0; c < 2; ++c)
                vf[dt][c] = BM ? swz_tr_operand_split<V8, D>(kvc + TILE, 32 * c, dt, r16, g)
                               : swz_tr_operand<V8, D>(kvc + TILE, 32 * c, dt, r16, g);
        // Slot j of chunk c is key k0 + 32c + 8g + j, or in the bias-MFMA order
        // k0 + 32c + 4g + j (j < 4) and k0 + 32c + 12 + 4g + j (j >= 4).
        V8 pf[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int lim = Sk - (k0 + 32 * c + (BM ? 4 : 8) * g);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                pf[c][j] = TR::from_f((BM && j >= 4 ? j + 12 : j) < lim ? 1.f : 0.f);
        }
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
            for (int c = 0; c < 2; ++c) lsum[qt] = TR::mfma(ones, pf[c], lsum[qt]);
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt)
#pragma unroll
                for (int c = 0; c < 2; ++c) acc[qt][dt] = TR::mfma(vf[dt][c], pf[c], acc[qt][dt]);
        }
    };
    if (PATCH && row_empty) {  // block-uniform
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) nm[qt] = 0.f;
        for (int kt = 0; kt < nrun; kt += 2) {
            tile_empty(kt, kv0, kv1, ca, cb);
            if (kt + 1 < nrun) tile_empty(kt + 1, kv1, kv0, cb, ca);
        }
    } else {
        for (int kt = 0; kt < nrun; kt += 2) {
            tile(kt, kv0, kv1, ca, cb);
            if (kt + 1 < nrun) tile(kt + 1, kv1, kv0, cb, ca);
        }
    }

    // Gate pre-activations in O^T's accumulator layout (lane: rows 16*dt + 4*g + i of head h's
    // columns, query r16), so gate and O pair up element for element.
    f32x4 gacc[GATE ? QT : 1][G::DT];
    if constexpr (GATE) {
        // G^T = Wg_h^T . X^T + bg_h, 2*kGateChannels channels per round: A = head h's wg
        // columns for kGateChannels channels per K/V buffer (both buffers hold 128 rows of D),
        // staged like a V tile and read transposed; B = eight consecutive channels of the
        // lane's query row of x, straight from global memory into registers (zero for rows past
        // Sq and channels past C). The first buffer's rows were fetched during the last key
        // tile, and the x loads are issued before the barrier, so a round costs one wait.
        const int C = ga.C, HD = ga.HD;
        // Thread coordinates recomputed from an opaque copy of the thread index: shared with
        // the key loop, the epilogue's offsets would stay live (in registers) through it.
        int tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        const int gr16 = tid & 15, gg = (tid >> 4) & 3;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
            const int d = 16 * dt + 4 * gg;
            f32x4 b0 = {0.f, 0.f, 0.f, 0.f};
            if (d < D)
#pragma unroll
                for (int i = 0; i < 4; ++i) b0[i] = TR::to_f(ga.bg[h * D + d + i]);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) gacc[qt][dt] = b0;
        }
        constexpr int GC = kGateChannels, NX = 2 * GC / 32;
        static_assert(GC * T::ROWB <= 2 * TILE, "a K/V buffer holds kGateChannels wg rows");
        char* const kfree = (nrun & 1) ? kv1 : kv0;  // not read by the last key tile
        char* const klast = (nrun & 1) ? kv0 : kv1;
        for (int c0 = 0; c0 < C; c0 += 2 * GC) {
            V8 xo[QT][NX];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const int row = qbase + qt * 16 + gr16;
#pragma unroll
                for (int j = 0; j < NX; ++j) {
                    const int c = c0 + 32 * j;
                    u32x4 raw = {0u, 0u, 0u, 0u};
                    if (c < C && row < Sq)
                        raw = ld16(ga.x + ((size_t)n * Sq + row) * C + c + 8 * gg);
                    xo[qt][j] = bits_as<V8>(raw);
                }
            }
            __syncthreads();  // every wave is done with both buffers
            if (c0 > 0 || nrun == 0) stage_rows_ld<D, GC, 256>(rw, c0, HD, kfree, tid);
            if (c0 + GC < C) stage_rows_ld<D, GC, 256>(rw, c0 + GC, HD, klast, tid);
            async_wait();
            __syncthreads();  // this round's wg rows are visible
#pragma unroll
            for (int half = 0; half < 2; ++half)
#pragma unroll
                for (int cc = 0; cc < GC / 32; ++cc) {
                    if (c0 + GC * half + 32 * cc >= C) break;  // wave-uniform
#pragma unroll
                    for (int dt = 0; dt < G::DT; ++dt) {
                        const V8 a =
                            swz_tr_operand<V8, D>(half ? klast : kfree, 32 * cc, dt, gr16, gg);
#pragma unroll
                        for (int qt = 0; qt < QT; ++qt)
                            gacc[qt][dt] = TR::mfma(a, xo[qt][(GC / 32) * half + cc], gacc[qt][dt]);
                    }
                }
        }
    }

    // Normalise and store: lane holds O[row][16*dt + 4*g + i], i = 0..3. With the gate, O is
    // stored only when `out` is given, and the gated row goes to its [N, Sq, HD] place (its
    // lane coordinates again from an opaque thread index, as in the gate products).
    int etid = threadIdx.x;
    if constexpr (GATE) asm volatile("" : "+v"(etid));
    const int er16 = etid & 15, eg = (etid >> 4) & 3;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float l_tot = lsum[qt][0];
        const float inv = 1.0f / fmaxf(l_tot, 1e-30f);
        const int row = qbase + qt * 16 + er16;
        if (row >= Sq) continue;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
            const int d = 16 * dt + 4 * eg;
            if (d >= D) continue;
            const f32x4 o = acc[qt][dt] * inv;
            if (!GATE || out) store4<TR>(op + (size_t)row * ld + d, o);
            if constexpr (GATE) {
                f32x4 r;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    r[i] = o[i] * fast_rcp(1.f + fast_exp2(-kLog2e * gacc[qt][dt][i]));
                store4<TR>(ga.gated + ((size_t)n * Sq + row) * ga.HD + h * D + d, r);
            }
        }
        // A row whose present-key logits all lie below the running max's start (half the masked
        // logit) has no weight: O = 0 and lse = +inf, so the backward's P is 0 there.
        if (lse && eg == 0)
            lse[nh * Sq + row] =
                l_tot > 0.f ? -nm[qt] * kLn2 + logf(l_tot) : INFINITY;
    }
}

template <typename TR, int D, int QT, bool GATE, bool NSHD>
void launch_fwd_qt(hipStream_t st, const void* q, const void* k, const void* v, const void* bias,
                   const uint8_t* kmask, void* out, float* lse, int N, int H, int Sq, int Sk,
                   float scale, GateArgs<typename TR::elem> ga) {
    using E = typename TR::elem;
    const dim3 grid(ceil_div(Sq, 64 * QT) * H * N);
    // The head-outer work-item order when the bias of all heads passes half of an XCD's 4 MB L2,
    // in groups of rows whose query tiles make about 48 work items, half an XCD's resident
    // blocks (32 CUs x 3): at N_res = 1024 (8 MB of bias) this cut the launch's fetch from 8.2 to
    // 0.9 GB and its time by 9% (any group of 4 to 24 rows within 1%). Otherwise the head stays
    // inside the row: the MSA shapes' gate rows and [N, S, H, D] rows are shared by the heads.
    const bool head_outer = (size_t)H * Sq * Sk * 2 > (2u << 20);
    const int grp = head_outer ? max(1, min(N, 48 / ceil_div(Sq, 64 * QT))) : 0;
    // The bias tile through LDS: whole 8-key pieces, 8-byte aligned mask rows and at most
    // kPresWords key tiles (masked bias tiles are changed in LDS from presence words kept there).
    const bool vec = Sk % 8 == 0 && (reinterpret_cast<uintptr_t>(kmask) & 7u) == 0 &&
                     Sk <= kPresWords * 64;
    BiasMfma bm{};
    if (vec && bias_mfma_for<TR>(scale, &bm))
        attn_fwd_kernel<TR, D, QT, true, GATE, true, NSHD><<<grid, 256, 0, st>>>(
            (const E*)q, (const E*)k, (const E*)v, (const E*)bias, kmask, (E*)out, lse, H, Sq, Sk,
            scale, ga, bm, grp);
    else if (vec)
        attn_fwd_kernel<TR, D, QT, true, GATE, false, NSHD><<<grid, 256, 0, st>>>(
            (const E*)q, (const E*)k, (const E*)v, (const E*)bias, kmask, (E*)out, lse, H, Sq, Sk,
            scale, ga, bm, grp);
    else
        attn_fwd_kernel<TR, D, QT, false, GATE, false, NSHD><<<grid, 256, 0, st>>>(
            (const E*)q, (const E*)k, (const E*)v, (const E*)bias, kmask, (E*)out, lse, H, Sq, Sk,
            scale, ga, bm, grp);
}

template <typename TR, int D, bool GATE>
void launch_fwd(hipStream_t st, const void* q, const void* k, const void* v, const void* bias,
                const uint8_t* kmask, void* out, float* lse, int N, int H, int Sq, int Sk,
                float scale, GateArgs<typename TR::elem> ga, int nshd) {
    KernelTimer timer(GATE ? "attn_fwd_gated" : "attn_fwd", st);
    // The [N, S, H, D] layout only for the ungated forward.
    if constexpr (!GATE) {
        if (nshd) {
            if (Sq <= 64)
                launch_fwd_qt<TR, D, 1, GATE, true>(st, q, k, v, bias, kmask, out, lse, N, H, Sq,
                                                    Sk, scale, ga);
            else
                launch_fwd_qt<TR, D, 2, GATE, true>(st, q, k, v, bias, kmask, out, lse, N, H, Sq,
                                                    Sk, scale, ga);
            return;
        }
    }
    if (Sq <= 64)
        launch_fwd_qt<TR, D, 1, GATE, false>(st, q, k, v, bias, kmask, out, lse, N, H, Sq, Sk,
                                             scale, ga);
    else
        launch_fwd_qt<TR, D, 2, GATE, false>(st, q, k, v, bias, kmask, out, lse, N, H, Sq, Sk,
                                             scale, ga);
}

template <typename TR, bool GATE>
void dispatch_fwd(hipStream_t st, int64_t D, const void* q, const void* k, const void* v,
                  const void* bias, const uint8_t* kmask, void* out, float* lse, int N, int H,
                  int Sq, int Sk, float scale, GateArgs<typename TR::elem> ga, int nshd = 0) {
    switch (D) {
#define CLK_FWD_D(DV)                                                                           \
    case DV:                                                                                    \
        launch_fwd<TR, DV, GATE>(st, q, k, v, bias, kmask, out, lse, N, H, Sq, Sk, scale, ga,   \
                                 nshd);                                                         \
        break;
        CLK_FWD_D(8) CLK_FWD_D(16) CLK_FWD_D(32)
#undef CLK_FWD_D
        default:
            launch_fwd<TR, 64, GATE>(st, q, k, v, bias, kmask, out, lse, N, H, Sq, Sk, scale, ga,
                                     nshd);
            break;
    }
}

template <typename TR>
GateArgs<typename TR::elem> gate_args(const void* x, const void* wg, const void* bg, void* gated,
                                      int C, int HD) {
    using E = typename TR::elem;
    return {(const E*)x, (const E*)wg, (const E*)bg, (E*)gated, C, HD};
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
        dispatch_fwd<BF16, false>(stream, D, q, k, v, bias, kmask, out, lse, (int)N, (int)H,
                                  (int)Sq, (int)Sk, scale, {});
    else
        dispatch_fwd<F16, false>(stream, D, q, k, v, bias, kmask, out, lse, (int)N, (int)H,
                                 (int)Sq, (int)Sk, scale, {});
    return check_launch("attention");
}

extern "C" clk_status clk_attention_fwd_nshd(hipStream_t stream, clk_dtype dtype, const void* q,
                                             const void* k, const void* v, const void* bias,
                                             const uint8_t* kmask, void* out, float* lse,
                                             int64_t N, int64_t H, int64_t Sq, int64_t Sk,
                                             int64_t D, float scale) {
    const char* who = "attention_nshd";
    clk_status s = validate_attention(who, dtype, N, H, Sq, Sk, D);
    if (s != CLK_OK) return s;
    // Byte offsets within the rows of one (n, h) are 32-bit: S*H*D*2 below 2^31.
    if ((Sq > Sk ? Sq : Sk) * H * D * 2 >= ((int64_t)1 << 31))
        return fail(CLK_INVALID_ARGUMENT, "%s: S*H*D too large for the [N,S,H,D] layout", who);
    if (N * H * Sq == 0) return ok();
    if (!q || !k || !v || !bias || !out)
        return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(bias) || !aligned16(out))
        return fail(CLK_INVALID_ARGUMENT, "%s: q, k, v, bias, out must be 16-byte aligned", who);
    if (dtype == CLK_BF16)
        dispatch_fwd<BF16, false>(stream, D, q, k, v, bias, kmask, out, lse, (int)N, (int)H,
                                  (int)Sq, (int)Sk, scale, {}, 1);
    else
        dispatch_fwd<F16, false>(stream, D, q, k, v, bias, kmask, out, lse, (int)N, (int)H,
                                 (int)Sq, (int)Sk, scale, {}, 1);
    return check_launch(who);
}

extern "C" clk_status clk_attention_fwd_gated(hipStream_t stream, clk_dtype dtype, const void* q,
                                              const void* k, const void* v, const void* bias,
                                              const uint8_t* kmask, const void* x, const void* wg,
                                              const void* bg, void* gated, void* out, float* lse,
                                              int64_t N, int64_t H, int64_t Sq, int64_t Sk,
                                              int64_t D, int64_t C, float scale) {
    const char* who = "attention_gated";
    clk_status s = validate_attention(who, dtype, N, H, Sq, Sk, D);
    if (s != CLK_OK) return s;
    if (C <= 0 || C % 32)
        return fail(CLK_INVALID_ARGUMENT, "%s: C=%lld must be a positive multiple of 32", who,
                    (long long)C);
    const int64_t HD = H * D;
    // Buffer offsets into a row block of x and into wg are 32-bit.
    if (Sq * C * 2 >= ((int64_t)1 << 30) || C * HD * 2 >= ((int64_t)1 << 30))
        return fail(CLK_INVALID_ARGUMENT, "%s: Sq*C or C*H*D too large", who);
    if (N * H * Sq == 0) return ok();
    if (!q || !k || !v || !bias || !x || !wg || !bg || !gated)
        return fail(CLK_INVALID_ARGUMENT, "%s: null operand pointer", who);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(bias) || !aligned16(x) ||
        !aligned16(wg) || !aligned16(gated) || (out && !aligned16(out)))
        return fail(CLK_INVALID_ARGUMENT,
                    "%s: q, k, v, bias, x, wg, gated, out must be 16-byte aligned", who);
    if (dtype == CLK_BF16)
        dispatch_fwd<BF16, true>(stream, D, q, k, v, bias, kmask, out, lse, (int)N, (int)H,
                                 (int)Sq, (int)Sk, scale,
                                 gate_args<BF16>(x, wg, bg, gated, (int)C, (int)HD));
    else
        dispatch_fwd<F16, true>(stream, D, q, k, v, bias, kmask, out, lse, (int)N, (int)H,
                                (int)Sq, (int)Sk, scale,
                                gate_args<F16>(x, wg, bg, gated, (int)C, (int)HD));
    return check_launch(who);
}
