/*
 * clk.h -- C ABI of the gfx950 Evoformer kernels (attention with pair bias, LayerNorm,
 * gated dual projection).
 *
 * Every entry point takes raw device pointers, sizes and a HIP stream, launches its kernels on
 * that stream in order and returns without synchronising. Nothing is allocated, retained or
 * freed: the caller owns every buffer, including the workspace of the backward passes. A
 * non-OK status leaves a message in clk_last_error() (thread-local). Validation of every shape,
 * dtype and pointer runs on the host before any HIP call, so an invalid call never launches.
 *
 * Status and dtype codes use the XLA FFI numbering (XLA_FFI_Error_Code, XLA_FFI_DataType), so
 * the XLA FFI handlers pass them through unchanged.
 *
 * Layouts (all row-major, contiguous):
 *   attention  q, out [N,H,Sq,D]; k, v [N,H,Sk,D] (the *_nshd entries: [N,Sq,H,D],
 *              [N,Sk,H,D]); bias [H,Sq,Sk] shared by the N rows; kmask [N,Sk] uint8
 *              (0 = key absent); lse [N,H,Sq] float32 (natural log)
 *   layer norm x, y [M,C]; scale, offset [C] float32
 *   gdp        x [M,K]; wp, wg [K,N]; bp, bg [N]; mask [M]; out [M,N]
 */
#ifndef CLK_H_
#define CLK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

typedef enum clk_status {
    CLK_OK = 0,
    CLK_INVALID_ARGUMENT = 3,
    CLK_UNIMPLEMENTED = 12,
    CLK_INTERNAL = 13,
} clk_status;

typedef enum clk_dtype {
    CLK_U8 = 6,
    CLK_F16 = 10,
    CLK_F32 = 11,
    CLK_BF16 = 16,
} clk_dtype;

/* Message of the last non-OK status returned on this thread ("" if none). */
const char* clk_last_error(void);

/* Library version string. */
const char* clk_version(void);

/*
 * Per-launch timing (no reference counterpart; the reference has no run-time tracing). While
 * enabled on a thread, every kernel an entry point launches from that thread is bracketed by a
 * pair of HIP events on its stream. clk_profile_collect waits for the recorded events, writes up
 * to `max` (kernel name, milliseconds) pairs in launch order, releases the events and returns
 * the number of records (which may exceed `max`). Names are static strings. Off by default;
 * creating events allocates host-side resources, so keep it out of graph capture.
 */
void clk_profile_enable(int on);
int clk_profile_collect(const char** names, float* ms, int max);

/*
 * Attention forward: out = softmax(scale * q.k^T + bias, masked keys at logit -1e9) . v.
 * Replaces VoltaMma (cuda/volta_mma_attn.cu:304-351) and VoltaWmma (cuda/volta_wmma_attn.cu:
 * 264-311): same operands, same attributes (scale, block_q, block_k). dtype is CLK_F16 or
 * CLK_BF16 for q, k, v, bias and out. D is 8, 16, 32 or 64. block_q and block_k are hints: any
 * value the reference dispatch accepts is accepted, and other positive values too.
 * kmask may be NULL (every key present). lse may be NULL (inference); when given, the natural-log
 * logsumexp of every query row is written for clk_attention_bwd.
 */
clk_status clk_attention_fwd(hipStream_t stream, clk_dtype dtype, const void* q, const void* k,
                             const void* v, const void* bias, const uint8_t* kmask, void* out,
                             float* lse, int64_t N, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                             float scale, int64_t block_q, int64_t block_k);

/*
 * Attention forward on AlphaFold's own [N, S, H, D] layout: q [N, Sq, H, D], k and v
 * [N, Sk, H, D], out [N, Sq, H, D] (contiguous), so a caller need not transpose them to the
 * [N, H, S, D] layout of VoltaMma first (the jnp caller does, around
 * cuda/volta_mma_attn.cu:304-351; four passes over the operands). bias [H, Sq, Sk], kmask
 * [N, Sk], lse [N, H, Sq] (may be NULL), dtype, D and scale as in clk_attention_fwd, and the
 * same kernel, so O and lse are bit-identical to clk_attention_fwd on the transposed operands.
 * S*H*D*2 must stay below 2^31 bytes.
 */
clk_status clk_attention_fwd_nshd(hipStream_t stream, clk_dtype dtype, const void* q,
                                  const void* k, const void* v, const void* bias,
                                  const uint8_t* kmask, void* out, float* lse, int64_t N,
                                  int64_t H, int64_t Sq, int64_t Sk, int64_t D, float scale);

/*
 * Attention forward with the output gate fused into its epilogue: the reference's epilogue
 * normalises and stores O (cuda/volta_mma_attn.cu:256-272) and its caller's Attention module
 * then gates it; here
 *   gated[n, s, h*D + d] = O[n, h, s, d] * sigmoid(x[n, s, :] . wg[:, h*D + d] + bg[h*D + d])
 * is written directly in the [N, Sq, H*D] layout the output projection reads, and O itself
 * never reaches memory unless `out` is given. q, k, v, bias, kmask, lse, scale as in
 * clk_attention_fwd; x [N, Sq, C] (the attention's query-side input), wg [C, H*D] row-major,
 * bg [H*D], all of the attention's dtype; C a positive multiple of 32. out (the ungated O
 * [N,H,Sq,D], for a backward pass) and lse may be NULL. The gate GEMM runs on MFMA with float32
 * accumulation; O is not rounded to the dtype before it is gated.
 */
clk_status clk_attention_fwd_gated(hipStream_t stream, clk_dtype dtype, const void* q,
                                   const void* k, const void* v, const void* bias,
                                   const uint8_t* kmask, const void* x, const void* wg,
                                   const void* bg, void* gated, void* out, float* lse, int64_t N,
                                   int64_t H, int64_t Sq, int64_t Sk, int64_t D, int64_t C,
                                   float scale);

/* Bytes of device workspace clk_attention_bwd needs for these sizes. */
size_t clk_attention_bwd_workspace_size(int64_t N, int64_t H, int64_t Sq, int64_t Sk, int64_t D);

/*
 * Attention backward. No reference counterpart (the reference is forward-only); it is the
 * gradient of clk_attention_fwd's math with the additive-mask convention: dS = P*(dP - D) at
 * every key, masked ones included. Inputs q, k, v, bias, kmask as in the forward, plus out and
 * lse from it and dout. Outputs dq, dk, dv (dtype) and dbias [H,Sq,Sk] float32 = sum over the N
 * rows of dS. Deterministic: fixed-order reductions, no floating-point atomics, so repeated
 * calls give identical bits. workspace must hold clk_attention_bwd_workspace_size() bytes,
 * 256-byte aligned.
 */
clk_status clk_attention_bwd(hipStream_t stream, clk_dtype dtype, const void* q, const void* k,
                             const void* v, const void* bias, const uint8_t* kmask,
                             const void* out, const void* dout, const float* lse, void* dq,
                             void* dk, void* dv, float* dbias, void* workspace,
                             size_t workspace_bytes, int64_t N, int64_t H, int64_t Sq, int64_t Sk,
                             int64_t D, float scale);

/*
 * Attention backward on AlphaFold's [N, S, H, D] layout: q, out, dout, dq [N, Sq, H, D] and k, v,
 * dk, dv [N, Sk, H, D]; bias, kmask, lse [N, H, Sq], dbias, workspace (the same
 * clk_attention_bwd_workspace_size) and scale as in clk_attention_bwd, whose kernels it runs with
 * rows H*D apart: the results are bit-identical to clk_attention_bwd on the transposed operands.
 * S*H*D*2 must stay below 2^31 bytes. No reference counterpart (as clk_attention_bwd).
 */
clk_status clk_attention_bwd_nshd(hipStream_t stream, clk_dtype dtype, const void* q,
                                  const void* k, const void* v, const void* bias,
                                  const uint8_t* kmask, const void* out, const void* dout,
                                  const float* lse, void* dq, void* dk, void* dv, float* dbias,
                                  void* workspace, size_t workspace_bytes, int64_t N, int64_t H,
                                  int64_t Sq, int64_t Sk, int64_t D, float scale);

/*
 * Attention backward that allocates nothing. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same operands and results as clk_attention_bwd, without the
 * workspace: it uses the library's fixed per-GPU scratch array of
 * clk_attention_bwd_noalloc_limit() bytes (64 MiB). The array sits in a code object of its own,
 * which the HIP runtime loads on a GPU at this entry's first call there: from then until the
 * process ends that GPU holds the 64 MiB (the other entry points never load it; measured on
 * MI355X, free device memory drops by the 64 MiB at the first call of this entry and not at
 * the other kernels' launches). Sizes whose clk_attention_bwd_workspace_size() exceeds the limit are rejected
 * with CLK_INVALID_ARGUMENT before any device work. Calls that overlap on one GPU (several
 * streams or threads) share that array and race: serialise them.
 */
size_t clk_attention_bwd_noalloc_limit(void);
clk_status clk_attention_bwd_noalloc(hipStream_t stream, clk_dtype dtype, const void* q,
                                     const void* k, const void* v, const void* bias,
                                     const uint8_t* kmask, const void* out, const void* dout,
                                     const float* lse, void* dq, void* dk, void* dv,
                                     float* dbias, int64_t N, int64_t H, int64_t Sq, int64_t Sk,
                                     int64_t D, float scale);

/*
 * Streaming device-to-device copy of `bytes` bytes (16-byte aligned, a multiple of 16) with the
 * access pattern of this library's HBM-bound kernels. No reference counterpart: it is the
 * measured HBM ceiling the benchmark reports the LayerNorm and projection rates against.
 */
clk_status clk_stream_copy(hipStream_t stream, const void* src, void* dst, size_t bytes);

/*
 * Instruction-issue calibration: `blocks` x `threads` threads (threads a multiple of 64, at most
 * 1024) each run `iters` rounds of one instruction mix and write one float to `sink` (blocks *
 * threads floats). A round is two copies of: kind 0, 32 float32 FMAs; 1, 32 float32
 * exponentials (v_exp_f32); 2, four 16x16x32 bf16 MFMAs; 3, kinds 0 and 1; 4, kinds 0 and 2;
 * 5, kinds 1 and 2; 6, kinds 0, 1 and 2 -- every instruction independent of the others in its
 * round. Timing the kinds gives each instruction's cost on a SIMD and how far MFMAs hide under
 * the other kinds. No reference counterpart: it measures the per-instruction costs of the
 * benchmark's instruction-issue floor.
 */
clk_status clk_issue_calibration(hipStream_t stream, int kind, int blocks, int threads,
                                 int iters, float* sink);

/*
 * LayerNorm forward over the last axis. Replaces VoltaLayerNorm (cuda/volta_ops.cu:62-95):
 * x and y of dtype CLK_F16, CLK_BF16 or CLK_F32; scale and offset float32; attribute eps.
 */
clk_status clk_layer_norm_fwd(hipStream_t stream, clk_dtype dtype, const void* x,
                              const float* scale, const float* offset, void* y, int64_t M,
                              int64_t C, float eps);

/* Bytes of device workspace clk_layer_norm_bwd needs for these sizes. */
size_t clk_layer_norm_bwd_workspace_size(int64_t M, int64_t C);

/*
 * LayerNorm backward. No reference counterpart. Statistics are recomputed from x. Outputs
 * dx (dtype) and dscale, doffset [C] float32 (deterministic two-stage column sums).
 */
clk_status clk_layer_norm_bwd(hipStream_t stream, clk_dtype dtype, const void* x,
                              const float* scale, const void* dy, void* dx, float* dscale,
                              float* doffset, void* workspace, size_t workspace_bytes, int64_t M,
                              int64_t C, float eps);

/*
 * Gated dual projection: out = mask[m] * (x.wp + bp) * sigmoid(x.wg + bg).
 * Replaces VoltaGdp (cuda/volta_ops.cu:210-265) and VoltaGdpWmma (cuda/volta_gdp_wmma.cu:
 * 99-140): the same six operands and result, all of dtype CLK_F16 or CLK_BF16. N must be a
 * multiple of 8 (volta_ops.cu:234-236); any K (the weights are staged 512 rows at a time).
 */
clk_status clk_gated_dual_proj(hipStream_t stream, clk_dtype dtype, const void* x,
                               const void* wp, const void* bp, const void* wg, const void* bg,
                               const void* mask, void* out, int64_t M, int64_t K, int64_t N);

/*
 * Backward of the gated dual projection (new; the reference is forward-only): for out = mask *
 * (x.wp + bp) * sigmoid(x.wg + bg) and the incoming gradient dout [M,N], writes dx [M,K] (added
 * to the existing dx when accumulate_dx != 0, for two branches reading the same x), dwp, dwg
 * [K,N] and dbp, dbg [N] in float32. x, weights, biases, mask, dout, dx of dtype CLK_F16 or
 * CLK_BF16. K and N in {64, 128}; M at most 2^31 - 64. Deterministic: the weight and bias
 * gradients are summed from per-block partials in a fixed order. Workspace:
 * clk_gated_dual_proj_bwd_workspace_size bytes. M = 0 writes zero weight and bias gradients
 * (sums over no rows).
 */
size_t clk_gated_dual_proj_bwd_workspace_size(int64_t M, int64_t K, int64_t N);
clk_status clk_gated_dual_proj_bwd(hipStream_t stream, clk_dtype dtype, const void* x,
                                   const void* wp, const void* bp, const void* wg, const void* bg,
                                   const void* mask, const void* dout, void* dx, float* dwp,
                                   float* dbp, float* dwg, float* dbg, void* workspace,
                                   size_t workspace_bytes, int64_t M, int64_t K, int64_t N,
                                   int accumulate_dx);

/*
 * LayerNorm fused with both gated-projection branches of the triangle multiplication:
 *   y = LN(z); a = mask*(y.wpa+bpa)*sigmoid(y.wga+bga); b = likewise with the b weights.
 * One pass over z instead of VoltaLayerNorm followed by two VoltaGdp calls. z, weights, biases,
 * mask, a and b of dtype CLK_F16 or CLK_BF16; ln_scale, ln_offset float32. C and N must be
 * multiples of 32, at most 128 each.
 */
clk_status clk_ln_gated_dual_proj(hipStream_t stream, clk_dtype dtype, const void* z,
                                  const float* ln_scale, const float* ln_offset, const void* wpa,
                                  const void* bpa, const void* wga, const void* bga,
                                  const void* wpb, const void* bpb, const void* wgb,
                                  const void* bgb, const void* mask, void* a, void* b, int64_t M,
                                  int64_t C, int64_t N, float eps);

/*
 * Pair-bias projection (new; the step before the attention kernels in AlphaFold's triangle and
 * MSA-row attention): bias[h, m] = sum_c LN(z)[m, c] * w[c, h] for z [M, C] (M = Sq*Sk pair
 * positions), LN with scale/offset float32 [C] and eps, w [C, H] row-major, bias [H, M] --
 * the [H, Sq, Sk] attention bias -- in one pass over z. z, w and bias of dtype CLK_F16 or
 * CLK_BF16; C = 64, 128 or 256; H = 1, 2, 4 or 8.
 */
clk_status clk_ln_pair_bias(hipStream_t stream, clk_dtype dtype, const void* z, const float* scale,
                            const float* offset, const void* w, void* bias, int64_t M, int64_t C,
                            int64_t H, float eps);

/*
 * Gated attention output (new; the reference leaves the gate to the caller's jnp code):
 *   out[n, s, h*D + d] = o[n, h, s, d] * sigmoid(x[n, s, :] . wg[:, h*D + d] + bg[h*D + d])
 * with o [N,H,Sq,D] the attention output, x [N,Sq,C] the attention's query-side input, wg
 * [C, H*D] row-major, bg [H*D], out [N,Sq,H*D] (the layout the output projection reads). All of
 * dtype CLK_F16 or CLK_BF16. C and H*D must each be 64, 128 or 256; D a multiple of 8.
 */
clk_status clk_attention_gate(hipStream_t stream, clk_dtype dtype, const void* o, const void* x,
                              const void* wg, const void* bg, void* out, int64_t N, int64_t H,
                              int64_t Sq, int64_t D, int64_t C);

/*
 * Backward of the gated attention output (new; the reference has neither the gate nor any
 * backward): for out = clk_attention_gate(o, x, wg, bg) and the incoming gradient dout
 * [N,Sq,H*D], with s = sigmoid(x.wg + bg) recomputed,
 *   d_o = dout * s           in o's layout [N,H,Sq,D] (the dout of clk_attention_bwd),
 *   dg  = dout * o * s * (1 - s),  dx = dg.wg^T [N,Sq,C] (added to the existing dx when
 *   accumulate_dx != 0: x also feeds the q, k, v projections),
 *   dwg = x^T.dg [C,H*D] and dbg = sum of dg over the N*Sq rows [H*D], both float32.
 * o, x, wg, bg, dout, d_o, dx of dtype CLK_F16 or CLK_BF16 (o, x, wg, dout, d_o, dx and the
 * workspace 16-byte aligned); C and H*D each 64, 128 or 256; D a multiple of 8; N*Sq at most
 * 2^31 - 64 rows and Sq*H*D*4 under 2^30 bytes. Deterministic: dwg and dbg are summed from
 * per-block partials in a fixed order.
 * Workspace: clk_attention_gate_bwd_workspace_size bytes (dg in the input dtype and the
 * partials). N*Sq = 0 writes zero dwg and dbg.
 */
size_t clk_attention_gate_bwd_workspace_size(int64_t N, int64_t H, int64_t Sq, int64_t D,
                                             int64_t C);
clk_status clk_attention_gate_bwd(hipStream_t stream, clk_dtype dtype, const void* o,
                                  const void* x, const void* wg, const void* bg, const void* dout,
                                  void* d_o, void* dx, float* dwg, float* dbg, void* workspace,
                                  size_t workspace_bytes, int64_t N, int64_t H, int64_t Sq,
                                  int64_t D, int64_t C, int accumulate_dx);

/*
 * Triangle-multiplication contraction, per channel (new; the reference stops at the gated
 * projection): x[c] = a[c] . b[c]^T for a, b, x [C][N][N] row-major, i.e. channel-major with the
 * contraction index last. With a[c][i][k] = a_pair[i,k,c] this is the outgoing update
 * x[i,j,c] = sum_k a[i,k,c] b[j,k,c]; with a[c][i][k] = a_pair[k,i,c] the incoming one. dtype
 * CLK_F16 or CLK_BF16, float32 accumulation. N must be a multiple of 8.
 */
clk_status clk_triangle_einsum(hipStream_t stream, clk_dtype dtype, const void* a, const void* b,
                               void* x, int64_t C, int64_t N);

/*
 * Triangle multiplication (new; AlphaFold's TriangleMultiplication after the reference's gated
 * projection): for the pair representation z [N,N,C] and mask [N,N],
 *   y = LN_in(z); left = mask*(y.w[0]+b[0])*sigmoid(y.w[2]+b[2]);
 *   right = mask*(y.w[1]+b[1])*sigmoid(y.w[3]+b[3]);
 *   x = outgoing ? einsum('ikc,jkc->ijc', left, right) : einsum('kjc,kic->ijc', left, right);
 *   out = (LN_c(x).w[4] + b[4]) * sigmoid(y.w[5] + b[5])
 * w[0..5] = left projection, right projection, left gate, right gate, output projection, output
 * gate, each [C,C] row-major (input channel first); b[0..5] their [C] biases; ln[0..3] = LN_in
 * scale, offset, LN_c scale, offset (float32 [C]). z, mask, weights, biases and out of dtype
 * CLK_F16 or CLK_BF16. C = 64 or 128; N up to 16384 (a ragged N runs on a zero-padded grid
 * of N rounded up to 8, the padded positions masked). The workspace holds left, right and x
 * channel-major, and for a ragged N the padded z, mask and output
 * (clk_triangle_multiply_workspace_size bytes).
 */
size_t clk_triangle_multiply_workspace_size(int64_t N, int64_t C);
clk_status clk_triangle_multiply(hipStream_t stream, clk_dtype dtype, const void* z,
                                 const void* mask, const float* const* ln, const void* const* w,
                                 const void* const* b, void* out, void* workspace,
                                 size_t workspace_bytes, int64_t N, int64_t C, int outgoing,
                                 float eps);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CLK_H_ */
