// XLA FFI custom-call targets for the gfx950 kernels, exported as C symbols so JAX can register
// them with jax.ffi.register_ffi_target(name, jax.ffi.pycapsule(getattr(lib, name)),
// platform="ROCM"). Each handler decodes the call frame (operands, results, attributes, the
// platform stream), checks every rank, dtype and shape on the host, and forwards to the C ABI in
// clk.h; the status code becomes the XLA error code. No handler allocates, retains or
// synchronises anything, so all of them declare the command-buffer-compatible trait.
//
// Target names and operand order follow the reference handlers:
//   VoltaMma, VoltaWmma   (cuda/volta_mma_attn.cu:338-351, cuda/volta_wmma_attn.cu:298-311)
//       q, k, v, bias, kmask -> out; attributes scale (f32), block_q, block_k (i64)
//   VoltaLayerNorm        (cuda/volta_ops.cu:87-95)      x, scale, offset -> y; attribute eps
//   VoltaGdp, VoltaGdpWmma (cuda/volta_ops.cu:254-265, cuda/volta_gdp_wmma.cu:130-140)
//       x, wp, bp, wg, bg, mask -> out
// and accept bf16 as well as f16. Targets without a reference counterpart:
//   ClkAttentionFwd   q, k, v, bias, kmask -> out, lse (f32 [N,H,Sq]); attribute scale
//   ClkAttentionNshd  q [N,Sq,H,D], k, v [N,Sk,H,D], bias, kmask -> out [N,Sq,H,D] (AlphaFold's
//                     layout, no transposes) and optionally lse (f32 [N,H,Sq]); attribute scale
//   ClkAttentionBwdNshd  ClkAttentionBwd with q, k, v, out, dout, dq, dk, dv in [N,S,H,D]
//   ClkAttentionGated q, k, v, bias, kmask, x [N,Sq,C], wg [C,H*D], bg [H*D] -> gated
//                     [N,Sq,H*D] (attention with the output gate fused in); attribute scale
//   ClkAttentionBwd   q, k, v, bias, kmask, out, dout, lse -> dq, dk, dv, dbias (f32 [H,Sq,Sk]),
//                     workspace (u8, clk_attention_bwd_workspace_size bytes); attribute scale
//   ClkLayerNormBwd   x, scale, dy -> dx, dscale, doffset, workspace (u8); attribute eps
//   ClkLnGdp          z, ln_scale, ln_offset, wpa, bpa, wga, bga, wpb, bpb, wgb, bgb, mask
//                     -> a, b; attribute eps
//   ClkAttentionGate  o [N,H,Sq,D], x [N,Sq,C], wg [C,H*D], bg [H*D] -> out [N,Sq,H*D]
//   ClkAttentionGateBwd  o, x, wg, bg, dout [N,Sq,H*D] -> do [N,H,Sq,D], dx [N,Sq,C], dwg (f32
//                     [C,H*D]), dbg (f32 [H*D]), workspace (u8,
//                     clk_attention_gate_bwd_workspace_size bytes)
//   ClkLnPairBias     z [..., C], scale, offset (f32 [C]), w [C,H] -> bias [H, ...]; attribute eps
//   ClkGdpBwd         x, wp, bp, wg, bg, mask, dout -> dx, dwp, dbp, dwg, dbg (f32), workspace (u8,
//                     clk_gated_dual_proj_bwd_workspace_size bytes)
//   ClkTriangleMultiply  z [N,N,C], mask [N,N], ln_in scale, offset, ln_c scale, offset (f32 [C]),
//                     six weights [C,C], six biases [C] -> out [N,N,C], workspace (u8,
//                     clk_triangle_multiply_workspace_size bytes); attributes eps (f32), outgoing
//                     (i64, 1 = 'ikc,jkc->ijc', 0 = 'kjc,kic->ijc')
#include <hip/hip_runtime.h>

#include <cstring>

#include "clk.h"
#include "xla_ffi_abi.h"

namespace clk {
clk_status fail(clk_status code, const char* fmt, ...);
}

namespace {

using namespace clk::xffi;

class Frame {
   public:
    explicit Frame(CallFrame* f) : f_(f) {}

    Error* error(clk_status code, const char* msg) const {
        ErrorCreateArgs a;
        a.struct_size = sizeof(ErrorCreateArgs);
        a.extension_start = nullptr;
        a.message = msg;
        a.errc = static_cast<ErrorCode>(code);
        return f_->api->error_create(&a);
    }

    int64_t nargs() const { return f_->args.size; }
    int64_t nrets() const { return f_->rets.size; }

    const Buffer* arg(int64_t i) const {
        if (i >= f_->args.size || f_->args.types[i] != kArgBuffer) return nullptr;
        return static_cast<const Buffer*>(f_->args.args[i]);
    }
    const Buffer* ret(int64_t i) const {
        if (i >= f_->rets.size || f_->rets.types[i] != kRetBuffer) return nullptr;
        return static_cast<const Buffer*>(f_->rets.rets[i]);
    }

    const Scalar* scalar(const char* name) const {
        const size_t len = std::strlen(name);
        for (int64_t i = 0; i < f_->attrs.size; ++i) {
            const ByteSpan* n = f_->attrs.names[i];
            if (n->len == len && std::memcmp(n->ptr, name, len) == 0 &&
                f_->attrs.types[i] == kAttrScalar)
                return static_cast<const Scalar*>(f_->attrs.attrs[i]);
        }
        return nullptr;
    }
    bool attr_f32(const char* name, float* out) const {
        const Scalar* s = scalar(name);
        if (!s) return false;
        if (s->dtype == kF32) *out = *static_cast<const float*>(s->value);
        else if (s->dtype == kF64) *out = (float)*static_cast<const double*>(s->value);
        else return false;
        return true;
    }
    bool attr_i64(const char* name, int64_t* out) const {
        const Scalar* s = scalar(name);
        if (!s) return false;
        if (s->dtype == kS64) *out = *static_cast<const int64_t*>(s->value);
        else if (s->dtype == kS32) *out = *static_cast<const int32_t*>(s->value);
        else return false;
        return true;
    }

    // Asks XLA for the platform stream of this call. On failure returns XLA's own error, which
    // the handler passes back unchanged: launching on the default stream instead would leave the
    // kernels unordered with XLA's work.
    Error* fetch_stream() {
        StreamGetArgs a;
        a.struct_size = sizeof(StreamGetArgs);
        a.extension_start = nullptr;
        a.ctx = f_->ctx;
        a.stream = nullptr;
        if (Error* e = f_->api->stream_get(&a)) return e;
        stream_ = static_cast<hipStream_t>(a.stream);
        return nullptr;
    }
    hipStream_t stream() const { return stream_; }

   private:
    CallFrame* f_;
    hipStream_t stream_ = nullptr;
};

// The metadata query XLA makes when it registers a handler: report the API version and traits.
bool answer_metadata(CallFrame* frame) {
    ExtensionBase* ext = frame->extension_start;
    while (ext && ext->type != kExtensionMetadata) ext = ext->next;
    if (!ext) return false;
    Metadata* md = reinterpret_cast<MetadataExtension*>(ext)->metadata;
    md->api_version.struct_size = sizeof(ApiVersion);
    md->api_version.extension_start = nullptr;
    md->api_version.major_version = kApiMajor;
    md->api_version.minor_version = kApiMinor;
    md->traits = kCommandBufferCompatible;
    return true;
}

template <typename Body>
Error* run(CallFrame* frame, Body body) {
    if (!frame) return nullptr;
    if (answer_metadata(frame)) return nullptr;
    if (frame->stage != kExecute) return nullptr;
    Frame f(frame);
    if (Error* e = f.fetch_stream()) return e;
    const clk_status s = body(f);
    if (s == CLK_OK) return nullptr;
    return f.error(s, clk_last_error());
}

// ---- shape helpers ---------------------------------------------------------------------------

int64_t numel(const Buffer* b) {
    int64_t n = 1;
    for (int64_t i = 0; i < b->rank; ++i) n *= b->dims[i];
    return n;
}

bool dims_are(const Buffer* b, std::initializer_list<int64_t> d) {
    if (!b || b->rank != (int64_t)d.size()) return false;
    int64_t i = 0;
    for (int64_t v : d)
        if (b->dims[i++] != v) return false;
    return true;
}

bool half_type(DataType t) { return t == kF16 || t == kBF16; }

clk_status bad(const char* who, const char* what) {
    return clk::fail(CLK_INVALID_ARGUMENT, "%s: %s", who, what);
}

struct AttnDims {
    int64_t N, H, Sq, Sk, D;
};

// q [N,H,Sq,D], k, v [N,H,Sk,D], bias [H,Sq,Sk], kmask u8 [N,Sk], all half types alike.
// Whether b is an attention operand of S rows: [N, H, S, D], or [N, S, H, D] with nshd.
bool rows_are(const Buffer* b, const AttnDims& d, int64_t S, bool nshd) {
    return nshd ? dims_are(b, {d.N, S, d.H, d.D}) : dims_are(b, {d.N, d.H, S, d.D});
}

clk_status decode_attention(const char* who, const Frame& f, AttnDims* d, bool nshd = false) {
    const Buffer *q = f.arg(0), *k = f.arg(1), *v = f.arg(2), *bias = f.arg(3), *km = f.arg(4);
    if (!q || !k || !v || !bias || !km) return bad(who, "expects buffers q, k, v, bias, kmask");
    if (q->rank != 4) return bad(who, nshd ? "q must be [N,S,H,D]" : "q must be [N,H,S,D]");
    d->N = q->dims[0];
    d->H = q->dims[nshd ? 2 : 1];
    d->Sq = q->dims[nshd ? 1 : 2];
    d->D = q->dims[3];
    if (k->rank != 4) return bad(who, nshd ? "k must be [N,S,H,D]" : "k must be [N,H,S,D]");
    d->Sk = k->dims[nshd ? 1 : 2];
    if (!rows_are(k, *d, d->Sk, nshd) || !rows_are(v, *d, d->Sk, nshd))
        return bad(who, nshd ? "k and v must be [N,Sk,H,D] matching q"
                             : "k and v must be [N,H,Sk,D] matching q");
    if (!dims_are(bias, {d->H, d->Sq, d->Sk})) return bad(who, "bias must be [H,Sq,Sk]");
    if (!dims_are(km, {d->N, d->Sk}) || km->dtype != kU8) return bad(who, "kmask must be u8 [N,Sk]");
    if (!half_type(q->dtype) || k->dtype != q->dtype || v->dtype != q->dtype ||
        bias->dtype != q->dtype)
        return bad(who, "q, k, v and bias must all be f16 or all bf16");
    return CLK_OK;
}

clk_status attention_fwd(const char* who, const Frame& f, bool with_lse) {
    AttnDims d;
    clk_status s = decode_attention(who, f, &d);
    if (s != CLK_OK) return s;
    const Buffer* out = f.ret(0);
    if (!dims_are(out, {d.N, d.H, d.Sq, d.D}) || out->dtype != f.arg(0)->dtype)
        return bad(who, "result must be [N,H,Sq,D] of the input dtype");
    float* lse = nullptr;
    float scale = 0.f;
    int64_t bq = 64, bk = 64;
    if (!f.attr_f32("scale", &scale)) return bad(who, "missing f32 attribute 'scale'");
    if (with_lse) {
        const Buffer* l = f.ret(1);
        if (!dims_are(l, {d.N, d.H, d.Sq}) || l->dtype != kF32)
            return bad(who, "second result must be f32 [N,H,Sq]");
        lse = static_cast<float*>(l->data);
    } else {
        if (!f.attr_i64("block_q", &bq) || !f.attr_i64("block_k", &bk))
            return bad(who, "missing i64 attributes 'block_q', 'block_k'");
    }
    return clk_attention_fwd(f.stream(), static_cast<clk_dtype>(f.arg(0)->dtype), f.arg(0)->data,
                             f.arg(1)->data, f.arg(2)->data, f.arg(3)->data,
                             static_cast<const uint8_t*>(f.arg(4)->data), out->data, lse, d.N,
                             d.H, d.Sq, d.Sk, d.D, scale, bq, bk);
}

clk_status attention_nshd(const Frame& f) {
    const char* who = "ClkAttentionNshd";
    if (f.nargs() != 5 || (f.nrets() != 1 && f.nrets() != 2))
        return bad(who, "expects 5 operands (q, k, v, bias, kmask) and 1 or 2 results");
    AttnDims d;
    clk_status s = decode_attention(who, f, &d, true);
    if (s != CLK_OK) return s;
    const Buffer* out = f.ret(0);
    if (!rows_are(out, d, d.Sq, true) || out->dtype != f.arg(0)->dtype)
        return bad(who, "result must be [N,Sq,H,D] of the input dtype");
    float* lse = nullptr;
    if (f.nrets() == 2) {  // the logsumexp for a backward pass
        const Buffer* l = f.ret(1);
        if (!dims_are(l, {d.N, d.H, d.Sq}) || l->dtype != kF32)
            return bad(who, "second result must be f32 [N,H,Sq]");
        lse = static_cast<float*>(l->data);
    }
    float scale = 0.f;
    if (!f.attr_f32("scale", &scale)) return bad(who, "missing f32 attribute 'scale'");
    return clk_attention_fwd_nshd(f.stream(), static_cast<clk_dtype>(f.arg(0)->dtype),
                                  f.arg(0)->data, f.arg(1)->data, f.arg(2)->data, f.arg(3)->data,
                                  static_cast<const uint8_t*>(f.arg(4)->data), out->data, lse,
                                  d.N, d.H, d.Sq, d.Sk, d.D, scale);
}

clk_status attention_gated(const Frame& f) {
    const char* who = "ClkAttentionGated";
    if (f.nargs() != 8 || f.nrets() != 1)
        return bad(who, "expects 8 operands (q, k, v, bias, kmask, x, wg, bg) and 1 result");
    AttnDims d;
    clk_status s = decode_attention(who, f, &d);
    if (s != CLK_OK) return s;
    const Buffer *x = f.arg(5), *wg = f.arg(6), *bg = f.arg(7), *gated = f.ret(0);
    if (!x || !wg || !bg || !gated) return bad(who, "operands must be buffers");
    if (x->rank != 3 || x->dims[0] != d.N || x->dims[1] != d.Sq)
        return bad(who, "x must be [N,Sq,C]");
    const int64_t C = x->dims[2], HD = d.H * d.D;
    if (!dims_are(wg, {C, HD}) || !dims_are(bg, {HD}) || !dims_are(gated, {d.N, d.Sq, HD}))
        return bad(who, "wg [C,H*D], bg [H*D], result [N,Sq,H*D] expected");
    const DataType t = f.arg(0)->dtype;
    if (x->dtype != t || wg->dtype != t || bg->dtype != t || gated->dtype != t)
        return bad(who, "x, wg, bg and the result must have the dtype of q");
    float scale = 0.f;
    if (!f.attr_f32("scale", &scale)) return bad(who, "missing f32 attribute 'scale'");
    return clk_attention_fwd_gated(f.stream(), static_cast<clk_dtype>(t), f.arg(0)->data,
                                   f.arg(1)->data, f.arg(2)->data, f.arg(3)->data,
                                   static_cast<const uint8_t*>(f.arg(4)->data), x->data,
                                   wg->data, bg->data, gated->data, nullptr, nullptr, d.N, d.H,
                                   d.Sq, d.Sk, d.D, C, scale);
}

clk_status attention_bwd(const Frame& f, bool nshd) {
    const char* who = nshd ? "ClkAttentionBwdNshd" : "ClkAttentionBwd";
    AttnDims d;
    clk_status s = decode_attention(who, f, &d, nshd);
    if (s != CLK_OK) return s;
    const DataType t = f.arg(0)->dtype;
    const Buffer *out = f.arg(5), *dout = f.arg(6), *lse = f.arg(7);
    if (!rows_are(out, d, d.Sq, nshd) || out->dtype != t || !rows_are(dout, d, d.Sq, nshd) ||
        dout->dtype != t)
        return bad(who, nshd ? "out and dout must be [N,Sq,H,D] of the input dtype"
                             : "out and dout must be [N,H,Sq,D] of the input dtype");
    if (!dims_are(lse, {d.N, d.H, d.Sq}) || lse->dtype != kF32)
        return bad(who, "lse must be f32 [N,H,Sq]");
    const Buffer *dq = f.ret(0), *dk = f.ret(1), *dv = f.ret(2), *db = f.ret(3), *ws = f.ret(4);
    if (!rows_are(dq, d, d.Sq, nshd) || dq->dtype != t || !rows_are(dk, d, d.Sk, nshd) ||
        dk->dtype != t || !rows_are(dv, d, d.Sk, nshd) || dv->dtype != t)
        return bad(who, "dq, dk, dv must match q, k, v");
    if (!dims_are(db, {d.H, d.Sq, d.Sk}) || db->dtype != kF32)
        return bad(who, "dbias must be f32 [H,Sq,Sk]");
    if (!ws || ws->dtype != kU8) return bad(who, "fifth result must be the u8 workspace");
    float scale;
    if (!f.attr_f32("scale", &scale)) return bad(who, "missing f32 attribute 'scale'");
    return (nshd ? clk_attention_bwd_nshd : clk_attention_bwd)(
        f.stream(), static_cast<clk_dtype>(t), f.arg(0)->data, f.arg(1)->data, f.arg(2)->data,
        f.arg(3)->data, static_cast<const uint8_t*>(f.arg(4)->data), out->data, dout->data,
        static_cast<const float*>(lse->data), dq->data, dk->data, dv->data,
        static_cast<float*>(db->data), ws->data, (size_t)numel(ws), d.N, d.H, d.Sq, d.Sk, d.D,
        scale);
}

clk_status layer_norm_fwd(const Frame& f) {
    const char* who = "VoltaLayerNorm";
    const Buffer *x = f.arg(0), *sc = f.arg(1), *of = f.arg(2), *y = f.ret(0);
    if (!x || !sc || !of || !y) return bad(who, "expects x, scale, offset -> y");
    if (x->rank < 1) return bad(who, "x must be [M,C]");
    const int64_t C = x->dims[x->rank - 1], M = C ? numel(x) / C : 0;
    if (!dims_are(sc, {C}) || !dims_are(of, {C}) || sc->dtype != kF32 || of->dtype != kF32)
        return bad(who, "scale and offset must be f32 [C]");
    if (numel(y) != numel(x) || y->dtype != x->dtype) return bad(who, "y must match x");
    float eps;
    if (!f.attr_f32("eps", &eps)) return bad(who, "missing f32 attribute 'eps'");
    return clk_layer_norm_fwd(f.stream(), static_cast<clk_dtype>(x->dtype), x->data,
                              static_cast<const float*>(sc->data),
                              static_cast<const float*>(of->data), y->data, M, C, eps);
}

clk_status layer_norm_bwd(const Frame& f) {
    const char* who = "ClkLayerNormBwd";
    const Buffer *x = f.arg(0), *sc = f.arg(1), *dy = f.arg(2);
    const Buffer *dx = f.ret(0), *ds = f.ret(1), *dof = f.ret(2), *ws = f.ret(3);
    if (!x || !sc || !dy || !dx || !ds || !dof || !ws)
        return bad(who, "expects x, scale, dy -> dx, dscale, doffset, workspace");
    if (x->rank < 1) return bad(who, "x must be [M,C]");
    const int64_t C = x->dims[x->rank - 1], M = C ? numel(x) / C : 0;
    if (!dims_are(sc, {C}) || sc->dtype != kF32) return bad(who, "scale must be f32 [C]");
    if (numel(dy) != numel(x) || dy->dtype != x->dtype || numel(dx) != numel(x) ||
        dx->dtype != x->dtype)
        return bad(who, "dy and dx must match x");
    if (!dims_are(ds, {C}) || !dims_are(dof, {C}) || ds->dtype != kF32 || dof->dtype != kF32)
        return bad(who, "dscale and doffset must be f32 [C]");
    if (ws->dtype != kU8) return bad(who, "fourth result must be the u8 workspace");
    float eps;
    if (!f.attr_f32("eps", &eps)) return bad(who, "missing f32 attribute 'eps'");
    return clk_layer_norm_bwd(f.stream(), static_cast<clk_dtype>(x->dtype), x->data,
                              static_cast<const float*>(sc->data), dy->data, dx->data,
                              static_cast<float*>(ds->data), static_cast<float*>(dof->data),
                              ws->data, (size_t)numel(ws), M, C, eps);
}

clk_status gdp(const char* who, const Frame& f) {
    const Buffer *x = f.arg(0), *wp = f.arg(1), *bp = f.arg(2), *wg = f.arg(3), *bg = f.arg(4),
                 *mask = f.arg(5), *out = f.ret(0);
    if (!x || !wp || !bp || !wg || !bg || !mask || !out)
        return bad(who, "expects x, wp, bp, wg, bg, mask -> out");
    if (x->rank != 2) return bad(who, "x must be [M,K]");
    const int64_t M = x->dims[0], K = x->dims[1];
    if (wp->rank != 2 || wp->dims[0] != K) return bad(who, "wp must be [K,N]");
    const int64_t N = wp->dims[1];
    if (!dims_are(wg, {K, N}) || !dims_are(bp, {N}) || !dims_are(bg, {N}) ||
        !dims_are(mask, {M}) || !dims_are(out, {M, N}))
        return bad(who, "wg [K,N], bp, bg [N], mask [M], out [M,N] expected");
    const DataType t = x->dtype;
    if (!half_type(t) || wp->dtype != t || bp->dtype != t || wg->dtype != t || bg->dtype != t ||
        mask->dtype != t || out->dtype != t)
        return bad(who, "all operands must be f16 or all bf16");
    return clk_gated_dual_proj(f.stream(), static_cast<clk_dtype>(t), x->data, wp->data,
                               bp->data, wg->data, bg->data, mask->data, out->data, M, K, N);
}

clk_status ln_gdp(const Frame& f) {
    const char* who = "ClkLnGdp";
    if (f.nargs() != 12 || f.nrets() != 2)
        return bad(who, "expects 12 operands (z, ln_scale, ln_offset, 8 weights/biases, mask) "
                        "and 2 results");
    const Buffer* z = f.arg(0);
    const Buffer *sc = f.arg(1), *of = f.arg(2), *mask = f.arg(11), *a = f.ret(0), *b = f.ret(1);
    if (!z || !sc || !of || !mask || !a || !b) return bad(who, "operands must be buffers");
    if (z->rank < 1) return bad(who, "z must be [M,C]");
    const int64_t C = z->dims[z->rank - 1], M = C ? numel(z) / C : 0;
    if (!dims_are(sc, {C}) || !dims_are(of, {C}) || sc->dtype != kF32 || of->dtype != kF32)
        return bad(who, "ln_scale and ln_offset must be f32 [C]");
    const Buffer* w[4] = {f.arg(3), f.arg(5), f.arg(7), f.arg(9)};
    const Buffer* bias[4] = {f.arg(4), f.arg(6), f.arg(8), f.arg(10)};
    if (!w[0] || w[0]->rank != 2 || w[0]->dims[0] != C) return bad(who, "weights must be [C,N]");
    const int64_t N = w[0]->dims[1];
    const DataType t = z->dtype;
    if (!half_type(t)) return bad(who, "z must be f16 or bf16");
    for (int i = 0; i < 4; ++i) {
        if (!dims_are(w[i], {C, N}) || w[i]->dtype != t) return bad(who, "weights must be [C,N]");
        if (!dims_are(bias[i], {N}) || bias[i]->dtype != t) return bad(who, "biases must be [N]");
    }
    if (numel(mask) != M || mask->dtype != t) return bad(who, "mask must have M elements");
    if (numel(a) != M * N || numel(b) != M * N || a->dtype != t || b->dtype != t)
        return bad(who, "a and b must be [M,N]");
    float eps;
    if (!f.attr_f32("eps", &eps)) return bad(who, "missing f32 attribute 'eps'");
    return clk_ln_gated_dual_proj(f.stream(), static_cast<clk_dtype>(t), z->data,
                                  static_cast<const float*>(sc->data),
                                  static_cast<const float*>(of->data), w[0]->data, bias[0]->data,
                                  w[1]->data, bias[1]->data, w[2]->data, bias[2]->data,
                                  w[3]->data, bias[3]->data, mask->data, a->data, b->data, M, C,
                                  N, eps);
}

clk_status attention_gate(const Frame& f) {
    const char* who = "ClkAttentionGate";
    if (f.nargs() != 4 || f.nrets() != 1)
        return bad(who, "expects 4 operands (o, x, wg, bg) and 1 result");
    const Buffer *o = f.arg(0), *x = f.arg(1), *wg = f.arg(2), *bg = f.arg(3), *out = f.ret(0);
    if (!o || !x || !wg || !bg || !out) return bad(who, "operands must be buffers");
    if (o->rank != 4) return bad(who, "o must be [N,H,Sq,D]");
    const int64_t N = o->dims[0], H = o->dims[1], Sq = o->dims[2], D = o->dims[3];
    if (x->rank != 3 || x->dims[0] != N || x->dims[1] != Sq) return bad(who, "x must be [N,Sq,C]");
    const int64_t C = x->dims[2];
    if (!dims_are(wg, {C, H * D}) || !dims_are(bg, {H * D}) || !dims_are(out, {N, Sq, H * D}))
        return bad(who, "wg [C,H*D], bg [H*D], out [N,Sq,H*D] expected");
    const DataType t = o->dtype;
    if (!half_type(t) || x->dtype != t || wg->dtype != t || bg->dtype != t || out->dtype != t)
        return bad(who, "all operands must be f16 or all bf16");
    return clk_attention_gate(f.stream(), static_cast<clk_dtype>(t), o->data, x->data, wg->data,
                              bg->data, out->data, N, H, Sq, D, C);
}

clk_status attention_gate_bwd(const Frame& f) {
    const char* who = "ClkAttentionGateBwd";
    if (f.nargs() != 5 || f.nrets() != 5)
        return bad(who, "expects 5 operands (o, x, wg, bg, dout) and 5 results (do, dx, dwg, dbg, "
                        "workspace)");
    const Buffer *o = f.arg(0), *x = f.arg(1), *wg = f.arg(2), *bg = f.arg(3), *dout = f.arg(4);
    const Buffer *dO = f.ret(0), *dx = f.ret(1), *dwg = f.ret(2), *dbg = f.ret(3), *ws = f.ret(4);
    if (!o || !x || !wg || !bg || !dout || !dO || !dx || !dwg || !dbg || !ws)
        return bad(who, "operands and results must be buffers");
    if (o->rank != 4) return bad(who, "o must be [N,H,Sq,D]");
    const int64_t N = o->dims[0], H = o->dims[1], Sq = o->dims[2], D = o->dims[3];
    if (x->rank != 3 || x->dims[0] != N || x->dims[1] != Sq) return bad(who, "x must be [N,Sq,C]");
    const int64_t C = x->dims[2];
    if (!dims_are(wg, {C, H * D}) || !dims_are(bg, {H * D}) || !dims_are(dout, {N, Sq, H * D}))
        return bad(who, "wg [C,H*D], bg [H*D], dout [N,Sq,H*D] expected");
    if (!dims_are(dO, {N, H, Sq, D}) || !dims_are(dx, {N, Sq, C}))
        return bad(who, "do [N,H,Sq,D] and dx [N,Sq,C] expected");
    const DataType t = o->dtype;
    if (!half_type(t) || x->dtype != t || wg->dtype != t || bg->dtype != t || dout->dtype != t ||
        dO->dtype != t || dx->dtype != t)
        return bad(who, "o, x, wg, bg, dout, do, dx must be all f16 or all bf16");
    if (!dims_are(dwg, {C, H * D}) || !dims_are(dbg, {H * D}) || dwg->dtype != kF32 ||
        dbg->dtype != kF32)
        return bad(who, "dwg f32 [C,H*D] and dbg f32 [H*D] expected");
    if (ws->dtype != kU8) return bad(who, "fifth result must be the u8 workspace");
    return clk_attention_gate_bwd(f.stream(), static_cast<clk_dtype>(t), o->data, x->data,
                                  wg->data, bg->data, dout->data, dO->data, dx->data,
                                  static_cast<float*>(dwg->data), static_cast<float*>(dbg->data),
                                  ws->data, (size_t)numel(ws), N, H, Sq, D, C, 0);
}

clk_status ln_pair_bias(const Frame& f) {
    const char* who = "ClkLnPairBias";
    if (f.nargs() != 4 || f.nrets() != 1)
        return bad(who, "expects 4 operands (z, scale, offset, w) and 1 result");
    const Buffer *z = f.arg(0), *sc = f.arg(1), *of = f.arg(2), *w = f.arg(3), *out = f.ret(0);
    if (!z || !sc || !of || !w || !out) return bad(who, "operands must be buffers");
    if (z->rank < 1) return bad(who, "z must be [..., C]");
    const int64_t C = z->dims[z->rank - 1], M = C ? numel(z) / C : 0;
    if (!dims_are(sc, {C}) || !dims_are(of, {C}) || sc->dtype != kF32 || of->dtype != kF32)
        return bad(who, "scale and offset must be f32 [C]");
    if (w->rank != 2 || w->dims[0] != C) return bad(who, "w must be [C,H]");
    const int64_t H = w->dims[1];
    const DataType t = z->dtype;
    if (!half_type(t) || w->dtype != t || out->dtype != t) return bad(who, "z, w, out f16 or bf16");
    if (numel(out) != H * M || out->rank != z->rank || out->dims[0] != H)
        return bad(who, "out must be [H, ...] over z's leading axes");
    float eps;
    if (!f.attr_f32("eps", &eps)) return bad(who, "missing f32 attribute 'eps'");
    return clk_ln_pair_bias(f.stream(), static_cast<clk_dtype>(t), z->data,
                            static_cast<const float*>(sc->data), static_cast<const float*>(of->data),
                            w->data, out->data, M, C, H, eps);
}

clk_status gdp_bwd(const Frame& f) {
    const char* who = "ClkGdpBwd";
    if (f.nargs() != 7 || f.nrets() != 6)
        return bad(who, "expects 7 operands (x, wp, bp, wg, bg, mask, dout) and 6 results "
                        "(dx, dwp, dbp, dwg, dbg, workspace)");
    const Buffer* a[7];
    for (int i = 0; i < 7; ++i)
        if (!(a[i] = f.arg(i))) return bad(who, "operands must be buffers");
    const Buffer* r[6];
    for (int i = 0; i < 6; ++i)
        if (!(r[i] = f.ret(i))) return bad(who, "results must be buffers");
    const Buffer* x = a[0];
    if (x->rank != 2 || a[1]->rank != 2 || a[1]->dims[0] != x->dims[1])
        return bad(who, "x [M,K] and wp [K,N] expected");
    const int64_t M = x->dims[0], K = x->dims[1], N = a[1]->dims[1];
    const DataType t = x->dtype;
    if (!half_type(t)) return bad(who, "x must be f16 or bf16");
    if (!dims_are(a[3], {K, N}) || !dims_are(a[2], {N}) || !dims_are(a[4], {N}) ||
        !dims_are(a[5], {M}) || !dims_are(a[6], {M, N}) || !dims_are(r[0], {M, K}))
        return bad(who, "wg [K,N], bp, bg [N], mask [M], dout [M,N], dx [M,K] expected");
    for (int i = 1; i < 7; ++i)
        if (a[i]->dtype != t) return bad(who, "all operands must share x's dtype");
    if (r[0]->dtype != t) return bad(who, "dx must have x's dtype");
    if (!dims_are(r[1], {K, N}) || !dims_are(r[3], {K, N}) || !dims_are(r[2], {N}) ||
        !dims_are(r[4], {N}) || r[1]->dtype != kF32 || r[2]->dtype != kF32 ||
        r[3]->dtype != kF32 || r[4]->dtype != kF32)
        return bad(who, "dwp, dwg f32 [K,N] and dbp, dbg f32 [N] expected");
    if (r[5]->dtype != kU8) return bad(who, "sixth result must be the u8 workspace");
    return clk_gated_dual_proj_bwd(
        f.stream(), static_cast<clk_dtype>(t), x->data, a[1]->data, a[2]->data, a[3]->data,
        a[4]->data, a[5]->data, a[6]->data, r[0]->data, static_cast<float*>(r[1]->data),
        static_cast<float*>(r[2]->data), static_cast<float*>(r[3]->data),
        static_cast<float*>(r[4]->data), r[5]->data, (size_t)numel(r[5]), M, K, N, 0);
}

clk_status triangle_multiply(const Frame& f) {
    const char* who = "ClkTriangleMultiply";
    if (f.nargs() != 18 || f.nrets() != 2)
        return bad(who, "expects 18 operands (z, mask, 4 LayerNorm vectors, 6 weights, 6 biases) "
                        "and 2 results (out, workspace)");
    const Buffer* z = f.arg(0);
    const Buffer* mask = f.arg(1);
    const Buffer *out = f.ret(0), *ws = f.ret(1);
    if (!z || !mask || !out || !ws) return bad(who, "operands must be buffers");
    if (z->rank != 3 || z->dims[0] != z->dims[1]) return bad(who, "z must be [N,N,C]");
    const int64_t N = z->dims[0], C = z->dims[2];
    const DataType t = z->dtype;
    if (!half_type(t)) return bad(who, "z must be f16 or bf16");
    if (!dims_are(mask, {N, N}) || mask->dtype != t) return bad(who, "mask must be [N,N]");
    if (!dims_are(out, {N, N, C}) || out->dtype != t) return bad(who, "out must be [N,N,C]");
    if (ws->dtype != kU8) return bad(who, "second result must be the u8 workspace");
    const float* ln[4];
    for (int i = 0; i < 4; ++i) {
        const Buffer* b = f.arg(2 + i);
        if (!b || !dims_are(b, {C}) || b->dtype != kF32)
            return bad(who, "LayerNorm scales and offsets must be f32 [C]");
        ln[i] = static_cast<const float*>(b->data);
    }
    const void *w[6], *bb[6];
    for (int i = 0; i < 6; ++i) {
        const Buffer *wi = f.arg(6 + i), *bi = f.arg(12 + i);
        if (!wi || !bi || !dims_are(wi, {C, C}) || !dims_are(bi, {C}) || wi->dtype != t ||
            bi->dtype != t)
            return bad(who, "weights must be [C,C] and biases [C] of z's dtype");
        w[i] = wi->data;
        bb[i] = bi->data;
    }
    float eps;
    int64_t outgoing;
    if (!f.attr_f32("eps", &eps)) return bad(who, "missing f32 attribute 'eps'");
    if (!f.attr_i64("outgoing", &outgoing)) return bad(who, "missing i64 attribute 'outgoing'");
    return clk_triangle_multiply(f.stream(), static_cast<clk_dtype>(t), z->data, mask->data, ln,
                                 w, bb, out->data, ws->data, (size_t)numel(ws), N, C,
                                 outgoing != 0, eps);
}

}  // namespace

#define CLK_FFI_EXPORT extern "C" __attribute__((visibility("default")))

CLK_FFI_EXPORT Error* VoltaMma(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return attention_fwd("VoltaMma", f, false); });
}
CLK_FFI_EXPORT Error* VoltaWmma(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return attention_fwd("VoltaWmma", f, false); });
}
CLK_FFI_EXPORT Error* ClkAttentionFwd(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return attention_fwd("ClkAttentionFwd", f, true); });
}
CLK_FFI_EXPORT Error* ClkAttentionNshd(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return attention_nshd(f); });
}
CLK_FFI_EXPORT Error* ClkAttentionGated(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return attention_gated(f); });
}
CLK_FFI_EXPORT Error* ClkAttentionBwd(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return attention_bwd(f, false); });
}
CLK_FFI_EXPORT Error* ClkAttentionBwdNshd(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return attention_bwd(f, true); });
}
CLK_FFI_EXPORT Error* VoltaLayerNorm(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return layer_norm_fwd(f); });
}
CLK_FFI_EXPORT Error* ClkLayerNormBwd(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return layer_norm_bwd(f); });
}
CLK_FFI_EXPORT Error* VoltaGdp(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return gdp("VoltaGdp", f); });
}
CLK_FFI_EXPORT Error* VoltaGdpWmma(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return gdp("VoltaGdpWmma", f); });
}
CLK_FFI_EXPORT Error* ClkLnGdp(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return ln_gdp(f); });
}
CLK_FFI_EXPORT Error* ClkAttentionGate(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return attention_gate(f); });
}
CLK_FFI_EXPORT Error* ClkAttentionGateBwd(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return attention_gate_bwd(f); });
}
CLK_FFI_EXPORT Error* ClkLnPairBias(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return ln_pair_bias(f); });
}
CLK_FFI_EXPORT Error* ClkGdpBwd(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return gdp_bwd(f); });
}
CLK_FFI_EXPORT Error* ClkTriangleMultiply(CallFrame* frame) {
    return run(frame, [](const Frame& f) { return triangle_multiply(f); });
}
