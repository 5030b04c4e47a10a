"""PyTorch front end of the gfx950 kernels: allocate outputs, pass pointers to the C ABI.

Each function mirrors one XLA FFI target of the reference -- the same operands in the same order,
the same attributes, the same errors -- with torch tensors on a ROCm device in place of XLA
buffers:

  attention(q, k, v, bias, kmask, scale, block_q, block_k)   VoltaMma   (cuda/volta_mma_attn.cu:338-351)
  layer_norm(x, scale, offset, eps)                          VoltaLayerNorm (cuda/volta_ops.cu:87-95)
  gated_dual_proj(x, wp, bp, wg, bg, mask)                   VoltaGdp   (cuda/volta_ops.cu:254-265)

and the targets the reference lacks: attention_fwd (also returns the logsumexp), attention_bwd,
layer_norm_bwd and ln_gated_dual_proj. An invalid call raises InvalidArgument (a ValueError), as
the reference handlers return ffi::Error::InvalidArgument; a launch failure raises InternalError.

Torch is used only for device memory and the current stream; all arithmetic runs in the HIP
library, and a missing library raises FileNotFoundError (there is no fallback path).
"""

import ctypes
import math

import torch

from . import _native

__all__ = [
    "ClkError", "InvalidArgument", "InternalError",
    "attention", "attention_fwd", "attention_bwd",
    "attention_gate", "attention_gate_bwd", "attention_gated", "attention_gated_fwd",
    "layer_norm", "layer_norm_bwd",
    "gated_dual_proj", "ln_gated_dual_proj",
    "AttentionFunction", "GatedAttentionFunction", "LayerNormFunction",
]


class ClkError(RuntimeError):
    """A non-OK status from the library; ``code`` is the clk_status value."""

    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


class InvalidArgument(ClkError, ValueError):
    pass


class InternalError(ClkError):
    pass


_DTYPES = {torch.float16: _native.F16, torch.bfloat16: _native.BF16,
           torch.float32: _native.F32}


def _check(status):
    if status == _native.OK:
        return
    msg = _native.last_error()
    if status == _native.INVALID_ARGUMENT:
        raise InvalidArgument(status, msg)
    raise InternalError(status, msg)


def _ptr(t):
    return None if t is None else t.data_ptr()


def _dtype_code(t, allowed, what):
    code = _DTYPES.get(t.dtype)
    if code is None or code not in allowed:
        raise InvalidArgument(_native.INVALID_ARGUMENT,
                              "%s: dtype %s not supported" % (what, t.dtype))
    return code


def _require(tensors, what):
    dev = None
    for name, t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise InvalidArgument(_native.INVALID_ARGUMENT,
                                  "%s: %s must be a tensor on a ROCm device" % (what, name))
        if not t.is_contiguous():
            raise InvalidArgument(_native.INVALID_ARGUMENT, "%s: %s must be contiguous" % (what, name))
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise InvalidArgument(_native.INVALID_ARGUMENT,
                                  "%s: all operands must be on one device" % what)
    return dev


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _shape_check(cond, what, msg):
    if not cond:
        raise InvalidArgument(_native.INVALID_ARGUMENT, "%s: %s" % (what, msg))


def _attn_dims(q, k, v, bias, kmask, what):
    _shape_check(q.dim() == 4, what, "q must be [N,H,S,D]")
    n, h, sq, d = q.shape
    _shape_check(k.dim() == 4 and k.shape[0] == n and k.shape[1] == h and k.shape[3] == d,
                 what, "k must be [N,H,Sk,D]")
    sk = k.shape[2]
    _shape_check(tuple(v.shape) == tuple(k.shape), what, "v must have the shape of k")
    _shape_check(tuple(bias.shape) == (h, sq, sk), what, "bias must be [H,Sq,Sk]")
    _shape_check(q.dtype == k.dtype == v.dtype == bias.dtype, what,
                 "q, k, v and bias must share one dtype")
    if kmask is not None:
        _shape_check(tuple(kmask.shape) == (n, sk) and kmask.dtype == torch.uint8, what,
                     "kmask must be uint8 [N,Sk]")
    return n, h, sq, sk, d


def _attention_call(q, k, v, bias, kmask, scale, block_q, block_k, want_lse, what):
    dev = _require([("q", q), ("k", k), ("v", v), ("bias", bias), ("kmask", kmask)], what)
    n, h, sq, sk, d = _attn_dims(q, k, v, bias, kmask, what)
    code = _dtype_code(q, (_native.F16, _native.BF16), what)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    out = torch.empty_like(q)
    lse = torch.empty((n, h, sq), device=dev, dtype=torch.float32) if want_lse else None
    lib = _native.lib()
    with torch.cuda.device(dev):
        _check(lib.clk_attention_fwd(_stream(dev), code, _ptr(q), _ptr(k), _ptr(v), _ptr(bias),
                                     _ptr(kmask), _ptr(out), _ptr(lse), n, h, sq, sk, d,
                                     float(scale), int(block_q), int(block_k)))
    return out, lse


def attention(q, k, v, bias, kmask=None, scale=None, block_q=64, block_k=64):
    """softmax(scale*q.k^T + bias, masked keys -> -1e9) . v for q [N,H,Sq,D], k/v [N,H,Sk,D],
    bias [H,Sq,Sk], kmask uint8 [N,Sk]. block_q/block_k are accepted as hints."""
    out, _ = _attention_call(q, k, v, bias, kmask, scale, block_q, block_k, False, "attention")
    return out


def attention_fwd(q, k, v, bias, kmask=None, scale=None):
    """(out, lse): the forward plus the float32 natural-log logsumexp [N,H,Sq] per query."""
    return _attention_call(q, k, v, bias, kmask, scale, 64, 64, True, "attention_fwd")


def attention_nshd(q, k, v, bias, kmask=None, scale=None, want_lse=False):
    """The forward on AlphaFold's [N,S,H,D] layout: q [N,Sq,H,D], k/v [N,Sk,H,D], bias
    [H,Sq,Sk], kmask uint8 [N,Sk]; returns (out [N,Sq,H,D], lse [N,H,Sq] or None), bit-identical
    to attention_fwd on the [N,H,S,D] transposes."""
    what = "attention_nshd"
    dev = _require([("q", q), ("k", k), ("v", v), ("bias", bias), ("kmask", kmask)], what)
    _shape_check(q.dim() == 4 and k.dim() == 4, what, "q and k must be [N,S,H,D]")
    n, h, sq, sk, d = _attn_dims(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), bias,
                                 kmask, what)
    code = _dtype_code(q, (_native.F16, _native.BF16), what)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    out = torch.empty_like(q)
    lse = torch.empty((n, h, sq), device=dev, dtype=torch.float32) if want_lse else None
    lib = _native.lib()
    with torch.cuda.device(dev):
        _check(lib.clk_attention_fwd_nshd(_stream(dev), code, _ptr(q), _ptr(k), _ptr(v),
                                          _ptr(bias), _ptr(kmask), _ptr(out), _ptr(lse), n, h, sq,
                                          sk, d, float(scale)))
    return out, lse


def attention_bwd(q, k, v, bias, kmask, out, dout, lse, scale=None):
    """(dq, dk, dv, dbias) with dbias [H,Sq,Sk] float32 summed over the N rows."""
    what = "attention_bwd"
    dev = _require([("q", q), ("k", k), ("v", v), ("bias", bias), ("kmask", kmask),
                    ("out", out), ("dout", dout), ("lse", lse)], what)
    n, h, sq, sk, d = _attn_dims(q, k, v, bias, kmask, what)
    code = _dtype_code(q, (_native.F16, _native.BF16), what)
    _shape_check(tuple(out.shape) == tuple(q.shape) and out.dtype == q.dtype, what,
                 "out must match q")
    _shape_check(tuple(dout.shape) == tuple(q.shape) and dout.dtype == q.dtype, what,
                 "dout must match q")
    _shape_check(tuple(lse.shape) == (n, h, sq) and lse.dtype == torch.float32, what,
                 "lse must be float32 [N,H,Sq]")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    lib = _native.lib()
    ws_bytes = lib.clk_attention_bwd_workspace_size(n, h, sq, sk, d)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dbias = torch.empty((h, sq, sk), device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        _check(lib.clk_attention_bwd(_stream(dev), code, _ptr(q), _ptr(k), _ptr(v), _ptr(bias),
                                     _ptr(kmask), _ptr(out), _ptr(dout), _ptr(lse), _ptr(dq),
                                     _ptr(dk), _ptr(dv), _ptr(dbias), _ptr(ws), ws_bytes, n, h,
                                     sq, sk, d, float(scale)))
    return dq, dk, dv, dbias


def attention_bwd_nshd(q, k, v, bias, kmask, out, dout, lse, scale=None):
    """attention_bwd on AlphaFold's [N,S,H,D] layout: q, out, dout [N,Sq,H,D], k, v [N,Sk,H,D],
    lse [N,H,Sq]; returns (dq, dk, dv) in the layout of q, k, v and dbias [H,Sq,Sk] float32,
    bit-identical to attention_bwd on the [N,H,S,D] transposes."""
    what = "attention_bwd_nshd"
    dev = _require([("q", q), ("k", k), ("v", v), ("bias", bias), ("kmask", kmask),
                    ("out", out), ("dout", dout), ("lse", lse)], what)
    _shape_check(q.dim() == 4 and k.dim() == 4, what, "q and k must be [N,S,H,D]")
    n, h, sq, sk, d = _attn_dims(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), bias,
                                 kmask, what)
    code = _dtype_code(q, (_native.F16, _native.BF16), what)
    _shape_check(tuple(out.shape) == tuple(q.shape) and out.dtype == q.dtype, what,
                 "out must match q")
    _shape_check(tuple(dout.shape) == tuple(q.shape) and dout.dtype == q.dtype, what,
                 "dout must match q")
    _shape_check(tuple(lse.shape) == (n, h, sq) and lse.dtype == torch.float32, what,
                 "lse must be float32 [N,H,Sq]")
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    lib = _native.lib()
    ws_bytes = lib.clk_attention_bwd_workspace_size(n, h, sq, sk, d)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dbias = torch.empty((h, sq, sk), device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        _check(lib.clk_attention_bwd_nshd(_stream(dev), code, _ptr(q), _ptr(k), _ptr(v),
                                          _ptr(bias), _ptr(kmask), _ptr(out), _ptr(dout),
                                          _ptr(lse), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dbias),
                                          _ptr(ws), ws_bytes, n, h, sq, sk, d, float(scale)))
    return dq, dk, dv, dbias


def _ln_dims(x, scale, what):
    _shape_check(x.dim() >= 1, what, "x must have at least one axis")
    c = x.shape[-1]
    m = x.numel() // c if c else 0
    _shape_check(tuple(scale.shape) == (c,) and scale.dtype == torch.float32, what,
                 "scale must be float32 [C]")
    return m, c


def layer_norm(x, scale, offset, eps=1e-5):
    """LayerNorm over the last axis of x (f16, bf16 or f32); scale and offset float32 [C]."""
    what = "layer_norm"
    dev = _require([("x", x), ("scale", scale), ("offset", offset)], what)
    m, c = _ln_dims(x, scale, what)
    _shape_check(tuple(offset.shape) == (c,) and offset.dtype == torch.float32, what,
                 "offset must be float32 [C]")
    code = _dtype_code(x, (_native.F16, _native.BF16, _native.F32), what)
    y = torch.empty_like(x)
    with torch.cuda.device(dev):
        _check(_native.lib().clk_layer_norm_fwd(_stream(dev), code, _ptr(x), _ptr(scale),
                                                _ptr(offset), _ptr(y), m, c, float(eps)))
    return y


def layer_norm_bwd(x, scale, dy, eps=1e-5):
    """(dx, dscale, doffset); dscale and doffset are float32 [C]."""
    what = "layer_norm_bwd"
    dev = _require([("x", x), ("scale", scale), ("dy", dy)], what)
    m, c = _ln_dims(x, scale, what)
    _shape_check(tuple(dy.shape) == tuple(x.shape) and dy.dtype == x.dtype, what,
                 "dy must match x")
    code = _dtype_code(x, (_native.F16, _native.BF16, _native.F32), what)
    lib = _native.lib()
    ws_bytes = lib.clk_layer_norm_bwd_workspace_size(m, c)
    ws = torch.empty(max(ws_bytes, 1), device=dev, dtype=torch.uint8)
    dx = torch.empty_like(x)
    dscale = torch.empty(c, device=dev, dtype=torch.float32)
    doffset = torch.empty(c, device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        _check(lib.clk_layer_norm_bwd(_stream(dev), code, _ptr(x), _ptr(scale), _ptr(dy),
                                      _ptr(dx), _ptr(dscale), _ptr(doffset), _ptr(ws), ws_bytes,
                                      m, c, float(eps)))
    return dx, dscale, doffset


def gated_dual_proj(x, wp, bp, wg, bg, mask):
    """mask[m] * (x.wp + bp) * sigmoid(x.wg + bg) for x [M,K], wp/wg [K,N], bp/bg [N], mask [M]."""
    what = "gated_dual_proj"
    dev = _require([("x", x), ("wp", wp), ("bp", bp), ("wg", wg), ("bg", bg), ("mask", mask)],
                   what)
    _shape_check(x.dim() == 2, what, "x must be [M,K]")
    m, kdim = x.shape
    _shape_check(wp.dim() == 2 and wp.shape[0] == kdim, what, "wp must be [K,N]")
    n = wp.shape[1]
    _shape_check(tuple(wg.shape) == (kdim, n), what, "wg must be [K,N]")
    _shape_check(tuple(bp.shape) == (n,) and tuple(bg.shape) == (n,), what, "bp, bg must be [N]")
    _shape_check(tuple(mask.shape) == (m,), what, "mask must be [M]")
    _shape_check(all(t.dtype == x.dtype for t in (wp, bp, wg, bg, mask)), what,
                 "all operands must share one dtype")
    code = _dtype_code(x, (_native.F16, _native.BF16), what)
    out = torch.empty((m, n), device=dev, dtype=x.dtype)
    with torch.cuda.device(dev):
        _check(_native.lib().clk_gated_dual_proj(_stream(dev), code, _ptr(x), _ptr(wp), _ptr(bp),
                                                 _ptr(wg), _ptr(bg), _ptr(mask), _ptr(out), m,
                                                 kdim, n))
    return out


def gated_dual_proj_bwd(x, wp, bp, wg, bg, mask, dout, dx=None):
    """Gradients of gated_dual_proj: (dx, dwp, dbp, dwg, dbg); dx in x's dtype, the rest
    float32. If dx is given, the input gradient is added to it in place (two branches that read
    the same x)."""
    what = "gated_dual_proj_bwd"
    dev = _require([("x", x), ("wp", wp), ("bp", bp), ("wg", wg), ("bg", bg), ("mask", mask),
                    ("dout", dout), ("dx", dx)], what)
    _shape_check(x.dim() == 2, what, "x must be [M,K]")
    m, kdim = x.shape
    _shape_check(wp.dim() == 2 and wp.shape[0] == kdim, what, "wp must be [K,N]")
    n = wp.shape[1]
    _shape_check(tuple(wg.shape) == (kdim, n), what, "wg must be [K,N]")
    _shape_check(tuple(bp.shape) == (n,) and tuple(bg.shape) == (n,), what, "bp, bg must be [N]")
    _shape_check(tuple(mask.shape) == (m,), what, "mask must be [M]")
    _shape_check(tuple(dout.shape) == (m, n), what, "dout must be [M,N]")
    _shape_check(all(t.dtype == x.dtype for t in (wp, bp, wg, bg, mask, dout)), what,
                 "all operands must share one dtype")
    code = _dtype_code(x, (_native.F16, _native.BF16), what)
    acc = dx is not None
    if acc:
        _shape_check(tuple(dx.shape) == (m, kdim) and dx.dtype == x.dtype, what,
                     "dx must be [M,K] of x's dtype")
    else:
        dx = torch.empty_like(x)
    f32 = dict(device=dev, dtype=torch.float32)
    dwp, dwg = torch.empty((kdim, n), **f32), torch.empty((kdim, n), **f32)
    dbp, dbg = torch.empty(n, **f32), torch.empty(n, **f32)
    lib = _native.lib()
    wsb = lib.clk_gated_dual_proj_bwd_workspace_size(m, kdim, n)
    ws = torch.empty(max(wsb, 1), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _check(lib.clk_gated_dual_proj_bwd(_stream(dev), code, _ptr(x), _ptr(wp), _ptr(bp),
                                           _ptr(wg), _ptr(bg), _ptr(mask), _ptr(dout), _ptr(dx),
                                           _ptr(dwp), _ptr(dbp), _ptr(dwg), _ptr(dbg), _ptr(ws),
                                           wsb, m, kdim, n, 1 if acc else 0))
    return dx, dwp, dbp, dwg, dbg


def ln_gated_dual_proj_bwd(z, ln_scale, ln_offset, branch_a, branch_b, mask, da, db, eps=1e-5):
    """Gradients of ln_gated_dual_proj: (dz, dln_scale, dln_offset, grads_a, grads_b) with
    grads_x = (dwp, dbp, dwg, dbg). Recomputes y = LN(z), runs the GDP backward of both branches
    into one dy, then the LayerNorm backward."""
    y = layer_norm(z, ln_scale, ln_offset, eps)
    c = z.shape[-1]
    y2, m2 = y.reshape(-1, c), mask.reshape(-1)
    dy, *ga = gated_dual_proj_bwd(y2, *branch_a, m2, da.reshape(y2.shape[0], -1))
    _, *gb = gated_dual_proj_bwd(y2, *branch_b, m2, db.reshape(y2.shape[0], -1), dx=dy)
    dz, dsc, dof = layer_norm_bwd(z, ln_scale, dy.reshape(z.shape), eps)
    return dz, dsc, dof, tuple(ga), tuple(gb)


def ln_gated_dual_proj(z, ln_scale, ln_offset, branch_a, branch_b, mask, eps=1e-5):
    """(a, b): LayerNorm(z) then both gated projections, in one pass. Each branch is
    (wp, bp, wg, bg); z [M,C] (or [..., C]); mask [M]."""
    what = "ln_gated_dual_proj"
    wpa, bpa, wga, bga = branch_a
    wpb, bpb, wgb, bgb = branch_b
    dev = _require([("z", z), ("ln_scale", ln_scale), ("ln_offset", ln_offset), ("wpa", wpa),
                    ("bpa", bpa), ("wga", wga), ("bga", bga), ("wpb", wpb), ("bpb", bpb),
                    ("wgb", wgb), ("bgb", bgb), ("mask", mask)], what)
    m, c = _ln_dims(z, ln_scale, what)
    _shape_check(wpa.dim() == 2 and wpa.shape[0] == c, what, "weights must be [C,N]")
    n = wpa.shape[1]
    for name, w in (("wga", wga), ("wpb", wpb), ("wgb", wgb)):
        _shape_check(tuple(w.shape) == (c, n), what, "%s must be [C,N]" % name)
    for name, b in (("bpa", bpa), ("bga", bga), ("bpb", bpb), ("bgb", bgb)):
        _shape_check(tuple(b.shape) == (n,), what, "%s must be [N]" % name)
    _shape_check(mask.numel() == m, what, "mask must have M elements")
    code = _dtype_code(z, (_native.F16, _native.BF16), what)
    a = torch.empty(tuple(z.shape[:-1]) + (n,), device=dev, dtype=z.dtype)
    b = torch.empty_like(a)
    with torch.cuda.device(dev):
        _check(_native.lib().clk_ln_gated_dual_proj(
            _stream(dev), code, _ptr(z), _ptr(ln_scale), _ptr(ln_offset), _ptr(wpa), _ptr(bpa),
            _ptr(wga), _ptr(bga), _ptr(wpb), _ptr(bpb), _ptr(wgb), _ptr(bgb), _ptr(mask),
            _ptr(a), _ptr(b), m, c, n, float(eps)))
    return a, b


def ln_pair_bias(z, scale, offset, w, eps=1e-5):
    """LN(z).w transposed to the attention bias layout: z [Sq,Sk,C] (or [M,C]), scale/offset
    float32 [C], w [C,H] -> [H,Sq,Sk] (or [H,M])."""
    what = "ln_pair_bias"
    dev = _require([("z", z), ("scale", scale), ("offset", offset), ("w", w)], what)
    m, c = _ln_dims(z, scale, what)
    _shape_check(w.dim() == 2 and w.shape[0] == c and w.dtype == z.dtype, what,
                 "w must be [C,H] of z's dtype")
    _shape_check(tuple(offset.shape) == (c,) and offset.dtype == torch.float32, what,
                 "offset must be float32 [C]")
    h = w.shape[1]
    code = _dtype_code(z, (_native.F16, _native.BF16), what)
    out = torch.empty((h,) + tuple(z.shape[:-1]), device=dev, dtype=z.dtype)
    with torch.cuda.device(dev):
        _check(_native.lib().clk_ln_pair_bias(_stream(dev), code, _ptr(z), _ptr(scale),
                                              _ptr(offset), _ptr(w), _ptr(out), m, c, h,
                                              float(eps)))
    return out


def attention_gate(o, x, wg, bg):
    """o * sigmoid(x.wg + bg), transposed to the output projection's layout: o [N,H,Sq,D] (the
    attention output), x [N,Sq,C], wg [C,H*D], bg [H*D] -> [N,Sq,H*D]."""
    what = "attention_gate"
    dev = _require([("o", o), ("x", x), ("wg", wg), ("bg", bg)], what)
    _shape_check(o.dim() == 4, what, "o must be [N,H,Sq,D]")
    n, h, sq, d = o.shape
    _shape_check(x.dim() == 3 and tuple(x.shape[:2]) == (n, sq), what, "x must be [N,Sq,C]")
    c = x.shape[2]
    _shape_check(tuple(wg.shape) == (c, h * d), what, "wg must be [C,H*D]")
    _shape_check(tuple(bg.shape) == (h * d,), what, "bg must be [H*D]")
    _shape_check(all(t.dtype == o.dtype for t in (x, wg, bg)), what,
                 "all operands must share one dtype")
    code = _dtype_code(o, (_native.F16, _native.BF16), what)
    out = torch.empty((n, sq, h * d), device=dev, dtype=o.dtype)
    with torch.cuda.device(dev):
        _check(_native.lib().clk_attention_gate(_stream(dev), code, _ptr(o), _ptr(x), _ptr(wg),
                                                _ptr(bg), _ptr(out), n, h, sq, d, c))
    return out


def attention_gate_bwd(o, x, wg, bg, dout, dx=None):
    """Gradients of attention_gate for dout [N,Sq,H*D]: (do, dx, dwg, dbg) with do [N,H,Sq,D]
    (the dout of attention_bwd) and dx [N,Sq,C] in o's dtype, dwg [C,H*D] and dbg [H*D] float32.
    If dx is given, the input gradient is added to it in place (x also feeds the q, k, v
    projections)."""
    what = "attention_gate_bwd"
    dev = _require([("o", o), ("x", x), ("wg", wg), ("bg", bg), ("dout", dout), ("dx", dx)],
                   what)
    _shape_check(o.dim() == 4, what, "o must be [N,H,Sq,D]")
    n, h, sq, d = o.shape
    _shape_check(x.dim() == 3 and tuple(x.shape[:2]) == (n, sq), what, "x must be [N,Sq,C]")
    c = x.shape[2]
    _shape_check(tuple(wg.shape) == (c, h * d), what, "wg must be [C,H*D]")
    _shape_check(tuple(bg.shape) == (h * d,), what, "bg must be [H*D]")
    _shape_check(tuple(dout.shape) == (n, sq, h * d), what, "dout must be [N,Sq,H*D]")
    _shape_check(all(t.dtype == o.dtype for t in (x, wg, bg, dout)), what,
                 "all operands must share one dtype")
    code = _dtype_code(o, (_native.F16, _native.BF16), what)
    acc = dx is not None
    if acc:
        _shape_check(tuple(dx.shape) == (n, sq, c) and dx.dtype == o.dtype, what,
                     "dx must be [N,Sq,C] of o's dtype")
    else:
        dx = torch.empty_like(x)
    do = torch.empty_like(o)
    f32 = dict(device=dev, dtype=torch.float32)
    dwg, dbg = torch.empty((c, h * d), **f32), torch.empty(h * d, **f32)
    lib = _native.lib()
    wsb = lib.clk_attention_gate_bwd_workspace_size(n, h, sq, d, c)
    ws = torch.empty(max(wsb, 1), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        _check(lib.clk_attention_gate_bwd(_stream(dev), code, _ptr(o), _ptr(x), _ptr(wg),
                                          _ptr(bg), _ptr(dout), _ptr(do), _ptr(dx), _ptr(dwg),
                                          _ptr(dbg), _ptr(ws), wsb, n, h, sq, d, c,
                                          1 if acc else 0))
    return do, dx, dwg, dbg


def _gated_call(q, k, v, bias, kmask, x, wg, bg, scale, residuals, what):
    dev = _require([("q", q), ("k", k), ("v", v), ("bias", bias), ("kmask", kmask), ("x", x),
                    ("wg", wg), ("bg", bg)], what)
    n, h, sq, sk, d = _attn_dims(q, k, v, bias, kmask, what)
    _shape_check(x.dim() == 3 and tuple(x.shape[:2]) == (n, sq), what, "x must be [N,Sq,C]")
    c = x.shape[2]
    _shape_check(tuple(wg.shape) == (c, h * d), what, "wg must be [C,H*D]")
    _shape_check(tuple(bg.shape) == (h * d,), what, "bg must be [H*D]")
    _shape_check(all(t.dtype == q.dtype for t in (x, wg, bg)), what,
                 "x, wg and bg must have the dtype of q")
    code = _dtype_code(q, (_native.F16, _native.BF16), what)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    gated = torch.empty((n, sq, h * d), device=dev, dtype=q.dtype)
    out = torch.empty_like(q) if residuals else None
    lse = torch.empty((n, h, sq), device=dev, dtype=torch.float32) if residuals else None
    with torch.cuda.device(dev):
        _check(_native.lib().clk_attention_fwd_gated(
            _stream(dev), code, _ptr(q), _ptr(k), _ptr(v), _ptr(bias), _ptr(kmask), _ptr(x),
            _ptr(wg), _ptr(bg), _ptr(gated), _ptr(out), _ptr(lse), n, h, sq, sk, d, c,
            float(scale)))
    return gated, out, lse


def attention_gated(q, k, v, bias, kmask, x, wg, bg, scale=None):
    """attention(q, k, v, bias, kmask) gated by sigmoid(x.wg + bg) in one kernel, in the output
    projection's layout: q [N,H,Sq,D], k/v [N,H,Sk,D], bias [H,Sq,Sk], kmask uint8 [N,Sk] or
    None, x [N,Sq,C] with C % 32 == 0, wg [C,H*D], bg [H*D] -> [N,Sq,H*D]. The ungated
    attention output never reaches memory."""
    gated, _, _ = _gated_call(q, k, v, bias, kmask, x, wg, bg, scale, False, "attention_gated")
    return gated


def attention_gated_fwd(q, k, v, bias, kmask, x, wg, bg, scale=None):
    """(gated, out, lse): attention_gated plus the ungated output [N,H,Sq,D] and the float32
    logsumexp [N,H,Sq] that attention_bwd needs."""
    return _gated_call(q, k, v, bias, kmask, x, wg, bg, scale, True, "attention_gated_fwd")


def triangle_einsum(a, b):
    """x[c] = a[c] . b[c]^T for channel-major a, b [C,N,N] (the triangle-multiplication
    contraction with the channel index first and the contracted index last); N % 8 == 0."""
    what = "triangle_einsum"
    dev = _require([("a", a), ("b", b)], what)
    _shape_check(a.dim() == 3 and a.shape[1] == a.shape[2], what, "a must be [C,N,N]")
    _shape_check(tuple(b.shape) == tuple(a.shape) and b.dtype == a.dtype, what,
                 "b must match a")
    c, n, _ = a.shape
    code = _dtype_code(a, (_native.F16, _native.BF16), what)
    x = torch.empty_like(a)
    with torch.cuda.device(dev):
        _check(_native.lib().clk_triangle_einsum(_stream(dev), code, _ptr(a), _ptr(b), _ptr(x), c,
                                                 n))
    return x


def triangle_multiply(z, mask, ln_in, weights, biases, ln_center, outgoing=True, eps=1e-5):
    """AlphaFold's triangle multiplication on the pair representation z [N,N,C] with mask [N,N].
    ln_in, ln_center: (scale, offset) float32 [C]; weights: the six [C,C] matrices (left
    projection, right projection, left gate, right gate, output projection, output gate), biases
    their [C] vectors, all of z's dtype. Returns [N,N,C]."""
    what = "triangle_multiply"
    ws6, bs6 = list(weights), list(biases)
    _shape_check(len(ws6) == 6 and len(bs6) == 6, what, "six weights and six biases")
    lns = [ln_in[0], ln_in[1], ln_center[0], ln_center[1]]
    dev = _require([("z", z), ("mask", mask)] + [("w%d" % i, w) for i, w in enumerate(ws6)]
                   + [("b%d" % i, b) for i, b in enumerate(bs6)]
                   + [("ln%d" % i, t) for i, t in enumerate(lns)], what)
    _shape_check(z.dim() == 3 and z.shape[0] == z.shape[1], what, "z must be [N,N,C]")
    n, _, c = z.shape
    _shape_check(tuple(mask.shape) == (n, n) and mask.dtype == z.dtype, what,
                 "mask must be [N,N] of z's dtype")
    _shape_check(all(tuple(w.shape) == (c, c) and w.dtype == z.dtype for w in ws6), what,
                 "weights must be [C,C] of z's dtype")
    _shape_check(all(tuple(b.shape) == (c,) and b.dtype == z.dtype for b in bs6), what,
                 "biases must be [C] of z's dtype")
    _shape_check(all(tuple(t.shape) == (c,) and t.dtype == torch.float32 for t in lns), what,
                 "LayerNorm scales and offsets must be float32 [C]")
    code = _dtype_code(z, (_native.F16, _native.BF16), what)
    lib = _native.lib()
    wsb = lib.clk_triangle_multiply_workspace_size(n, c)
    ws = torch.empty(max(wsb, 1), device=dev, dtype=torch.uint8)
    out = torch.empty_like(z)
    arr = lambda ts: (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])  # noqa: E731
    with torch.cuda.device(dev):
        _check(lib.clk_triangle_multiply(_stream(dev), code, _ptr(z), _ptr(mask), arr(lns),
                                         arr(ws6), arr(bs6), _ptr(out), _ptr(ws), wsb, n, c,
                                         1 if outgoing else 0, float(eps)))
    return out


class AttentionFunction(torch.autograd.Function):
    """Differentiable attention: forward saves (out, lse); backward calls attention_bwd."""

    @staticmethod
    def forward(ctx, q, k, v, bias, kmask, scale):
        out, lse = attention_fwd(q, k, v, bias, kmask, scale)
        ctx.save_for_backward(q, k, v, bias, kmask, out, lse)
        ctx.scale = scale
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, bias, kmask, out, lse = ctx.saved_tensors
        dq, dk, dv, dbias = attention_bwd(q, k, v, bias, kmask, out, dout.contiguous(), lse,
                                          ctx.scale)
        return dq, dk, dv, dbias.to(bias.dtype), None, None


class GatedAttentionFunction(torch.autograd.Function):
    """Differentiable gated attention, o(q, k, v, bias, kmask) * sigmoid(x.wg + bg) in the output
    projection's [N,Sq,H*D] layout. forward: attention_gated_fwd (one launch) when fused, else
    attention_fwd then attention_gate (the faster pair on MSA row shapes); both keep the ungated
    output and the logsumexp. backward: attention_gate_bwd (do, dx, dwg, dbg), then
    attention_bwd with that do. Gradients for q, k, v, bias, x, wg, bg."""

    @staticmethod
    def forward(ctx, q, k, v, bias, kmask, x, wg, bg, scale, fused=False):
        if fused:
            gated, out, lse = attention_gated_fwd(q, k, v, bias, kmask, x, wg, bg, scale)
        else:
            out, lse = attention_fwd(q, k, v, bias, kmask, scale)
            gated = attention_gate(out, x, wg, bg)
        ctx.save_for_backward(q, k, v, bias, kmask, x, wg, bg, out, lse)
        ctx.scale = scale
        return gated

    @staticmethod
    def backward(ctx, dgated):
        q, k, v, bias, kmask, x, wg, bg, out, lse = ctx.saved_tensors
        do, dx, dwg, dbg = attention_gate_bwd(out, x, wg, bg, dgated.contiguous())
        dq, dk, dv, dbias = attention_bwd(q, k, v, bias, kmask, out, do, lse, ctx.scale)
        return (dq, dk, dv, dbias.to(bias.dtype), None, dx, dwg.to(wg.dtype), dbg.to(bg.dtype),
                None, None)


class LayerNormFunction(torch.autograd.Function):
    """Differentiable LayerNorm over the last axis (statistics recomputed in backward)."""

    @staticmethod
    def forward(ctx, x, scale, offset, eps):
        ctx.save_for_backward(x, scale)
        ctx.eps = eps
        return layer_norm(x, scale, offset, eps)

    @staticmethod
    def backward(ctx, dy):
        x, scale = ctx.saved_tensors
        dx, dscale, doffset = layer_norm_bwd(x, scale, dy.contiguous(), ctx.eps)
        return dx, dscale, doffset, None
