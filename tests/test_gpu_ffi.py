"""The XLA FFI targets run on device buffers through a fake XLA runtime and agree bit-for-bit with
the C ABI calls they forward to (and hence with the oracle-checked results of the other tests)."""
import ctypes

import pytest
import torch

import colabfold_legacy_kernels as clk
from colabfold_legacy_kernels import ops
from colabfold_legacy_kernels.workloads import attention_inputs, gdp_weights, layer_norm_inputs
from _xla_ffi import BF16, F16, F32, S64, U8, FakeXla

pytestmark = pytest.mark.gpu

DT = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32, torch.uint8: U8}


def buf(x, t):
    return x.buffer(DT[t.dtype], tuple(t.shape), t.data_ptr())


def lib_and_runtime(dev):
    lib = ctypes.CDLL(clk.library_path("attention", "gfx950"))
    return lib, FakeXla(stream=torch.cuda.current_stream(dev).cuda_stream)


def test_volta_mma_and_attention_bwd_targets(cuda):
    lib, x = lib_and_runtime(cuda)
    inp = attention_inputs(3, 2, 100, 90, 32, torch.bfloat16, seed=8, device=cuda,
                           masked_tail=0.1, masked_rows=1)
    q, k, v, bias, km, dout = (inp[n] for n in ("q", "k", "v", "bias", "kmask", "dout"))
    out = torch.empty_like(q)
    fr = x.frame([buf(x, q), buf(x, k), buf(x, v), buf(x, bias), buf(x, km)], [buf(x, out)],
                 [("scale", F32, inp["scale"]), ("block_q", S64, 64), ("block_k", S64, 64)])
    assert x.call(lib, "VoltaMma", fr) is None, x.errors
    ref_out, ref_lse = ops.attention_fwd(q, k, v, bias, km, inp["scale"])
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out)

    out2 = torch.empty_like(q)
    lse = torch.empty_like(ref_lse)
    fr = x.frame([buf(x, q), buf(x, k), buf(x, v), buf(x, bias), buf(x, km)],
                 [buf(x, out2), buf(x, lse)], [("scale", F32, inp["scale"])])
    assert x.call(lib, "ClkAttentionFwd", fr) is None, x.errors
    torch.cuda.synchronize()
    assert torch.equal(out2, ref_out) and torch.equal(lse, ref_lse)

    n, h, sq, d = q.shape
    sk = k.shape[2]
    ws = torch.empty(lib.clk_attention_bwd_workspace_size(n, h, sq, sk, d), device=cuda,
                     dtype=torch.uint8)
    grads = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
             torch.empty((h, sq, sk), device=cuda, dtype=torch.float32)]
    fr = x.frame([buf(x, t) for t in (q, k, v, bias, km, ref_out, dout, ref_lse)],
                 [buf(x, t) for t in grads] + [buf(x, ws)], [("scale", F32, inp["scale"])])
    assert x.call(lib, "ClkAttentionBwd", fr) is None, x.errors
    ref = ops.attention_bwd(q, k, v, bias, km, ref_out, dout, ref_lse, inp["scale"])
    torch.cuda.synchronize()
    for a, b in zip(grads, ref):
        assert torch.equal(a, b)

    # The [N,S,H,D] targets: forward with lse, then the backward, on the transposed operands.
    t = lambda x_: x_.transpose(1, 2).contiguous()  # noqa: E731
    qs, ks, vs, outs_ref, douts = t(q), t(k), t(v), t(ref_out), t(dout)
    outs, lses = torch.empty_like(qs), torch.empty_like(ref_lse)
    fr = x.frame([buf(x, tt) for tt in (qs, ks, vs, bias, km)], [buf(x, outs), buf(x, lses)],
                 [("scale", F32, inp["scale"])])
    assert x.call(lib, "ClkAttentionNshd", fr) is None, x.errors
    gs = [torch.empty_like(qs), torch.empty_like(ks), torch.empty_like(vs),
          torch.empty((h, sq, sk), device=cuda, dtype=torch.float32)]
    fr = x.frame([buf(x, tt) for tt in (qs, ks, vs, bias, km, outs_ref, douts, ref_lse)],
                 [buf(x, tt) for tt in gs] + [buf(x, ws)], [("scale", F32, inp["scale"])])
    assert x.call(lib, "ClkAttentionBwdNshd", fr) is None, x.errors
    torch.cuda.synchronize()
    assert torch.equal(outs, outs_ref) and torch.equal(lses, ref_lse)
    for a, b in zip(gs[:3], ref[:3]):
        assert torch.equal(t(a), b)
    assert torch.equal(gs[3], ref[3])


# The (D, block_q, block_k) sets each reference target dispatches (cuda/volta_mma_attn.cu:323-331,
# cuda/volta_wmma_attn.cu:286-292), called with f16 buffers as the reference's callers do.
VOLTA_SETS = {
    "VoltaMma": [(8, 64, 64), (8, 64, 32), (8, 32, 32), (8, 128, 64), (8, 32, 64), (32, 64, 64),
                 (32, 64, 32), (32, 32, 64), (32, 32, 32), (32, 128, 64), (32, 16, 64),
                 (16, 64, 64), (16, 32, 32), (16, 64, 32), (64, 64, 64), (64, 32, 32)],
    "VoltaWmma": [(32, 64, 64), (32, 64, 32), (32, 32, 64), (32, 32, 32), (32, 128, 64),
                  (32, 128, 32), (16, 64, 64), (16, 32, 32), (16, 64, 32), (64, 64, 64),
                  (64, 32, 32), (64, 64, 32), (8, 64, 64), (8, 64, 32), (8, 32, 32)],
}


@pytest.mark.parametrize("target", sorted(VOLTA_SETS))
def test_volta_targets_take_every_reference_block_config(cuda, target):
    lib, x = lib_and_runtime(cuda)
    for d in sorted({c[0] for c in VOLTA_SETS[target]}):
        inp = attention_inputs(2, 2, 70, 90, d, torch.float16, seed=d, device=cuda,
                               masked_tail=0.1, with_dout=False)
        q, k, v, bias, km = (inp[n] for n in ("q", "k", "v", "bias", "kmask"))
        ref = ops.attention(q, k, v, bias, km, inp["scale"])
        for dd, bq, bk in VOLTA_SETS[target]:
            if dd != d:
                continue
            out = torch.empty_like(q)
            fr = x.frame([buf(x, q), buf(x, k), buf(x, v), buf(x, bias), buf(x, km)],
                         [buf(x, out)], [("scale", F32, inp["scale"]), ("block_q", S64, bq),
                                         ("block_k", S64, bk)])
            assert x.call(lib, target, fr) is None, (d, bq, bk, x.errors)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), (d, bq, bk)


def test_layer_norm_and_gdp_targets(cuda):
    lib, x = lib_and_runtime(cuda)
    li = layer_norm_inputs(500, 128, torch.bfloat16, seed=2, device=cuda)
    y = torch.empty_like(li["x"])
    fr = x.frame([buf(x, li["x"]), buf(x, li["scale"]), buf(x, li["offset"])], [buf(x, y)],
                 [("eps", F32, 1e-5)])
    assert x.call(lib, "VoltaLayerNorm", fr) is None, x.errors
    assert torch.equal(y, ops.layer_norm(li["x"], li["scale"], li["offset"], 1e-5))

    dx, ds, do = (torch.empty_like(li["x"]), torch.empty(128, device=cuda),
                  torch.empty(128, device=cuda))
    ws = torch.empty(lib.clk_layer_norm_bwd_workspace_size(500, 128), device=cuda,
                     dtype=torch.uint8)
    fr = x.frame([buf(x, li["x"]), buf(x, li["scale"]), buf(x, li["dy"])],
                 [buf(x, dx), buf(x, ds), buf(x, do), buf(x, ws)], [("eps", F32, 1e-5)])
    assert x.call(lib, "ClkLayerNormBwd", fr) is None, x.errors
    for a, b in zip((dx, ds, do), ops.layer_norm_bwd(li["x"], li["scale"], li["dy"], 1e-5)):
        assert torch.equal(a, b)

    wp, bp, wg, bg = gdp_weights(128, 128, torch.bfloat16, seed=4, device=cuda, bias_std=0.1)
    out = torch.empty_like(y)
    fr = x.frame([buf(x, t) for t in (y, wp, bp, wg, bg, li["mask"])], [buf(x, out)])
    assert x.call(lib, "VoltaGdp", fr) is None, x.errors
    assert torch.equal(out, ops.gated_dual_proj(y, wp, bp, wg, bg, li["mask"]))

    wb = gdp_weights(128, 128, torch.bfloat16, seed=5, device=cuda, bias_std=0.1)
    a, b = torch.empty_like(y), torch.empty_like(y)
    fr = x.frame([buf(x, t) for t in (li["x"], li["scale"], li["offset"], wp, bp, wg, bg) + wb
                  + (li["mask"],)], [buf(x, a), buf(x, b)], [("eps", F32, 1e-5)])
    assert x.call(lib, "ClkLnGdp", fr) is None, x.errors
    ra, rb = ops.ln_gated_dual_proj(li["x"], li["scale"], li["offset"], (wp, bp, wg, bg), wb,
                                    li["mask"])
    torch.cuda.synchronize()
    assert torch.equal(a, ra) and torch.equal(b, rb)


def test_new_targets_match_the_c_abi(cuda):
    """ClkAttentionGate, ClkAttentionGateBwd, ClkAttentionGated, ClkAttentionNshd, ClkLnPairBias,
    ClkGdpBwd and ClkTriangleMultiply on device buffers."""
    lib, x = lib_and_runtime(cuda)
    g = torch.Generator().manual_seed(21)
    bf = lambda *s, std=1.0: (torch.randn(s, generator=g) * std).to(torch.bfloat16).to(cuda)  # noqa
    f32 = lambda *s, base=0.0: (base + 0.1 * torch.randn(s, generator=g)).to(cuda)  # noqa

    o, xin, wgt, bgt = bf(2, 8, 40, 32), bf(2, 40, 256), bf(256, 256, std=1 / 16), bf(256, std=0.3)
    out = torch.empty((2, 40, 256), dtype=torch.bfloat16, device=cuda)
    fr = x.frame([buf(x, t) for t in (o, xin, wgt, bgt)], [buf(x, out)])
    assert x.call(lib, "ClkAttentionGate", fr) is None, x.errors
    torch.cuda.synchronize()
    assert torch.equal(out, ops.attention_gate(o, xin, wgt, bgt))

    dgate = bf(2, 40, 256)
    gws = lib.clk_attention_gate_bwd_workspace_size
    gws.restype = ctypes.c_size_t
    gws.argtypes = [ctypes.c_int64] * 5
    ws = torch.empty(gws(2, 8, 40, 32, 256), dtype=torch.uint8, device=cuda)
    grets = [torch.empty_like(o), torch.empty_like(xin), torch.empty((256, 256), device=cuda),
             torch.empty((256,), device=cuda)]
    fr = x.frame([buf(x, t) for t in (o, xin, wgt, bgt, dgate)],
                 [buf(x, t) for t in grets] + [buf(x, ws)])
    assert x.call(lib, "ClkAttentionGateBwd", fr) is None, x.errors
    ref = ops.attention_gate_bwd(o, xin, wgt, bgt, dgate)
    torch.cuda.synchronize()
    for a, b in zip(grets, ref):
        assert torch.equal(a, b)

    q, k, v = bf(2, 8, 40, 32), bf(2, 8, 40, 32), bf(2, 8, 40, 32)
    ab, km = bf(8, 40, 40), (torch.rand((2, 40), generator=g) > 0.2).to(torch.uint8).to(cuda)
    gated = torch.empty((2, 40, 256), dtype=torch.bfloat16, device=cuda)
    fr = x.frame([buf(x, t) for t in (q, k, v, ab, km, xin, wgt, bgt)], [buf(x, gated)],
                 [("scale", F32, 0.17)])
    assert x.call(lib, "ClkAttentionGated", fr) is None, x.errors
    torch.cuda.synchronize()
    assert torch.equal(gated, ops.attention_gated(q, k, v, ab, km, xin, wgt, bgt, 0.17))

    qs, ks, vs = (t.transpose(1, 2).contiguous() for t in (q, k, v))  # [N, S, H, D]
    outs = torch.empty_like(qs)
    fr = x.frame([buf(x, t) for t in (qs, ks, vs, ab, km)], [buf(x, outs)],
                 [("scale", F32, 0.17)])
    assert x.call(lib, "ClkAttentionNshd", fr) is None, x.errors
    torch.cuda.synchronize()
    assert torch.equal(outs, ops.attention_nshd(qs, ks, vs, ab, km, 0.17)[0])
    assert torch.equal(outs.transpose(1, 2), ops.attention(q, k, v, ab, km, 0.17))

    z, sc, of, w = bf(16, 24, 128), f32(128, base=1.0), f32(128), bf(128, 4, std=1 / 11.3)
    bias = torch.empty((4, 16, 24), dtype=torch.bfloat16, device=cuda)
    fr = x.frame([buf(x, t) for t in (z, sc, of, w)], [buf(x, bias)], [("eps", F32, 1e-5)])
    assert x.call(lib, "ClkLnPairBias", fr) is None, x.errors
    torch.cuda.synchronize()
    assert torch.equal(bias, ops.ln_pair_bias(z, sc, of, w))

    li = layer_norm_inputs(300, 128, torch.bfloat16, seed=22, device=cuda)
    wts = gdp_weights(128, 128, torch.bfloat16, seed=23, device=cuda, bias_std=0.2)
    dout = bf(300, 128)
    ws_bytes = lib.clk_gated_dual_proj_bwd_workspace_size
    ws_bytes.restype = ctypes.c_size_t
    ws_bytes.argtypes = [ctypes.c_int64] * 3
    ws = torch.empty(ws_bytes(300, 128, 128), dtype=torch.uint8, device=cuda)
    rets = [torch.empty_like(li["x"])] + [torch.empty(s, device=cuda)
                                          for s in ((128, 128), (128,), (128, 128), (128,))]
    fr = x.frame([buf(x, t) for t in (li["x"],) + tuple(wts) + (li["mask"], dout)],
                 [buf(x, t) for t in rets] + [buf(x, ws)])
    assert x.call(lib, "ClkGdpBwd", fr) is None, x.errors
    ref = ops.gated_dual_proj_bwd(li["x"], *wts, li["mask"], dout)
    torch.cuda.synchronize()
    for a, b in zip(rets, ref):
        assert torch.equal(a, b)

    n, c = 24, 128
    zt, mask = bf(n, n, c), (torch.rand((n, n), generator=g) > 0.1).to(torch.bfloat16).to(cuda)
    lns = [f32(c, base=1.0), f32(c), f32(c, base=1.0), f32(c)]
    ws6 = [bf(c, c, std=c ** -0.5) for _ in range(6)]
    bs6 = [bf(c, std=0.2) for _ in range(6)]
    tws = lib.clk_triangle_multiply_workspace_size
    tws.restype = ctypes.c_size_t
    tws.argtypes = [ctypes.c_int64] * 2
    ws = torch.empty(tws(n, c), dtype=torch.uint8, device=cuda)
    for outgoing in (1, 0):
        out = torch.empty_like(zt)
        fr = x.frame([buf(x, t) for t in [zt, mask] + lns + ws6 + bs6], [buf(x, out), buf(x, ws)],
                     [("eps", F32, 1e-5), ("outgoing", S64, outgoing)])
        assert x.call(lib, "ClkTriangleMultiply", fr) is None, x.errors
        ref = ops.triangle_multiply(zt, mask, lns[:2], ws6, bs6, lns[2:], bool(outgoing))
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
