"""GPU kernels against the committed golden fixtures, and the pair micro-block (LayerNorm, both
gated projections, pair-bias projection and triangle-start attention, 4 heads x 32) at its full
64x64x128 size against the float64 oracle."""
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from _util import TOL, assert_close, np64
from colabfold_legacy_kernels import ops
from oracle import evoformer as EV

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name, dev):
    d = np.load(GOLDEN / (name + ".npz"))
    out = {}
    for k in d.files:
        a = d[k]
        if a.dtype == np.float32 and a.ndim > 0 and k not in ("scale", "offset", "ln_scale",
                                                              "ln_offset"):
            out[k] = torch.from_numpy(a).to(dev).to(torch.bfloat16)
        elif a.ndim > 0 and a.dtype != np.float64:
            out[k] = torch.from_numpy(a).to(dev)
        else:
            out[k] = a
    return out


def test_attention_fixture(cuda):
    g = load("attention_small", cuda)
    scale = float(g["scale"])
    out, lse = ops.attention_fwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], scale)
    assert_close("O", out, g["o"], TOL["bf16"]["o"])
    grads = ops.attention_bwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], out, g["dout"], lse,
                              scale)
    for name, got in zip(("dq", "dk", "dv", "dbias"), grads):
        assert_close(name, got, g[name], TOL["bf16"]["grad"])


def test_layer_norm_fixture(cuda):
    g = load("layer_norm_small", cuda)
    eps = float(g["eps"])
    y = ops.layer_norm(g["x"], g["scale"], g["offset"], eps)
    assert_close("y", y, g["y"], TOL["bf16"]["ln"])
    dx, ds, do = ops.layer_norm_bwd(g["x"], g["scale"], g["dy"], eps)
    assert_close("dx", dx, g["dx"], TOL["bf16"]["ln"])
    assert_close("dscale", ds, g["dscale"], TOL["bf16"]["ln"])
    assert_close("doffset", do, g["doffset"], TOL["bf16"]["ln"])


def test_gdp_fixtures(cuda):
    g = load("gdp_small", cuda)
    out = ops.gated_dual_proj(g["x"], g["wp"], g["bp"], g["wg"], g["bg"], g["mask"])
    assert_close("gdp", out, g["out"], TOL["bf16"]["gdp"])
    g = load("ln_gdp_small", cuda)
    a, b = ops.ln_gated_dual_proj(g["z"], g["ln_scale"], g["ln_offset"],
                                  (g["wpa"], g["bpa"], g["wga"], g["bga"]),
                                  (g["wpb"], g["bpb"], g["wgb"], g["bgb"]), g["mask"])
    assert_close("a", a, g["a"], TOL["bf16"]["gdp"])
    assert_close("b", b, g["b"], TOL["bf16"]["gdp"])


def test_pair_block_64(cuda):
    """The float32 pair micro-block workload: z [64,64,128] ~N(0,1); LN eps 1e-5, gamma = 1 +
    N(0,0.1), beta ~ N(0,0.1); four 128x128 GDP weights ~N(0,1/128), no biases; pair bias [4,64,64]
    = LN(z).W_b; q, k, v = LN(z).W as [64 rows, 4 heads, 64, 32]; mask all ones. LayerNorm runs in
    float32 on the GPU, the projections feed bf16 GDP and attention kernels."""
    gen = torch.Generator().manual_seed(0)
    rnd = lambda *s, std=1.0: torch.randn(s, generator=gen) * std  # noqa: E731
    c, h, d = 128, 4, 32
    z = rnd(64, 64, c)
    gamma = 1 + rnd(c, std=math.sqrt(0.1))
    beta = rnd(c, std=math.sqrt(0.1))
    ws = [rnd(c, c, std=1 / math.sqrt(c)) for _ in range(4)]
    zeros = torch.zeros(c)
    wbias = rnd(c, h, std=1 / math.sqrt(c))
    wq, wk, wv = (rnd(c, h * d, std=1 / math.sqrt(c)) for _ in range(3))
    ref = EV.pair_block_fwd(z.numpy(), gamma.numpy(), beta.numpy(), 1e-5,
                            (ws[0].numpy(), zeros.numpy(), ws[1].numpy(), zeros.numpy()),
                            (ws[2].numpy(), zeros.numpy(), ws[3].numpy(), zeros.numpy()),
                            wbias.numpy(), wq.numpy(), wk.numpy(), wv.numpy(), h, d)

    dev = cuda
    y = ops.layer_norm(z.to(dev).reshape(-1, c), gamma.to(dev), beta.to(dev), 1e-5)
    assert_close("y(f32)", y, ref["y"], TOL["f32"]["ln"])
    yb = y.to(torch.bfloat16)
    bf = lambda t: t.to(dev).to(torch.bfloat16)  # noqa: E731
    ones = torch.ones(64 * 64, device=dev, dtype=torch.bfloat16)
    a = ops.gated_dual_proj(yb, bf(ws[0]), bf(zeros), bf(ws[1]), bf(zeros), ones)
    b = ops.gated_dual_proj(yb, bf(ws[2]), bf(zeros), bf(ws[3]), bf(zeros), ones)
    assert_close("a", a, ref["a"], TOL["bf16"]["gdp"])
    assert_close("b", b, ref["b"], TOL["bf16"]["gdp"])
    # The pair bias through the library's LayerNorm-folded projection (16-bit operands: z and
    # W_b rounded to bf16), written straight in the [H, Sq, Sk] attention-bias layout.
    bias = ops.ln_pair_bias(z.to(dev).to(torch.bfloat16), gamma.to(dev), beta.to(dev),
                            bf(wbias))
    assert bias.shape == (h, 64, 64)
    assert_close("bias", bias, ref["bias"], TOL["bf16"]["ln"])
    heads = lambda w: (y @ w.to(dev)).reshape(64, 64, h, d).permute(0, 2, 1, 3).contiguous()  # noqa
    q, k, v = (heads(w).to(torch.bfloat16) for w in (wq, wk, wv))
    o = ops.attention(q, k, v, bias, None, 1 / math.sqrt(d))
    assert_close("o", o, ref["o"], TOL["bf16"]["o"])
    _ = np64
