"""Seeded synthetic inputs for the Evoformer hot-path workloads.

Each workload is the triangle/MSA attention, LayerNorm or gated-projection shape that ColabFold's
pair and MSA stacks call the kernels with. Values are drawn in float32 with a seeded torch
generator and rounded once to the compute dtype; anything that checks a result (the CPU oracle)
reads those same rounded values. N(mu, var) below names a variance.

  pair_block_c0       z [64,64,128] fp32, LN + GDP + triangle-start attention (4 heads x 32)
  triangle_attn_256   q,k,v [256,4,256,32] ~N(0,1), bias [4,256,256] ~N(0,1), keys >= 230 masked
  triangle_attn_384   the same recipe at N_res = 384 (keys >= 346 masked)
  msa_row_attn        q,k,v [512,8,256,32], bias [8,256,256], 102 fully padded sequences,
                      sigmoid gate from a 256x256 weight ~N(0,1/256)
  ln_gdp_512          z [512,512,128], Bernoulli(0.95) mask, four 128x128 weights ~N(0,1/128)
  triangle_attn_1024  q,k,v [1024,4,1024,32], bias ~N(0,2), keys >= 870 masked (forward only),
                      sigmoid gate from x [1024,1024,128] by a 128x128 weight ~N(0,1/128)
"""

import math

import torch

__all__ = ["attention_inputs", "gate_inputs", "layer_norm_inputs", "gdp_weights",
           "ATTENTION_WORKLOADS", "GATED_ATTENTION_WORKLOADS"]


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def _randn(shape, g, device, std=1.0, mean=0.0):
    t = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        t.mul_(std)
    if mean != 0.0:
        t.add_(mean)
    return t


def attention_inputs(n, h, sq, sk, d, dtype=torch.bfloat16, seed=0, device="cpu",
                     bias_var=1.0, masked_tail=0.0, masked_rows=0, with_dout=True):
    """q, k, v [N,H,S,D], bias [H,Sq,Sk], kmask uint8 [N,Sk], dout [N,H,Sq,D] (or None).

    masked_tail: fraction of trailing keys padded in every row; masked_rows: number of rows
    (chosen by the generator) whose keys are all padded.
    """
    g = _gen(seed, device)
    q = _randn((n, h, sq, d), g, device).to(dtype)
    k = _randn((n, h, sk, d), g, device).to(dtype)
    v = _randn((n, h, sk, d), g, device).to(dtype)
    bias = _randn((h, sq, sk), g, device, std=math.sqrt(bias_var)).to(dtype)
    kmask = torch.ones((n, sk), dtype=torch.uint8, device=device)
    tail = int(round(masked_tail * sk))
    if tail:
        kmask[:, sk - tail:] = 0
    if masked_rows:
        rows = torch.randperm(n, generator=g, device=device)[:masked_rows]
        kmask[rows] = 0
    dout = _randn((n, h, sq, d), g, device).to(dtype) if with_dout else None
    return {"q": q, "k": k, "v": v, "bias": bias, "kmask": kmask, "dout": dout,
            "scale": 1.0 / math.sqrt(d)}


# name -> (N, H, S, D, seed, bias_var, masked_tail, masked_rows, backward?)
ATTENTION_WORKLOADS = {
    "triangle_attn_256": (256, 4, 256, 32, 1, 1.0, 0.10, 0, True),
    "triangle_attn_384": (384, 4, 384, 32, 1, 1.0, 0.10, 0, True),
    "msa_row_attn": (512, 8, 256, 32, 2, 1.0, 0.0, 102, True),
    "triangle_attn_1024": (1024, 4, 1024, 32, 4, 2.0, 0.15, 0, False),
}


def attention_workload(name, dtype=torch.bfloat16, device="cpu", with_dout=None):
    n, h, s, d, seed, bvar, tail, rows, bwd = ATTENTION_WORKLOADS[name]
    return attention_inputs(n, h, s, s, d, dtype, seed, device, bvar, tail, rows,
                            bwd if with_dout is None else with_dout)


# Attention workloads whose output is gated: name -> gate input channels C (the gate maps
# x [N,Sq,C] to H*D columns).
GATED_ATTENTION_WORKLOADS = {"msa_row_attn": 256, "triangle_attn_1024": 128}


def gate_inputs(n, sq, c, hd, dtype=torch.bfloat16, seed=0, device="cpu", bias_std=0.0):
    """x [N,Sq,C] ~N(0,1), wg [C,HD] ~N(0,1/C), bg [HD] ~N(0,bias_std^2): the output gate."""
    g = _gen(seed + 2000, device)
    x = _randn((n, sq, c), g, device).to(dtype)
    wg = _randn((c, hd), g, device, std=1.0 / math.sqrt(c)).to(dtype)
    bg = _randn((hd,), g, device, std=bias_std).to(dtype)
    return x, wg, bg


def layer_norm_inputs(m, c, dtype=torch.bfloat16, seed=3, device="cpu", mask_p=0.95):
    """x, dy [M,C]; LN scale = 1+N(0,0.1), offset ~N(0,0.1) float32; a Bernoulli row mask."""
    g = _gen(seed, device)
    x = _randn((m, c), g, device).to(dtype)
    scale = _randn((c,), g, device, std=math.sqrt(0.1), mean=1.0)
    offset = _randn((c,), g, device, std=math.sqrt(0.1))
    mask = (torch.rand((m,), generator=g, device=device) < mask_p).to(dtype)
    dy = _randn((m, c), g, device).to(dtype)
    return {"x": x, "scale": scale, "offset": offset, "mask": mask, "dy": dy}


def gdp_weights(k, n, dtype=torch.bfloat16, seed=3, device="cpu", bias_std=0.0):
    """(wp, bp, wg, bg): weights ~N(0,1/K) [K,N], biases ~N(0,bias_std^2) [N]."""
    g = _gen(seed + 1000, device)
    wp = _randn((k, n), g, device, std=1.0 / math.sqrt(k)).to(dtype)
    wg = _randn((k, n), g, device, std=1.0 / math.sqrt(k)).to(dtype)
    bp = _randn((n,), g, device, std=bias_std).to(dtype)
    bg = _randn((n,), g, device, std=bias_std).to(dtype)
    return wp, bp, wg, bg
