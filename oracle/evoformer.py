"""Float64 pair micro-block built from the three hot-path ops (forward only).

  y      = LayerNorm(z)                                     [I*J, C]
  a, b   = gated_dual_proj(y, branch_a), (y, branch_b)      [I*J, C]  (triangle-multiply inputs)
  bias   = (y @ w_bias) as [H, J, K]                        pair bias of triangle-start attention
  q,k,v  = (y @ w_q|w_k|w_v) as [I, H, J, D]                one attention per row i
  o      = attention(q, k, v, bias, kmask, 1/sqrt(D))

This composes oracle.layer_norm, oracle.gdp and oracle.attention exactly as the ColabFold pair
stack calls VoltaLayerNorm, VoltaGdp and VoltaMma (cuda/volta_ops.cu:87-95, :254-265,
cuda/volta_mma_attn.cu:338-351); the projections between them are plain matmuls of the caller.
"""

import numpy as np

from .attention import attention_fwd
from .gdp import gated_dual_proj
from .layer_norm import layer_norm_fwd

__all__ = ["pair_block_fwd"]


def pair_block_fwd(z, ln_scale, ln_offset, eps, branch_a, branch_b, w_bias, w_q, w_k, w_v,
                   heads, head_dim, kmask=None):
    """Returns dict with y, a, b, bias, q, k, v, o (all float64)."""
    z = np.asarray(z, np.float64)
    ni, nj, c = z.shape
    y, _, _ = layer_norm_fwd(z.reshape(ni * nj, c), ln_scale, ln_offset, eps)
    ones = np.ones(ni * nj)
    a = gated_dual_proj(y, *branch_a, ones)
    b = gated_dual_proj(y, *branch_b, ones)
    bias = (y @ np.asarray(w_bias, np.float64)).reshape(ni, nj, heads).transpose(2, 0, 1)

    def heads_first(w):
        t = (y @ np.asarray(w, np.float64)).reshape(ni, nj, heads, head_dim)
        return t.transpose(0, 2, 1, 3)

    q, k, v = heads_first(w_q), heads_first(w_k), heads_first(w_v)
    o, lse = attention_fwd(q, k, v, bias, kmask, 1.0 / np.sqrt(head_dim))
    return {"y": y, "a": a, "b": b, "bias": bias, "q": q, "k": k, "v": v, "o": o, "lse": lse}
