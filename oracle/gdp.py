"""Float64 restatement of the gated dual projection.

gated_dual_proj follows cuda/volta_ops.cu:97 and its epilogue at :185-207 (the same contract as
cuda/volta_gdp_wmma.cu:76-96):
  out[m, n] = mask[m] * (sum_k x[m,k] wp[k,n] + bp[n]) * sigmoid(sum_k x[m,k] wg[k,n] + bg[n])
with wp, wg row-major [K,N], biases [N] and a per-row mask [M]. The bias is added before the
sigmoid, the row mask multiplies last (volta_ops.cu:201-204).

gated_dual_proj_bwd is the derivative of gated_dual_proj (no reference code; the reference is
forward-only): with p = x.wp + bp, s = sigmoid(x.wg + bg),
  dp = dout * mask * s, dg = dout * mask * p * s * (1 - s),
  dx = dp.wp^T + dg.wg^T, dwp = x^T.dp, dwg = x^T.dg, dbp = sum_m dp, dbg = sum_m dg.

ln_gated_dual_proj is the pair-stack use in ColabFold's triangle multiplication: the two GDP
branches a and b read the same LayerNorm(z). The reference runs it as one VoltaLayerNorm call and
two VoltaGdp calls (volta_ops.cu:62-95 then :210-265 twice); here it is their composition.
"""

import numpy as np

from .layer_norm import layer_norm_fwd

__all__ = ["sigmoid", "gated_dual_proj", "ln_gated_dual_proj", "gated_dual_proj_bwd"]


def sigmoid(x):
    x = np.asarray(x, np.float64)
    return 0.5 * (1.0 + np.tanh(0.5 * x))


def gated_dual_proj(x, wp, bp, wg, bg, mask):
    """out [M,N] float64 for x [M,K]."""
    x = np.asarray(x, np.float64)
    p = x @ np.asarray(wp, np.float64) + np.asarray(bp, np.float64)
    g = x @ np.asarray(wg, np.float64) + np.asarray(bg, np.float64)
    return np.asarray(mask, np.float64)[:, None] * p * sigmoid(g)


def ln_gated_dual_proj(z, ln_scale, ln_offset, eps, branch_a, branch_b, mask):
    """(a, b) [M,N] float64. Each branch is a tuple (wp, bp, wg, bg)."""
    y, _, _ = layer_norm_fwd(z, ln_scale, ln_offset, eps)
    a = gated_dual_proj(y, *branch_a, mask)
    b = gated_dual_proj(y, *branch_b, mask)
    return a, b


def gated_dual_proj_bwd(x, wp, bp, wg, bg, mask, dout):
    """(dx [M,K], dwp [K,N], dbp [N], dwg [K,N], dbg [N]) float64."""
    x = np.asarray(x, np.float64)
    wp = np.asarray(wp, np.float64)
    wg = np.asarray(wg, np.float64)
    p = x @ wp + np.asarray(bp, np.float64)
    s = sigmoid(x @ wg + np.asarray(bg, np.float64))
    dm = np.asarray(dout, np.float64) * np.asarray(mask, np.float64)[:, None]
    dp = dm * s
    dg = dm * p * s * (1.0 - s)
    return dp @ wp.T + dg @ wg.T, x.T @ dp, dp.sum(0), x.T @ dg, dg.sum(0)
