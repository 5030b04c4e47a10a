"""Float64 restatement of the attention output gate.

The reference library has no gate: its attention targets return O (cuda/volta_mma_attn.cu:
256-272) and the caller's jnp Attention module gates it before the output projection
[ColabFold/AlphaFold, not under the reference]:
  gate = sigmoid(x . Wg + bg)   x the query-side input [N, Sq, C], Wg [C, H, D], bg [H, D]
  out  = O^T * gate             O [N, H, Sq, D] seen as [N, Sq, H, D]
Wg and bg are flattened over (H, D) here and the result is [N, Sq, H*D], the layout the output
projection reads. The sigmoid is the reference GDP's (cuda/volta_ops.cu:203), evaluated exactly.

attention_gate_bwd is its derivative (no reference code: the reference has no gate and no
backward): with s = sigmoid(x . Wg + bg) and O' = O^T,
  dO' = dout * s (returned in O's [N, H, Sq, D] layout), dg = dout * O' * s * (1 - s),
  dx = dg . Wg^T, dWg = x^T . dg (over all N * Sq rows), dbg = sum of dg over the rows.

Pinned in tests/test_oracle.py by closed forms that need no formula of this module: Wg = 0 and
bg = 0 give 0.5 * O^T; bg -> +inf gives O^T and bg -> -inf gives 0; a single large weight
Wg[c0, j0] gates column j0 by the sign of x[..., c0] and leaves the rest at 0.5 * O^T. The
backward against torch float64 autograd of the gate written independently, and central finite
differences of attention_gate on a tiny case.
"""

import numpy as np

from .gdp import sigmoid

__all__ = ["attention_gate", "attention_gate_bwd"]


def attention_gate(o, x, wg, bg):
    """out [N, Sq, H*D] float64 for o [N, H, Sq, D], x [N, Sq, C], wg [C, H*D], bg [H*D]."""
    o = np.asarray(o, np.float64)
    n, h, sq, d = o.shape
    g = np.asarray(x, np.float64) @ np.asarray(wg, np.float64) + np.asarray(bg, np.float64)
    return o.transpose(0, 2, 1, 3).reshape(n, sq, h * d) * sigmoid(g)


def attention_gate_bwd(o, x, wg, bg, dout):
    """(do [N, H, Sq, D], dx [N, Sq, C], dwg [C, H*D], dbg [H*D]) float64 for the gradient dout
    [N, Sq, H*D] of attention_gate(o, x, wg, bg)."""
    o = np.asarray(o, np.float64)
    n, h, sq, d = o.shape
    x = np.asarray(x, np.float64)
    wg = np.asarray(wg, np.float64)
    c = x.shape[-1]
    s = sigmoid(x @ wg + np.asarray(bg, np.float64))
    dout = np.asarray(dout, np.float64)
    ot = o.transpose(0, 2, 1, 3).reshape(n, sq, h * d)
    dot = dout * s
    dg = dout * ot * s * (1.0 - s)
    do = dot.reshape(n, sq, h, d).transpose(0, 2, 1, 3)
    x2, dg2 = x.reshape(-1, c), dg.reshape(-1, h * d)
    return do, dg @ wg.T, x2.T @ dg2, dg2.sum(0)
