"""Float64 restatement of the attention output gate.

The reference library has no gate: its attention targets return O (cuda/volta_mma_attn.cu:
256-272) and the caller's jnp Attention module gates it before the output projection
[ColabFold/AlphaFold, not under the reference]:
  gate = sigmoid(x . Wg + bg)   x the query-side input [N, Sq, C], Wg [C, H, D], bg [H, D]
  out  = O^T * gate             O [N, H, Sq, D] seen as [N, Sq, H, D]
Wg and bg are flattened over (H, D) here and the result is [N, Sq, H*D], the layout the output
projection reads. The sigmoid is the reference GDP's (cuda/volta_ops.cu:203), evaluated exactly.

Pinned in tests/test_oracle.py by closed forms that need no formula of this module: Wg = 0 and
bg = 0 give 0.5 * O^T; bg -> +inf gives O^T and bg -> -inf gives 0; a single large weight
Wg[c0, j0] gates column j0 by the sign of x[..., c0] and leaves the rest at 0.5 * O^T.
"""

import numpy as np

from .gdp import sigmoid

__all__ = ["attention_gate"]


def attention_gate(o, x, wg, bg):
    """out [N, Sq, H*D] float64 for o [N, H, Sq, D], x [N, Sq, C], wg [C, H*D], bg [H*D]."""
    o = np.asarray(o, np.float64)
    n, h, sq, d = o.shape
    g = np.asarray(x, np.float64) @ np.asarray(wg, np.float64) + np.asarray(bg, np.float64)
    return o.transpose(0, 2, 1, 3).reshape(n, sq, h * d) * sigmoid(g)
