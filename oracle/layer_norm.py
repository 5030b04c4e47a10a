"""Float64 restatement of LayerNorm over the last axis, forward and backward.

Forward follows cuda/volta_ops.cu:40-58:
  mu = sum(x)/C ; var = E[(x - mu)^2] ; y = (x - mu) * rsqrt(var + eps) * scale[c] + offset[c]
The reference kernel forms var as max(E[x^2] - mu^2, 0) in float32 (volta_ops.cu:53); in
float64 that is the same number as the two-pass form used here up to rounding, and the HIP kernel
uses a Chan/Welford merge, which tracks the two-pass value.

Backward (no reference code), with xhat = (x - mu) * r and g = scale * dy:
  dx = r * (g - mean_c(g) - xhat * mean_c(g * xhat)),
  dscale = sum_m dy * xhat, doffset = sum_m dy.
"""

import numpy as np

__all__ = ["layer_norm_fwd", "layer_norm_bwd"]


def _stats(x, eps):
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    return mu, 1.0 / np.sqrt(var + eps)


def layer_norm_fwd(x, scale, offset, eps=1e-5):
    """y [M,C] float64, plus mean [M] and rstd [M]."""
    x = np.asarray(x, np.float64)
    mu, r = _stats(x, eps)
    y = (x - mu) * r * np.asarray(scale, np.float64) + np.asarray(offset, np.float64)
    return y, mu[..., 0], r[..., 0]


def layer_norm_bwd(x, scale, dy, eps=1e-5):
    """dx [M,C], dscale [C], doffset [C], all float64."""
    x = np.asarray(x, np.float64)
    dy = np.asarray(dy, np.float64)
    mu, r = _stats(x, eps)
    xhat = (x - mu) * r
    g = dy * np.asarray(scale, np.float64)
    dx = r * (g - g.mean(axis=-1, keepdims=True)
              - xhat * (g * xhat).mean(axis=-1, keepdims=True))
    red = tuple(range(x.ndim - 1))
    return dx, (dy * xhat).sum(axis=red), dy.sum(axis=red)
