"""Float64 restatement of LayerNorm over the last axis, forward and backward.

Forward follows cuda/volta_ops.cu:40-58:
  mu = sum(x)/C ; var = E[(x - mu)^2] ; y = (x - mu) * rsqrt(var + eps) * scale[c] + offset[c]
The reference kernel forms var as max(E[x^2] - mu^2, 0) in float32 (volta_ops.cu:53); in
float64 that is the same number as the two-pass form used here up to rounding, and the HIP kernel
uses a Chan/Welford merge, which tracks the two-pass value.

Backward (no reference code), with xhat = (x - mu) * r and g = scale * dy:
  dx = r * (g - mean_c(g) - xhat * mean_c(g * xhat)),
  dscale = sum_m dy * xhat, doffset = sum_m dy.

ln_pair_bias (no reference code: AlphaFold's attention bias from the pair representation, the
step before the reference's attention targets): bias[h, ...] = sum_c LN(z)[..., c] * w[c, h],
the LN(z).w product with the head axis moved first ([H, Sq, Sk], the attention bias layout).
"""

import numpy as np

__all__ = ["layer_norm_fwd", "layer_norm_bwd", "ln_pair_bias"]


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


def ln_pair_bias(z, scale, offset, w, eps=1e-5):
    """[H, ...] float64 for z [..., C] and w [C, H]."""
    z = np.asarray(z, np.float64)
    c = z.shape[-1]
    y, _, _ = layer_norm_fwd(z.reshape(-1, c), scale, offset, eps)
    b = y @ np.asarray(w, np.float64)
    return np.moveaxis(b.reshape(z.shape[:-1] + (b.shape[-1],)), -1, 0)
