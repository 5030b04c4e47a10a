"""Float64 restatement of attention with a per-head pair bias and a per-row key mask.

Forward (follows cuda/volta_mma_attn.cu):
  * logits = scale * (q . k) + bias              -- scale on Q.K^T only, bias added unscaled
                                                    (volta_mma_attn.cu:137,189-190)
  * a key with kmask == 0 gets a fixed logit     -- volta_mma_attn.cu:186-188 replaces the
                                                    logit by a constant (-1e4 there)
  * softmax over keys, O = P . V                  -- online form at volta_mma_attn.cu:204-231,
                                                    normalised by 1/max(l, 1e-30) at :265
Mask convention. The ColabFold caller adds ``1e9 * (mask - 1)`` to float32 logits. In float32 the
score and bias of a masked key are far below the rounding unit of 1e9 (64), so the masked logit
IS the constant -1e9, and a fully masked row gets uniform weights over its Sk keys. The
derivative of the additive form is 1 for every key, so the gradient of a masked logit is the
ordinary dS = P * (dP - D) and it reaches dQ, dK and dBias. This module states exactly that:
``MASKED_LOGIT`` replaces the logit, and the backward differentiates through every position.
For rows with at least one unmasked key this equals the reference kernel's output (its -1e4
constant and this -1e9 both give P = 0 to float precision); for fully masked rows it is the
jnp value mean(V) (the reference kernel divides by the tile-padded key count instead).

Backward (no reference code; the reference is forward-only):
  D = rowsum(dO * O), dS = P * (dO . V^T - D),
  dQ = scale * dS . K, dK = scale * dS^T . Q, dV = P^T . dO, dBias[h] = sum_n dS[n, h].
"""

import numpy as np

MASKED_LOGIT = -1.0e9

__all__ = ["MASKED_LOGIT", "logits", "attention_fwd", "attention_bwd"]


def _f64(x):
    return np.asarray(x, dtype=np.float64)


def _valid(kmask, n, sk):
    if kmask is None:
        return np.ones((n, sk), dtype=bool)
    return np.asarray(kmask) != 0


def logits(q, k, bias, kmask, scale):
    """Masked logits [N,H,Sq,Sk] in float64 (volta_mma_attn.cu:185-192)."""
    q, k, bias = _f64(q), _f64(k), _f64(bias)
    s = np.einsum("nhqd,nhkd->nhqk", q, k) * scale + bias[None]
    valid = _valid(kmask, q.shape[0], k.shape[2])[:, None, None, :]
    return np.where(valid, s, MASKED_LOGIT)


def _softmax(s):
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    return e / l, (m + np.log(l))[..., 0]


def _chunks(n, chunk):
    step = max(1, int(chunk))
    for a in range(0, n, step):
        yield a, min(n, a + step)


def attention_fwd(q, k, v, bias, kmask, scale, chunk=64):
    """O [N,H,Sq,D] and the natural-log row logsumexp [N,H,Sq], both float64.

    q [N,H,Sq,D]; k, v [N,H,Sk,D]; bias [H,Sq,Sk]; kmask [N,Sk] (nonzero = key present) or None.
    Rows N are processed ``chunk`` at a time to bound memory.
    """
    q, k, v, bias = _f64(q), _f64(k), _f64(v), _f64(bias)
    n, h, sq, d = q.shape
    o = np.empty((n, h, sq, v.shape[3]))
    lse = np.empty((n, h, sq))
    km = None if kmask is None else np.asarray(kmask)
    for a, b in _chunks(n, chunk):
        s = logits(q[a:b], k[a:b], bias, None if km is None else km[a:b], scale)
        p, lse[a:b] = _softmax(s)
        o[a:b] = p @ v[a:b]
    return o, lse


def attention_bwd(q, k, v, bias, kmask, scale, dout, chunk=64):
    """dQ, dK, dV [as inputs] and dBias [H,Sq,Sk], all float64.

    P is recomputed from the inputs; D = rowsum(dO * O) uses the exact O, so D = sum_k P * dP.
    """
    q, k, v, bias, dout = _f64(q), _f64(k), _f64(v), _f64(bias), _f64(dout)
    n = q.shape[0]
    dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    dbias = np.zeros(bias.shape)
    km = None if kmask is None else np.asarray(kmask)
    for a, b in _chunks(n, chunk):
        s = logits(q[a:b], k[a:b], bias, None if km is None else km[a:b], scale)
        p, _ = _softmax(s)
        o = p @ v[a:b]
        dp = dout[a:b] @ np.swapaxes(v[a:b], -1, -2)
        dvec = (dout[a:b] * o).sum(axis=-1, keepdims=True)
        ds = p * (dp - dvec)
        dq[a:b] = scale * (ds @ k[a:b])
        dk[a:b] = scale * (np.swapaxes(ds, -1, -2) @ q[a:b])
        dv[a:b] = np.swapaxes(p, -1, -2) @ dout[a:b]
        dbias += ds.sum(axis=0)
    return dq, dk, dv, dbias
