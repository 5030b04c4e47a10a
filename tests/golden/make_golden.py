"""Writes the small golden fixtures in this directory from the float64 oracle.

    python tests/golden/make_golden.py

Inputs come from numpy's PCG64 generator (stable across numpy versions) and are rounded to
bf16 once (round-to-nearest-even on the float32 bits), so the fixture holds exactly the values a
bf16 kernel reads. Outputs are the oracle's float64 results. The reference ships no golden vectors
for this path; these fixtures pin the oracle against regressions (tests/test_golden.py) and give
the GPU tests data that does not depend on any generator (tests/test_gpu_golden.py).
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import attention as A  # noqa: E402
from oracle import gdp as G  # noqa: E402
from oracle import layer_norm as L  # noqa: E402


def bf16(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def attention(r):
    n, h, sq, sk, d = 3, 2, 20, 24, 16
    q, k, v = (bf16(r.standard_normal(s)) for s in ((n, h, sq, d), (n, h, sk, d), (n, h, sk, d)))
    bias = bf16(r.standard_normal((h, sq, sk)))
    dout = bf16(r.standard_normal((n, h, sq, d)))
    kmask = np.ones((n, sk), np.uint8)
    kmask[:, sk - 3:] = 0
    kmask[1] = 0
    scale = np.float32(1 / np.sqrt(d))
    o, lse = A.attention_fwd(q, k, v, bias, kmask, scale)
    dq, dk, dv, db = A.attention_bwd(q, k, v, bias, kmask, scale, dout)
    return dict(q=q, k=k, v=v, bias=bias, dout=dout, kmask=kmask, scale=scale, o=o, lse=lse,
                dq=dq, dk=dk, dv=dv, dbias=db)


def layer_norm(r):
    m, c = 10, 128
    x = bf16(r.standard_normal((m, c)) * 2 + 0.5)
    scale = (1 + np.sqrt(0.1) * r.standard_normal(c)).astype(np.float32)
    offset = (np.sqrt(0.1) * r.standard_normal(c)).astype(np.float32)
    dy = bf16(r.standard_normal((m, c)))
    y, _, _ = L.layer_norm_fwd(x, scale, offset, 1e-5)
    dx, ds, do = L.layer_norm_bwd(x, scale, dy, 1e-5)
    return dict(x=x, scale=scale, offset=offset, dy=dy, eps=np.float32(1e-5), y=y, dx=dx,
                dscale=ds, doffset=do)


def weights(r, k, n):
    return (bf16(r.standard_normal((k, n)) / np.sqrt(k)), bf16(0.2 * r.standard_normal(n)),
            bf16(r.standard_normal((k, n)) / np.sqrt(k)), bf16(0.2 * r.standard_normal(n)))


def gdp(r):
    m, k, n = 12, 64, 32
    x = bf16(r.standard_normal((m, k)))
    wp, bp, wg, bg = weights(r, k, n)
    mask = bf16((r.random(m) > 0.2).astype(np.float32))
    out = G.gated_dual_proj(x, wp, bp, wg, bg, mask)
    return dict(x=x, wp=wp, bp=bp, wg=wg, bg=bg, mask=mask, out=out)


def ln_gdp(r):
    m, c, n = 12, 64, 32
    z = bf16(r.standard_normal((m, c)))
    g = (1 + np.sqrt(0.1) * r.standard_normal(c)).astype(np.float32)
    b = (np.sqrt(0.1) * r.standard_normal(c)).astype(np.float32)
    wa, wb = weights(r, c, n), weights(r, c, n)
    mask = bf16((r.random(m) > 0.2).astype(np.float32))
    a, bb = G.ln_gated_dual_proj(z, g, b, 1e-5, wa, wb, mask)
    out = dict(z=z, ln_scale=g, ln_offset=b, mask=mask, a=a, b=bb)
    for name, w in zip(("pa", "ga"), ((wa[0], wa[1]), (wa[2], wa[3]))):
        out["w" + name], out["b" + name] = w
    for name, w in zip(("pb", "gb"), ((wb[0], wb[1]), (wb[2], wb[3]))):
        out["w" + name], out["b" + name] = w
    return out


FIXTURES = {"attention_small": (attention, 101), "layer_norm_small": (layer_norm, 102),
            "gdp_small": (gdp, 103), "ln_gdp_small": (ln_gdp, 104)}


def build(name):
    fn, seed = FIXTURES[name]
    return fn(np.random.default_rng(seed))


def main():
    for name in FIXTURES:
        data = build(name)
        np.savez_compressed(HERE / (name + ".npz"), **data)
        print("wrote", name, sum(np.asarray(v).nbytes for v in data.values()), "bytes")


if __name__ == "__main__":
    main()
