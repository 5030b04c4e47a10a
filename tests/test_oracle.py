"""Pins the float64 oracle before anything is compared with it.

The reference has no tests, fixtures or golden vectors for this path and its CUDA/CUTLASS/XLA
build cannot run here, so each oracle function is checked against what the mathematics fixes:
  * independent textbook routines in float64 on the CPU: torch scaled_dot_product_attention,
    softmax, layer_norm and torch.autograd;
  * the caller's convention itself: torch float32 autograd of the jnp additive mask
    1e9*(mask-1), which fixes fully masked rows (uniform weights) and their gradients;
  * central finite differences on tiny shapes;
  * closed forms and invariants (Sk = 1 gives V, a row constant in the bias changes nothing,
    key permutations, masked V is ignored, sum_k dBias = 0, sum_c dx = 0, mask = 0 gives 0, ...);
  * a planted mistake (a dropped bias term, a wrong scale) fails the pins.
"""
import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import evoformer as EV
from oracle import gate as GT
from oracle import gdp as G
from oracle import layer_norm as L
from oracle import triangle as TM



def attn_case(seed, n=2, h=3, sq=7, sk=9, d=8, tail=2, empty_row=False):
    r = np.random.default_rng(seed)
    q = r.standard_normal((n, h, sq, d))
    k = r.standard_normal((n, h, sk, d))
    v = r.standard_normal((n, h, sk, d))
    bias = r.standard_normal((h, sq, sk))
    dout = r.standard_normal((n, h, sq, d))
    kmask = np.ones((n, sk), np.uint8)
    if tail:
        kmask[:, sk - tail:] = 0
    if empty_row:
        kmask[0] = 0
    return q, k, v, bias, kmask, dout, 1.0 / np.sqrt(d)


def T(x):
    return torch.tensor(np.asarray(x, np.float64))


# ---- attention forward -----------------------------------------------------------------------

def test_fwd_matches_torch_sdpa():
    q, k, v, bias, kmask, _, scale = attn_case(0)
    o, lse = A.attention_fwd(q, k, v, bias, kmask, scale)
    add = torch.where(T(kmask) == 0, -torch.inf, 0.0)[:, None, None, :]
    mask = T(bias)[None] + add
    ref = torch.nn.functional.scaled_dot_product_attention(T(q), T(k), T(v), attn_mask=mask,
                                                           scale=scale)
    np.testing.assert_allclose(o, ref.numpy(), rtol=1e-12, atol=1e-12)
    logits = scale * T(q) @ T(k).transpose(-1, -2) + mask
    np.testing.assert_allclose(lse, torch.logsumexp(logits, -1).numpy(), rtol=1e-12)


def test_fwd_rows_of_p_sum_to_one():
    q, k, v, bias, kmask, _, scale = attn_case(1, empty_row=True)
    s = A.logits(q, k, bias, kmask, scale)
    _, lse = A.attention_fwd(q, k, v, bias, kmask, scale)
    # float64 holds -1e9 + ln(Sk) to about 1e-7, which bounds the all-masked row
    np.testing.assert_allclose(np.exp(s - lse[..., None]).sum(-1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(np.exp(s[1:] - lse[1:, ..., None]).sum(-1), 1.0, rtol=1e-12)


def test_fully_masked_row_is_uniform_mean_of_v():
    q, k, v, bias, kmask, _, scale = attn_case(2, empty_row=True)
    o, lse = A.attention_fwd(q, k, v, bias, kmask, scale)
    np.testing.assert_allclose(o[0], np.broadcast_to(v[0].mean(axis=1, keepdims=True), o[0].shape),
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse[0], A.MASKED_LOGIT + np.log(k.shape[2]), rtol=1e-15)


def test_fwd_invariants():
    q, k, v, bias, kmask, _, scale = attn_case(3, tail=3)
    o, _ = A.attention_fwd(q, k, v, bias, kmask, scale)
    # a per-row constant added to the bias cancels in the softmax
    shift = np.random.default_rng(9).standard_normal((bias.shape[0], bias.shape[1], 1)) * 5
    o2, _ = A.attention_fwd(q, k, v, bias + shift, kmask, scale)
    np.testing.assert_allclose(o, o2, rtol=1e-10, atol=1e-12)
    # permuting keys (k, v, bias columns and mask together) changes nothing
    perm = np.random.default_rng(10).permutation(k.shape[2])
    o3, _ = A.attention_fwd(q, k[:, :, perm], v[:, :, perm], bias[:, :, perm], kmask[:, perm], scale)
    np.testing.assert_allclose(o, o3, rtol=1e-10, atol=1e-12)
    # values of masked keys are ignored
    v4 = v.copy()
    v4[:, :, kmask[0] == 0] = 1e6
    o4, _ = A.attention_fwd(q, k, v4, bias, kmask, scale)
    np.testing.assert_allclose(o, o4, rtol=1e-10, atol=1e-12)


def test_fwd_special_cases():
    q, k, v, bias, kmask, _, scale = attn_case(4, sk=1, tail=0)
    o, _ = A.attention_fwd(q, k, v, bias, kmask, scale)
    np.testing.assert_allclose(o, np.broadcast_to(v, o.shape), rtol=1e-14)
    q, k, v, bias, kmask, _, scale = attn_case(5, tail=0)
    b = np.full_like(bias, -1e30)
    b[:, :, 4] = 0.0
    o, _ = A.attention_fwd(q, k, v, b, kmask, scale)
    np.testing.assert_allclose(o, np.broadcast_to(v[:, :, 4:5], o.shape), rtol=1e-14)


def test_fwd_brute_force_loops():
    """Scalar loops over one tiny case, no vectorised algebra."""
    q, k, v, bias, kmask, _, scale = attn_case(6, n=1, h=1, sq=3, sk=4, d=2, tail=1)
    o, _ = A.attention_fwd(q, k, v, bias, kmask, scale)
    for i in range(3):
        ws = []
        for j in range(4):
            s = sum(q[0, 0, i, t] * k[0, 0, j, t] for t in range(2)) * scale + bias[0, i, j]
            ws.append(np.exp(s) if kmask[0, j] else 0.0)
        tot = sum(ws)
        for t in range(2):
            assert abs(o[0, 0, i, t] - sum(w * v[0, 0, j, t] for j, w in enumerate(ws)) / tot) < 1e-12


# ---- attention backward ----------------------------------------------------------------------

def torch_attention(q, k, v, bias, kmask, scale, additive_value, dtype):
    tq, tk, tv, tb = (T(a).to(dtype).requires_grad_(True) for a in (q, k, v, bias))
    if additive_value == torch.inf:
        add = torch.where(T(kmask) == 0, -torch.inf, 0.0).to(dtype)[:, None, None, :]
    else:
        add = (T(kmask).to(dtype) - 1.0)[:, None, None, :] * additive_value
    logits = scale * (tq @ tk.transpose(-1, -2)) + tb[None] + add
    o = torch.softmax(logits, -1) @ tv
    return o, (tq, tk, tv, tb)


def test_bwd_matches_torch_autograd_fp64():
    q, k, v, bias, kmask, dout, scale = attn_case(7)
    grads = A.attention_bwd(q, k, v, bias, kmask, scale, dout)
    o, leaves = torch_attention(q, k, v, bias, kmask, scale, torch.inf, torch.float64)
    o.backward(T(dout))
    for g, leaf in zip(grads, leaves):
        np.testing.assert_allclose(g, leaf.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_bwd_matches_jnp_additive_mask_in_float32():
    """The caller adds 1e9*(mask-1) to float32 logits. Autodiff of that, in float32, fixes the
    convention for a fully masked row: uniform P, and dS = P*(dP - D) reaching dQ, dK, dBias."""
    q, k, v, bias, kmask, dout, scale = attn_case(8, empty_row=True)
    grads = A.attention_bwd(q, k, v, bias, kmask, scale, dout)
    o, leaves = torch_attention(q, k, v, bias, kmask, scale, 1e9, torch.float32)
    o.backward(T(dout).float())
    ofwd, _ = A.attention_fwd(q, k, v, bias, kmask, scale)
    np.testing.assert_allclose(ofwd, o.detach().double().numpy(), rtol=2e-5, atol=2e-5)
    for g, leaf in zip(grads, leaves):
        np.testing.assert_allclose(g, leaf.grad.double().numpy(), rtol=1e-4, atol=1e-4)
    assert np.abs(grads[0][0]).max() > 1e-3  # the fully masked row does carry a gradient


def test_bwd_central_finite_differences():
    q, k, v, bias, kmask, dout, scale = attn_case(9, n=1, h=2, sq=4, sk=5, d=3, tail=1)
    grads = A.attention_bwd(q, k, v, bias, kmask, scale, dout)

    def f(qq, kk, vv, bb):
        o, _ = A.attention_fwd(qq, kk, vv, bb, kmask, scale)
        return float((o * dout).sum())

    args = [q, k, v, bias]
    r = np.random.default_rng(0)
    eps = 1e-6
    for which in range(4):
        for _ in range(6):
            idx = tuple(r.integers(0, s) for s in args[which].shape)
            plus = [a.copy() for a in args]
            minus = [a.copy() for a in args]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            fd = (f(*plus) - f(*minus)) / (2 * eps)
            assert abs(fd - grads[which][idx]) < 1e-6 * max(1.0, abs(fd)), (which, idx)


def test_dbias_rows_sum_to_zero():
    q, k, v, bias, kmask, dout, scale = attn_case(10, empty_row=True)
    _, _, _, dbias = A.attention_bwd(q, k, v, bias, kmask, scale, dout)
    assert np.abs(dbias.sum(-1)).max() < 1e-12 * np.abs(dbias).max() * dbias.shape[-1]


def test_chunking_does_not_change_results():
    q, k, v, bias, kmask, dout, scale = attn_case(11, n=5)
    a = A.attention_bwd(q, k, v, bias, kmask, scale, dout, chunk=2)
    b = A.attention_bwd(q, k, v, bias, kmask, scale, dout, chunk=64)
    for x, y in zip(a, b):
        np.testing.assert_allclose(x, y, rtol=1e-13, atol=1e-14)


def test_planted_mistakes_fail_the_pins(monkeypatch):
    """A dropped bias term or a wrong scale in the oracle is caught by the SDPA pin."""
    q, k, v, bias, kmask, _, scale = attn_case(12)
    add = torch.where(T(kmask) == 0, -torch.inf, 0.0)[:, None, None, :]
    ref = torch.nn.functional.scaled_dot_product_attention(
        T(q), T(k), T(v), attn_mask=T(bias)[None] + add, scale=scale).numpy()
    orig = A.logits
    monkeypatch.setattr(A, "logits", lambda q_, k_, b_, m_, s_: orig(q_, k_, 0 * b_, m_, s_))
    o, _ = A.attention_fwd(q, k, v, bias, kmask, scale)
    assert np.abs(o - ref).max() > 1e-2
    monkeypatch.setattr(A, "logits", lambda q_, k_, b_, m_, s_: orig(q_, k_, b_, m_, 1.0))
    o, _ = A.attention_fwd(q, k, v, bias, kmask, scale)
    assert np.abs(o - ref).max() > 1e-2


# ---- LayerNorm ---------------------------------------------------------------------------------

def ln_case(seed, m=11, c=24):
    r = np.random.default_rng(seed)
    return (r.standard_normal((m, c)) * 3 + 1, 1 + r.standard_normal(c) * 0.3,
            r.standard_normal(c) * 0.3, r.standard_normal((m, c)))


def test_layer_norm_matches_torch():
    x, g, b, dy = ln_case(0)
    y, mu, r = L.layer_norm_fwd(x, g, b, 1e-5)
    tx = T(x).requires_grad_(True)
    tg, tb = T(g).requires_grad_(True), T(b).requires_grad_(True)
    ty = torch.nn.functional.layer_norm(tx, (x.shape[1],), tg, tb, 1e-5)
    np.testing.assert_allclose(y, ty.detach().numpy(), rtol=1e-12, atol=1e-12)
    ty.backward(T(dy))
    dx, dg, db = L.layer_norm_bwd(x, g, dy, 1e-5)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dg, tg.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(db, tb.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_layer_norm_invariants():
    x, g, b, dy = ln_case(1, m=7, c=128)
    y, _, _ = L.layer_norm_fwd(x, np.ones(128), np.zeros(128), 0.0)
    np.testing.assert_allclose(y.mean(1), 0, atol=1e-12)
    np.testing.assert_allclose(y.var(1), 1, rtol=1e-12)
    dx, _, db = L.layer_norm_bwd(x, g, dy, 1e-5)
    np.testing.assert_allclose(dx.sum(1), 0, atol=1e-10)
    np.testing.assert_allclose(db, dy.sum(0), rtol=1e-14)


def test_layer_norm_finite_differences():
    x, g, b, dy = ln_case(2, m=3, c=6)
    dx, dg, _ = L.layer_norm_bwd(x, g, dy, 1e-5)
    f = lambda xx, gg: float((L.layer_norm_fwd(xx, gg, b, 1e-5)[0] * dy).sum())  # noqa: E731
    eps = 1e-6
    for i in range(3):
        for j in range(6):
            xp, xm = x.copy(), x.copy()
            xp[i, j] += eps
            xm[i, j] -= eps
            assert abs((f(xp, g) - f(xm, g)) / (2 * eps) - dx[i, j]) < 1e-6
    for j in range(6):
        gp, gm = g.copy(), g.copy()
        gp[j] += eps
        gm[j] -= eps
        assert abs((f(x, gp) - f(x, gm)) / (2 * eps) - dg[j]) < 1e-6


# ---- gated dual projection ---------------------------------------------------------------------

def gdp_case(seed, m=9, k=16, n=8):
    r = np.random.default_rng(seed)
    return (r.standard_normal((m, k)), r.standard_normal((k, n)) / 4, r.standard_normal(n),
            r.standard_normal((k, n)) / 4, r.standard_normal(n), (r.random(m) > 0.3).astype(float))


def test_gdp_matches_torch():
    x, wp, bp, wg, bg, mask = gdp_case(0)
    out = G.gated_dual_proj(x, wp, bp, wg, bg, mask)
    ref = T(mask)[:, None] * (T(x) @ T(wp) + T(bp)) * torch.sigmoid(T(x) @ T(wg) + T(bg))
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-12, atol=1e-14)


def test_gdp_special_cases():
    x, wp, bp, wg, bg, mask = gdp_case(1)
    assert not G.gated_dual_proj(x, wp, bp, wg, bg, np.zeros_like(mask)).any()
    one = np.ones_like(mask)
    lin = x @ wp + bp
    np.testing.assert_allclose(G.gated_dual_proj(x, wp, bp, 0 * wg, 0 * bg, one), 0.5 * lin,
                               rtol=1e-14)
    np.testing.assert_allclose(G.gated_dual_proj(x, wp, bp, 0 * wg, 0 * bg + 60, one), lin,
                               rtol=1e-14)


def test_ln_gdp_is_the_composition():
    x, g, b, _ = ln_case(3, m=9, c=16)
    _, wp, bp, wg, bg, mask = gdp_case(4, m=9, k=16, n=8)
    a, bb = G.ln_gated_dual_proj(x, g, b, 1e-5, (wp, bp, wg, bg), (wg, bg, wp, bp), mask)
    y = torch.nn.functional.layer_norm(T(x), (16,), T(g), T(b), 1e-5)
    ref_a = T(mask)[:, None] * (y @ T(wp) + T(bp)) * torch.sigmoid(y @ T(wg) + T(bg))
    np.testing.assert_allclose(a, ref_a.numpy(), rtol=1e-12, atol=1e-14)
    ref_b = T(mask)[:, None] * (y @ T(wg) + T(bg)) * torch.sigmoid(y @ T(wp) + T(bp))
    np.testing.assert_allclose(bb, ref_b.numpy(), rtol=1e-12, atol=1e-14)


def gate_case(seed, n=2, h=3, sq=5, d=4, c=6):
    r = np.random.default_rng(seed)
    return (r.standard_normal((n, h, sq, d)), r.standard_normal((n, sq, c)),
            r.standard_normal((c, h * d)), r.standard_normal(h * d))


def test_gate_closed_forms():
    """Closed forms fixed by the definition alone: a zero gate pre-activation halves the
    transposed O, saturated biases pass it or zero it, and one large weight gates a single
    column by the sign of one input channel (which pins the orientation of wg and of the
    [N,H,Sq,D] -> [N,Sq,H*D] transpose)."""
    o, x, wg, bg = gate_case(0)
    n, h, sq, d = o.shape
    ot = np.stack([np.concatenate([o[b, hh, s] for hh in range(h)]) for b in range(n)
                   for s in range(sq)]).reshape(n, sq, h * d)
    np.testing.assert_array_equal(GT.attention_gate(o, x, 0 * wg, 0 * bg), 0.5 * ot)
    np.testing.assert_array_equal(GT.attention_gate(o, x, 0 * wg, 0 * bg + 800), ot)
    assert not GT.attention_gate(o, x, 0 * wg, 0 * bg - 800).any()
    w1 = np.zeros_like(wg)
    c0, j0 = 4, 7
    w1[c0, j0] = 1e4
    out = GT.attention_gate(o, x, w1, 0 * bg)
    want = 0.5 * ot
    want[..., j0] = ot[..., j0] * (x[..., c0] > 0)
    np.testing.assert_allclose(out, want, rtol=0, atol=1e-300)


def test_gate_matches_torch():
    o, x, wg, bg = gate_case(1, n=3, h=2, sq=4, d=8, c=5)
    ref = T(o).permute(0, 2, 1, 3).reshape(3, 4, 16) * torch.sigmoid(
        torch.einsum("nsc,cj->nsj", T(x), T(wg)) + T(bg))
    np.testing.assert_allclose(GT.attention_gate(o, x, wg, bg), ref.numpy(), rtol=1e-13,
                               atol=1e-15)


def test_gate_bwd_matches_torch_autograd():
    """The gate's backward against float64 autograd of the gate written out in torch (per-head
    einsum form, no transpose shared with the oracle)."""
    n, h, sq, d, c = 2, 3, 5, 4, 6
    o, x, wg, bg = gate_case(12, n=n, h=h, sq=sq, d=d, c=c)
    dout = np.random.default_rng(13).standard_normal((n, sq, h * d))
    to, tx, twg, tbg = (T(a).requires_grad_() for a in (o, x, wg, bg))
    gate = torch.sigmoid(torch.einsum("nsc,chd->nshd", tx, twg.reshape(c, h, d)) +
                         tbg.reshape(h, d))
    out = torch.einsum("nhsd,nshd->nshd", to, gate).reshape(n, sq, h * d)
    out.backward(T(dout))
    got = GT.attention_gate_bwd(o, x, wg, bg, dout)
    for name, a, b in zip(("do", "dx", "dwg", "dbg"), got,
                          (to.grad, tx.grad, twg.grad, tbg.grad)):
        assert a.shape == tuple(b.shape), name
        np.testing.assert_allclose(a, b.numpy(), rtol=1e-12, atol=1e-13, err_msg=name)


def test_gate_bwd_central_finite_differences():
    """Every gradient of the gate's backward against central differences of attention_gate."""
    o, x, wg, bg = gate_case(14, n=1, h=2, sq=3, d=2, c=3)
    dout = np.random.default_rng(15).standard_normal((1, 3, 4))
    grads = GT.attention_gate_bwd(o, x, wg, bg, dout)

    def f(oo, xx, ww, bb):
        return float((GT.attention_gate(oo, xx, ww, bb) * dout).sum())

    args = [o, x, wg, bg]
    r = np.random.default_rng(16)
    eps = 1e-6
    for which in range(4):
        for _ in range(5):
            idx = tuple(r.integers(0, s) for s in args[which].shape)
            plus = [a.copy() for a in args]
            minus = [a.copy() for a in args]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            fd = (f(*plus) - f(*minus)) / (2 * eps)
            assert abs(fd - grads[which][idx]) < 1e-7 * max(1.0, abs(fd)), (which, idx)


def test_pair_block_composes_the_ops():
    r = np.random.default_rng(5)
    z = r.standard_normal((6, 6, 16))
    g, b = 1 + 0.3 * r.standard_normal(16), 0.3 * r.standard_normal(16)
    br = tuple(r.standard_normal(s) / 4 for s in ((16, 16), (16,), (16, 16), (16,)))
    wb = r.standard_normal((16, 2)) / 4
    wq, wk, wv = (r.standard_normal((16, 8)) / 4 for _ in range(3))
    out = EV.pair_block_fwd(z, g, b, 1e-5, br, br, wb, wq, wk, wv, heads=2, head_dim=4)
    y = torch.nn.functional.layer_norm(T(z), (16,), T(g), T(b), 1e-5)
    bias = (y @ T(wb)).permute(2, 0, 1)
    heads = lambda w: (y @ T(w)).reshape(6, 6, 2, 4).permute(0, 2, 1, 3)  # noqa: E731
    ref = torch.nn.functional.scaled_dot_product_attention(heads(wq), heads(wk), heads(wv),
                                                           attn_mask=bias[None], scale=0.5)
    np.testing.assert_allclose(out["o"], ref.numpy(), rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(out["a"], out["b"], rtol=0, atol=0)


# ---- triangle multiplication -------------------------------------------------------------------

def test_triangle_einsum_matches_torch():
    r = np.random.default_rng(3)
    a, b = r.standard_normal((5, 6, 3)), r.standard_normal((5, 6, 3))
    out = TM.pair_einsum(a[:, :5], b[:, :5], outgoing=True)
    ref = torch.einsum("ikc,jkc->ijc", T(a[:, :5]), T(b[:, :5]))
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-13, atol=1e-14)
    a, b = r.standard_normal((6, 6, 3)), r.standard_normal((6, 6, 3))
    out = TM.pair_einsum(a, b, outgoing=False)
    ref = torch.einsum("kjc,kic->ijc", T(a), T(b))
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-13, atol=1e-14)
    ac, bc = r.standard_normal((2, 7, 9)), r.standard_normal((2, 5, 9))
    np.testing.assert_allclose(TM.einsum(ac, bc), torch.einsum("cik,cjk->cij", T(ac), T(bc)),
                               rtol=1e-13, atol=1e-14)


def test_triangle_einsum_closed_forms():
    """b = 1 turns the contraction into row sums of a; permuting k in both changes nothing."""
    r = np.random.default_rng(4)
    a = r.standard_normal((7, 7, 2))
    ones = np.ones_like(a)
    out = TM.pair_einsum(a, ones, outgoing=True)
    np.testing.assert_allclose(out, np.repeat(a.sum(1)[:, None, :], 7, axis=1), rtol=1e-13)
    out = TM.pair_einsum(ones, a, outgoing=False)   # x[i,j] = sum_k right[k,i]
    np.testing.assert_allclose(out, np.repeat(a.sum(0)[:, None, :], 7, axis=1), rtol=1e-13)
    b = r.standard_normal((7, 7, 2))
    p = r.permutation(7)
    np.testing.assert_allclose(TM.pair_einsum(a[:, p], b[:, p]), TM.pair_einsum(a, b),
                               rtol=1e-12, atol=1e-13)


def test_triangle_multiply_matches_torch():
    """The whole module against an independent torch float64 statement of AlphaFold's
    TriangleMultiplication (layer_norm, linear layers, sigmoid gates, einsum)."""
    r = np.random.default_rng(5)
    n, c = 6, 4
    z = r.standard_normal((n, n, c))
    mask = (r.random((n, n)) > 0.2).astype(np.float64)
    ln_in = (1 + 0.1 * r.standard_normal(c), 0.1 * r.standard_normal(c))
    ln_c = (1 + 0.1 * r.standard_normal(c), 0.1 * r.standard_normal(c))
    ws = [r.standard_normal((c, c)) / 2 for _ in range(6)]
    bs = [r.standard_normal(c) / 2 for _ in range(6)]
    F = torch.nn.functional
    for outgoing, eq in ((True, "ikc,jkc->ijc"), (False, "kjc,kic->ijc")):
        y = F.layer_norm(T(z), (c,), T(ln_in[0]), T(ln_in[1]), 1e-5)
        m = T(mask)[..., None]
        left = m * (y @ T(ws[0]) + T(bs[0])) * torch.sigmoid(y @ T(ws[2]) + T(bs[2]))
        right = m * (y @ T(ws[1]) + T(bs[1])) * torch.sigmoid(y @ T(ws[3]) + T(bs[3]))
        x = F.layer_norm(torch.einsum(eq, left, right), (c,), T(ln_c[0]), T(ln_c[1]), 1e-5)
        ref = (x @ T(ws[4]) + T(bs[4])) * torch.sigmoid(y @ T(ws[5]) + T(bs[5]))
        out = TM.triangle_multiply(z, mask, ln_in, ws, bs, ln_c, outgoing)
        np.testing.assert_allclose(out, ref.numpy(), rtol=1e-12, atol=1e-13)


def test_triangle_multiply_at_matches_the_whole_grid():
    """The position-sampled statement equals the whole-grid one at every position, both
    directions (a swapped i/j, row/column or left/right fails it: the module is not symmetric)."""
    r = np.random.default_rng(9)
    n, c = 7, 5
    z = r.standard_normal((n, n, c))
    mask = (r.random((n, n)) > 0.2).astype(np.float64)
    ln_in = (1 + 0.1 * r.standard_normal(c), 0.1 * r.standard_normal(c))
    ln_c = (1 + 0.1 * r.standard_normal(c), 0.1 * r.standard_normal(c))
    ws = [r.standard_normal((c, c)) / 2 for _ in range(6)]
    bs = [r.standard_normal(c) / 2 for _ in range(6)]
    line = lambda kind, i: (z[i], mask[i]) if kind == "row" else (z[:, i], mask[:, i])  # noqa
    pos = [(i, j) for i in range(n) for j in range(n)]
    for outgoing in (True, False):
        full = TM.triangle_multiply(z, mask, ln_in, ws, bs, ln_c, outgoing)
        at = TM.triangle_multiply_at(line, ln_in, ws, bs, ln_c, pos, outgoing)
        np.testing.assert_allclose(at, full.reshape(n * n, c), rtol=1e-12, atol=1e-13)


def test_ln_pair_bias_matches_torch_and_pair_block():
    """LN(z).w with the head axis first: an independent torch float64 einsum, and the bias that
    the pair micro-block composes (evoformer.pair_block_fwd)."""
    r = np.random.default_rng(6)
    z = r.standard_normal((5, 7, 16))
    g, b = 1 + 0.1 * r.standard_normal(16), 0.1 * r.standard_normal(16)
    w = r.standard_normal((16, 4))
    out = L.ln_pair_bias(z, g, b, w, 1e-5)
    y = torch.nn.functional.layer_norm(T(z), (16,), T(g), T(b), 1e-5)
    np.testing.assert_allclose(out, torch.einsum("qkc,ch->hqk", y, T(w)).numpy(), rtol=1e-12,
                               atol=1e-13)
    assert out.shape == (4, 5, 7)


def test_gdp_bwd_matches_torch_autograd():
    x, wp, bp, wg, bg, mask = gdp_case(8, m=9, k=12, n=7)
    r = np.random.default_rng(9)
    dout = r.standard_normal((9, 7))
    tx, twp, tbp, twg, tbg = (T(a).requires_grad_() for a in (x, wp, bp, wg, bg))
    out = T(mask)[:, None] * (tx @ twp + tbp) * torch.sigmoid(tx @ twg + tbg)
    out.backward(T(dout))
    got = G.gated_dual_proj_bwd(x, wp, bp, wg, bg, mask, dout)
    for a, b in zip(got, (tx.grad, twp.grad, tbp.grad, twg.grad, tbg.grad)):
        np.testing.assert_allclose(a, b.numpy(), rtol=1e-12, atol=1e-13)
