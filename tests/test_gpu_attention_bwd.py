"""Attention backward on the GPU against the float64 oracle (through the C ABI)."""
import numpy as np
import pytest
import torch

from _util import TOL, assert_close, dname, np64
from colabfold_legacy_kernels import ops
from colabfold_legacy_kernels.workloads import attention_inputs, attention_workload
from oracle import attention as ref

pytestmark = pytest.mark.gpu

# (N, H, Sq, Sk, D, masked_tail, masked_rows)
CASES = [
    (2, 2, 64, 64, 32, 0.0, 0),
    (3, 2, 100, 77, 32, 0.1, 1),
    (2, 1, 130, 200, 64, 0.2, 0),
    (2, 4, 64, 64, 16, 0.0, 1),
    (2, 2, 48, 40, 8, 0.1, 0),
    (1, 1, 1, 1, 32, 0.0, 0),
    (5, 3, 257, 129, 32, 0.05, 2),
    (2, 2, 33, 300, 64, 0.0, 0),
    (4, 2, 96, 600, 32, 0.1, 1),   # Sk > 384: two key ranges, dQ partials
    (3, 2, 70, 456, 16, 0.1, 1),   # D = 16 over two key ranges
    (2, 1, 16, 8, 8, 0.0, 0),
    (1, 1, 16, 4100, 32, 0.1, 0),  # more than 64 key tiles, ragged last tile
]


def _run(inp, dev):
    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out, lse = ops.attention_fwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"])
    grads = ops.attention_bwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], out, g["dout"], lse,
                              g["scale"])
    return g, out, lse, grads


def _oracle(inp, rows=None):
    sel = slice(None) if rows is None else rows
    return ref.attention_bwd(np64(inp["q"][sel]), np64(inp["k"][sel]), np64(inp["v"][sel]),
                             np64(inp["bias"]), inp["kmask"][sel].cpu().numpy(), inp["scale"],
                             np64(inp["dout"][sel]))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])))
def test_attention_bwd_parity(cuda, case, dtype):
    n, h, sq, sk, d, tail, rows = case
    inp = attention_inputs(n, h, sq, sk, d, dtype, seed=sq * 13 + sk, masked_tail=tail,
                           masked_rows=rows)
    _, _, _, (dq, dk, dv, dbias) = _run(inp, cuda)
    rq, rk, rv, rb = _oracle(inp)
    tol = TOL[dname(dtype)]["grad"]
    assert_close("dQ", dq, rq, tol)
    assert_close("dK", dk, rk, tol)
    assert_close("dV", dv, rv, tol)
    assert_close("dBias", dbias, rb, tol)


@pytest.mark.parametrize("shape", [(3, 2, 100, 130), (2, 2, 200, 384)], ids=str)
def test_attention_bwd_bias_past_float16_range(cuda, shape):
    """bfloat16 biases beyond float16's range (the reference's operand type) stay exact: a query
    row whose bias is -70000 for every key, one key at +70000 and one at -70000 in other rows."""
    n, h, sq, sk = shape
    inp = attention_inputs(n, h, sq, sk, 32, torch.bfloat16, seed=77, masked_tail=0.1)
    b = inp["bias"].float()
    b[0, 5, :] = -70000.0
    b[1, sq - 3, 7] = 70000.0
    b[1, 40, sk // 2] = -70000.0
    inp["bias"] = b.to(torch.bfloat16)
    _, out, lse, (dq, dk, dv, dbias) = _run(inp, cuda)
    for t in (out, lse, dq, dk, dv, dbias):
        assert torch.isfinite(t).all()
    rq, rk, rv, rb = _oracle(inp)
    tol = TOL["bf16"]["grad"]
    assert_close("dQ", dq, rq, tol)
    assert_close("dK", dk, rk, tol)
    assert_close("dV", dv, rv, tol)
    assert_close("dBias", dbias, rb, tol)


# (N, H, Sq, Sk, D, masked_tail, masked_rows): the mask-byte path (Sk % 8 != 0), two key ranges
# (dQ partials), D = 8, 16 and 64 (the D = 64 kernels), rows with no present key.
NSHD_CASES = [(3, 2, 100, 77, 32, 0.1, 1), (4, 2, 96, 600, 32, 0.1, 1),
              (3, 2, 70, 456, 16, 0.1, 1), (2, 1, 130, 200, 64, 0.2, 0),
              (2, 2, 48, 40, 8, 0.1, 0), (3, 4, 64, 128, 32, 0.3, 1)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("case", NSHD_CASES, ids=lambda c: "x".join(map(str, c[:5])))
def test_attention_bwd_nshd_layout(cuda, case, dtype):
    """The [N,S,H,D] backward runs the same kernels with rows H*D apart: dq, dk, dv (in
    [N,S,H,D]) and dbias are bit-identical to the [N,H,S,D] entry on the transposed operands."""
    n, h, sq, sk, d, tail, rows = case
    inp = attention_inputs(n, h, sq, sk, d, dtype, seed=sq * 3 + sk + d, masked_tail=tail,
                           masked_rows=rows)
    g, out, lse, (dq, dk, dv, dbias) = _run(inp, cuda)
    t = lambda x: x.transpose(1, 2).contiguous()  # [N,H,S,D] <-> [N,S,H,D]
    gs = ops.attention_bwd_nshd(t(g["q"]), t(g["k"]), t(g["v"]), g["bias"], g["kmask"], t(out),
                                t(g["dout"]), lse, g["scale"])
    for name, a, b in zip(("dQ", "dK", "dV"), gs[:3], (dq, dk, dv)):
        assert a.shape == (n, b.shape[2], h, d), name
        assert torch.equal(t(a), b), name
    assert torch.equal(gs[3], dbias)


# (N, H, Sq, Sk, D): key counts that fill whole 32-key chunks and ones that end inside a chunk,
# Sk % 8 == 0 (presence words) and not (mask bytes), one and two key ranges.
MIXED_MASK_SHAPES = [(24, 2, 70, 200, 32), (20, 2, 64, 77, 32), (12, 2, 40, 456, 16),
                     (16, 1, 64, 384, 32)]


@pytest.mark.parametrize("shape", MIXED_MASK_SHAPES, ids=lambda c: "x".join(map(str, c)))
def test_attention_bwd_mixed_masks(cuda, shape):
    """Keys absent in every row (a padding tail: their bias is replaced by -inf inside the
    kernel), keys absent in some rows only (random holes: per-score selects), rows with no
    present key, and rows with everything present, all in the blocks of one call."""
    n, h, sq, sk, d = shape
    inp = attention_inputs(n, h, sq, sk, d, torch.bfloat16, seed=sk + n)
    g = torch.Generator().manual_seed(sk * 7 + n)
    km = (torch.rand((n, sk), generator=g) > 0.15).to(torch.uint8)
    tail = sk - sk // 6
    km[:, tail:] = 0
    km[n // 3] = 0
    km[n // 2, :tail] = 1
    km[n - 1, :tail] = 1
    km[n - 1, tail + 1] = 1  # one row reaches into the tail
    inp["kmask"] = km
    _, _, _, (dq, dk, dv, dbias) = _run(inp, cuda)
    rq, rk, rv, rb = _oracle(inp)
    tol = TOL["bf16"]["grad"]
    assert_close("dQ", dq, rq, tol)
    assert_close("dK", dk, rk, tol)
    assert_close("dV", dv, rv, tol)
    assert_close("dBias", dbias, rb, tol)
    absent = (km == 0).nonzero().tolist()
    present_rows = (km != 0).any(dim=1)
    zero_dk = [(i, k) for i, k in absent if present_rows[i]]
    assert all(torch.count_nonzero(dk[i, :, k]).item() == 0 for i, k in zero_dk[:50])


@pytest.mark.parametrize("scale", [-0.17, -1.0 / np.sqrt(32)], ids=lambda s: "%.3f" % s)
@pytest.mark.parametrize("shape", [(3, 2, 100, 77, 32, 0.1), (2, 2, 64, 200, 32, 0.0),
                                   (3, 2, 70, 456, 16, 0.1), (2, 2, 48, 40, 8, 0.1)],
                         ids=lambda c: "x".join(map(str, c[:5])))
def test_attention_bwd_negative_scale(cuda, shape, scale):
    """A negative scale: the keys past Sk (key counts ending inside a 32-key chunk) and the
    masked tail still get P = 0, so no infinity reaches dQ; every gradient against the oracle."""
    n, h, sq, sk, d, tail = shape
    inp = attention_inputs(n, h, sq, sk, d, torch.bfloat16, seed=sk + 5, masked_tail=tail,
                           masked_rows=1)
    inp["scale"] = scale
    _, out, lse, (dq, dk, dv, dbias) = _run(inp, cuda)
    ro, rl = ref.attention_fwd(np64(inp["q"]), np64(inp["k"]), np64(inp["v"]), np64(inp["bias"]),
                               inp["kmask"].numpy(), scale)
    assert_close("O", out, ro, TOL["bf16"]["o"])
    rq, rk, rv, rb = _oracle(inp)
    tol = TOL["bf16"]["grad"]
    assert_close("dQ", dq, rq, tol)
    assert_close("dK", dk, rk, tol)
    assert_close("dV", dv, rv, tol)
    assert_close("dBias", dbias, rb, tol)


def test_attention_bwd_deterministic(cuda):
    inp = attention_inputs(6, 4, 200, 200, 32, torch.bfloat16, seed=21, masked_tail=0.1,
                           masked_rows=1)
    g, out, lse, first = _run(inp, cuda)
    for _ in range(2):
        again = ops.attention_bwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], out, g["dout"],
                                  lse, g["scale"])
        for a, b in zip(first, again):
            assert torch.equal(a, b)


def test_attention_bwd_empty_axes(cuda):
    dt = torch.bfloat16
    for n, h, sq, sk in [(0, 2, 16, 16), (2, 2, 16, 0), (2, 2, 0, 16)]:
        q = torch.randn((n, h, sq, 32), device=cuda).to(dt)
        k = torch.randn((n, h, sk, 32), device=cuda).to(dt)
        bias = torch.randn((h, sq, sk), device=cuda).to(dt)
        km = torch.ones((n, sk), device=cuda, dtype=torch.uint8)
        lse = torch.zeros((n, h, sq), device=cuda)
        dq, dk, dv, db = ops.attention_bwd(q, k, k, bias, km, q, q, lse)
        for t in (dq, dk, dv, db):
            assert torch.count_nonzero(t).item() == 0


def test_attention_bwd_full_triangle_256(cuda):
    """The 256-residue triangle attention: every gradient against the full float64 oracle."""
    inp = attention_workload("triangle_attn_256", torch.bfloat16, device=cuda)
    _, _, _, (dq, dk, dv, dbias) = _run(inp, cuda)
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    rq, rk, rv, rb = _oracle(cpu)
    tol = TOL["bf16"]["grad"]
    assert_close("dQ", dq, rq, tol)
    assert_close("dK", dk, rk, tol)
    assert_close("dV", dv, rv, tol)
    assert_close("dBias", dbias, rb, tol)


@pytest.mark.parametrize("name", ["triangle_attn_384", "msa_row_attn"])
def test_attention_bwd_full_size(cuda, name):
    """The headline workload (N_res = 384, ten row chunks of dBias partials) and MSA row
    attention (512 rows, 102 of them fully padded): every element of dQ, dK, dV and of the
    whole dBias [H,Sq,Sk] against the float64 oracle (which processes rows in chunks, so its
    memory stays bounded). An all-zero or wrongly scaled dBias fails here. Also: the rows of dS
    sum to zero, so sum_k dBias[h,q,k] = 0; a repeated run is bit-identical."""
    inp = attention_workload(name, torch.bfloat16, device=cuda)
    g, out, lse, (dq, dk, dv, dbias) = _run(inp, cuda)
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    rq, rk, rv, rb = _oracle(cpu)
    tol = TOL["bf16"]["grad"]
    padded = (cpu["kmask"] == 0).all(dim=1).nonzero().flatten().tolist()
    if name == "msa_row_attn":
        assert len(padded) == 102
        assert_close("dQ[padded rows]", dq[padded], rq[padded], tol)
        assert_close("dK[padded rows]", dk[padded], rk[padded], tol)
    assert_close("dQ", dq, rq, tol)
    assert_close("dK", dk, rk, tol)
    assert_close("dV", dv, rv, tol)
    assert_close("dBias", dbias, rb, tol)
    row_sum = dbias.double().sum(dim=-1).abs().max().item()
    assert row_sum <= 2e-2 * dbias.double().abs().sum(dim=-1).max().item()
    again = ops.attention_bwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], out, g["dout"], lse,
                              g["scale"])
    assert torch.equal(dbias, again[3]) and torch.equal(dq, again[0])


def test_attention_autograd_function(cuda):
    inp = attention_inputs(2, 2, 64, 64, 32, torch.bfloat16, seed=4, masked_tail=0.1)
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    q, k, v, b = (g[x].clone().requires_grad_(True) for x in ("q", "k", "v", "bias"))
    out = ops.AttentionFunction.apply(q, k, v, b, g["kmask"], g["scale"])
    out.backward(g["dout"])
    rq, rk, rv, rb = _oracle(inp)
    tol = TOL["bf16"]["grad"]
    assert_close("q.grad", q.grad, rq, tol)
    assert_close("bias.grad", b.grad.float(), rb, tol)
    _ = np
