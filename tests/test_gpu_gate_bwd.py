"""Backward of the gated attention output on the GPU against the float64 oracle: parity over every
supported (C, H*D) pair, ragged row counts and many tiles per block, exact special cases that pin
the layouts, dx accumulation, repeatability and the MSA-size workload; and gated attention's
whole forward + backward through ops.GatedAttentionFunction against the oracle's composition
(attention, gate, gate backward, attention backward)."""
import pytest
import torch

from _util import TOL, assert_close, dname, np64
from colabfold_legacy_kernels import ops
from colabfold_legacy_kernels.workloads import attention_inputs, gate_inputs
from oracle import attention as ref_attn
from oracle import gate as ref

pytestmark = pytest.mark.gpu

# (N, H, Sq, D, C): every (C, H*D) pair of {64, 128, 256}, with ragged query counts (not
# multiples of the 64-row tile, one row) and the head dims the forward gate takes.
GATE_BWD_SHAPES = [(2, 8, 70, 32, 256), (3, 4, 64, 32, 128), (1, 8, 33, 8, 64),
                   (2, 4, 45, 32, 64), (1, 8, 66, 32, 64), (2, 2, 90, 32, 128),
                   (2, 8, 40, 32, 128), (1, 4, 100, 32, 256), (1, 4, 200, 16, 256),
                   (3, 2, 1, 32, 64), (1, 2, 130, 64, 128)]


def case(n, h, sq, d, c, dtype, seed, dev, bias_std=0.5):
    g = torch.Generator().manual_seed(seed)
    o = torch.randn((n, h, sq, d), generator=g)
    x = torch.randn((n, sq, c), generator=g)
    wg = torch.randn((c, h * d), generator=g) / c ** 0.5
    bg = torch.randn((h * d,), generator=g) * bias_std
    dout = torch.randn((n, sq, h * d), generator=g)
    return [t.to(dtype).to(dev) for t in (o, x, wg, bg, dout)]


def check(got, o, x, wg, bg, dout, tol):
    r = ref.attention_gate_bwd(np64(o), np64(x), np64(wg), np64(bg), np64(dout))
    for name, a, b in zip(("do", "dx", "dwg", "dbg"), got, r):
        assert_close(name, a, b, tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("n,h,sq,d,c", GATE_BWD_SHAPES)
def test_gate_bwd_parity(cuda, n, h, sq, d, c, dtype):
    t = case(n, h, sq, d, c, dtype, n * 1000 + sq + c + h * d, cuda)
    check(ops.attention_gate_bwd(*t), *t, TOL[dname(dtype)]["grad"])


# Enough 64-row tiles that every block of the recompute kernel runs several (256 blocks at
# C = 256, 768 at C = 128) and each weight-gradient block sums a run of tiles.
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("n,h,sq,d,c", [(773, 8, 64, 32, 256), (1100, 4, 64, 32, 128),
                                        (301, 4, 100, 32, 256), (517, 8, 33, 8, 128)])
def test_gate_bwd_many_tiles(cuda, n, h, sq, d, c, dtype):
    t = case(n, h, sq, d, c, dtype, n + c, cuda)
    check(ops.attention_gate_bwd(*t), *t, TOL[dname(dtype)]["grad"])


def test_gate_bwd_exact_cases(cuda):
    """A zero gate pre-activation gives do = dout / 2 exactly and no dx; a saturated positive
    bias gives do = dout exactly and no other gradient; a saturated negative one gives zeros.
    do lands in o's [N,H,Sq,D] layout."""
    n, h, sq, d, c = 2, 8, 70, 32, 256
    o, x, wg, bg, dout = case(n, h, sq, d, c, torch.bfloat16, 5, cuda)
    dt = dout.reshape(n, sq, h, d).permute(0, 2, 1, 3)
    z = torch.zeros_like(wg)
    do, dx, dwg, dbg = ops.attention_gate_bwd(o, x, z, torch.zeros_like(bg), dout)
    assert torch.equal(do, 0.5 * dt)
    assert torch.count_nonzero(dx) == 0
    do, dx, dwg, dbg = ops.attention_gate_bwd(o, x, z, torch.full_like(bg, 100.0), dout)
    assert torch.equal(do, dt)
    for g in (dx, dwg, dbg):
        assert torch.count_nonzero(g) == 0
    do, dx, dwg, dbg = ops.attention_gate_bwd(o, x, z, torch.full_like(bg, -100.0), dout)
    for g in (do, dx, dwg, dbg):
        assert torch.count_nonzero(g) == 0


def test_gate_bwd_accumulates_dx(cuda):
    """dx added into an existing gradient (x also feeds the q, k, v projections)."""
    n, h, sq, d, c = 3, 4, 64, 32, 128
    o, x, wg, bg, dout = case(n, h, sq, d, c, torch.bfloat16, 21, cuda)
    prev = torch.randn((n, sq, c), generator=torch.Generator().manual_seed(22)).to(x)
    dx = prev.clone()
    ops.attention_gate_bwd(o, x, wg, bg, dout, dx=dx)
    r = ref.attention_gate_bwd(np64(o), np64(x), np64(wg), np64(bg), np64(dout))
    assert_close("dx+prev", dx, r[1] + np64(prev), TOL["bf16"]["grad"])


def test_gate_bwd_no_rows(cuda):
    """N = 0: dwg and dbg are sums over no rows, zero even where their buffers held values."""
    h, sq, d, c = 8, 16, 32, 256
    o = torch.empty((0, h, sq, d), device=cuda, dtype=torch.bfloat16)
    x = torch.empty((0, sq, c), device=cuda, dtype=torch.bfloat16)
    wg = torch.randn((c, h * d), device=cuda).to(torch.bfloat16)
    bg = torch.randn((h * d,), device=cuda).to(torch.bfloat16)
    dout = torch.empty((0, sq, h * d), device=cuda, dtype=torch.bfloat16)
    junk = [torch.full((c * h * d,), 7.0, device=cuda) for _ in range(4)]
    del junk  # the gradients below reuse these nonzero blocks
    do, dx, dwg, dbg = ops.attention_gate_bwd(o, x, wg, bg, dout)
    assert do.shape == o.shape and dx.shape == x.shape
    assert torch.count_nonzero(dwg) == 0 and torch.count_nonzero(dbg) == 0


def test_gate_bwd_msa_workload(cuda):
    """MSA row attention's gate (N=512 rows, 256 queries, 8 x 32 heads on 256 channels): the
    full gradients against the oracle, and two calls bit-identical."""
    n, h, sq, d, c = 512, 8, 256, 32, 256
    t = case(n, h, sq, d, c, torch.bfloat16, 9, cuda)
    a = ops.attention_gate_bwd(*t)
    b = ops.attention_gate_bwd(*t)
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    check(a, *t, TOL["bf16"]["grad"])


def test_gate_bwd_beyond_one_gib(cuda):
    """N = 8200 MSA rows of 256 queries, 8 x 32 heads on 256 channels: each operand 1.07 GB, past
    2^30 bytes. Sampled samples' do and dx at the start, around the 2^30-byte point and at the
    end against the oracle, and dwg, dbg against the oracle summed over sample chunks."""
    n, h, sq, d, c = 8200, 8, 256, 32, 256
    dt = torch.bfloat16
    g = torch.Generator(device=cuda).manual_seed(51)
    o = torch.randn((n, h, sq, d), generator=g, device=cuda).to(dt)
    x = torch.randn((n, sq, c), generator=g, device=cuda).to(dt)
    wg = (torch.randn((c, h * d), generator=g, device=cuda) / c ** 0.5).to(dt)
    bg = (0.5 * torch.randn((h * d,), generator=g, device=cuda)).to(dt)
    dout = torch.randn((n, sq, h * d), generator=g, device=cuda).to(dt)
    do, dx, dwg, dbg = ops.attention_gate_bwd(o, x, wg, bg, dout)
    wn, bn = np64(wg), np64(bg)
    tol = TOL["bf16"]["grad"]
    mid = (1 << 30) // (sq * h * d * 2)  # the first sample past 2^30 bytes
    for a in (0, mid - 2, n - 3):
        r = ref.attention_gate_bwd(np64(o[a:a + 3]), np64(x[a:a + 3]), wn, bn,
                                   np64(dout[a:a + 3]))
        assert_close("do[%d:]" % a, do[a:a + 3], r[0], tol)
        assert_close("dx[%d:]" % a, dx[a:a + 3], r[1], tol)
    sums = None
    step = 512
    for a in range(0, n, step):
        r = ref.attention_gate_bwd(np64(o[a:a + step]), np64(x[a:a + step]), wn, bn,
                                   np64(dout[a:a + step]))[2:]
        sums = list(r) if sums is None else [u + v for u, v in zip(sums, r)]
    assert_close("dwg", dwg, sums[0], tol)
    assert_close("dbg", dbg, sums[1], tol)


@pytest.mark.parametrize("fused", [False, True], ids=["separate", "fused"])
@pytest.mark.parametrize("n,h,sq,sk,d,c,tail", [(2, 8, 70, 70, 32, 256, 0.1),
                                                (3, 4, 64, 64, 32, 128, 0.0),
                                                (2, 4, 33, 40, 16, 64, 0.2)])
def test_gated_attention_autograd(cuda, n, h, sq, sk, d, c, tail, fused):
    """Gradients of q, k, v, bias, x, wg and bg through the library's gated attention (forward
    fused or as two launches; backward = gate backward, then attention backward) against the
    float64 oracle's chain."""
    dt = torch.bfloat16
    inp = attention_inputs(n, h, sq, sk, d, dt, seed=sq + c, masked_tail=tail, with_dout=False)
    x, wg, bg = gate_inputs(n, sq, c, h * d, dt, seed=sq + c, bias_std=0.5)
    dgated = torch.randn((n, sq, h * d), generator=torch.Generator().manual_seed(7)).to(dt)
    kmask, scale = inp["kmask"], inp["scale"]
    host = [inp["q"], inp["k"], inp["v"], inp["bias"], x, wg, bg]
    q, k, v, b, xx, w, bb = (t.to(cuda).requires_grad_(True) for t in host)
    gated = ops.GatedAttentionFunction.apply(q, k, v, b, kmask.to(cuda), xx, w, bb, scale, fused)
    gated.backward(dgated.to(cuda))
    qh, kh, vh, bh = (np64(t) for t in host[:4])
    o, _ = ref_attn.attention_fwd(qh, kh, vh, bh, kmask.numpy(), scale)
    r_do, r_dx, r_dwg, r_dbg = ref.attention_gate_bwd(o, np64(x), np64(wg), np64(bg),
                                                      np64(dgated))
    rq, rk, rv, rb = ref_attn.attention_bwd(qh, kh, vh, bh, kmask.numpy(), scale, r_do)
    tol = TOL["bf16"]["grad"]
    for name, t, r in (("dq", q, rq), ("dk", k, rk), ("dv", v, rv), ("dbias", b, rb),
                       ("dx", xx, r_dx), ("dwg", w, r_dwg), ("dbg", bb, r_dbg)):
        assert t.grad is not None and t.grad.dtype == dt, name
        assert_close(name, t.grad, r, tol)
