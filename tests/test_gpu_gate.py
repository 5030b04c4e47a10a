"""Gated attention output on the GPU against the float64 oracle, and its exact special cases."""
import pytest
import torch

from _util import TOL, assert_close, dname, np64
from colabfold_legacy_kernels import ops
from oracle import gate as ref

pytestmark = pytest.mark.gpu

# (N, H, Sq, D, C): MSA row attention (8 x 32 heads on 256 channels), triangle attention
# (4 x 32 on 128), extra-MSA (8 x 8 on 64), template stack (4 x 16 on 64), D = 64 heads, and
# ragged query counts (not multiples of the 64-row tile, one row, one full tile).
GATE_SHAPES = [(2, 8, 70, 32, 256), (3, 4, 64, 32, 128), (1, 8, 33, 8, 64), (2, 4, 17, 16, 64),
               (1, 2, 130, 64, 128), (2, 8, 40, 32, 128), (1, 4, 50, 64, 256), (3, 2, 1, 32, 64),
               (1, 4, 200, 16, 256)]


def case(n, h, sq, d, c, dtype, seed, dev, bias_std=0.5):
    g = torch.Generator().manual_seed(seed)
    o = torch.randn((n, h, sq, d), generator=g)
    x = torch.randn((n, sq, c), generator=g)
    wg = torch.randn((c, h * d), generator=g) / c ** 0.5
    bg = torch.randn((h * d,), generator=g) * bias_std
    return [t.to(dtype).to(dev) for t in (o, x, wg, bg)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("n,h,sq,d,c", GATE_SHAPES)
def test_gate_parity(cuda, n, h, sq, d, c, dtype):
    o, x, wg, bg = case(n, h, sq, d, c, dtype, n * 1000 + sq + c, cuda)
    out = ops.attention_gate(o, x, wg, bg)
    r = ref.attention_gate(np64(o), np64(x), np64(wg), np64(bg))
    assert_close("gated", out, r, TOL[dname(dtype)]["o"])


# Enough 64-query tiles that the resident blocks (256 at H*D = 256, 512 at 128) run two to four
# each: the staged tile handed from one tile step to the next, and the flush of a block's last
# tile.
@pytest.mark.parametrize("n,h,sq,d,c", [(773, 8, 64, 32, 256), (1100, 4, 64, 32, 128)])
def test_gate_many_tiles(cuda, n, h, sq, d, c):
    o, x, wg, bg = case(n, h, sq, d, c, torch.bfloat16, n + c, cuda)
    out = ops.attention_gate(o, x, wg, bg)
    r = ref.attention_gate(np64(o), np64(x), np64(wg), np64(bg))
    assert_close("gated", out, r, TOL["bf16"]["o"])


def test_gate_exact_cases(cuda):
    """A zero gate pre-activation halves O exactly; saturated biases pass O or zero it exactly;
    every result lands in the [N,Sq,H*D] layout."""
    n, h, sq, d, c = 2, 8, 70, 32, 256
    o, x, wg, bg = case(n, h, sq, d, c, torch.bfloat16, 5, cuda)
    ot = o.permute(0, 2, 1, 3).reshape(n, sq, h * d)
    z = torch.zeros_like(wg)
    assert torch.equal(ops.attention_gate(o, x, z, torch.zeros_like(bg)), 0.5 * ot)
    assert torch.equal(ops.attention_gate(o, x, z, torch.full_like(bg, 100.0)), ot)
    assert torch.count_nonzero(ops.attention_gate(o, x, z, torch.full_like(bg, -100.0))) == 0


def test_gate_repeatable_and_large(cuda):
    """The metric-size MSA gate (N=512 rows, 256 queries, 8 x 32 heads on 256 channels): two
    calls agree bit for bit and a strided sample of rows matches the oracle."""
    n, h, sq, d, c = 512, 8, 256, 32, 256
    o, x, wg, bg = case(n, h, sq, d, c, torch.bfloat16, 9, cuda)
    a = ops.attention_gate(o, x, wg, bg)
    b = ops.attention_gate(o, x, wg, bg)
    assert torch.equal(a, b)
    rows = slice(3, None, 61)
    r = ref.attention_gate(np64(o[rows]), np64(x[rows]), np64(wg), np64(bg))
    assert_close("gated", a[rows], r, TOL["bf16"]["o"])
