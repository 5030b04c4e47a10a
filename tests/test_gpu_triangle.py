"""Triangle-multiplication contraction on the GPU against the float64 oracle."""
import pytest
import torch

from _util import TOL, assert_close, dname, np64
from colabfold_legacy_kernels import ops
from oracle import triangle as ref

pytestmark = pytest.mark.gpu

# (C, N): one tile, ragged tiles (N not a multiple of the 256 tile or of the 32-wide k slice),
# several tiles per channel, the smallest N.
EINSUM_SHAPES = [(4, 64), (3, 264), (2, 384), (1, 8), (5, 520), (2, 40)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("c,n", EINSUM_SHAPES)
def test_einsum_parity(cuda, c, n, dtype):
    g = torch.Generator().manual_seed(c * 1000 + n)
    a = torch.randn((c, n, n), generator=g).to(dtype)
    b = torch.randn((c, n, n), generator=g).to(dtype)
    x = ops.triangle_einsum(a.to(cuda), b.to(cuda))
    r = ref.einsum(np64(a), np64(b))
    assert_close("x", x, r, TOL[dname(dtype)]["o"])


def test_einsum_pair_directions(cuda):
    """Both pair-layout directions through the channel-major kernel: outgoing takes a[c][i][k] =
    a[i,k,c], incoming a[c][i][k] = a[k,i,c]."""
    n, c = 72, 6
    g = torch.Generator().manual_seed(7)
    a = torch.randn((n, n, c), generator=g).to(torch.bfloat16)
    b = torch.randn((n, n, c), generator=g).to(torch.bfloat16)
    for outgoing in (True, False):
        perm = (2, 0, 1) if outgoing else (2, 1, 0)
        ac = a.permute(*perm).contiguous().to(cuda)
        bc = b.permute(*perm).contiguous().to(cuda)
        x = ops.triangle_einsum(ac, bc).permute(1, 2, 0)
        assert_close("x", x, ref.pair_einsum(np64(a), np64(b), outgoing), TOL["bf16"]["o"])


def test_einsum_large_repeatable(cuda):
    """128 channels at N = 512: two calls agree bit for bit, sampled channels match the oracle."""
    c, n = 128, 512
    g = torch.Generator().manual_seed(11)
    a = torch.randn((c, n, n), generator=g).to(torch.bfloat16).to(cuda)
    b = torch.randn((c, n, n), generator=g).to(torch.bfloat16).to(cuda)
    x = ops.triangle_einsum(a, b)
    assert torch.equal(x, ops.triangle_einsum(a, b))
    for ch in (0, 37, 127):
        assert_close("x[%d]" % ch, x[ch], ref.einsum(np64(a[ch:ch + 1]), np64(b[ch:ch + 1]))[0],
                     TOL["bf16"]["o"])
