"""Triangle-multiplication contraction on the GPU against the float64 oracle."""
import numpy as np
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
    """Both pair-layout directions through the channel-major kernel (left = a, right = b)."""
    n, c = 72, 6
    g = torch.Generator().manual_seed(7)
    a = torch.randn((n, n, c), generator=g).to(torch.bfloat16)
    b = torch.randn((n, n, c), generator=g).to(torch.bfloat16)
    for outgoing in (True, False):
        if outgoing:   # A[c][i][k] = left[i,k,c], B[c][j][k] = right[j,k,c]
            ac, bc = a.permute(2, 0, 1), b.permute(2, 0, 1)
        else:          # A[c][i][k] = right[k,i,c], B[c][j][k] = left[k,j,c]
            ac, bc = b.permute(2, 1, 0), a.permute(2, 1, 0)
        x = ops.triangle_einsum(ac.contiguous().to(cuda), bc.contiguous().to(cuda))
        assert_close("x", x.permute(1, 2, 0), ref.pair_einsum(np64(a), np64(b), outgoing),
                     TOL["bf16"]["o"])


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


def module_case(n, c, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    rnd = lambda *s, std=1.0: torch.randn(s, generator=g) * std  # noqa: E731
    z = rnd(n, n, c).to(dtype)
    mask = (torch.rand((n, n), generator=g) > 0.1).to(dtype)
    ln_in = (1 + rnd(c, std=0.1), rnd(c, std=0.1))
    ln_c = (1 + rnd(c, std=0.1), rnd(c, std=0.1))
    ws = [rnd(c, c, std=c ** -0.5).to(dtype) for _ in range(6)]
    bs = [rnd(c, std=0.3).to(dtype) for _ in range(6)]
    d = lambda t: t.to(dev)  # noqa: E731
    return (d(z), d(mask), tuple(map(d, ln_in)), [d(w) for w in ws], [d(b) for b in bs],
            tuple(map(d, ln_c)))


# (N, C): the pair stack's 128 channels and the template stack's 64, one 64-position tile,
# several tiles, N not a multiple of 64 (ragged contraction tiles), more than one 256-wide
# contraction tile per channel (N = 264).
MODULE_SHAPES = [(8, 128), (64, 128), (72, 128), (40, 64), (136, 64), (264, 64)]
# Ragged N (not a multiple of 8): run on a zero-padded grid internally.
RAGGED_SHAPES = [(1, 64), (13, 128), (50, 64), (261, 64)]


@pytest.mark.parametrize("outgoing", [True, False], ids=["outgoing", "incoming"])
@pytest.mark.parametrize("n,c", MODULE_SHAPES)
def test_triangle_multiply_parity(cuda, n, c, outgoing):
    z, mask, ln_in, ws, bs, ln_c = module_case(n, c, torch.bfloat16, n + c, cuda)
    out = ops.triangle_multiply(z, mask, ln_in, ws, bs, ln_c, outgoing)
    r = ref.triangle_multiply(np64(z), np64(mask), tuple(map(np64, ln_in)), [np64(w) for w in ws],
                              [np64(b) for b in bs], tuple(map(np64, ln_c)), outgoing)
    assert_close("out", out, r, 2e-2)


@pytest.mark.parametrize("outgoing", [True, False], ids=["outgoing", "incoming"])
@pytest.mark.parametrize("n,c", RAGGED_SHAPES)
def test_triangle_multiply_ragged_n(cuda, n, c, outgoing):
    z, mask, ln_in, ws, bs, ln_c = module_case(n, c, torch.bfloat16, 2 * n + c, cuda)
    out = ops.triangle_multiply(z, mask, ln_in, ws, bs, ln_c, outgoing)
    r = ref.triangle_multiply(np64(z), np64(mask), tuple(map(np64, ln_in)), [np64(w) for w in ws],
                              [np64(b) for b in bs], tuple(map(np64, ln_c)), outgoing)
    assert_close("out", out, r, 2e-2)


def test_triangle_multiply_incoming_f16(cuda):
    z, mask, ln_in, ws, bs, ln_c = module_case(72, 64, torch.float16, 5, cuda)
    out = ops.triangle_multiply(z, mask, ln_in, ws, bs, ln_c, False)
    r = ref.triangle_multiply(np64(z), np64(mask), tuple(map(np64, ln_in)), [np64(w) for w in ws],
                              [np64(b) for b in bs], tuple(map(np64, ln_c)), False)
    assert_close("out", out, r, 1e-2)


def test_triangle_multiply_f16_and_repeatable(cuda):
    z, mask, ln_in, ws, bs, ln_c = module_case(64, 128, torch.float16, 3, cuda)
    out = ops.triangle_multiply(z, mask, ln_in, ws, bs, ln_c, True)
    assert torch.equal(out, ops.triangle_multiply(z, mask, ln_in, ws, bs, ln_c, True))
    r = ref.triangle_multiply(np64(z), np64(mask), tuple(map(np64, ln_in)), [np64(w) for w in ws],
                              [np64(b) for b in bs], tuple(map(np64, ln_c)), True)
    assert_close("out", out, r, 1e-2)


# Grids whose channel-major planes pass 2^31 bytes (N^2 * C * 2 at C = 128 from N = 2897): offsets
# into the projection planes, x and out need more than 31 bits. Outgoing at N = 3000 (a multiple
# of 8); incoming at a ragged N = 2901 (run on the zero-padded 2904 grid). Positions: the four
# corners, the last 64-position tile, and random ones; every channel of each.
@pytest.mark.parametrize("n,outgoing", [(3000, True), (2901, False)],
                         ids=["3000-outgoing", "2901-incoming"])
def test_triangle_multiply_large_grid_sampled(cuda, n, outgoing):
    c = 128
    gd = torch.Generator(device=cuda).manual_seed(n)
    z = torch.randn((n, n, c), generator=gd, device=cuda).to(torch.bfloat16)
    mask = (torch.rand((n, n), generator=gd, device=cuda) > 0.1).to(torch.bfloat16)
    _, _, ln_in, ws, bs, ln_c = module_case(8, c, torch.bfloat16, n, cuda)
    out = ops.triangle_multiply(z, mask, ln_in, ws, bs, ln_c, outgoing)
    rng = np.random.default_rng(n)
    pos = [(0, 0), (n - 1, n - 1), (n - 1, 0), (0, n - 1), (n - 1, n - 40), (n - 2, n - 7)]
    pos += [tuple(map(int, rng.integers(0, n, 2))) for _ in range(6)]

    def line(kind, idx):
        if kind == "row":
            return np64(z[idx]), np64(mask[idx])
        return np64(z[:, idx]), np64(mask[:, idx])

    r = ref.triangle_multiply_at(line, tuple(map(np64, ln_in)), [np64(w) for w in ws],
                                 [np64(b) for b in bs], tuple(map(np64, ln_c)), pos, outgoing)
    got = torch.stack([out[i, j] for i, j in pos])
    assert_close("out", got, r, 2e-2)
