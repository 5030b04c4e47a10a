"""LayerNorm forward/backward on the GPU against the float64 oracle (through the C ABI)."""
import numpy as np
import pytest
import torch

from _util import TOL, assert_close, dname, np64
from colabfold_legacy_kernels import ops
from colabfold_legacy_kernels.workloads import layer_norm_inputs
from oracle import layer_norm as ref

pytestmark = pytest.mark.gpu

# (M, C): fast-path shapes (16-byte vectors, 4..64 lanes per row) and generic-path shapes.
SHAPES = [(1000, 128), (77, 256), (33, 384), (5, 64), (64, 96), (300, 512), (16, 100), (9, 7)]
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


@pytest.mark.parametrize("dtype", DTYPES, ids=dname)
@pytest.mark.parametrize("m,c", SHAPES)
def test_layer_norm_fwd_bwd(cuda, m, c, dtype):
    inp = layer_norm_inputs(m, c, dtype, seed=m * 1000 + c, device="cpu")
    x, scale, offset, dy = (inp[k].to(cuda) for k in ("x", "scale", "offset", "dy"))
    eps = 1e-5
    y = ops.layer_norm(x, scale, offset, eps)
    yr, _, _ = ref.layer_norm_fwd(np64(x), np64(scale), np64(offset), eps)
    tol = TOL[dname(dtype)]["ln"]
    assert_close("y", y, yr, tol)
    dx, dscale, doffset = ops.layer_norm_bwd(x, scale, dy, eps)
    dxr, dsr, dor = ref.layer_norm_bwd(np64(x), np64(scale), np64(dy), eps)
    assert_close("dx", dx, dxr, tol)
    # Column sums over M rows of float32 products: float32 accumulation tolerance.
    assert_close("dscale", dscale, dsr, 1e-4 if dtype == torch.float32 else tol)
    assert_close("doffset", doffset, dor, 1e-4 if dtype == torch.float32 else tol)


def test_layer_norm_empty_rows(cuda):
    x = torch.empty((0, 128), device=cuda, dtype=torch.bfloat16)
    scale = torch.ones(128, device=cuda)
    offset = torch.zeros(128, device=cuda)
    assert ops.layer_norm(x, scale, offset).shape == (0, 128)
    dx, ds, do = ops.layer_norm_bwd(x, scale, x)
    assert dx.shape == (0, 128)
    assert torch.count_nonzero(ds).item() == 0 and torch.count_nonzero(do).item() == 0


def test_layer_norm_full_pair_rep(cuda):
    """The 512x512x128 pair representation: sampled rows against the oracle, plus the
    size-independent properties (gamma=1, beta=0 rows have mean 0 and variance ~1; sum_c dx = 0;
    doffset is the column sum of dy; bit-identical repeat)."""
    m, c = 512 * 512, 128
    inp = layer_norm_inputs(m, c, torch.bfloat16, seed=3, device=cuda)
    x, scale, offset, dy = inp["x"], inp["scale"], inp["offset"], inp["dy"]
    y = ops.layer_norm(x, scale, offset)
    rows = torch.tensor([0, 1, 4095, 131072, m - 1], device=cuda)
    yr, _, _ = ref.layer_norm_fwd(np64(x[rows]), np64(scale), np64(offset), 1e-5)
    assert_close("y[rows]", y[rows], yr, TOL["bf16"]["ln"])
    one, zero = torch.ones_like(scale), torch.zeros_like(offset)
    y1 = ops.layer_norm(x, one, zero).float()
    assert y1.mean(dim=1).abs().max().item() < 2e-2
    assert (y1.var(dim=1, unbiased=False) - 1).abs().max().item() < 2e-2
    dx, dscale, doffset = ops.layer_norm_bwd(x, scale, dy)
    assert dx.float().sum(dim=1).abs().max().item() < 0.15
    col = dy.double().sum(dim=0)
    assert (doffset.double() - col).abs().max().item() < 1e-3 * col.abs().max().item() + 1e-3
    # The whole dscale and doffset (column sums over all 262144 rows, reduced through the
    # kernel's per-block partials) against the float64 oracle, summed over row chunks.
    dsr, dor = np.zeros(c), np.zeros(c)
    for a in range(0, m, 32768):
        _, ds_c, do_c = ref.layer_norm_bwd(np64(x[a:a + 32768]), np64(scale),
                                           np64(dy[a:a + 32768]), 1e-5)
        dsr += ds_c
        dor += do_c
    assert_close("dscale", dscale, dsr, TOL["bf16"]["ln"])
    assert_close("doffset", doffset, dor, TOL["bf16"]["ln"])
    dx2, dscale2, doffset2 = ops.layer_norm_bwd(x, scale, dy)
    assert torch.equal(dx, dx2) and torch.equal(dscale, dscale2) and torch.equal(doffset, doffset2)
    dxr, dsr, dor = ref.layer_norm_bwd(np64(x[rows]), np64(scale), np64(dy[rows]), 1e-5)
    assert_close("dx[rows]", dx[rows], dxr, TOL["bf16"]["ln"])
    _ = np


def test_layer_norm_rejects_bad_operands(cuda):
    x = torch.randn(4, 128, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(ops.InvalidArgument):
        ops.layer_norm(x, torch.ones(64, device=cuda), torch.zeros(64, device=cuda))
    with pytest.raises(ops.InvalidArgument):
        ops.layer_norm(x.to(torch.float64), torch.ones(128, device=cuda),
                       torch.zeros(128, device=cuda))


# (Sq, Sk, C, H): triangle attention (4 heads on 128 channels), MSA row attention's pair bias
# (8 heads), the template stack (64 channels), 256 channels, one head, ragged row counts.
BIAS_SHAPES = [(64, 64, 128, 4), (37, 53, 128, 8), (40, 40, 64, 4), (9, 11, 256, 2), (3, 5, 128, 1)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("sq,sk,c,h", BIAS_SHAPES)
def test_ln_pair_bias_parity(cuda, sq, sk, c, h, dtype):
    g = torch.Generator().manual_seed(sq * sk + c + h)
    z = (torch.randn((sq, sk, c), generator=g) * 2 + 0.5).to(dtype)
    sc = 1 + 0.1 * torch.randn(c, generator=g)
    of = 0.1 * torch.randn(c, generator=g)
    w = (torch.randn((c, h), generator=g) / c ** 0.5).to(dtype)
    out = ops.ln_pair_bias(z.to(cuda), sc.to(cuda), of.to(cuda), w.to(cuda))
    r = ref.ln_pair_bias(np64(z), np64(sc), np64(of), np64(w))
    assert_close("bias", out, r, TOL[dname(dtype)]["ln"])


@pytest.mark.parametrize("nbytes", [16, 4096 + 48, 3 << 20])
def test_stream_copy(cuda, nbytes):
    """The HBM ceiling probe copies exactly (ragged tails included)."""
    from colabfold_legacy_kernels import _native
    a = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=cuda)
    b = torch.zeros_like(a)
    lib = _native.lib()
    st = lib.clk_stream_copy(torch.cuda.current_stream(cuda).cuda_stream, a.data_ptr(),
                             b.data_ptr(), nbytes)
    assert st == _native.OK, _native.last_error()
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("kind", range(7))
def test_issue_calibration_mixes_run(cuda, kind):
    """Every instruction mix of the issue calibration runs and writes one finite float per
    thread (a short launch: 4 blocks of 128 threads, 3 rounds)."""
    from colabfold_legacy_kernels import _native
    sink = torch.full((4 * 128,), float("nan"), device=cuda)
    lib = _native.lib()
    st = lib.clk_issue_calibration(torch.cuda.current_stream(cuda).cuda_stream, kind, 4, 128, 3,
                                   sink.data_ptr())
    assert st == _native.OK, _native.last_error()
    torch.cuda.synchronize()
    assert torch.isfinite(sink).all()
