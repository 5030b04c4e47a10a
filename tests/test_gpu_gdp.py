"""Gated dual projection and LayerNorm-fused GDP on the GPU against the float64 oracle."""
import numpy as np
import pytest
import torch

from _util import TOL, assert_close, dname, np64
from colabfold_legacy_kernels import ops
from colabfold_legacy_kernels.workloads import gdp_weights, layer_norm_inputs
from oracle import gdp as ref

pytestmark = pytest.mark.gpu

# (M, K, N): reference shapes (128x128), the MSA width, ragged rows, K/N not multiples of 32/64,
# K not a multiple of 8 and K above the 512 weight rows staged at a time (both taken by the
# reference's bounds-checked K loop, cuda/volta_ops.cu:143-183).
GDP_SHAPES = [(1000, 128, 128), (77, 256, 256), (300, 128, 64), (33, 64, 200), (5, 40, 8),
              (129, 512, 72), (1, 8, 8), (70, 100, 64), (41, 3, 16), (90, 1100, 128),
              (65, 777, 40), (200, 64, 64), (130, 64, 128), (100, 32, 96), (64, 96, 128),
              (3, 128, 128)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("m,k,n", GDP_SHAPES)
def test_gdp_parity(cuda, m, k, n, dtype):
    li = layer_norm_inputs(m, k, dtype, seed=m + k + n)
    w = gdp_weights(k, n, dtype, seed=n, bias_std=0.3)
    x, mask = li["x"], li["mask"]
    out = ops.gated_dual_proj(x.to(cuda), *(t.to(cuda) for t in w), mask.to(cuda))
    r = ref.gated_dual_proj(np64(x), *(np64(t) for t in w), np64(mask))
    assert_close("gdp", out, r, TOL[dname(dtype)]["gdp"])


def test_gdp_special_cases(cuda):
    """mask = 0 gives 0; wg = bg = 0 gives 0.5*(x.wp + bp); a large bg gives x.wp + bp."""
    dt = torch.bfloat16
    li = layer_norm_inputs(256, 128, dt, seed=1)
    wp, bp, wg, bg = (t.to(cuda) for t in gdp_weights(128, 128, dt, seed=2, bias_std=0.2))
    x = li["x"].to(cuda)
    zero_mask = torch.zeros(256, device=cuda, dtype=dt)
    assert torch.count_nonzero(ops.gated_dual_proj(x, wp, bp, wg, bg, zero_mask)).item() == 0
    ones = torch.ones(256, device=cuda, dtype=dt)
    half = ops.gated_dual_proj(x, wp, bp, torch.zeros_like(wg), torch.zeros_like(bg), ones)
    lin = np64(x) @ np64(wp) + np64(bp)
    assert_close("0.5*lin", half, 0.5 * lin, 1e-2)
    open_gate = ops.gated_dual_proj(x, wp, bp, torch.zeros_like(wg),
                                    torch.full_like(bg, 60.0), ones)
    assert_close("lin", open_gate, lin, 1e-2)


def test_gdp_rejects_bad_operands(cuda):
    dt = torch.bfloat16
    x = torch.zeros((4, 128), device=cuda, dtype=dt)
    w = torch.zeros((128, 12), device=cuda, dtype=dt)
    b = torch.zeros(12, device=cuda, dtype=dt)
    with pytest.raises(ops.InvalidArgument):   # N % 8 != 0, as the reference requires
        ops.gated_dual_proj(x, w, b, w, b, torch.ones(4, device=cuda, dtype=dt))


LN_GDP_SHAPES = [(1000, 128, 128), (77, 64, 64), (130, 128, 32), (33, 32, 128), (9, 96, 96)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("m,c,n", LN_GDP_SHAPES)
def test_ln_gdp_parity(cuda, m, c, n, dtype):
    li = layer_norm_inputs(m, c, dtype, seed=m * 3 + c)
    wa = gdp_weights(c, n, dtype, seed=11, bias_std=0.2)
    wb = gdp_weights(c, n, dtype, seed=12, bias_std=0.2)
    dev = lambda ts: tuple(t.to(cuda) for t in ts)  # noqa: E731
    a, b = ops.ln_gated_dual_proj(li["x"].to(cuda), li["scale"].to(cuda), li["offset"].to(cuda),
                                  dev(wa), dev(wb), li["mask"].to(cuda), 1e-5)
    ra, rb = ref.ln_gated_dual_proj(np64(li["x"]), np64(li["scale"]), np64(li["offset"]), 1e-5,
                                    tuple(np64(t) for t in wa), tuple(np64(t) for t in wb),
                                    np64(li["mask"]))
    tol = TOL[dname(dtype)]["gdp"]
    assert_close("a", a, ra, tol)
    assert_close("b", b, rb, tol)


# Row counts around the 64-row tile and the grid of 256 resident blocks per launch: one row, a
# tile short by one and long by one, and enough tiles that blocks run two and three of them --
# both staging buffers of the whole-row output stores and the flush of a block's last tile.
TILE_ROWS = [1, 63, 65, 16581, 33000]


@pytest.mark.parametrize("m", TILE_ROWS)
@pytest.mark.parametrize("c,n", [(128, 128), (64, 64), (128, 32)])
def test_ln_gdp_tile_boundaries(cuda, m, c, n):
    dtype = torch.bfloat16
    li = layer_norm_inputs(m, c, dtype, seed=m + c * 7 + n)
    wa = gdp_weights(c, n, dtype, seed=21, bias_std=0.2)
    wb = gdp_weights(c, n, dtype, seed=22, bias_std=0.2)
    dev = lambda ts: tuple(t.to(cuda) for t in ts)  # noqa: E731
    a, b = ops.ln_gated_dual_proj(li["x"].to(cuda), li["scale"].to(cuda), li["offset"].to(cuda),
                                  dev(wa), dev(wb), li["mask"].to(cuda), 1e-5)
    ra, rb = ref.ln_gated_dual_proj(np64(li["x"]), np64(li["scale"]), np64(li["offset"]), 1e-5,
                                    tuple(np64(t) for t in wa), tuple(np64(t) for t in wb),
                                    np64(li["mask"]))
    tol = TOL[dname(dtype)]["gdp"]
    assert_close("a", a, ra, tol)
    assert_close("b", b, rb, tol)


@pytest.mark.parametrize("m", TILE_ROWS)
@pytest.mark.parametrize("k,n", [(128, 128), (64, 128)])
def test_gdp_tile_boundaries(cuda, m, k, n):
    dtype = torch.bfloat16
    li = layer_norm_inputs(m, k, dtype, seed=m + k + 3 * n)
    w = gdp_weights(k, n, dtype, seed=n + 1, bias_std=0.3)
    out = ops.gated_dual_proj(li["x"].to(cuda), *(t.to(cuda) for t in w), li["mask"].to(cuda))
    r = ref.gated_dual_proj(np64(li["x"]), *(np64(t) for t in w), np64(li["mask"]))
    assert_close("gdp", out, r, TOL[dname(dtype)]["gdp"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
def test_ln_gdp_offset_and_constant_rows(cuda, dtype):
    """Rows whose mean is large against their spread (|mean|/std up to 50) and constant rows
    (variance 0, so LN(z) = beta): the one-pass sum / sum-of-squares statistics stay within the
    same tolerance as the two-pass oracle."""
    m, c = 192, 128
    li = layer_norm_inputs(m, c, dtype, seed=5)
    g = torch.Generator().manual_seed(6)
    z = li["x"].float()
    mean = torch.empty(m).uniform_(-100.0, 100.0, generator=g)
    std = torch.empty(m).uniform_(2.0, 4.0, generator=g)
    z = mean[:, None] + std[:, None] * z
    z[::7] = mean[::7, None]  # constant rows
    z = z.to(dtype)
    wa = gdp_weights(c, c, dtype, seed=13, bias_std=0.2)
    wb = gdp_weights(c, c, dtype, seed=14, bias_std=0.2)
    dev = lambda ts: tuple(t.to(cuda) for t in ts)  # noqa: E731
    a, b = ops.ln_gated_dual_proj(z.to(cuda), li["scale"].to(cuda), li["offset"].to(cuda),
                                  dev(wa), dev(wb), li["mask"].to(cuda), 1e-5)
    ra, rb = ref.ln_gated_dual_proj(np64(z), np64(li["scale"]), np64(li["offset"]), 1e-5,
                                    tuple(np64(t) for t in wa), tuple(np64(t) for t in wb),
                                    np64(li["mask"]))
    tol = TOL[dname(dtype)]["gdp"]
    assert_close("a", a, ra, tol)
    assert_close("b", b, rb, tol)


def test_ln_gdp_full_pair_rep(cuda):
    """The 512x512x128 pair representation with a 5% padding mask: sampled rows against the
    oracle, masked rows exactly zero, and agreement with LayerNorm followed by two GDP calls."""
    m, c = 512 * 512, 128
    li = layer_norm_inputs(m, c, torch.bfloat16, seed=3, device=cuda)
    wa = gdp_weights(c, c, torch.bfloat16, seed=21, device=cuda)
    wb = gdp_weights(c, c, torch.bfloat16, seed=22, device=cuda)
    a, b = ops.ln_gated_dual_proj(li["x"], li["scale"], li["offset"], wa, wb, li["mask"])
    rows = torch.tensor([0, 7, 65536, 200000, m - 1], device=cuda)
    ra, rb = ref.ln_gated_dual_proj(np64(li["x"][rows]), np64(li["scale"]), np64(li["offset"]),
                                    1e-5, tuple(np64(t) for t in wa), tuple(np64(t) for t in wb),
                                    np64(li["mask"][rows]))
    assert_close("a[rows]", a[rows], ra, TOL["bf16"]["gdp"])
    assert_close("b[rows]", b[rows], rb, TOL["bf16"]["gdp"])
    masked = li["mask"] == 0
    assert torch.count_nonzero(a[masked]).item() == 0
    y = ops.layer_norm(li["x"], li["scale"], li["offset"])
    a2 = ops.gated_dual_proj(y, *wa, li["mask"])
    err = (a.float() - a2.float()).abs().max().item()
    assert err <= 2e-2 * a2.float().abs().max().item()
    _ = np


# (M, K, N): the pair stack (128 -> 128), the template stack (64), mixed widths, ragged row
# counts (not multiples of the 64-row tile), one row.
GDP_BWD_SHAPES = [(1000, 128, 128), (77, 64, 64), (300, 128, 64), (33, 64, 128), (1, 128, 128),
                  (4096, 128, 128)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("m,k,n", GDP_BWD_SHAPES)
def test_gdp_bwd_parity(cuda, m, k, n, dtype):
    li = layer_norm_inputs(m, k, dtype, seed=m + 3 * k + n)
    w = gdp_weights(k, n, dtype, seed=n + 1, bias_std=0.3)
    g = torch.Generator().manual_seed(m)
    dout = torch.randn((m, n), generator=g).to(dtype)
    x, mask = li["x"], li["mask"]
    got = ops.gated_dual_proj_bwd(x.to(cuda), *(t.to(cuda) for t in w), mask.to(cuda),
                                  dout.to(cuda))
    r = ref.gated_dual_proj_bwd(np64(x), *(np64(t) for t in w), np64(mask), np64(dout))
    tol = TOL[dname(dtype)]["grad"]
    for name, a, b in zip(("dx", "dwp", "dbp", "dwg", "dbg"), got, r):
        assert_close(name, a, b, tol)


@pytest.mark.parametrize("k,n", [(128, 128), (64, 128)])
def test_gdp_bwd_no_rows_gives_zero_weight_grads(cuda, k, n):
    """M = 0: the weight and bias gradients are sums over no rows, so they must come back zero
    even when their buffers held other values."""
    dt = torch.bfloat16
    w = [t.to(cuda) for t in gdp_weights(k, n, dt, seed=3, bias_std=0.3)]
    x = torch.empty((0, k), device=cuda, dtype=dt)
    mask = torch.empty((0,), device=cuda, dtype=dt)
    dout = torch.empty((0, n), device=cuda, dtype=dt)
    junk = [torch.full((k * n,), 7.0, device=cuda) for _ in range(8)]
    del junk  # the gradients below reuse these nonzero blocks
    dx, dwp, dbp, dwg, dbg = ops.gated_dual_proj_bwd(x, *w, mask, dout)
    assert dx.shape == (0, k)
    for t in (dwp, dbp, dwg, dbg):
        assert torch.count_nonzero(t).item() == 0


def test_gdp_bwd_accumulates_and_repeats(cuda):
    """dx accumulation (two branches reading one x) and bit-identical repeated runs."""
    dt = torch.bfloat16
    m, k, n = 2000, 128, 128
    li = layer_norm_inputs(m, k, dt, seed=5)
    wa = [t.to(cuda) for t in gdp_weights(k, n, dt, seed=6, bias_std=0.3)]
    wb = [t.to(cuda) for t in gdp_weights(k, n, dt, seed=7, bias_std=0.3)]
    g = torch.Generator().manual_seed(8)
    da, db = (torch.randn((m, n), generator=g).to(dt).to(cuda) for _ in range(2))
    x, mask = li["x"].to(cuda), li["mask"].to(cuda)
    dx, *ga = ops.gated_dual_proj_bwd(x, *wa, mask, da)
    again = ops.gated_dual_proj_bwd(x, *wa, mask, da)
    for u, v in zip([dx] + ga, again):
        assert torch.equal(u, v)
    dx2 = dx.clone()
    ops.gated_dual_proj_bwd(x, *wb, mask, db, dx=dx2)
    ra = ref.gated_dual_proj_bwd(np64(x), *(np64(t) for t in wa), np64(mask), np64(da))
    rb = ref.gated_dual_proj_bwd(np64(x), *(np64(t) for t in wb), np64(mask), np64(db))
    assert_close("dx_a+dx_b", dx2, ra[0] + rb[0], TOL["bf16"]["grad"])


def test_ln_gdp_bwd_composition(cuda):
    """LayerNorm + both branches backward (recomputed LN, two GDP backwards into one dy, LN
    backward) against the float64 composition of the oracle functions."""
    from oracle import layer_norm as L
    dt = torch.bfloat16
    m, c, n = 1500, 128, 128
    li = layer_norm_inputs(m, c, dt, seed=11)
    wa = [t.to(cuda) for t in gdp_weights(c, n, dt, seed=12, bias_std=0.3)]
    wb = [t.to(cuda) for t in gdp_weights(c, n, dt, seed=13, bias_std=0.3)]
    g = torch.Generator().manual_seed(14)
    da, db = (torch.randn((m, n), generator=g).to(dt).to(cuda) for _ in range(2))
    z, sc, of, mask = (li[k].to(cuda) for k in ("x", "scale", "offset", "mask"))
    dz, dsc, dof, ga, gb = ops.ln_gated_dual_proj_bwd(z, sc, of, wa, wb, mask, da, db)
    y, _, _ = L.layer_norm_fwd(np64(z), np64(sc), np64(of), 1e-5)
    ra = ref.gated_dual_proj_bwd(y, *(np64(t) for t in wa), np64(mask), np64(da))
    rb = ref.gated_dual_proj_bwd(y, *(np64(t) for t in wb), np64(mask), np64(db))
    rdz, rdsc, rdof = L.layer_norm_bwd(np64(z), np64(sc), ra[0] + rb[0], 1e-5)
    tol = TOL["bf16"]["grad"]
    assert_close("dz", dz, rdz, tol)
    assert_close("dscale", dsc, rdsc, tol)
    assert_close("doffset", dof, rdof, tol)
    for name, a, b in zip(("dwpa", "dbpa", "dwga", "dbga"), ga, ra[1:]):
        assert_close(name, a, b, tol)
    for name, a, b in zip(("dwpb", "dbpb", "dwgb", "dbgb"), gb, rb[1:]):
        assert_close(name, a, b, tol)


def test_ln_gdp_bwd_full_pair_rep(cuda):
    """The LN + GDP backward on the 512x512x128 pair representation (Bernoulli(0.95) row mask):
    sampled rows of dz, and every element of the eight weight and bias gradients and of the
    LayerNorm's dscale and doffset (sums over all 262144 rows) against the float64 oracle,
    which runs over row chunks."""
    from oracle import layer_norm as L
    dt = torch.bfloat16
    m, c, n = 512 * 512, 128, 128
    li = layer_norm_inputs(m, c, dt, seed=3, device=cuda)
    wa = [t.to(cuda) for t in gdp_weights(c, n, dt, seed=12, bias_std=0.3)]
    wb = [t.to(cuda) for t in gdp_weights(c, n, dt, seed=13, bias_std=0.3)]
    g = torch.Generator(device=cuda).manual_seed(14)
    da, db = (torch.randn((m, n), generator=g, device=cuda).to(dt) for _ in range(2))
    z, sc, of, mask = (li[k] for k in ("x", "scale", "offset", "mask"))
    dz, dsc, dof, ga, gb = ops.ln_gated_dual_proj_bwd(z, sc, of, wa, wb, mask, da, db)
    torch.cuda.synchronize()
    wa64, wb64 = [np64(t) for t in wa], [np64(t) for t in wb]
    sc64, of64 = np64(sc), np64(of)
    acc_a, acc_b = [0.0] * 4, [0.0] * 4
    rdsc, rdof = np.zeros(c), np.zeros(c)
    rows = [0, 1, 70001, 131072, 200000, m - 1]
    rdz = {}
    step = 16384
    for a in range(0, m, step):
        zc, mc = np64(z[a:a + step]), np64(mask[a:a + step])
        y, _, _ = L.layer_norm_fwd(zc, sc64, of64, 1e-5)
        ra = ref.gated_dual_proj_bwd(y, *wa64, mc, np64(da[a:a + step]))
        rb = ref.gated_dual_proj_bwd(y, *wb64, mc, np64(db[a:a + step]))
        dyc = ra[0] + rb[0]
        dzc, ds_c, do_c = L.layer_norm_bwd(zc, sc64, dyc, 1e-5)
        rdsc += ds_c
        rdof += do_c
        acc_a = [s + t for s, t in zip(acc_a, ra[1:])]
        acc_b = [s + t for s, t in zip(acc_b, rb[1:])]
        for r in rows:
            if a <= r < a + step:
                rdz[r] = dzc[r - a]
    tol = TOL["bf16"]["grad"]
    assert_close("dz[rows]", dz[rows], np.stack([rdz[r] for r in rows]), tol)
    assert_close("dscale", dsc, rdsc, tol)
    assert_close("doffset", dof, rdof, tol)
    for name, a, b in zip(("dwpa", "dbpa", "dwga", "dbga"), ga, acc_a):
        assert_close(name, a, b, tol)
    for name, a, b in zip(("dwpb", "dbpb", "dwgb", "dbgb"), gb, acc_b):
        assert_close(name, a, b, tol)


def test_gdp_bwd_beyond_two_gib(cuda):
    """M = 2048*2048 + 37 rows at K = N = 128: the projection gradient dpg (2.1 GB) and x, dout,
    dx (1.07 GB each) exceed 2^31 bytes. Sampled rows of dx at the start, across the 2^31-byte
    point of dpg and at the end against the oracle, and every weight and bias gradient against
    the oracle summed over row chunks."""
    m, k, n = 2048 * 2048 + 37, 128, 128
    dt = torch.bfloat16
    g = torch.Generator(device=cuda).manual_seed(41)
    x = torch.randn((m, k), generator=g, device=cuda).to(dt)
    dout = torch.randn((m, n), generator=g, device=cuda).to(dt)
    mask = (torch.rand((m,), generator=g, device=cuda) > 0.05).to(dt)
    w = [t.to(cuda) for t in gdp_weights(k, n, dt, seed=42, bias_std=0.3)]
    dx, dwp, dbp, dwg, dbg = ops.gated_dual_proj_bwd(x, *w, mask, dout)
    wn = [np64(t) for t in w]
    tol = TOL["bf16"]["grad"]
    half = (1 << 31) // (2 * n * 2)  # first row of dpg past 2^31 bytes
    for a in (0, half - 300, m - 300):
        r = ref.gated_dual_proj_bwd(np64(x[a:a + 300]), *wn, np64(mask[a:a + 300]),
                                    np64(dout[a:a + 300]))
        assert_close("dx[%d:]" % a, dx[a:a + 300], r[0], tol)
    sums = None
    step = 1 << 18
    for a in range(0, m, step):
        r = ref.gated_dual_proj_bwd(np64(x[a:a + step]), *wn, np64(mask[a:a + step]),
                                    np64(dout[a:a + step]))[1:]
        sums = list(r) if sums is None else [u + v for u, v in zip(sums, r)]
    for name, got, want in zip(("dwp", "dbp", "dwg", "dbg"), (dwp, dbp, dwg, dbg), sums):
        assert_close(name, got, want, tol)
