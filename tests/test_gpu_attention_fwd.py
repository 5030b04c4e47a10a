"""Attention forward on the GPU against the float64 oracle (through the C ABI)."""
import numpy as np
import pytest
import torch

from _util import TOL, assert_close, dname, np64
from colabfold_legacy_kernels import ops
from colabfold_legacy_kernels.workloads import attention_inputs, attention_workload, gate_inputs
from oracle import attention as ref

pytestmark = pytest.mark.gpu

# (N, H, Sq, Sk, D, masked_tail, masked_rows): aligned, ragged, every head dim, masks.
CASES = [
    (2, 2, 64, 64, 32, 0.0, 0),
    (3, 2, 100, 77, 32, 0.1, 1),
    (2, 1, 130, 200, 64, 0.2, 0),
    (2, 4, 64, 64, 16, 0.0, 1),
    (2, 2, 48, 40, 8, 0.1, 0),
    (1, 1, 1, 1, 32, 0.0, 0),
    (2, 3, 257, 129, 32, 0.05, 1),
    (2, 2, 33, 300, 64, 0.0, 0),
    (1, 1, 16, 4100, 32, 0.1, 0),  # more than 64 key tiles, ragged last tile
    (1, 1, 16, 16400, 32, 0.1, 0),  # more key tiles than the masked-bias patching covers
    (3, 2, 64, 320, 32, 0.6, 1),    # a padding tail of whole key tiles
    # Biases over 2 MB run the head-outer work-item order in groups of rows: 13 rows in groups
    # of 9 and 4 (a ragged last group), and 5 rows in one group smaller than the group size.
    (13, 4, 640, 640, 32, 0.1, 1),
    (5, 2, 1024, 1024, 16, 0.0, 0),
]


def _oracle(inp, rows=None):
    sel = slice(None) if rows is None else rows
    return ref.attention_fwd(np64(inp["q"][sel]), np64(inp["k"][sel]), np64(inp["v"][sel]),
                             np64(inp["bias"]), inp["kmask"][sel].cpu().numpy(), inp["scale"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:5])))
def test_attention_fwd_parity(cuda, case, dtype):
    n, h, sq, sk, d, tail, rows = case
    inp = attention_inputs(n, h, sq, sk, d, dtype, seed=sq * 7 + sk, bias_var=1.0,
                           masked_tail=tail, masked_rows=rows, with_dout=False)
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out, lse = ops.attention_fwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"])
    o_ref, lse_ref = _oracle(inp)
    tol = TOL[dname(dtype)]["o"]
    assert_close("O", out, o_ref, tol)
    # lse is float32 from float32 logits: absolute error on the logit scale. A row with no
    # present key reports ln(Sk) (relative to its masked logit); the oracle's value is
    # -1e9 + ln(Sk), which float32 cannot hold.
    empty = (inp["kmask"].numpy() == 0).all(axis=1)[:, None, None]
    lse_ref = np.where(empty, np.log(sk), lse_ref)
    assert np.abs(np64(lse) - lse_ref).max() < 5e-2
    # The inference entry (VoltaMma contract) gives the same bits as the training entry.
    out2 = ops.attention(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"], 64, 64)
    assert torch.equal(out, out2)


# (N, H, Sq, Sk, D, masked_tail, masked_rows): every head dim, one- and two-sub-tile query
# blocks, the bias-tile and element-wise paths (Sk % 8), a padding tail, rows with no key, H = 1.
NSHD_CASES = [(3, 4, 100, 77, 32, 0.1, 1), (2, 2, 64, 384, 32, 0.2, 1),
              (2, 3, 130, 200, 64, 0.0, 0), (2, 4, 48, 40, 8, 0.1, 0), (2, 2, 33, 136, 16, 0.0, 1),
              (4, 1, 70, 96, 32, 0.5, 0)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("case", NSHD_CASES, ids=lambda c: "x".join(map(str, c[:5])))
def test_attention_fwd_nshd_layout(cuda, case, dtype):
    """The [N,S,H,D] entry runs the same kernel with rows H*D apart: O (in [N,S,H,D]) and lse
    are bit-identical to the [N,H,S,D] entry on the transposed operands, and match the oracle."""
    n, h, sq, sk, d, tail, rows = case
    inp = attention_inputs(n, h, sq, sk, d, dtype, seed=sq * 5 + sk + d, bias_var=1.0,
                           masked_tail=tail, masked_rows=rows, with_dout=False)
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out, lse = ops.attention_fwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"])
    t = lambda x: x.transpose(1, 2).contiguous()  # [N,H,S,D] <-> [N,S,H,D]
    out_s, lse_s = ops.attention_nshd(t(g["q"]), t(g["k"]), t(g["v"]), g["bias"], g["kmask"],
                                      g["scale"], want_lse=True)
    assert out_s.shape == (n, sq, h, d)
    assert torch.equal(t(out_s), out)
    assert torch.equal(lse_s, lse)
    assert_close("O", t(out_s), _oracle(inp)[0], TOL[dname(dtype)]["o"])
    out_n, lse_n = ops.attention_nshd(t(g["q"]), t(g["k"]), t(g["v"]), g["bias"], g["kmask"],
                                      g["scale"])
    assert lse_n is None and torch.equal(out_n, out_s)


# (N, H, Sq, Sk, D): whole and ragged key tiles, the element-wise mask path (Sk % 8 != 0).
MIXED_MASK_SHAPES = [(8, 2, 70, 200, 32), (6, 2, 64, 77, 32), (6, 2, 40, 456, 16),
                     (4, 1, 130, 384, 64), (5, 2, 64, 136, 8)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("shape", MIXED_MASK_SHAPES, ids=lambda c: "x".join(map(str, c)))
def test_attention_fwd_mixed_masks(cuda, shape, dtype):
    """Per-row masks of every kind in one call: random holes with a padding tail, a row with no
    present key, a row whose first 64-key tile is entirely absent (its running max starts on
    absent keys), a row with everything present, and one whose only present key is the last."""
    n, h, sq, sk, d = shape
    inp = attention_inputs(n, h, sq, sk, d, dtype, seed=sk + 3 * n, with_dout=False)
    gen = torch.Generator().manual_seed(sk * 5 + n)
    km = (torch.rand((n, sk), generator=gen) > 0.2).to(torch.uint8)
    km[:, sk - sk // 5:] = 0
    km[1] = 0
    km[2, :min(64, sk - 1)] = 0
    km[2, sk - 1] = 1
    km[3] = 1
    km[n - 1] = 0
    km[n - 1, sk - 1] = 1
    inp["kmask"] = km
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out, lse = ops.attention_fwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"])
    o_ref, lse_ref = _oracle(inp)
    assert_close("O", out, o_ref, TOL[dname(dtype)]["o"])
    empty = (km.numpy() == 0).all(axis=1)[:, None, None]
    lse_ref = np.where(empty, np.log(sk), lse_ref)
    assert np.abs(np64(lse) - lse_ref).max() < 5e-2


def test_attention_fwd_no_mask_is_all_present(cuda):
    inp = attention_inputs(2, 2, 64, 96, 32, torch.bfloat16, seed=5, with_dout=False)
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    a = ops.attention(g["q"], g["k"], g["v"], g["bias"], None, g["scale"])
    b = ops.attention(g["q"], g["k"], g["v"], g["bias"], torch.ones_like(g["kmask"]), g["scale"])
    assert torch.equal(a, b)


def test_attention_fwd_fully_masked_row_is_mean_v(cuda):
    """jnp's float32 additive mask: a row with every key masked attends uniformly over its Sk
    keys (not over tile padding), so O = mean(V)."""
    inp = attention_inputs(2, 2, 40, 70, 32, torch.bfloat16, seed=9, with_dout=False)
    inp["kmask"][1] = 0
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out = ops.attention(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"])
    mean_v = np64(inp["v"][1]).mean(axis=1, keepdims=True).repeat(40, axis=1)
    assert_close("O[masked]", out[1], mean_v, TOL["bf16"]["o"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("slope", [0.02, 0.06, 0.3, -0.3])
def test_attention_fwd_rising_and_falling_logits(cuda, slope, dtype):
    """Bias ramps along the keys, so a row's running max rises tile after tile by less than,
    about, or more than the forward's rescale slack (2^8 in P: 5.5 logit units; a 64-key tile
    rises by 64*slope), or falls (slope < 0: the first tile holds the max). O and the
    logsumexp against the oracle."""
    n, h, sq, sk, d = 2, 2, 70, 320, 32
    inp = attention_inputs(n, h, sq, sk, d, dtype, seed=13, bias_var=0.25, masked_tail=0.05,
                           with_dout=False)
    ramp = slope * torch.arange(sk, dtype=torch.float32)
    inp["bias"] = (inp["bias"].float() + ramp).to(dtype)
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out, lse = ops.attention_fwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"])
    o_ref, lse_ref = _oracle(inp)
    assert_close("O", out, o_ref, TOL[dname(dtype)]["o"])
    assert np.abs(np64(lse) - lse_ref).max() < 5e-2


# Every (D, block_q, block_k) that VoltaMma (cuda/volta_mma_attn.cu:323-331) or VoltaWmma
# (cuda/volta_wmma_attn.cu:286-292) dispatches, plus one neither knows: block sizes are hints.
REFERENCE_BLOCKS = {
    8: [(64, 64), (64, 32), (32, 32), (128, 64), (32, 64), (7, 5)],
    16: [(64, 64), (32, 32), (64, 32)],
    32: [(64, 64), (64, 32), (32, 64), (32, 32), (128, 64), (16, 64), (128, 32), (7, 5)],
    64: [(64, 64), (32, 32), (64, 32)],
}


@pytest.mark.parametrize("d,block", [(d, b) for d, bs in REFERENCE_BLOCKS.items() for b in bs],
                         ids=lambda v: str(v))
def test_attention_fwd_accepts_reference_block_hints(cuda, d, block):
    inp = attention_inputs(1, 2, 70, 90, d, torch.float16, seed=3, masked_tail=0.1,
                           with_dout=False)
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    base = ops.attention(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"])
    out = ops.attention(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"], *block)
    assert torch.equal(base, out)
    o_ref, _ = _oracle(inp)
    assert_close("O", out, o_ref, TOL["f16"]["o"])


@pytest.mark.parametrize("name", ["triangle_attn_256", "triangle_attn_384", "msa_row_attn",
                                  "triangle_attn_1024"])
def test_attention_fwd_full_size_rows(cuda, name):
    """Full workload on the GPU; sampled rows n against the oracle (rows are independent),
    including two fully padded rows (no present key) where the workload has them."""
    inp = attention_workload(name, torch.bfloat16, device=cuda, with_dout=False)
    out, lse = ops.attention_fwd(inp["q"], inp["k"], inp["v"], inp["bias"], inp["kmask"],
                                 inp["scale"])
    n = inp["q"].shape[0]
    padded = (inp["kmask"] == 0).all(dim=1).nonzero().flatten().tolist()
    if name == "msa_row_attn":
        assert len(padded) == 102
    rows = sorted({0, 1, n // 2, n - 1} | set(padded[:1] + padded[-1:]))
    cpu = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    o_ref, _ = _oracle(cpu, rows)
    assert_close("O[rows]", out[rows], o_ref, TOL["bf16"]["o"])
    assert torch.isfinite(lse).all()


def test_attention_rejects_bad_operands(cuda):
    inp = attention_inputs(1, 2, 16, 16, 32, torch.bfloat16, seed=1, with_dout=False)
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    with pytest.raises(ops.InvalidArgument):
        ops.attention(g["q"], g["k"], g["v"], g["bias"][:, :8], g["kmask"])
    q24 = torch.zeros((1, 2, 16, 24), device=cuda, dtype=torch.bfloat16)
    with pytest.raises(ops.InvalidArgument):
        ops.attention(q24, q24, q24, g["bias"], g["kmask"])
    with pytest.raises(ops.InvalidArgument):
        ops.attention(g["q"], g["k"], g["v"], g["bias"], g["kmask"], None, 0, 64)


@pytest.mark.parametrize("gated", [False, True], ids=["plain", "gated"])
def test_attention_fwd_nan_propagates(cuda, gated):
    """A NaN in one query row, and a NaN bias entry at one present key, make exactly the output
    rows they reach NaN (every head dim), with and without the fused gate; every other row stays
    finite. (The forward's device code assumes no NaN operand for its maxima; the exponentials
    and the sums still carry a NaN score into its row.)"""
    n, h, sq, sk, d = 2, 4, 70, 96, 32
    inp = attention_inputs(n, h, sq, sk, d, torch.bfloat16, seed=5, masked_tail=0.1,
                           with_dout=False)
    q, bias = inp["q"].clone(), inp["bias"].clone()
    q[1, 2, 5, 3] = float("nan")
    bias[3, 40, 17] = float("nan")  # key 17 is present in every row
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    g["q"], g["bias"] = q.to(cuda), bias.to(cuda)
    nan_rows = torch.zeros((n, h, sq), dtype=torch.bool)
    nan_rows[1, 2, 5] = True
    nan_rows[:, 3, 40] = True
    if gated:
        c = 128
        x, wg, bg = gate_inputs(n, sq, c, h * d, torch.bfloat16, seed=5, bias_std=0.5)
        out = ops.attention_gated(g["q"], g["k"], g["v"], g["bias"], g["kmask"], x.to(cuda),
                                  wg.to(cuda), bg.to(cuda), g["scale"]).cpu()
        out = out.reshape(n, sq, h, d).transpose(1, 2)
    else:
        out = ops.attention(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"]).cpu()
    isnan = torch.isnan(out.float())
    assert isnan[nan_rows].all()
    assert torch.isfinite(out.float()[~nan_rows]).all()


def test_attention_row_with_no_weight(cuda):
    """Present-key logits below -5e8 (a bias of -1e9, the masked-logit convention, on every
    present key of one query row): that row has no weight, O = 0 and lse = +inf, and its
    gradients are zero; every other row is unaffected. The backward is compared with the oracle
    on inputs whose dO of that row is zero (which removes the row from every gradient there)."""
    n, h, sq, sk, d = 3, 2, 70, 96, 32
    inp = attention_inputs(n, h, sq, sk, d, torch.bfloat16, seed=8, masked_tail=0.1)
    b = inp["bias"].float()
    b[1, 20, :] = -1e9
    inp["bias"] = b.to(torch.bfloat16)
    inp["dout"][:, 1, 20, :] = 0
    g = {k: (v.to(cuda) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out, lse = ops.attention_fwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"])
    assert torch.count_nonzero(out[:, 1, 20]).item() == 0
    assert torch.isinf(lse[:, 1, 20]).all() and (lse[:, 1, 20] > 0).all()
    o_ref, _ = _oracle(inp)
    assert_close("O[h0]", out[:, 0], o_ref[:, 0], TOL["bf16"]["o"])
    assert_close("O[h1, :20]", out[:, 1, :20], o_ref[:, 1, :20], TOL["bf16"]["o"])
    assert_close("O[h1, 21:]", out[:, 1, 21:], o_ref[:, 1, 21:], TOL["bf16"]["o"])
    dq, dk, dv, dbias = ops.attention_bwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], out,
                                          g["dout"], lse, g["scale"])
    assert torch.count_nonzero(dq[:, 1, 20]).item() == 0
    assert torch.count_nonzero(dbias[1, 20]).item() == 0
    rq, rk, rv, rb = ref.attention_bwd(np64(inp["q"]), np64(inp["k"]), np64(inp["v"]),
                                       np64(inp["bias"]), inp["kmask"].numpy(), inp["scale"],
                                       np64(inp["dout"]))
    tol = TOL["bf16"]["grad"]
    assert_close("dQ", dq, rq, tol)
    assert_close("dK", dk, rk, tol)
    assert_close("dV", dv, rv, tol)
    assert_close("dBias", dbias, rb, tol)
