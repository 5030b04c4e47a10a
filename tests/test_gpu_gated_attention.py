"""Attention with the output gate fused into the forward's epilogue, on the GPU, against the
float64 oracle composed as oracle.attention then oracle.gate (the reference's epilogue stores O,
cuda/volta_mma_attn.cu:256-272, and its caller gates it)."""
import numpy as np
import pytest
import torch

from _util import TOL, assert_close, dname, np64
from colabfold_legacy_kernels import ops
from colabfold_legacy_kernels.workloads import (GATED_ATTENTION_WORKLOADS, attention_inputs,
                                                attention_workload, gate_inputs)
from oracle import attention as ref_attn
from oracle import gate as ref_gate

pytestmark = pytest.mark.gpu

# (N, H, Sq, Sk, D, C, masked_tail, masked_rows): every head dim; one- and two-sub-tile query
# blocks (Sq <= 64 and above) with ragged ends; gate channel counts that fill whole 64-channel
# chunks and ones that end on a half chunk (C % 64 == 32); odd Sk (the element-wise mask path).
CASES = [
    (2, 8, 70, 70, 32, 256, 0.1, 1),
    (3, 4, 64, 64, 32, 128, 0.0, 0),
    (2, 8, 33, 40, 8, 64, 0.1, 0),
    (2, 4, 17, 23, 16, 64, 0.0, 1),
    (1, 2, 130, 96, 64, 128, 0.2, 0),
    (2, 3, 129, 77, 32, 96, 0.05, 1),
    (1, 2, 200, 64, 16, 32, 0.0, 0),
    (2, 1, 1, 1, 32, 160, 0.0, 0),
    (2, 4, 70, 300, 32, 128, 0.5, 1),  # the last two key tiles hold no present key
    (2, 2, 40, 256, 16, 64, 0.7, 0),   # ... the last three
    # More than 256 gate channels: the epilogue's later rounds stage Wg rows into the freed K/V
    # buffer, 128 channels per buffer; 544 ends on a 32-channel round.
    (2, 4, 70, 130, 32, 384, 0.5, 1),  # and a padding tail: the last key tile is never run
    (2, 2, 64, 64, 32, 544, 0.0, 0),
    (1, 8, 33, 200, 16, 544, 0.6, 1),
]


def _inputs(n, h, sq, sk, d, c, tail, rows, dtype, seed, bias_std=0.5):
    inp = attention_inputs(n, h, sq, sk, d, dtype, seed=seed, bias_var=1.0, masked_tail=tail,
                           masked_rows=rows, with_dout=False)
    x, wg, bg = gate_inputs(n, sq, c, h * d, dtype, seed=seed, bias_std=bias_std)
    inp.update(x=x, wg=wg, bg=bg)
    return inp


def _cuda(inp, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}


def _oracle(inp, rows=slice(None)):
    o, _ = ref_attn.attention_fwd(np64(inp["q"][rows]), np64(inp["k"][rows]),
                                  np64(inp["v"][rows]), np64(inp["bias"]),
                                  inp["kmask"][rows].cpu().numpy(), inp["scale"])
    return ref_gate.attention_gate(o, np64(inp["x"][rows]), np64(inp["wg"]), np64(inp["bg"]))


def _call(g, fn=ops.attention_gated):
    return fn(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["x"], g["wg"], g["bg"],
              g["scale"])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=dname)
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:6])))
def test_attention_gated_parity(cuda, case, dtype):
    n, h, sq, sk, d, c, tail, rows = case
    inp = _inputs(n, h, sq, sk, d, c, tail, rows, dtype, seed=sq * 11 + sk + c)
    g = _cuda(inp, cuda)
    gated = _call(g)
    assert gated.shape == (n, sq, h * d) and gated.dtype == dtype
    assert_close("gated", gated, _oracle(inp), TOL[dname(dtype)]["o"])


@pytest.mark.parametrize("case", [CASES[0], CASES[4], CASES[5]],
                         ids=lambda c: "x".join(map(str, c[:6])))
def test_attention_gated_residuals_match_the_plain_forward(cuda, case):
    """The training entry writes the same gated bits as the inference entry, and its ungated O
    and lse are bit-identical to clk_attention_fwd's: the key loop is the same code."""
    n, h, sq, sk, d, c, tail, rows = case
    g = _cuda(_inputs(n, h, sq, sk, d, c, tail, rows, torch.bfloat16, seed=3), cuda)
    gated, out, lse = _call(g, ops.attention_gated_fwd)
    out_ref, lse_ref = ops.attention_fwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"],
                                         g["scale"])
    assert torch.equal(out, out_ref)
    assert torch.equal(lse, lse_ref)
    assert torch.equal(gated, _call(g))


def test_attention_gated_exact_cases(cuda):
    """A zero gate pre-activation halves O exactly; saturated biases pass O through or zero it;
    either way the result sits in the [N,Sq,H*D] layout."""
    n, h, sq, sk, d, c = 2, 8, 70, 70, 32, 256
    g = _cuda(_inputs(n, h, sq, sk, d, c, 0.1, 1, torch.bfloat16, seed=5), cuda)
    _, out, _ = _call(g, ops.attention_gated_fwd)
    ot = out.permute(0, 2, 1, 3).reshape(n, sq, h * d)
    g["wg"] = torch.zeros_like(g["wg"])
    g["bg"] = torch.zeros_like(g["bg"])
    assert torch.equal(_call(g), 0.5 * ot)
    g["bg"] = torch.full_like(g["bg"], 100.0)
    assert torch.equal(_call(g), ot)
    g["bg"] = torch.full_like(g["bg"], -100.0)
    assert torch.count_nonzero(_call(g)) == 0


def test_attention_gated_without_mask(cuda):
    n, h, sq, sk, d, c = 2, 4, 64, 96, 32, 128
    g = _cuda(_inputs(n, h, sq, sk, d, c, 0.0, 0, torch.bfloat16, seed=6), cuda)
    a = ops.attention_gated(g["q"], g["k"], g["v"], g["bias"], None, g["x"], g["wg"], g["bg"])
    b = _call(g)
    assert torch.equal(a, b)


@pytest.mark.parametrize("name", sorted(GATED_ATTENTION_WORKLOADS))
def test_attention_gated_workload(cuda, name):
    """The full-size gated workloads (MSA row attention with its 256-channel gate, 20% of the
    rows fully padded; 1024-residue triangle attention with its 128-channel gate): two calls
    agree bit for bit, and rows sampled across the batch -- fully padded ones included --
    match the oracle."""
    inp = attention_workload(name, torch.bfloat16, with_dout=False)
    n, h, sq, d = inp["q"].shape
    c = GATED_ATTENTION_WORKLOADS[name]
    x, wg, bg = gate_inputs(n, sq, c, h * d, torch.bfloat16, seed=7)
    inp.update(x=x, wg=wg, bg=bg)
    g = _cuda(inp, cuda)
    a = _call(g)
    assert torch.equal(a, _call(g))
    empty = np.flatnonzero((inp["kmask"].numpy() == 0).all(axis=1))
    rows = sorted(set([0, n - 1, n // 3] + list(empty[:2])))
    assert_close("gated", a[rows], _oracle(inp, rows), TOL["bf16"]["o"])
