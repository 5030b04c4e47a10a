"""Every entry point under HIP graph capture. The handlers of the reference declare XLA's
command-buffer trait (cuda/volta_mma_attn.cu:338-351, cuda/volta_ops.cu:87-95, :254-265), so a
caller may capture them; the library records only kernel launches on the given stream (no
allocation, synchronisation or memset). Each graph is captured once after an eager warm-up call,
then replayed several times with eager work in between that overwrites its outputs; every replay
must give the eager result bit for bit. Also: calls from several host threads at once."""
import pytest
import torch

from colabfold_legacy_kernels import ops
from colabfold_legacy_kernels.workloads import (attention_inputs, gate_inputs, gdp_weights,
                                                layer_norm_inputs)
from test_gpu_triangle import module_case

pytestmark = pytest.mark.gpu


def _flatten(x):
    if isinstance(x, torch.Tensor):
        return [x]
    out = []
    for t in x:
        out += _flatten(t)
    return out


def _check_replays(fn, replays=3):
    eager = [t.clone() for t in _flatten(fn())]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static = _flatten(fn())
    for r in range(replays):
        for t in static:  # eager work between the replays, on the outputs themselves
            t.fill_(float("nan") if t.is_floating_point() else 0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(static, eager)):
            assert torch.equal(a, b), (r, i)


def test_attention_fwd_bwd_graph(cuda):
    inp = attention_inputs(3, 2, 100, 90, 32, torch.bfloat16, seed=21, device=cuda,
                           masked_tail=0.1, masked_rows=1)
    q, k, v, bias, km, dout, s = (inp[n] for n in ("q", "k", "v", "bias", "kmask", "dout", "scale"))

    def step():
        out, lse = ops.attention_fwd(q, k, v, bias, km, s)
        return out, lse, ops.attention_bwd(q, k, v, bias, km, out, dout, lse, s)

    _check_replays(step)


def test_attention_layouts_gates_and_pair_bias_graph(cuda):
    """The [N,S,H,D] forward and backward, the forward with the gate fused, the separate gate and
    its backward, and the pair-bias projection."""
    inp = attention_inputs(2, 4, 70, 96, 32, torch.bfloat16, seed=23, device=cuda,
                           masked_tail=0.1, masked_rows=1)
    q, k, v, bias, km, s = (inp[n] for n in ("q", "k", "v", "bias", "kmask", "scale"))
    qs, ks, vs, dos = (t.transpose(1, 2).contiguous() for t in (q, k, v, inp["dout"]))
    x, wg, bg = gate_inputs(2, 70, 128, 4 * 32, torch.bfloat16, seed=24, device=cuda)
    g = torch.Generator().manual_seed(25)
    z = torch.randn((16, 24, 128), generator=g).to(torch.bfloat16).to(cuda)
    sc = (1.0 + 0.1 * torch.randn(128, generator=g)).to(cuda)
    of = (0.1 * torch.randn(128, generator=g)).to(cuda)
    w = (torch.randn((128, 4), generator=g) / 11.3).to(torch.bfloat16).to(cuda)
    dgate = torch.randn((2, 70, 128), generator=g).to(torch.bfloat16).to(cuda)

    def step():
        o = ops.attention(q, k, v, bias, km, s)
        os_, lse = ops.attention_nshd(qs, ks, vs, bias, km, s, want_lse=True)
        return (os_, lse, ops.attention_bwd_nshd(qs, ks, vs, bias, km, os_, dos, lse, s),
                ops.attention_gated(q, k, v, bias, km, x, wg, bg, s),
                ops.attention_gate(o, x, wg, bg), ops.attention_gate_bwd(o, x, wg, bg, dgate),
                ops.ln_pair_bias(z, sc, of, w))

    _check_replays(step)


def test_layer_norm_and_gdp_graph(cuda):
    li = layer_norm_inputs(3000, 128, torch.bfloat16, seed=5, device=cuda)
    w = gdp_weights(128, 128, torch.bfloat16, seed=6, device=cuda, bias_std=0.3)
    wb = gdp_weights(128, 128, torch.bfloat16, seed=7, device=cuda, bias_std=0.3)
    x, sc, off, mask, dy = li["x"], li["scale"], li["offset"], li["mask"], li["dy"]

    def step():
        y = ops.layer_norm(x, sc, off)
        return (y, ops.layer_norm_bwd(x, sc, dy), ops.gated_dual_proj(y, *w, mask),
                ops.gated_dual_proj_bwd(x, *w, mask, dy),
                ops.ln_gated_dual_proj(x, sc, off, w, wb, mask))

    _check_replays(step)


@pytest.mark.parametrize("outgoing", [True, False], ids=["outgoing", "incoming"])
def test_triangle_multiply_graph(cuda, outgoing):
    z, mask, ln_in, ws, bs, ln_c = module_case(72, 64, torch.bfloat16, 9, cuda)
    _check_replays(lambda: ops.triangle_multiply(z, mask, ln_in, ws, bs, ln_c, outgoing))


def test_entry_points_from_concurrent_host_threads(cuda):
    """Re-entrancy (no mutable statics; errors are thread-local): four host threads, each on its
    own stream, call the attention forward and backward and LayerNorm at the same time; each
    thread's results equal the same calls made one after another."""
    import threading

    cases = [attention_inputs(2, 2, 70 + 10 * i, 64, 32, torch.bfloat16, seed=40 + i,
                              device=cuda, masked_tail=0.1) for i in range(4)]
    lis = [layer_norm_inputs(500 + i, 128, torch.bfloat16, seed=60 + i, device=cuda)
           for i in range(4)]

    def work(i):
        c, li = cases[i], lis[i]
        out, lse = ops.attention_fwd(c["q"], c["k"], c["v"], c["bias"], c["kmask"], c["scale"])
        grads = ops.attention_bwd(c["q"], c["k"], c["v"], c["bias"], c["kmask"], out, c["dout"],
                                  lse, c["scale"])
        return _flatten((out, lse, grads, ops.layer_norm(li["x"], li["scale"], li["offset"])))

    serial = [[t.clone() for t in work(i)] for i in range(4)]
    torch.cuda.synchronize()
    results, errors = [None] * 4, []

    def run(i):
        try:
            s = torch.cuda.Stream(device=cuda)
            with torch.cuda.stream(s):
                for _ in range(3):
                    r = work(i)
                s.synchronize()
            results[i] = r
        except Exception as e:  # reported below, in the main thread
            errors.append((i, repr(e)))

    threads = [threading.Thread(target=run, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    for i in range(4):
        for a, b in zip(results[i], serial[i]):
            assert torch.equal(a, b), i
