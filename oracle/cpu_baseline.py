"""CPU baseline: the ColabFold jnp math restated in torch float32 on the host cores.

The caller's jnp attention (logits materialised as [N,H,Sq,Sk], additive 1e9*(mask-1) mask,
softmax, P.V; gradients by autodiff) cannot run here -- there is no jax -- so this is the same
math in torch float32 with torch.autograd standing in for jax.grad. It is timed beside the GPU
numbers as a speed-up reference, never as a roofline, and it is test/bench infrastructure only.
"""

import time

import torch

__all__ = ["attention_fwd_bwd", "time_attention_fwd_bwd", "time_layer_norm"]


def attention_fwd_bwd(q, k, v, bias, kmask, scale, dout):
    """float32 forward + backward on the CPU; returns (o, dq, dk, dv, dbias)."""
    q = q.float().requires_grad_(True)
    k = k.float().requires_grad_(True)
    v = v.float().requires_grad_(True)
    bias = bias.float().requires_grad_(True)
    add = (kmask.float() - 1.0)[:, None, None, :] * 1e9
    logits = torch.matmul(q * scale, k.transpose(-1, -2)) + bias[None] + add
    p = torch.softmax(logits, dim=-1)
    o = torch.matmul(p, v)
    o.backward(dout.float())
    return o.detach(), q.grad, k.grad, v.grad, bias.grad


def time_attention_fwd_bwd(inp, rows, threads, min_seconds=10.0, reps_min=3):
    """Median seconds for fwd+bwd over the first ``rows`` rows of ``inp`` (CPU tensors)."""
    torch.set_num_threads(threads)
    sl = slice(0, rows)
    args = (inp["q"][sl], inp["k"][sl], inp["v"][sl], inp["bias"], inp["kmask"][sl],
            inp["scale"], inp["dout"][sl])
    attention_fwd_bwd(*args)  # warm-up
    times = []
    start = time.perf_counter()
    while len(times) < reps_min or (time.perf_counter() - start < min_seconds and len(times) < 50):
        t0 = time.perf_counter()
        attention_fwd_bwd(*args)
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def time_layer_norm(x, scale, offset, threads, reps=5, eps=1e-5):
    """Median seconds of torch float32 LayerNorm over x (CPU)."""
    torch.set_num_threads(threads)
    xf = x.float()
    torch.nn.functional.layer_norm(xf, (x.shape[-1],), scale, offset, eps)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        torch.nn.functional.layer_norm(xf, (x.shape[-1],), scale, offset, eps)
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]
