"""Benchmark of the Evoformer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--min-warmup-ms T] [--no-cpu-baseline]

Headline (one JSON line on stdout): triangle attention forward + backward at N_res = 384
(q, k, v [384 rows, 4 heads, 384 residues, 32], bf16 in, float32 accumulate), in TFLOP/s of
algorithmic work 12*N*H*Sq*Sk*D per step. A step is one forward and one backward over the whole
batch, through the C ABI with preallocated buffers; inputs rotate over 3 sets (~0.9 GB) so the
256 MB Infinity Cache cannot hold them. Exactly K steps are timed after W untimed warm-up steps;
the warm-up continues past W steps until T ms (default 100) have passed, because the GPU's
clocks ramp up over its first ~20 ms of work (the first 50 steps of a process run ~8% slower
than every later pass); the JSON line reports the warm-up steps actually run. ms_per_step is the
mean over the bracket of K steps (one HIP event before the first and one after the last, a device
synchronize on both sides, nothing recorded in between); the median, min and max of a second
pass with an event after every step are reported beside it (those events add 2-4 us to each
step). Every secondary figure is a bracket mean the same way. Secondary figures: LayerNorm
forward/backward, LayerNorm + gated dual projection, the plain projection and its backward and
the pair-bias projection on the 512x512x128 pair representation; the attention output gate of
MSA row attention (512 rows x 256 queries, 8 x 32 heads, 256 channels) and its backward; gated
attention fused and separate on MSA rows and at N_res = 1024; the triangle multiplication
(outgoing, incoming) on z [512,512,128] per kernel; the library's streaming copy as the HBM
ceiling.

The roofline block names the kernel with the most time per step, its algorithmic work per launch
divided by its average duration from per-launch HIP events on the launch stream (the library's
clk_profile_* hooks), against MI355X's dense bf16 MFMA peak (2516.6 TFLOP/s) or HBM (8 TB/s).
roofline.traffic is the dominant kernel's HBM bytes per launch as recorded by the committed
rocprofv3 FETCH_SIZE/WRITE_SIZE summaries in profiles/*hbm_traffic*.md (lines
"traffic_bytes_per_launch[<kernel>]: <bytes>"), null when none covers the kernel. Those runs
scale each counter by what it reads for a plain device copy of known size, which
"--copy-calibration MIB" performs (and nothing else). roofline.issue is the same kernel's
instruction-issue floor -- its VALU, transcendental and MFMA wave instructions per launch, from
the committed profiles/*instruction_mix*.md, at 4, 8 and 16 cycles each over the 1024 SIMDs at
2.4 GHz (the costs "--issue-calibration" measures) -- and frac = floor / measured duration.
cpu_baseline times the same math in torch float32 on the host cores (oracle/cpu_baseline.py) on
all 384 rows by default (--cpu-rows for fewer), repeated for about --cpu-seconds (10 s) and
reported as the median run in the same unit.
"""

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "colabfold-legacy-kernels_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "attn fwd+bwd TFLOP/s (% bf16 MFMA peak) at N_res=384; LN/GDP HBM GB/s"
MFMA_PEAK_BF16 = 2516.6  # TFLOP/s, dense
HBM_PEAK = 8000.0        # GB/s

N_ROWS, HEADS, NRES, HEAD_DIM = 384, 4, 384, 32
ROTATE = 3

# Issue costs of one MI355X (256 CUs x 4 SIMDs at 2.4 GHz): a wave64 VALU instruction occupies a
# 16-lane SIMD for 4 cycles (the published 157.3 TFLOP/s vector fp32 counts two lanes per packed
# instruction); a float32 transcendental (v_exp_f32) 8 cycles; a 16x16x32 bf16 MFMA (16384 flops)
# 16 cycles at the 2516.6 TFLOP/s peak. "--issue-calibration" measures them: 4.3, 8.6 and 17.4
# cycles at three waves per SIMD; FMAs and exponentials share the issue slots, while half to
# three quarters of the MFMAs' time hides under them.
SIMDS, CLOCK_HZ = 1024, 2.4e9
VALU_CYCLES, TRANS_CYCLES, MFMA_CYCLES = 4, 8, 16


def _cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def attention_flops(n, h, sq, sk, d):
    fwd = 4.0 * n * h * sq * sk * d
    return {"fwd": fwd, "bwd": 2.0 * fwd, "step": 3.0 * fwd,
            # per kernel: the products whose results the kernel owns (recomputes excluded)
            "attn_fwd": fwd, "attn_bwd_dkv": 1.5 * fwd, "attn_bwd_dq": 0.5 * fwd}


class AttentionSet:
    """One rotating set of inputs and preallocated outputs for the C ABI."""

    def __init__(self, torch, workloads, native, dev, seed, dtype=None):
        dtype = torch.bfloat16 if dtype is None else dtype
        inp = workloads.attention_inputs(N_ROWS, HEADS, NRES, NRES, HEAD_DIM, dtype,
                                         seed=seed, device=dev, masked_tail=0.10)
        self.__dict__.update(inp)
        self.code = native.BF16 if dtype == torch.bfloat16 else native.F16
        self.out = torch.empty_like(self.q)
        self.lse = torch.empty((N_ROWS, HEADS, NRES), device=dev, dtype=torch.float32)
        self.dq = torch.empty_like(self.q)
        self.dk = torch.empty_like(self.k)
        self.dv = torch.empty_like(self.v)
        self.dbias = torch.empty((HEADS, NRES, NRES), device=dev, dtype=torch.float32)
        lib = native.lib()
        self.ws_bytes = lib.clk_attention_bwd_workspace_size(N_ROWS, HEADS, NRES, NRES, HEAD_DIM)
        self.ws = torch.empty(max(self.ws_bytes, 1), device=dev, dtype=torch.uint8)


def attention_step(lib, native, stream, s):
    dims = (N_ROWS, HEADS, NRES, NRES, HEAD_DIM)
    st = lib.clk_attention_fwd(stream, s.code, s.q.data_ptr(), s.k.data_ptr(),
                               s.v.data_ptr(), s.bias.data_ptr(), s.kmask.data_ptr(),
                               s.out.data_ptr(), s.lse.data_ptr(), *dims, s.scale, 64, 64)
    if st != 0:
        raise RuntimeError(native.last_error())
    st = lib.clk_attention_bwd(stream, s.code, s.q.data_ptr(), s.k.data_ptr(),
                               s.v.data_ptr(), s.bias.data_ptr(), s.kmask.data_ptr(),
                               s.out.data_ptr(), s.dout.data_ptr(), s.lse.data_ptr(),
                               s.dq.data_ptr(), s.dk.data_ptr(), s.dv.data_ptr(),
                               s.dbias.data_ptr(), s.ws.data_ptr(), s.ws_bytes, *dims, s.scale)
    if st != 0:
        raise RuntimeError(native.last_error())


# Minimum warm-up wall time of every timed section (--min-warmup-ms).
MIN_WARMUP_MS = 100.0


def timed(torch, fn, steps, warmup, stream_obj, stats=None, min_warmup_ms=None):
    """Mean ms per step over `steps` timed steps after `warmup` untimed ones: one HIP event on
    the launch stream before the first step and one after the last, with a device synchronize
    on both sides (nothing else is recorded between the steps: an event recorded after every
    step puts a timestamp between each pair of launches, measured at 2-4 us per step on the
    short kernels). The warm-up continues past `warmup` steps until min_warmup_ms (default
    MIN_WARMUP_MS) of wall time has passed: the GPU's clocks ramp up over its first ~20 ms of work
    and again after each idle stretch, such as building the next section's inputs. `stats`
    (a dict), when given, also receives the warm-up actually run and, from a second pass of
    `steps` steps with an event after every step, the median, min and max step."""
    if min_warmup_ms is None:
        min_warmup_ms = MIN_WARMUP_MS
    t0 = time.perf_counter()
    i = 0
    while i < warmup:
        fn(i)
        i += 1
    if min_warmup_ms > 0:
        torch.cuda.synchronize()
        while (time.perf_counter() - t0) * 1e3 < min_warmup_ms:
            fn(i)
            i += 1
            if i % 16 == 0:
                torch.cuda.synchronize()
    torch.cuda.synchronize()
    if stats is not None:
        stats["warmup_run"] = i
        stats["warmup_ms"] = (time.perf_counter() - t0) * 1e3
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream_obj)
    for i in range(steps):
        fn(i)
    e1.record(stream_obj)
    torch.cuda.synchronize()
    mean = e0.elapsed_time(e1) / steps
    if stats is not None:
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        ev[0].record(stream_obj)
        for i in range(steps):
            fn(i)
            ev[i + 1].record(stream_obj)
        torch.cuda.synchronize()
        per = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
        mid = len(per) // 2
        stats["median_ms"] = per[mid] if len(per) % 2 else 0.5 * (per[mid - 1] + per[mid])
        stats["min_ms"], stats["max_ms"] = per[0], per[-1]
    return mean


def per_kernel(torch, native, fn, steps):
    """Average ms per launch of each kernel, from the library's per-launch HIP events."""
    torch.cuda.synchronize()
    with native.profile() as prof:
        for i in range(steps):
            fn(i)
    torch.cuda.synchronize()
    agg = {}
    for name, ms in prof.records:
        tot, cnt = agg.get(name, (0.0, 0))
        agg[name] = (tot + ms, cnt + 1)
    return {k: {"avg_ms": t / c, "launches_per_step": c / steps} for k, (t, c) in agg.items()}


def bench_attention_f16(torch, workloads, native, dev, stream, steps, warmup):
    """The headline step in float16, the reference's own operand type (same shapes, 3 rotating
    sets)."""
    lib = native.lib()
    sets = [AttentionSet(torch, workloads, native, dev, seed=11 + r, dtype=torch.float16)
            for r in range(ROTATE)]

    def step(i):
        attention_step(lib, native, stream, sets[i % ROTATE])

    ms = timed(torch, step, steps, warmup, torch.cuda.current_stream(dev))
    flops = attention_flops(N_ROWS, HEADS, NRES, NRES, HEAD_DIM)["step"]
    return {"attn_f16_ms": ms, "attn_f16_TFLOPs": flops / (ms * 1e-3) / 1e12}


def bench_layer_norm(torch, workloads, native, dev, stream, steps, warmup):
    """LayerNorm fwd and bwd on [512*512, 128] bf16; rotates 4 sets (> 512 MB)."""
    m, c = 512 * 512, 128
    lib = native.lib()
    sets = []
    for r in range(4):
        li = workloads.layer_norm_inputs(m, c, torch.bfloat16, seed=3 + r, device=dev)
        li["y"] = torch.empty_like(li["x"])
        li["dx"] = torch.empty_like(li["x"])
        li["ds"] = torch.empty(c, device=dev)
        li["do"] = torch.empty(c, device=dev)
        wsb = lib.clk_layer_norm_bwd_workspace_size(m, c)
        li["ws"] = torch.empty(wsb, device=dev, dtype=torch.uint8)
        li["wsb"] = wsb
        sets.append(li)

    def fwd(i):
        s = sets[i % len(sets)]
        lib.clk_layer_norm_fwd(stream, native.BF16, s["x"].data_ptr(), s["scale"].data_ptr(),
                               s["offset"].data_ptr(), s["y"].data_ptr(), m, c, 1e-5)

    def bwd(i):
        s = sets[i % len(sets)]
        lib.clk_layer_norm_bwd(stream, native.BF16, s["x"].data_ptr(), s["scale"].data_ptr(),
                               s["dy"].data_ptr(), s["dx"].data_ptr(), s["ds"].data_ptr(),
                               s["do"].data_ptr(), s["ws"].data_ptr(), s["wsb"], m, c, 1e-5)

    so = torch.cuda.current_stream(dev)
    t_f = timed(torch, fwd, steps, warmup, so)
    t_b = timed(torch, bwd, steps, warmup, so)
    bytes_f = m * c * 4.0
    bytes_b = m * c * 6.0
    kf = per_kernel(torch, native, fwd, steps)
    kb = per_kernel(torch, native, bwd, steps)
    return {
        "ln_fwd_GBps": bytes_f / (t_f * 1e-3) / 1e9, "ln_fwd_ms": t_f,
        "ln_bwd_GBps": bytes_b / (t_b * 1e-3) / 1e9, "ln_bwd_ms": t_b,
        "ln_fwd_kernel_ms": kf.get("ln_fwd", {}).get("avg_ms"),
        "ln_bwd_kernel_ms": kb.get("ln_bwd", {}).get("avg_ms"),
        "ln_bwd_colsum_ms": kb.get("ln_bwd_colsum", {}).get("avg_ms"),
        "ln_bytes_fwd": bytes_f, "ln_bytes_bwd": bytes_b,
    }


def bench_hbm_copy(torch, native, dev, stream, steps, warmup):
    """The library's own streaming copy (clk_stream_copy) of 512 MiB, two rotating buffer pairs
    (2 GiB): the HBM rate its HBM-bound kernels can reach, read + write bytes per second."""
    lib = native.lib()
    nbytes = 512 << 20
    pairs = [(torch.empty(nbytes, device=dev, dtype=torch.uint8).fill_(r),
              torch.empty(nbytes, device=dev, dtype=torch.uint8)) for r in range(2)]

    def run(i):
        a, b = pairs[i % 2]
        st = lib.clk_stream_copy(stream, a.data_ptr(), b.data_ptr(), nbytes)
        if st != 0:
            raise RuntimeError(native.last_error())

    t = timed(torch, run, steps, warmup, torch.cuda.current_stream(dev))
    return {"hbm_copy_GBps": 2.0 * nbytes / (t * 1e-3) / 1e9, "hbm_copy_ms": t}


def bench_ln_gdp(torch, workloads, native, dev, stream, steps, warmup):
    """LayerNorm + both gated branches on z [512*512, 128] bf16 (a, b [512*512, 128])."""
    m, c, n = 512 * 512, 128, 128
    lib = native.lib()
    sets = []
    for r in range(3):
        li = workloads.layer_norm_inputs(m, c, torch.bfloat16, seed=3 + r, device=dev)
        wa = workloads.gdp_weights(c, n, torch.bfloat16, seed=21 + r, device=dev)
        wb = workloads.gdp_weights(c, n, torch.bfloat16, seed=41 + r, device=dev)
        sets.append((li, wa, wb, torch.empty((m, n), device=dev, dtype=torch.bfloat16),
                     torch.empty((m, n), device=dev, dtype=torch.bfloat16)))

    # The call's sixteen device pointers per set, taken once: the timed loop then issues the
    # launches well ahead of the GPU.
    args = [(li["x"].data_ptr(), li["scale"].data_ptr(), li["offset"].data_ptr(),
             *(t.data_ptr() for t in wa), *(t.data_ptr() for t in wb), li["mask"].data_ptr(),
             a.data_ptr(), b.data_ptr()) for li, wa, wb, a, b in sets]

    def run(i):
        st = lib.clk_ln_gated_dual_proj(stream, native.BF16, *args[i % len(args)], m, c, n, 1e-5)
        if st != 0:
            raise RuntimeError(native.last_error())

    so = torch.cuda.current_stream(dev)
    t = timed(torch, run, steps, warmup, so)
    nbytes = m * c * 2.0 + m * 2.0 + 2.0 * m * n * 2.0 + 4.0 * c * n * 2.0
    k = per_kernel(torch, native, run, steps)
    return {"ln_gdp_GBps": nbytes / (t * 1e-3) / 1e9, "ln_gdp_ms": t,
            "ln_gdp_kernel_ms": k.get("ln_gdp", {}).get("avg_ms"), "ln_gdp_bytes": nbytes,
            "ln_gdp_TFLOPs": 4 * 2.0 * m * c * n / (t * 1e-3) / 1e12}


def bench_gdp(torch, workloads, native, dev, stream, steps, warmup):
    """The reference's gated dual projection (VoltaGdp) on x [512*512, 128] bf16, 128x128
    weights, one branch per call; 4 rotating sets."""
    m, k, n = 512 * 512, 128, 128
    lib = native.lib()
    sets = []
    for r in range(4):
        li = workloads.layer_norm_inputs(m, k, torch.bfloat16, seed=60 + r, device=dev)
        w = workloads.gdp_weights(k, n, torch.bfloat16, seed=70 + r, device=dev)
        sets.append((li, w, torch.empty((m, n), device=dev, dtype=torch.bfloat16)))

    def run(i):
        li, w, out = sets[i % len(sets)]
        st = lib.clk_gated_dual_proj(stream, native.BF16, li["x"].data_ptr(),
                                     *(t.data_ptr() for t in w), li["mask"].data_ptr(),
                                     out.data_ptr(), m, k, n)
        if st != 0:
            raise RuntimeError(native.last_error())

    t = timed(torch, run, steps, warmup, torch.cuda.current_stream(dev))
    nbytes = m * k * 2.0 + m * 2.0 + m * n * 2.0 + 2.0 * k * n * 2.0
    kt = per_kernel(torch, native, run, steps)
    return {"gdp_GBps": nbytes / (t * 1e-3) / 1e9, "gdp_ms": t,
            "gdp_kernel_ms": kt.get("gdp", {}).get("avg_ms"), "gdp_bytes": nbytes}


def bench_gdp_bwd(torch, workloads, native, dev, stream, steps, warmup):
    """Gated dual projection backward on x [512*512, 128] bf16, 128x128 weights, dout ~N(0,1);
    2 rotating sets. Reports the call time and each kernel's."""
    m, k, n = 512 * 512, 128, 128
    lib = native.lib()
    wsb = lib.clk_gated_dual_proj_bwd_workspace_size(m, k, n)
    sets = []
    for r in range(2):
        li = workloads.layer_norm_inputs(m, k, torch.bfloat16, seed=30 + r, device=dev)
        w = workloads.gdp_weights(k, n, torch.bfloat16, seed=50 + r, device=dev)
        dout = torch.randn((m, n), device=dev).to(torch.bfloat16)
        f32 = dict(device=dev, dtype=torch.float32)
        grads = (torch.empty_like(li["x"]), torch.empty((k, n), **f32), torch.empty(n, **f32),
                 torch.empty((k, n), **f32), torch.empty(n, **f32))
        sets.append((li, w, dout, grads, torch.empty(wsb, dtype=torch.uint8, device=dev)))

    def run(i):
        li, w, dout, gr, ws = sets[i % len(sets)]
        st = lib.clk_gated_dual_proj_bwd(stream, native.BF16, li["x"].data_ptr(),
                                         *(t.data_ptr() for t in w), li["mask"].data_ptr(),
                                         dout.data_ptr(), *(t.data_ptr() for t in gr),
                                         ws.data_ptr(), wsb, m, k, n, 0)
        if st != 0:
            raise RuntimeError(native.last_error())

    t = timed(torch, run, steps, warmup, torch.cuda.current_stream(dev))
    kt = per_kernel(torch, native, run, steps)
    out = {"gdp_bwd_ms": t}
    for name, v in kt.items():
        out["gdp_bwd_%s_ms" % name.replace("gdp_bwd_", "")] = v["avg_ms"]
    return out


def bench_pair_bias(torch, workloads, native, dev, stream, steps, warmup):
    """Pair-bias projection LN(z).w -> [4, 512, 512] on z [512*512, 128] bf16; 4 rotating sets."""
    m, c, h = 512 * 512, 128, 4
    lib = native.lib()
    sets = []
    for r in range(4):
        li = workloads.layer_norm_inputs(m, c, torch.bfloat16, seed=7 + r, device=dev)
        w = (torch.randn((c, h)) / c ** 0.5).to(torch.bfloat16).to(dev)
        sets.append((li, w, torch.empty((h, m), dtype=torch.bfloat16, device=dev)))

    def run(i):
        li, w, out = sets[i % len(sets)]
        st = lib.clk_ln_pair_bias(stream, native.BF16, li["x"].data_ptr(), li["scale"].data_ptr(),
                                  li["offset"].data_ptr(), w.data_ptr(), out.data_ptr(), m, c, h,
                                  1e-5)
        if st != 0:
            raise RuntimeError(native.last_error())

    t = timed(torch, run, steps, warmup, torch.cuda.current_stream(dev))
    nbytes = m * c * 2.0 + h * m * 2.0
    k = per_kernel(torch, native, run, steps)
    return {"pair_bias_GBps": nbytes / (t * 1e-3) / 1e9, "pair_bias_ms": t,
            "pair_bias_kernel_ms": k.get("ln_bias", {}).get("avg_ms")}


def bench_attn_gate(torch, native, dev, stream, steps, warmup):
    """Attention output gate of MSA row attention: o [512,8,256,32], x [512,256,256] ~N(0,1),
    wg [256,256] ~N(0,1/256), bg = 0, bf16 -> [512,256,256]; rotates 3 sets (600 MB)."""
    n, h, sq, d, c = 512, 8, 256, 32, 256
    lib = native.lib()
    sets = []
    for r in range(3):
        g = torch.Generator(device="cpu").manual_seed(60 + r)
        o = torch.randn((n, h, sq, d), generator=g).to(torch.bfloat16).to(dev)
        x = torch.randn((n, sq, c), generator=g).to(torch.bfloat16).to(dev)
        wg = (torch.randn((c, h * d), generator=g) / c ** 0.5).to(torch.bfloat16).to(dev)
        bg = torch.zeros(h * d, dtype=torch.bfloat16, device=dev)
        sets.append((o, x, wg, bg, torch.empty((n, sq, h * d), dtype=torch.bfloat16, device=dev)))

    def run(i):
        o, x, wg, bg, out = sets[i % len(sets)]
        st = lib.clk_attention_gate(stream, native.BF16, o.data_ptr(), x.data_ptr(),
                                    wg.data_ptr(), bg.data_ptr(), out.data_ptr(), n, h, sq, d, c)
        if st != 0:
            raise RuntimeError(native.last_error())

    so = torch.cuda.current_stream(dev)
    t = timed(torch, run, steps, warmup, so)
    nbytes = 2.0 * n * sq * (2 * h * d + c) + 2.0 * c * h * d
    k = per_kernel(torch, native, run, steps)
    return {"attn_gate_GBps": nbytes / (t * 1e-3) / 1e9, "attn_gate_ms": t,
            "attn_gate_kernel_ms": k.get("attn_gate", {}).get("avg_ms"),
            "attn_gate_bytes": nbytes}


def bench_attn_gate_bwd(torch, native, dev, stream, steps, warmup):
    """Backward of the MSA row attention's output gate (the shapes of bench_attn_gate, dout
    ~N(0,1), bg ~N(0,0.25)): do, dx, dwg, dbg; rotates 2 sets (~0.8 GB). Bytes counted: one read
    of o, x and dout and one write of do and dx (the op's inputs and outputs; the kernels also
    write and re-read the gate-logit gradient dg and re-read x for dwg)."""
    n, h, sq, d, c = 512, 8, 256, 32, 256
    lib = native.lib()
    bf = dict(dtype=torch.bfloat16, device=dev)
    wsb = lib.clk_attention_gate_bwd_workspace_size(n, h, sq, d, c)
    sets = []
    for r in range(2):
        g = torch.Generator(device="cpu").manual_seed(70 + r)
        o = torch.randn((n, h, sq, d), generator=g).to(**bf)
        x = torch.randn((n, sq, c), generator=g).to(**bf)
        wg = (torch.randn((c, h * d), generator=g) / c ** 0.5).to(**bf)
        bg = (0.5 * torch.randn(h * d, generator=g)).to(**bf)
        dout = torch.randn((n, sq, h * d), generator=g).to(**bf)
        outs = (torch.empty_like(o), torch.empty_like(x),
                torch.empty((c, h * d), device=dev), torch.empty(h * d, device=dev),
                torch.empty(wsb, dtype=torch.uint8, device=dev))
        sets.append((o, x, wg, bg, dout) + outs)

    def run(i):
        o, x, wg, bg, dout, do, dx, dwg, dbg, ws = sets[i % len(sets)]
        st = lib.clk_attention_gate_bwd(stream, native.BF16, o.data_ptr(), x.data_ptr(),
                                        wg.data_ptr(), bg.data_ptr(), dout.data_ptr(),
                                        do.data_ptr(), dx.data_ptr(), dwg.data_ptr(),
                                        dbg.data_ptr(), ws.data_ptr(), wsb, n, h, sq, d, c, 0)
        if st != 0:
            raise RuntimeError(native.last_error())

    so = torch.cuda.current_stream(dev)
    t = timed(torch, run, steps, warmup, so)
    nbytes = 2.0 * n * sq * (2 * h * d + c) + 2.0 * n * sq * (h * d + c)
    k = per_kernel(torch, native, run, steps)
    res = {"attn_gate_bwd_GBps": nbytes / (t * 1e-3) / 1e9, "attn_gate_bwd_ms": t,
           "attn_gate_bwd_bytes": nbytes}
    for name in ("gate_bwd_grad", "gate_bwd_dx", "gate_bwd_dw", "gate_bwd_sum"):
        res[name + "_ms"] = k.get(name, {}).get("avg_ms")
    return res


def bench_gated_attention(torch, workloads, native, dev, stream, steps, warmup):
    """Gated attention forward on the two gated workloads (MSA row attention with a 256-channel
    gate, 1024-residue triangle attention with a 128-channel gate), bf16: the fused entry
    (clk_attention_fwd_gated, O never stored) against the forward followed by the separate gate
    kernel. Two rotating sets each (> 512 MB)."""
    lib = native.lib()
    res = {}
    for name, tag in (("msa_row_attn", "msa"), ("triangle_attn_1024", "tri1024")):
        c = workloads.GATED_ATTENTION_WORKLOADS[name]
        sets = []
        for r in range(2):
            inp = workloads.attention_workload(name, torch.bfloat16, device=dev, with_dout=False)
            n, h, sq, d = inp["q"].shape
            sk = inp["k"].shape[2]
            x, wg, bg = workloads.gate_inputs(n, sq, c, h * d, torch.bfloat16, seed=70 + r,
                                              device=dev)
            inp.update(x=x, wg=wg, bg=bg, out=torch.empty_like(inp["q"]),
                       gated=torch.empty((n, sq, h * d), dtype=torch.bfloat16, device=dev))
            sets.append(inp)
        dims = (n, h, sq, sk, d)

        def fused(i):
            s = sets[i % 2]
            st = lib.clk_attention_fwd_gated(
                stream, native.BF16, s["q"].data_ptr(), s["k"].data_ptr(), s["v"].data_ptr(),
                s["bias"].data_ptr(), s["kmask"].data_ptr(), s["x"].data_ptr(),
                s["wg"].data_ptr(), s["bg"].data_ptr(), s["gated"].data_ptr(), None, None,
                *dims, c, s["scale"])
            if st != 0:
                raise RuntimeError(native.last_error())

        def separate(i):
            s = sets[i % 2]
            st = lib.clk_attention_fwd(stream, native.BF16, s["q"].data_ptr(),
                                       s["k"].data_ptr(), s["v"].data_ptr(),
                                       s["bias"].data_ptr(), s["kmask"].data_ptr(),
                                       s["out"].data_ptr(), None, *dims, s["scale"], 64, 64)
            if st == 0:
                st = lib.clk_attention_gate(stream, native.BF16, s["out"].data_ptr(),
                                            s["x"].data_ptr(), s["wg"].data_ptr(),
                                            s["bg"].data_ptr(), s["gated"].data_ptr(), n, h, sq,
                                            d, c)
            if st != 0:
                raise RuntimeError(native.last_error())

        so = torch.cuda.current_stream(dev)
        tf = timed(torch, fused, steps, warmup, so)
        ts = timed(torch, separate, steps, warmup, so)
        flops = attention_flops(n, h, sq, sk, d)["fwd"]
        res.update({"gated_%s_fused_ms" % tag: tf, "gated_%s_separate_ms" % tag: ts,
                    "gated_%s_fused_TFLOPs" % tag: flops / (tf * 1e-3) / 1e12,
                    "gated_%s_speedup" % tag: ts / tf})
        del sets
    return res


def bench_attention_nshd(torch, workloads, native, dev, stream, steps, warmup):
    """MSA row attention's forward (bf16) with q, k, v and O in AlphaFold's [N,S,H,D] layout:
    clk_attention_fwd_nshd on them directly, against transposing q, k, v to [N,H,S,D] (torch
    copies), clk_attention_fwd, and transposing O back -- what a caller of the [N,H,S,D] entry
    does -- and against clk_attention_fwd alone. Two rotating sets."""
    lib = native.lib()
    sets = []
    for r in range(2):
        inp = workloads.attention_workload("msa_row_attn", torch.bfloat16, device=dev,
                                           with_dout=False)
        t = {key: inp[key].transpose(1, 2).contiguous() for key in ("q", "k", "v")}
        inp.update(qs=t["q"], ks=t["k"], vs=t["v"], outs=torch.empty_like(t["q"]),
                   out=torch.empty_like(inp["q"]))
        sets.append(inp)
    n, h, sq, d = sets[0]["q"].shape
    sk = sets[0]["k"].shape[2]

    def run(st):
        if st != 0:
            raise RuntimeError(native.last_error())

    def nshd(i):
        s = sets[i % 2]
        run(lib.clk_attention_fwd_nshd(stream, native.BF16, s["qs"].data_ptr(),
                                       s["ks"].data_ptr(), s["vs"].data_ptr(),
                                       s["bias"].data_ptr(), s["kmask"].data_ptr(),
                                       s["outs"].data_ptr(), None, n, h, sq, sk, d, s["scale"]))

    def nhsd(s, q, k, v):
        run(lib.clk_attention_fwd(stream, native.BF16, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                  s["bias"].data_ptr(), s["kmask"].data_ptr(), s["out"].data_ptr(),
                                  None, n, h, sq, sk, d, s["scale"], 64, 64))

    def plain(i):
        s = sets[i % 2]
        nhsd(s, s["q"], s["k"], s["v"])

    def transposed(i):
        s = sets[i % 2]
        q, k, v = (s[key].transpose(1, 2).contiguous() for key in ("qs", "ks", "vs"))
        nhsd(s, q, k, v)
        s["outs"].copy_(s["out"].transpose(1, 2))

    so = torch.cuda.current_stream(dev)
    res = {"attn_nshd_msa_ms": timed(torch, nshd, steps, warmup, so),
           "attn_nhsd_msa_ms": timed(torch, plain, steps, warmup, so),
           "attn_nhsd_transposed_msa_ms": timed(torch, transposed, steps, warmup, so)}
    del sets
    return res


def bench_triangle(torch, native, dev, stream, steps, warmup):
    """Triangle multiplication (outgoing and incoming) on z [512,512,128] bf16 ~N(0,1), mask
    Bernoulli(0.95), six 128x128 weights ~N(0,1/128), biases 0, LayerNorm scales 1 + N(0,0.1)
    and offsets N(0,0.1); 2 rotating sets. Reports each kernel's time per call and the
    contraction's TFLOP/s (2*N^3*C flops)."""
    import ctypes
    n, c = 512, 128
    lib = native.lib()
    g = torch.Generator(device="cpu").manual_seed(80)
    rnd = lambda *s, std=1.0: (torch.randn(s, generator=g) * std)  # noqa: E731
    wsb = lib.clk_triangle_multiply_workspace_size(n, c)
    sets = []
    for _ in range(2):
        z = rnd(n, n, c).to(torch.bfloat16).to(dev)
        mask = (torch.rand((n, n), generator=g) < 0.95).to(torch.bfloat16).to(dev)
        lns = [(1 + rnd(c, std=0.1)).to(dev), rnd(c, std=0.1).to(dev),
               (1 + rnd(c, std=0.1)).to(dev), rnd(c, std=0.1).to(dev)]
        ws = [rnd(c, c, std=c ** -0.5).to(torch.bfloat16).to(dev) for _ in range(6)]
        bs = [torch.zeros(c, dtype=torch.bfloat16, device=dev) for _ in range(6)]
        sets.append((z, mask, lns, ws, bs, torch.empty_like(z),
                     torch.empty(wsb, dtype=torch.uint8, device=dev)))
    arr = lambda ts: (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])  # noqa: E731
    out = {}
    for outgoing, tag in ((1, "tri_out"), (0, "tri_in")):
        def run(i, outgoing=outgoing):
            z, mask, lns, ws, bs, o, w = sets[i % len(sets)]
            st = lib.clk_triangle_multiply(stream, native.BF16, z.data_ptr(), mask.data_ptr(),
                                           arr(lns), arr(ws), arr(bs), o.data_ptr(),
                                           w.data_ptr(), wsb, n, c, outgoing, 1e-5)
            if st != 0:
                raise RuntimeError(native.last_error())
        t = timed(torch, run, steps, warmup, torch.cuda.current_stream(dev))
        k = per_kernel(torch, native, run, steps)
        out[tag + "_ms"] = t
        for name, v in k.items():
            out["%s_%s_ms_per_call" % (tag, name)] = v["avg_ms"] * v["launches_per_step"]
        ke = k.get("tri_einsum", {}).get("avg_ms")
        if ke:
            out[tag + "_einsum_TFLOPs"] = 2.0 * n ** 3 * c / (ke * 1e-3) / 1e12
    return out


def recorded_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summaries."""
    pat = re.compile(r"^traffic_bytes_per_launch\[(\w+)\]:\s*([0-9.eE+]+)\s*$")
    found = None
    for f in sorted((ROOT / "profiles").glob("*hbm_traffic*.md")):
        for line in f.read_text().splitlines():
            m = pat.match(line.strip())
            if m and m.group(1) == kernel:
                found = float(m.group(2))
    return found


def recorded_instructions(kernel):
    """{"valu", "trans", "mfma"}: wave instructions per launch of `kernel` (VALU excluding MFMA
    and transcendentals; float32 transcendentals; MFMA) from the committed rocprofv3
    instruction-mix summaries, lines "<kind>_instructions_per_launch[<kernel>]: <n>"; None when
    no summary covers the kernel."""
    pat = re.compile(r"^(valu|trans|mfma)_instructions_per_launch\[(\w+)\]:\s*([0-9.eE+]+)\s*$")
    found = {}
    for f in sorted((ROOT / "profiles").glob("*instruction_mix*.md")):
        for line in f.read_text().splitlines():
            m = pat.match(line.strip())
            if m and m.group(2) == kernel:
                found[m.group(1)] = float(m.group(3))
    return found if len(found) == 3 else None


def issue_cycles(valu, trans, mfma):
    """(VALU + transcendental, MFMA) SIMD cycles of that many wave instructions."""
    return valu * VALU_CYCLES + trans * TRANS_CYCLES, mfma * MFMA_CYCLES


def issue_bound(kernel, avg_ms, scores):
    """The kernel's instruction-issue floor: its recorded wave instructions at VALU_CYCLES,
    TRANS_CYCLES and MFMA_CYCLES SIMD cycles each over all SIMDs at CLOCK_HZ. bound_ms adds
    them all (a wave issues one instruction at a time; the calibration finds FMAs and
    exponentials sharing the issue slots); bound_ms_mfma_hidden counts the VALU and
    transcendental part only, the floor if every MFMA hid under other waves' work (half to three
    quarters does in the calibration). frac = bound_ms / measured duration."""
    rec = recorded_instructions(kernel)
    if rec is None:
        return None
    cyc = SIMDS * CLOCK_HZ / 1e3
    v, m = issue_cycles(rec["valu"], rec["trans"], rec["mfma"])
    valu_ms, mfma_ms = v / cyc, m / cyc
    lane_ops = (rec["valu"] + rec["trans"]) * 64
    return {"valu_instructions": rec["valu"], "trans_instructions": rec["trans"],
            "mfma_instructions": rec["mfma"], "scores": scores,
            "valu_lane_ops_per_score": lane_ops / scores if scores else None,
            "cycles": {"valu": VALU_CYCLES, "trans": TRANS_CYCLES, "mfma": MFMA_CYCLES},
            "valu_ms": valu_ms, "mfma_ms": mfma_ms, "bound_ms": valu_ms + mfma_ms,
            "bound_ms_mfma_hidden": valu_ms, "frac": (valu_ms + mfma_ms) / avg_ms}


def _kernel_key(r):
    name = r["Kernel_Name"].replace("(anonymous namespace)::", "")
    name = re.sub(r"^void |clk::", "", name.split("(")[0])
    if "Grid_Size" in r:
        grid, wg = int(r["Grid_Size"]), int(r["Workgroup_Size"])
    else:
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
    return name, grid // max(1, wg)


def trace_summary(path):
    """Markdown rows from a rocprofv3 --kernel-trace csv: per kernel and grid, calls and the
    average / min / max duration in microseconds and the share of all kernel time."""
    import csv
    per = {}
    for r in csv.DictReader(open(path)):
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        per.setdefault(_kernel_key(r), []).append(d)
    total = sum(sum(v) for v in per.values())
    print("| kernel | workgroups | calls | avg us | min us | max us | total % |")
    print("|---|---|---|---|---|---|---|")
    for (name, wgs), v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        if name.startswith(("at::", "rocprim::")):  # input generation and timing scaffolding
            continue
        print("| `%s` | %d | %d | %.1f | %.1f | %.1f | %.1f |" % (
            name, wgs, len(v), sum(v) / len(v), min(v), max(v), 100.0 * sum(v) / total))
    return 0


def counter_summary(paths):
    """Markdown rows: per kernel and grid (workgroups; one workload each), dispatch count and the
    median per dispatch of each counter in rocprofv3 --pmc csv files (values of one dispatch
    summed over its dimension instances). A --kernel-trace csv gives durations instead."""
    import csv
    import statistics
    if len(paths) == 1 and "Counter_Name" not in open(paths[0]).readline():
        return trace_summary(paths[0])
    per = {}
    for path in paths:
        with open(path) as fh:
            for r in csv.DictReader(fh):
                name, wgs = _kernel_key(r)
                key = (r["Dispatch_Id"], r["Counter_Name"])
                d = per.setdefault((name, wgs), {})
                d[key] = d.get(key, 0.0) + float(r["Counter_Value"])
    counters = sorted({c for d in per.values() for (_, c) in d})
    print("| kernel | workgroups | dispatches | " + " | ".join(counters) + " |")
    print("|---" * (len(counters) + 3) + "|")
    for (name, wgs), d in sorted(per.items()):
        if name.startswith(("at::", "rocprim::")):  # input generation and timing scaffolding
            continue
        cols = []
        for c in counters:
            vals = [v for (disp, cn), v in d.items() if cn == c]
            cols.append("%.4g" % statistics.median(vals) if vals else "-")
        disp = len({disp for (disp, _) in d})
        print("| `%s` | %d | %d | %s |" % (name, wgs, disp, " | ".join(cols)))
    mix = ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_VALU_TRANS_F32",
           "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE")
    if all(c in counters for c in mix):
        # Derived per-dispatch medians: VALU = SQ_INSTS_VALU less MFMA and transcendentals; the
        # SIMDs' cycles in a launch = SIMDS * GRBM_GUI_ACTIVE / 8 (that counter sums the XCDs).
        print()
        print("| kernel | workgroups | MFMA busy | MFMA instr | VALU instr | trans instr | "
              "(VALU+trans) per MFMA | issue |")
        print("|---|---|---|---|---|---|---|---|")
        for (name, wgs), d in sorted(per.items()):
            if name.startswith(("at::", "rocprim::")):
                continue
            med = {c: statistics.median([v for (disp, cn), v in d.items() if cn == c] or [0.0])
                   for c in mix}
            mf, tr = med["SQ_INSTS_MFMA"], med["SQ_INSTS_VALU_TRANS_F32"]
            plain = med["SQ_INSTS_VALU"] - mf - tr
            simd = SIMDS * med["GRBM_GUI_ACTIVE"] / 8
            if simd <= 0:
                continue
            v, m = issue_cycles(plain, tr, mf)
            print("| `%s` | %d | %.1f%% | %.3g | %.3g | %.3g | %s | %.0f%% |" % (
                name, wgs, 100 * med["SQ_VALU_MFMA_BUSY_CYCLES"] / simd, mf, plain, tr,
                "%.1f" % ((plain + tr) / mf) if mf else "-", 100 * (v + m) / simd))
    return 0


def copy_calibration(mib, reps=5):
    """A plain device-to-device copy of `mib` MiB, `reps` times: the known-size reference that
    the FETCH_SIZE / WRITE_SIZE counters are scaled by (reads and writes mib MiB each)."""
    import torch
    dev = torch.device("cuda:0")
    n = mib * (1 << 20) // 4
    a = torch.randn(n, device=dev)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "reps": reps}),
          flush=True)
    return 0


def issue_calibration(iters=20000):
    """What one wave instruction costs a SIMD on this device, from the library's
    clk_issue_calibration mixes: each kind on 256 blocks of 256, 512 and 768 threads (one, two
    and three waves per SIMD, the blocks one per CU), timed with HIP events on the launch stream,
    in SIMD cycles at CLOCK_HZ. Per wave count, one JSON line: the cycles of an FMA, an
    exponential and a 16x16x32 bf16 MFMA alone; the share of the MFMAs' own time that a mix with
    FMAs, exponentials or both hides; and the share of the shorter of FMAs and exponentials that
    overlaps the other (0: they share the issue slots)."""
    import torch
    from colabfold_legacy_kernels import _native as native
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = native.lib()
    st = torch.cuda.current_stream(dev)
    blocks = 256
    sink = torch.empty(blocks * 1024, device=dev)
    names = ["fma", "exp", "mfma", "fma+exp", "fma+mfma", "exp+mfma", "fma+exp+mfma"]
    per_round = {0: 64, 1: 64, 2: 8}  # instructions of the kind in one round (two copies)
    for threads in (256, 512, 768):
        waves_per_simd = blocks * threads // 64 / SIMDS

        def run(kind, n):
            if lib.clk_issue_calibration(st.cuda_stream, kind, blocks, threads, n,
                                         sink.data_ptr()) != native.OK:
                raise RuntimeError(native.last_error())

        cyc = {}
        for kind in range(7):
            run(kind, 10)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(st)
            run(kind, iters)
            e1.record(st)
            e1.synchronize()
            # SIMD cycles per wave and round
            cyc[kind] = e0.elapsed_time(e1) * 1e-3 * CLOCK_HZ / iters / waves_per_simd
        print(json.dumps({
            "waves_per_simd": waves_per_simd,
            "cycles_per_instruction": {names[k]: cyc[k] / per_round[k] for k in (0, 1, 2)},
            "round_cycles": {names[k]: round(cyc[k], 1) for k in range(7)},
            "mfma_hidden": {"under fma": (cyc[0] + cyc[2] - cyc[4]) / cyc[2],
                            "under exp": (cyc[1] + cyc[2] - cyc[5]) / cyc[2],
                            "under fma+exp": (cyc[3] + cyc[2] - cyc[6]) / cyc[2]},
            "fma_exp_overlap": (cyc[0] + cyc[1] - cyc[3]) / min(cyc[0], cyc[1])}), flush=True)
    return 0


def cpu_baseline(torch, workloads, rows, min_seconds):
    from oracle import cpu_baseline as cb
    cores = _cores()
    inp = workloads.attention_inputs(rows, HEADS, NRES, NRES, HEAD_DIM, torch.bfloat16, seed=1,
                                     device="cpu", masked_tail=0.10)
    sec = cb.time_attention_fwd_bwd(inp, rows, cores, min_seconds=min_seconds)
    flops = attention_flops(rows, HEADS, NRES, NRES, HEAD_DIM)["step"]
    return {"value": flops / sec / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": "torch float32 jnp restatement (materialised logits + autograd), fwd+bwd of "
                      "%d of the %d rows at N_res=%d, median of >=3 runs (%.2f s each), scaled "
                      "by algorithmic flops" % (rows, N_ROWS, NRES, sec)}


def main(argv=None):
    ap = argparse.ArgumentParser(description="Evoformer hot-path benchmark (one MI355X)")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--min-warmup-ms", type=float, default=100.0,
                    help="keep warming up past --warmup steps until this much time has passed "
                         "(every timed section)")
    ap.add_argument("--cpu-rows", type=int, default=N_ROWS)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (counter calibration)")
    ap.add_argument("--issue-calibration", action="store_true",
                    help="only measure the per-instruction issue costs (FMA, exponential, MFMA)")
    ap.add_argument("--counter-summary", nargs="+", metavar="CSV",
                    help="only summarise rocprofv3 --pmc (or one --kernel-trace) csv files per "
                         "kernel (no GPU)")
    args = ap.parse_args(argv)
    if args.counter_summary:
        return counter_summary(args.counter_summary)
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.issue_calibration:
        return issue_calibration()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the attention rows "
              "would shard across GPUs with one dBias all-reduce; not built). Use --gpus 1.",
              file=sys.stderr)
        return 2

    global MIN_WARMUP_MS
    MIN_WARMUP_MS = args.min_warmup_ms
    import torch
    from colabfold_legacy_kernels import _native as native
    from colabfold_legacy_kernels import workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = native.lib()
    so = torch.cuda.current_stream(dev)
    stream = so.cuda_stream
    print("bench: building %d attention input sets" % ROTATE, file=sys.stderr, flush=True)
    sets = [AttentionSet(torch, workloads, native, dev, seed=1 + r) for r in range(ROTATE)]

    def step(i):
        attention_step(lib, native, stream, sets[i % ROTATE])

    print("bench: timing attention fwd+bwd", file=sys.stderr, flush=True)
    step_stats = {}
    ms = timed(torch, step, args.steps, args.warmup, so, step_stats)
    fl = attention_flops(N_ROWS, HEADS, NRES, NRES, HEAD_DIM)
    tflops = fl["step"] / (ms * 1e-3) / 1e12
    kernels = per_kernel(torch, native, step, args.steps)
    per_step = {k: v["avg_ms"] * v["launches_per_step"] for k, v in kernels.items()}
    dom = max(per_step, key=per_step.get)
    dom_flops = fl.get(dom, 0.0)
    achieved = dom_flops / (kernels[dom]["avg_ms"] * 1e-3) / 1e12 if dom_flops else None
    roofline = {"bound": "mfma", "kernel": dom, "achieved": achieved, "peak": MFMA_PEAK_BF16,
                "unit": "TFLOP/s", "frac": (achieved / MFMA_PEAK_BF16) if achieved else None,
                "traffic": recorded_traffic(dom), "avg_ms": kernels[dom]["avg_ms"],
                "algorithmic_flops_per_launch": dom_flops,
                "issue": issue_bound(dom, kernels[dom]["avg_ms"], N_ROWS * HEADS * NRES * NRES)}

    result = {
        "metric": METRIC, "value": tflops, "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "warmup_run": step_stats["warmup_run"],
        "warmup_ms": step_stats["warmup_ms"], "ms_per_step": ms,
        "ms_per_step_median": step_stats["median_ms"], "ms_per_step_min": step_stats["min_ms"],
        "ms_per_step_max": step_stats["max_ms"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "triangle attention fwd+bwd, N_res=384", "rows": N_ROWS,
                   "heads": HEADS, "seq_q": NRES, "seq_k": NRES, "head_dim": HEAD_DIM,
                   "masked_keys": "last 10%", "rotating_sets": ROTATE,
                   "parallelism": "single GPU"},
        "frac_of_mfma_peak": tflops / MFMA_PEAK_BF16,
        "roofline": roofline,
        "kernels_ms_per_step": per_step,
    }
    if not args.no_secondary:
        print("bench: timing the streaming copy", file=sys.stderr, flush=True)
        sec = bench_hbm_copy(torch, native, dev, stream, args.steps, args.warmup)
        print("bench: timing LayerNorm", file=sys.stderr, flush=True)
        sec.update(bench_layer_norm(torch, workloads, native, dev, stream, args.steps,
                                    args.warmup))
        print("bench: timing the attention step in float16", file=sys.stderr, flush=True)
        sec.update(bench_attention_f16(torch, workloads, native, dev, stream, args.steps,
                                       args.warmup))
        sec["ln_fwd_frac_hbm"] = sec["ln_fwd_GBps"] / HBM_PEAK
        sec["ln_bwd_frac_hbm"] = sec["ln_bwd_GBps"] / HBM_PEAK
        sec["ln_fwd_frac_copy"] = sec["ln_fwd_GBps"] / sec["hbm_copy_GBps"]
        sec["ln_bwd_frac_copy"] = sec["ln_bwd_GBps"] / sec["hbm_copy_GBps"]
        print("bench: timing LayerNorm + gated dual projection", file=sys.stderr, flush=True)
        sec.update(bench_ln_gdp(torch, workloads, native, dev, stream, args.steps, args.warmup))
        sec["ln_gdp_frac_hbm"] = sec["ln_gdp_GBps"] / HBM_PEAK
        print("bench: timing the gated dual projection", file=sys.stderr, flush=True)
        sec.update(bench_gdp(torch, workloads, native, dev, stream, args.steps, args.warmup))
        sec["gdp_frac_hbm"] = sec["gdp_GBps"] / HBM_PEAK
        print("bench: timing the gated dual projection backward", file=sys.stderr, flush=True)
        sec.update(bench_gdp_bwd(torch, workloads, native, dev, stream, args.steps, args.warmup))
        print("bench: timing the pair-bias projection", file=sys.stderr, flush=True)
        sec.update(bench_pair_bias(torch, workloads, native, dev, stream, args.steps, args.warmup))
        sec["pair_bias_frac_hbm"] = sec["pair_bias_GBps"] / HBM_PEAK
        print("bench: timing the attention output gate", file=sys.stderr, flush=True)
        sec.update(bench_attn_gate(torch, native, dev, stream, args.steps, args.warmup))
        sec["attn_gate_frac_hbm"] = sec["attn_gate_GBps"] / HBM_PEAK
        print("bench: timing the attention output gate backward", file=sys.stderr, flush=True)
        sec.update(bench_attn_gate_bwd(torch, native, dev, stream, args.steps, args.warmup))
        print("bench: timing gated attention, fused and separate", file=sys.stderr, flush=True)
        sec.update(bench_gated_attention(torch, workloads, native, dev, stream, args.steps,
                                         args.warmup))
        print("bench: timing the forward on the [N,S,H,D] layout", file=sys.stderr, flush=True)
        sec.update(bench_attention_nshd(torch, workloads, native, dev, stream, args.steps,
                                        args.warmup))
        print("bench: timing the triangle multiplication", file=sys.stderr, flush=True)
        sec.update(bench_triangle(torch, native, dev, stream, args.steps, args.warmup))
        result["secondary"] = sec
    if not args.no_cpu_baseline:
        print("bench: timing CPU baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(torch, workloads, args.cpu_rows, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
