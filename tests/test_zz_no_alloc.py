"""clk_attention_bwd_noalloc: the attention backward with its workspace in the library's fixed
per-GPU scratch array, called through the C ABI. Its results must be bit-identical to
clk_attention_bwd with a caller workspace (the same kernels and the same fixed-order
reductions), on two calls in a row, the second with a smaller problem, so whatever the first
call left in the shared array cannot leak into the second."""
import pytest
import torch

from colabfold_legacy_kernels import _native, ops
from colabfold_legacy_kernels.workloads import attention_inputs


def _lib():
    return _native.lib()  # declares the prototypes of include/clk.h


def _grads(dev, inp):
    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    n, h, sq, d = g["q"].shape
    sk = g["k"].shape[2]
    out, lse = ops.attention_fwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], g["scale"])
    ref = ops.attention_bwd(g["q"], g["k"], g["v"], g["bias"], g["kmask"], out, g["dout"], lse,
                            g["scale"])
    got = [torch.full_like(t, float("nan")) for t in ref]
    lib = _lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    code = _native.BF16 if g["q"].dtype == torch.bfloat16 else _native.F16
    st = lib.clk_attention_bwd_noalloc(
        stream, code, g["q"].data_ptr(), g["k"].data_ptr(), g["v"].data_ptr(),
        g["bias"].data_ptr(), g["kmask"].data_ptr(), out.data_ptr(), g["dout"].data_ptr(),
        lse.data_ptr(), *(t.data_ptr() for t in got), n, h, sq, sk, d, g["scale"])
    assert st == _native.OK, _native.last_error()
    torch.cuda.synchronize(dev)
    return ref, got


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_twice(cuda):
    # First: two key ranges (dQ partials) and several row chunks (dBias partials); second: a
    # smaller problem in another dtype and head dim on the same scratch array.
    first = attention_inputs(6, 2, 130, 450, 32, torch.bfloat16, seed=31, masked_tail=0.1,
                             masked_rows=1)
    second = attention_inputs(3, 2, 64, 100, 16, torch.float16, seed=32, masked_tail=0.2)
    for inp in (first, second):
        ref, got = _grads(cuda, inp)
        for name, a, b in zip(("dq", "dk", "dv", "dbias"), ref, got):
            assert torch.equal(a, b), name
