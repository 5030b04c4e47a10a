"""Error metrics and tolerances shared by the parity tests.

Every comparison reports, per tensor, max-abs error and max-rel = max-abs / max|ref|, against a
float64 oracle evaluated on the same rounded inputs. Tolerances (max-rel):
  bf16: O 1e-2; dQ, dK, dV, dBias 2e-2; LayerNorm y and dx 8e-3; GDP 1e-2
  f16:  one quarter of the bf16 value;  f32 LayerNorm: 1e-5
"""
import numpy as np
import torch

TOL = {
    "bf16": {"o": 1e-2, "grad": 2e-2, "ln": 8e-3, "gdp": 1e-2},
    "f16": {"o": 2.5e-3, "grad": 5e-3, "ln": 2e-3, "gdp": 2.5e-3},
    "f32": {"ln": 1e-5},
}


def dname(dtype):
    return {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[dtype]


def np64(t):
    return t.detach().to("cpu", torch.float64).numpy()


def errors(got, ref):
    got = np64(got) if isinstance(got, torch.Tensor) else np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), "non-finite values in result"
    mabs = float(np.abs(got - ref).max()) if ref.size else 0.0
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    return mabs, (mabs / scale if scale > 0 else mabs)


def assert_close(name, got, ref, rel):
    mabs, mrel = errors(got, ref)
    print("%-10s max-abs %.3e  max-rel %.3e  (tol %.1e)" % (name, mabs, mrel, rel))
    assert mrel <= rel, "%s: max-rel %.3e > %.1e (max-abs %.3e)" % (name, mrel, rel, mabs)
