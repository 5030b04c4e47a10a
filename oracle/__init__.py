"""CPU oracle for the Evoformer hot path: a float64 NumPy restatement of the math.

This package is TEST INFRASTRUCTURE. It is the checker, never the thing measured or shipped:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The product path (``colabfold_legacy_kernels``) never calls into it, and fails
loudly when its HIP library is missing instead of falling back to anything here.

Modules
-------
attention     flash attention with pair bias and key mask, forward and backward
              (restates cuda/volta_mma_attn.cu:70-273 and cuda/volta_wmma_attn.cu:47-234;
              the backward has no reference code and is the autodiff of that forward)
layer_norm    LayerNorm forward and backward (restates cuda/volta_ops.cu:28-60)
gdp           gated dual projection and the LayerNorm-fused variant
              (restates cuda/volta_ops.cu:97-208 and cuda/volta_gdp_wmma.cu:16-97)
gate          the attention output gate O * sigmoid(x.Wg + bg) (no reference code: the caller's
              jnp step after the attention targets)
triangle      the triangle-multiplication contraction, outgoing and incoming (no reference code:
              the step after the gated dual projection)
evoformer     the pair micro-block composed from the three (LN -> GDP, LN -> bias -> attention)

How each function is pinned (tests/test_oracle.py): against independent textbook routines
(torch.nn.functional.layer_norm / softmax / scaled_dot_product_attention and torch.autograd,
all float64 on the CPU), against torch float32 autograd of the additive -1e9 mask form that the
jnp caller uses, against central finite differences on tiny shapes, and against closed forms
and invariants (rows of P sum to 1, sum_k dBias = 0, mask=0 -> 0, ...). The reference ships no
golden vectors or tests for this path, and its CUDA/CUTLASS/XLA build cannot run here, so no
reference binary is used.
"""

from . import attention, layer_norm, gdp, gate, triangle, evoformer  # noqa: F401

__all__ = ["attention", "layer_norm", "gdp", "gate", "triangle", "evoformer"]
