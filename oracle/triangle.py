"""Float64 restatement of AlphaFold's triangle multiplication (the step after the gated dual
projection; the reference library has no code for it and stops at cuda/volta_ops.cu:97-208).

  outgoing  x[i,j,c] = sum_k a[i,k,c] b[j,k,c]      incoming  x[i,j,c] = sum_k a[k,i,c] b[k,j,c]

``einsum`` states the per-channel product the kernels compute on channel-major operands,
x[c] = a[c] . b[c]^T for a, b [C, N, N]; ``pair_einsum`` states the two directions on the
pair-layout tensors [N, N, C] and is the composition of a channel-major transpose with it.

Pinned in tests/test_oracle.py by torch.einsum in float64 (an independent routine) and by closed
forms: b = 1 gives row sums of a; a permutation of k applied to both operands changes nothing.
"""

import numpy as np

__all__ = ["einsum", "pair_einsum"]


def einsum(a, b):
    """x [C, N, N] float64: x[c] = a[c] @ b[c]^T."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.matmul(a, b.transpose(0, 2, 1))


def pair_einsum(a, b, outgoing=True):
    """x [N, N, C] float64 from pair-layout a, b [N, N, C]."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if outgoing:
        ac, bc = a.transpose(2, 0, 1), b.transpose(2, 0, 1)   # [c][i][k], [c][j][k]
    else:
        ac, bc = a.transpose(2, 1, 0), b.transpose(2, 1, 0)   # [c][i][k] = a[k,i,c]
    return einsum(ac, bc).transpose(1, 2, 0)
