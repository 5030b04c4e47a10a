"""Float64 restatement of AlphaFold's triangle multiplication (the step after the gated dual
projection; the reference library has no code for it and stops at cuda/volta_ops.cu:97-208).

  outgoing  'ikc,jkc->ijc'  x[i,j,c] = sum_k left[i,k,c] right[j,k,c]
  incoming  'kjc,kic->ijc'  x[i,j,c] = sum_k left[k,j,c] right[k,i,c]

``einsum`` states the per-channel product the kernels compute on channel-major operands,
x[c] = a[c] . b[c]^T for a, b [C, N, N]; ``pair_einsum`` states the two directions on the
pair-layout tensors [N, N, C] through it (outgoing: a = left, b = right; incoming: a = right^T,
b = left^T per channel); ``triangle_multiply`` is the whole module around the contraction;
``triangle_multiply_at`` is the same module evaluated at chosen positions only (for grids too
large to compute whole: output (i, j) needs the two rows, or columns, of z it contracts over).

Pinned in tests/test_oracle.py by torch.einsum in float64 (an independent routine) and by closed
forms: b = 1 gives row sums of a; a permutation of k applied to both operands changes nothing.
``triangle_multiply_at`` is pinned there against ``triangle_multiply`` at every position.
"""

import numpy as np

__all__ = ["einsum", "pair_einsum", "triangle_multiply", "triangle_multiply_at"]


def einsum(a, b):
    """x [C, N, N] float64: x[c] = a[c] @ b[c]^T."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.matmul(a, b.transpose(0, 2, 1))


def pair_einsum(left, right, outgoing=True):
    """x [N, N, C] float64 from pair-layout left, right [N, N, C]."""
    left = np.asarray(left, np.float64)
    right = np.asarray(right, np.float64)
    if outgoing:
        ac, bc = left.transpose(2, 0, 1), right.transpose(2, 0, 1)   # [c][i][k], [c][j][k]
    else:
        ac, bc = right.transpose(2, 1, 0), left.transpose(2, 1, 0)   # right[k,i], left[k,j]
    return einsum(ac, bc).transpose(1, 2, 0)


def triangle_multiply(z, mask, ln_in, weights, biases, ln_center, outgoing=True, eps=1e-5):
    """out [N, N, C] float64: AlphaFold's TriangleMultiplication on z [N, N, C], mask [N, N].

    weights / biases: (left projection, right projection, left gate, right gate, output
    projection, output gate), each [C, C] (input channel first) / [C]; ln_in, ln_center:
    (scale, offset). The projections are the reference GDP's form (cuda/volta_ops.cu:97,
    201-204) on the input LayerNorm (volta_ops.cu:40-58).
    """
    from .gdp import gated_dual_proj, sigmoid
    from .layer_norm import layer_norm_fwd
    z = np.asarray(z, np.float64)
    n, _, c = z.shape
    w = [np.asarray(t, np.float64) for t in weights]
    b = [np.asarray(t, np.float64) for t in biases]
    y, _, _ = layer_norm_fwd(z.reshape(-1, c), ln_in[0], ln_in[1], eps)
    m = np.asarray(mask, np.float64).reshape(-1)
    left = gated_dual_proj(y, w[0], b[0], w[2], b[2], m).reshape(n, n, c)
    right = gated_dual_proj(y, w[1], b[1], w[3], b[3], m).reshape(n, n, c)
    x = pair_einsum(left, right, outgoing)
    xc, _, _ = layer_norm_fwd(x.reshape(-1, c), ln_center[0], ln_center[1], eps)
    out = (xc @ w[4] + b[4]) * sigmoid(y @ w[5] + b[5])
    return out.reshape(n, n, c)


def triangle_multiply_at(line, ln_in, weights, biases, ln_center, positions, outgoing=True,
                         eps=1e-5):
    """out[i, j, :] float64 [P, C] of ``triangle_multiply`` at positions [(i, j), ...].

    line(kind, idx) returns (z, mask) of one line of the grid as arrays [N, C], [N]: kind "row"
    gives z[idx, :, :], "col" gives z[:, idx, :]. Outgoing, x[i, j] contracts row i (left) with
    row j (right); incoming, column j (left) with column i (right). y[i, j] for the output gate
    is read from row i.
    """
    from .gdp import gated_dual_proj, sigmoid
    from .layer_norm import layer_norm_fwd
    w = [np.asarray(t, np.float64) for t in weights]
    b = [np.asarray(t, np.float64) for t in biases]
    kind = "row" if outgoing else "col"
    cache = {}

    def branch(idx, side):  # side 0: left, 1: right; the gated projection of one line
        key = (idx, side)
        if key not in cache:
            z, m = line(kind, idx)
            y, _, _ = layer_norm_fwd(np.asarray(z, np.float64), ln_in[0], ln_in[1], eps)
            cache[key] = gated_dual_proj(y, w[side], b[side], w[side + 2], b[side + 2],
                                         np.asarray(m, np.float64))
        return cache[key]

    out = []
    for i, j in positions:
        left, right = (branch(i, 0), branch(j, 1)) if outgoing else (branch(j, 0), branch(i, 1))
        x = (left * right).sum(axis=0)
        zi, _ = line("row", i)
        y, _, _ = layer_norm_fwd(np.asarray(zi, np.float64)[j:j + 1], ln_in[0], ln_in[1], eps)
        xc, _, _ = layer_norm_fwd(x[None], ln_center[0], ln_center[1], eps)
        out.append(((xc @ w[4] + b[4]) * sigmoid(y @ w[5] + b[5]))[0])
    return np.stack(out)
