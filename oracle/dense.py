"""The MoE-HLM expert layer through BLAS, in float64 (oracle for full-size shapes).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

``moe.geom_matmul`` follows the reference's operation order and is therefore a
Python loop over the contraction; it finishes a few thousand rows of a BASELINE
config in a test's time, not all of them.  This module evaluates the same
mathematics -- CliffordLinear (``holograph/layers/clifford_linear.py:101-123``,
i.e. ``geom_matmul``, ``rune/ops/batched.py:320-344``), the CliffordFFN of every
expert (``holograph/models/hlm_block.py:55-61``) and the layer's weighted combine
(``hlm_block.py:154-183``) -- as dense matrix products in float64, so that every
row of a full-size config is recomputed in seconds.  float64 is the truth the
build's fp32 and bf16 results are measured against; the reference's own fp32
result lies within fp32 rounding of it.

The product.  With ``e_a e_b = SIGN[a, b] e_IDX[a, b]``,
    y[m, j, c] = sum_i sum_{a, b : IDX[a, b] = c} SIGN[a, b] W[j, i, a] x[m, i, b].
For each (a, c) exactly one b = b(a, c) has ``IDX[a, b] = c`` (left multiplication
by a basis blade permutes the basis), so the layer is one matrix product
    Y[j, (c, m)] = sum_(i, a) W[j, (i, a)] Xs[(i, a), (c, m)],
    Xs[(i, a), (c, m)] = SIGN[a, b(a, c)] x[m, i, b(a, c)],
with W in its own (d_out, d_in * 8) layout and Xs the signed, permuted input
planes (8 times the input, built once per chunk of rows; W is read once per chunk).
The backward uses the left-multiplication matrix ``L(W)`` (``cl3.left_mul_matrix``):
``Y = X L^T``, so ``dX = dY L`` and ``dL = dY^T X``, folded back onto the weight
components ``L(W)[r, q] = SIGN * W[src[r, q]]``.

Pinning (``tests/test_oracle_dense.py``): ``linear`` equals ``moe.geom_matmul_f64``
(the dense ``L(W)`` einsum) to 1e-12 and ``moe.clifford_linear`` (the reference's
fp32 order, bit-exact against its compiled ``cl3_geom_matmul_flat``) to fp32
rounding; scalar-only weights reduce it to a plain matrix product; ``moe_layer``
equals ``moe.moe_forward_reference`` (the reference-order layer that reproduces
the reference goldens) to fp32 rounding; ``linear_backward`` and
``moe_layer_backward`` equal ``backward.clifford_linear_backward`` and
``backward.moe_backward_reference`` (both pinned by central finite differences).
"""

from __future__ import annotations

import numpy as np

from . import backward as bw
from .cl3 import L_SIGN, L_SRC, PRODUCT_IDX, PRODUCT_SIGN

F64 = np.float64

# _B_OF[a, c]: the b with IDX[a, b] = c; _S_OF[a, c]: SIGN[a, b] for that b
_B_OF = np.zeros((8, 8), dtype=np.int64)
_S_OF = np.zeros((8, 8), dtype=F64)
for _a in range(8):
    for _b in range(8):
        _B_OF[_a, PRODUCT_IDX[_a, _b]] = _b
        _S_OF[_a, PRODUCT_IDX[_a, _b]] = PRODUCT_SIGN[_a, _b]
assert all(sorted(_B_OF[a]) == list(range(8)) for a in range(8))


_BUFS: dict = {}


def _buf(name, n):
    """A reused float64 scratch array of at least n elements (fresh large arrays cost a page fault per page)."""
    a = _BUFS.get(name)
    if a is None or a.size < n:
        a = _BUFS[name] = np.empty(n, F64)
    return a[:n]


def linear(x, W, b=None, chunk_bytes: int = 32 << 20):
    """``y[m, j] = sum_i W[j, i] x[m, i] (+ b[j])``; x (M, d_in, 8), W (d_out, d_in, 8) -> (M, d_out, 8) float64."""
    x = np.asarray(x, F64)
    W = np.asarray(W, F64)
    M, d_in, _ = x.shape
    d_out = W.shape[0]
    assert W.shape == (d_out, d_in, 8)
    A = W.reshape(d_out, d_in * 8)  # columns (i, a)
    y = np.empty((M, d_out, 8), F64)
    chunk = max(16, chunk_bytes // (64 * 8 * d_in))
    for m0 in range(0, M, chunk):
        m1 = min(M, m0 + chunk)
        mc = m1 - m0
        planes = _buf("planes", d_in * 8 * mc).reshape(d_in, 8, mc)
        planes[...] = np.transpose(x[m0:m1], (1, 2, 0))  # (i, b, m)
        Xs = _buf("xs", d_in * 64 * mc).reshape(d_in, 64, mc)
        np.take(planes, _B_OF.reshape(-1), axis=1, out=Xs)  # (i, (a, c), m)
        Xs *= _S_OF.reshape(1, 64, 1)
        Y = _buf("y", d_out * 8 * mc).reshape(d_out, 8 * mc)
        np.matmul(A, Xs.reshape(d_in * 8, 8 * mc), out=Y)  # (j, (c, m))
        y[m0:m1] = np.transpose(Y.reshape(d_out, 8, mc), (2, 0, 1))
    if b is not None:
        y += np.asarray(b, F64)
    return y


def left_mul_dense(W):
    """``L(W)`` of a CliffordLinear weight as one matrix, rows (j, r), columns (i, q): (8 d_out, 8 d_in)."""
    W = np.asarray(W, F64)
    d_out, d_in, _ = W.shape
    L = W[..., L_SRC] * L_SIGN.astype(F64)  # (d_out, d_in, 8 r, 8 q)
    return np.ascontiguousarray(np.transpose(L, (0, 2, 1, 3))).reshape(d_out * 8, d_in * 8)


def linear_backward(x, W, dy):
    """Gradients of ``linear`` (no bias term needed): x (M, d_in, 8), W (d_out, d_in, 8), dy (M, d_out, 8)
    -> (dx, dW, db) in float64 (``clifford_linear.py:125-163``)."""
    x = np.asarray(x, F64)
    dy = np.asarray(dy, F64)
    d_out, d_in, _ = np.shape(W)
    M = x.shape[0]
    L = left_mul_dense(W)
    X = x.reshape(M, d_in * 8)
    DY = dy.reshape(M, d_out * 8)
    dx = (DY @ L).reshape(M, d_in, 8)
    dL = (DY.T @ X).reshape(d_out, 8, d_in, 8)  # [j, r, i, q]
    dW = np.zeros((d_out, d_in, 8), F64)
    for r in range(8):
        for q in range(8):
            dW[:, :, L_SRC[r, q]] += float(L_SIGN[r, q]) * dL[:, r, :, q]
    return dx, dW, dy.sum(axis=0)


def _slots_by_expert(idx, e):
    """Tokens and slots that hold expert e, ascending token order (``hlm_block.py:165-178``)."""
    return np.nonzero(np.asarray(idx) == e)


def moe_layer(x, idx, w, w_up, b_up, w_down, b_down, act="gelu", residual=None, progress=None):
    """``_moe_forward`` for a given routing, float64: x (N, d, 8); idx, w (N, k); stacked expert weights
    w_up (E, F, d, 8), b_up (E, F, 8) or None, w_down (E, d, F, 8), b_down (E, d, 8) or None.

    The combine adds each token's expert outputs in ascending expert order
    (``hlm_block.py:180-181``); ``residual`` (N, d, 8) is added first when given
    (``hlm_block.py:151``).  ``progress(e)``, when given, is called after each expert.
    """
    x = np.asarray(x, F64)
    idx = np.asarray(idx)
    w = np.asarray(w, F64)
    N, k = idx.shape
    E = np.shape(w_up)[0]
    y_slot = np.zeros((N, k) + x.shape[1:], F64)
    for e in range(E):
        tok, slot = _slots_by_expert(idx, e)
        if tok.size == 0:
            continue
        h = bw.activation_f64(act, linear(x[tok], w_up[e], None if b_up is None else b_up[e]))
        y_slot[tok, slot] = linear(h, w_down[e], None if b_down is None else b_down[e])
        if progress is not None:
            progress(e)
    out = np.zeros_like(x) if residual is None else np.array(residual, F64)
    order = np.argsort(idx, axis=-1, kind="stable")  # ascending expert per token
    rows = np.arange(N)
    for j in range(k):
        s = order[:, j]
        out += w[rows, s][:, None, None] * y_slot[rows, s]
    return out


def moe_layer_backward(x, idx, w, w_up, b_up, w_down, b_down, dout, act="gelu", residual=False, progress=None):
    """Backward of ``moe_layer`` for its routing: returns ``(dx, dW_up, db_up, dW_down, db_down)``, float64,
    the weight gradients stacked over experts (zero for an expert without rows).  ``progress(e)``, when
    given, is called after each expert."""
    x = np.asarray(x, F64)
    dout = np.asarray(dout, F64)
    w = np.asarray(w, F64)
    E = np.shape(w_up)[0]
    dx = dout.copy() if residual else np.zeros_like(x)
    dWu = np.zeros(np.shape(w_up), F64)
    dbu = np.zeros(np.shape(w_up)[:2] + (8,), F64)
    dWd = np.zeros(np.shape(w_down), F64)
    dbd = np.zeros(np.shape(w_down)[:2] + (8,), F64)
    for e in range(E):
        tok, slot = _slots_by_expert(idx, e)
        if tok.size == 0:
            continue
        xe = x[tok]
        h_pre = linear(xe, w_up[e], None if b_up is None else b_up[e])
        h = bw.activation_f64(act, h_pre)
        dy = w[tok, slot][:, None, None] * dout[tok]
        dh, dWd[e], dbd[e] = linear_backward(h, w_down[e], dy)
        dh_pre = bw.activation_backward(act, h_pre, dh, dtype=F64)
        dxe, dWu[e], dbu[e] = linear_backward(xe, w_up[e], dh_pre)
        np.add.at(dx, tok, dxe)
        if progress is not None:
            progress(e)
    return dx, dWu, dbu, dWd, dbd
