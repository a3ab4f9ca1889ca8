"""NumPy restatement of the expert-FFN backward pass (oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

* ``clifford_linear_backward`` restates ``CliffordLinear.backward``
  (``holograph/layers/clifford_linear.py:125-163``): with the forward
  ``y_t = geom_matmul(W, x_t)``, ``grad_W = geom_matmul(dy_t, reverse(x))``,
  ``grad_x = geom_matmul(reverse(W)^T, dy_t)^T`` and ``grad_b = sum dy``.
* ``activation_backward`` restates ``clifford_gelu_backward``,
  ``clifford_relu_backward`` (zero thresholds) and
  ``clifford_sigmoid_backward`` (``holograph/layers/activations.py:135-287``).
* ``moe_backward_reference`` is the backward of ``_moe_forward``
  (``hlm_block.py:154-183``), which the reference does not have
  (``hlm_block.py:202-206``): per expert, in the forward's grouping, the
  CliffordFFN backward (``hlm_block.py:63-86``) of ``w * dout`` and the
  gradient of the routing weights ``<dout, y>``; the token gradients are
  added back per token.

Pinning (``tests/test_oracle_backward.py``), as the reference's own harness
does (``holograph/tests/test_backward_numerical.py:28-98``): central finite
differences in float64 of the forward restatement, for every parameter and
input, each activation and the whole MoE; plus the closed forms of the
geometric-algebra adjoints (``<a b, c> = <b, ~a c> = <a, c ~b>``).
"""

from __future__ import annotations

import numpy as np

from . import moe
from .cl3 import reverse

F32 = np.float32


def clifford_linear_backward(x, W, dy):
    """x (M, d_in, 8), W (d_out, d_in, 8), dy (M, d_out, 8) -> (dx, dW, db), fp32."""
    x = np.asarray(x, F32)
    dy = np.asarray(dy, F32)
    x_t = np.ascontiguousarray(np.transpose(x, (1, 0, 2)))
    dy_t = np.ascontiguousarray(np.transpose(dy, (1, 0, 2)))
    x_rev_mt = np.ascontiguousarray(np.transpose(reverse(x_t), (1, 0, 2)))
    dW = moe.geom_matmul(dy_t, x_rev_mt)                                   # (d_out, d_in, 8)
    w_rev_t = np.ascontiguousarray(np.transpose(reverse(np.asarray(W, F32)), (1, 0, 2)))
    dx = np.transpose(moe.geom_matmul(w_rev_t, dy_t), (1, 0, 2))            # (M, d_in, 8)
    db = dy.sum(axis=0)
    return np.ascontiguousarray(dx), dW, db


def _gelu_derivative(v):
    c = np.sqrt(2.0 / np.pi)
    inner = c * (v + 0.044715 * v ** 3)
    t = np.tanh(inner)
    return 0.5 * (1.0 + t) + 0.5 * v * (1.0 - t ** 2) * (c * (1.0 + 3.0 * 0.044715 * v ** 2))


def _sigmoid_derivative(v):
    s = moe._sigmoid(v)
    return s * (1.0 - s)


def _gate_backward(c, g, fn, dfn):
    """``_magnitude_gate_backward`` (``activations.py:150-178``)."""
    mag = np.sqrt(np.sum(c ** 2, axis=-1, keepdims=True) + 1e-12)
    direction = c / mag
    gated = fn(mag)
    dot = np.sum(direction * g, axis=-1, keepdims=True)
    return (gated / mag) * g + (dfn(mag) - gated / mag) * direction * dot


def activation_backward(act, h, g, dtype=F32):
    """Gradient w.r.t. the activation input ``h`` (..., 8) given ``g`` w.r.t. its output, in ``dtype``."""
    h = np.asarray(h, dtype)
    g = np.asarray(g, dtype)
    if act == "none":
        return g.copy()
    out = np.zeros_like(h)
    if act == "relu":
        out[..., 0:1] = g[..., 0:1] * (h[..., 0:1] > 0).astype(dtype)
        for sl in (slice(1, 4), slice(4, 7)):
            c = h[..., sl]
            mag = np.sqrt(np.sum(c ** 2, axis=-1, keepdims=True) + 1e-12)
            active = (mag > 0).astype(dtype)
            direction = c / mag
            dot = np.sum(direction * g[..., sl], axis=-1, keepdims=True)
            gated = np.maximum(mag, 0.0)
            out[..., sl] = active * ((gated / mag) * g[..., sl] + (1.0 - gated / mag) * direction * dot)
        out[..., 7:8] = g[..., 7:8] * (np.abs(h[..., 7:8]) > 0).astype(dtype)
        return out
    fn, dfn = (moe._gelu, _gelu_derivative) if act == "gelu" else (moe._sigmoid, _sigmoid_derivative)
    out[..., 0:1] = g[..., 0:1] * dfn(h[..., 0:1])
    out[..., 1:4] = _gate_backward(h[..., 1:4], g[..., 1:4], fn, dfn)
    out[..., 4:7] = _gate_backward(h[..., 4:7], g[..., 4:7], fn, dfn)
    out[..., 7:8] = g[..., 7:8] * (1.0 - np.tanh(h[..., 7:8]) ** 2)
    return out


def moe_backward_reference(x, idx, w, experts, dout, act="gelu", residual=False):
    """Backward of ``_moe_forward`` for a fixed routing ``(idx, w)`` (N, k).

    ``x``, ``dout``: (N, d, 8).  ``experts``: list of (w_up, b_up, w_down, b_down).
    Returns ``(dx, grads, dw)``: ``grads[e] = (dW_up, db_up, dW_down, db_down)``
    (zeros for an expert with no rows) and ``dw`` (N, k) the gradient of the
    routing weights.  ``residual``: the forward added x to its output.
    """
    x = np.asarray(x, F32)
    dout = np.asarray(dout, F32)
    N, k = idx.shape
    dx = dout.copy() if residual else np.zeros_like(x)
    dw = np.zeros((N, k), F32)
    grads = []
    for e, (wu, bu, wd, bd) in enumerate(experts):
        tok, slot = np.nonzero(idx == e)           # ascending token order
        if tok.size == 0:
            grads.append(tuple(np.zeros_like(a) for a in (wu, bu, wd, bd)))
            continue
        xe = x[tok]
        h_pre = moe.clifford_linear(xe, wu, bu)
        h = moe.ACTIVATIONS[act](h_pre)
        y = moe.clifford_linear(h, wd, bd)
        we = w[tok, slot].astype(F32)
        dw[tok, slot] = np.sum(dout[tok] * y, axis=(1, 2))
        dy = we[:, None, None] * dout[tok]
        dh, dWd, dbd = clifford_linear_backward(h, wd, dy)
        dh_pre = activation_backward(act, h_pre, dh)
        dxe, dWu, dbu = clifford_linear_backward(xe, wu, dh_pre)
        np.add.at(dx, tok, dxe)
        grads.append((dWu, dbu, dWd, dbd))
    return dx, grads, dw


def moe_forward_fixed_routing_f64(x, idx, w, experts, act="gelu", residual=False):
    """float64 forward for a fixed routing -- the function the finite differences probe."""
    x = np.asarray(x, np.float64)
    out = x.copy() if residual else np.zeros_like(x)
    for e, (wu, bu, wd, bd) in enumerate(experts):
        tok, slot = np.nonzero(idx == e)
        if tok.size == 0:
            continue
        h = linear_f64(x[tok], wu, bu)
        h = activation_f64(act, h)
        y = linear_f64(h, wd, bd)
        out[tok] += np.asarray(w, np.float64)[tok, slot][:, None, None] * y
    return out


def linear_f64(x, W, b):
    xt = np.transpose(np.asarray(x, np.float64), (1, 0, 2))
    y = np.transpose(moe.geom_matmul_f64(np.asarray(W, np.float64), xt), (1, 0, 2))
    return y + np.asarray(b, np.float64) if b is not None else y


def activation_f64(act, h):
    h = np.asarray(h, np.float64)
    if act == "none":
        return h.copy()
    out = np.zeros_like(h)
    if act == "relu":
        out[..., 0:1] = np.maximum(h[..., 0:1], 0.0)
        for sl in (slice(1, 4), slice(4, 7)):
            c = h[..., sl]
            mag = np.sqrt(np.sum(c ** 2, axis=-1, keepdims=True) + 1e-12)
            out[..., sl] = (c / mag) * np.maximum(mag, 0.0)
        out[..., 7:8] = h[..., 7:8]
        return out
    fn = moe._gelu if act == "gelu" else moe._sigmoid
    out[..., 0:1] = fn(h[..., 0:1])
    for sl in (slice(1, 4), slice(4, 7)):
        c = h[..., sl]
        mag = np.sqrt(np.sum(c ** 2, axis=-1, keepdims=True) + 1e-12)
        out[..., sl] = (c / mag) * fn(mag)
    out[..., 7:8] = np.tanh(h[..., 7:8])
    return out
