"""Pins of the float64 BLAS oracle (``oracle/dense.py``) that the full-size GPU tests use.

Each check compares it with something fixed independently of it: the dense
``L(W)`` einsum and the reference-order fp32 restatement (bit-exact with the
reference's compiled code), plain matrix products in the scalar-only special
cases, the reference's own golden layer outputs, and central finite
differences.  A transposed operand (``x W`` for ``W x``), a dropped or
mis-signed (a, b) block or a wrong gradient fold fails one of them.
"""

import numpy as np
import pytest

from _fixtures import layer_weights, load_case
from oracle import backward as bw
from oracle import dense, moe


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


@pytest.mark.parametrize("M,d_in,d_out", [(5, 3, 4), (17, 9, 2), (40, 16, 33)])
def test_linear_equals_the_dense_einsum_and_the_reference_order(M, d_in, d_out):
    g = np.random.default_rng(M * 100 + d_in)
    x = g.standard_normal((M, d_in, 8))
    W = g.standard_normal((d_out, d_in, 8))
    b = g.standard_normal((d_out, 8))
    got = dense.linear(x, W, b, chunk_bytes=1)  # chunks of 16 rows
    assert _rel(got, bw.linear_f64(x, W, b)) < 1e-12
    ref32 = moe.clifford_linear(x.astype(np.float32), W.astype(np.float32), b.astype(np.float32))
    assert _rel(got, ref32) < 1e-5


def test_linear_weight_is_on_the_left():
    """Cl(3,0) does not commute: the product must be W x, as clifford_linear.py:114 computes it."""
    g = np.random.default_rng(3)
    x = g.standard_normal((6, 4, 8))
    W = g.standard_normal((5, 4, 8))
    got = dense.linear(x, W)
    from oracle.cl3 import geom_prod_f64

    want = np.einsum("mjic->mjc", geom_prod_f64(W[None, :, :, :], x[:, None, :, :]))
    wrong = np.einsum("mjic->mjc", geom_prod_f64(x[:, None, :, :], W[None, :, :, :]))
    assert _rel(got, want) < 1e-12
    assert _rel(got, wrong) > 0.1


def test_linear_scalar_special_cases_are_plain_matmuls():
    g = np.random.default_rng(4)
    x = g.standard_normal((9, 5, 8))
    W = g.standard_normal((7, 5, 8))
    Ws = np.zeros_like(W)
    Ws[..., 0] = W[..., 0]  # scalar-only weights: every blade is an ordinary matmul
    assert _rel(dense.linear(x, Ws), np.einsum("ji,mic->mjc", W[..., 0], x)) < 1e-12
    xs = np.zeros_like(x)
    xs[..., 0] = x[..., 0]  # scalar-only inputs: y[m, j] = sum_i W[j, i] x_i
    assert _rel(dense.linear(xs, W), np.einsum("jic,mi->mjc", W, x[..., 0])) < 1e-12


@pytest.mark.parametrize("name", ["c1_layer", "c3_small", "c4_small", "small_gelu", "small_relu", "small_sigmoid"])
def test_moe_layer_reproduces_the_reference_goldens(name):
    """On the reference's own routing, the float64 layer is within fp32 rounding of the reference's output."""
    p, inp, ref = load_case(name)
    wu, bu, wd, bd, _ = layer_weights(p, inp)
    N = p["B"] * p["T"]
    x = inp["x"].reshape(N, p["d"], 8)
    got = dense.moe_layer(x, ref["idx"], ref["w"], wu, bu, wd, bd, p["act"])
    assert _rel(got, ref["out"].reshape(N, p["d"], 8)) < 1e-5


def test_moe_layer_stack_reproduces_the_reference_golden():
    p, inp, ref = load_case("c5_small")
    assert p["kind"] == "stack"
    N = p["B"] * p["T"]
    x = inp["x"].reshape(N, p["d"], 8).astype(np.float64)
    for li in range(p["layers"]):
        pre = f"l{li}_"
        wu, bu, wd, bd, _ = layer_weights(p, inp, pre)
        probs = moe.softmax(inp[pre + "logits"])
        idx, w = moe.topk_reference(probs, p["k"])
        x = dense.moe_layer(x, idx, w, wu, bu, wd, bd, p["act"], residual=x)
    assert _rel(x, ref["out"].reshape(N, p["d"], 8)) < 1e-5


def test_moe_layer_against_the_reference_order_restatement():
    g = np.random.default_rng(11)
    N, d, F, E, k = 40, 6, 10, 5, 2
    x = g.standard_normal((1, N, d, 8)).astype(np.float32)
    wu = (g.standard_normal((E, F, d, 8)) / 7).astype(np.float32)
    bu = g.standard_normal((E, F, 8)).astype(np.float32)
    wd = (g.standard_normal((E, d, F, 8)) / 9).astype(np.float32)
    bd = g.standard_normal((E, d, 8)).astype(np.float32)
    logits = g.standard_normal((N, E)).astype(np.float32)
    for act in ("gelu", "relu", "sigmoid"):
        ref, info = moe.moe_forward_reference(x, None, None, [(wu[e], bu[e], wd[e], bd[e]) for e in range(E)], k,
                                              act, logits=logits)
        got = dense.moe_layer(x[0], info["idx"], info["w"], wu, bu, wd, bd, act)
        assert _rel(got, ref[0]) < 1e-5, act


def test_linear_backward_finite_differences():
    g = np.random.default_rng(5)
    M, d_in, d_out = 4, 3, 2
    x = g.standard_normal((M, d_in, 8))
    W = g.standard_normal((d_out, d_in, 8))
    b = g.standard_normal((d_out, 8))
    c = g.standard_normal((M, d_out, 8))
    dx, dW, db = dense.linear_backward(x, W, c)
    f = lambda xx, WW, bb: float(np.sum(dense.linear(xx, WW, bb) * c))
    h = 1e-6
    for arr, grad in ((x, dx), (W, dW), (b, db)):
        num = np.zeros_like(arr)
        for i in np.ndindex(arr.shape):
            orig = arr[i]
            arr[i] = orig + h
            fp = f(x, W, b)
            arr[i] = orig - h
            fm = f(x, W, b)
            arr[i] = orig
            num[i] = (fp - fm) / (2 * h)
        assert _rel(grad, num) < 1e-7


def test_linear_backward_against_the_reference_formulas():
    g = np.random.default_rng(6)
    x = g.standard_normal((30, 7, 8)).astype(np.float32)
    W = g.standard_normal((5, 7, 8)).astype(np.float32)
    dy = g.standard_normal((30, 5, 8)).astype(np.float32)
    for got, want in zip(dense.linear_backward(x, W, dy), bw.clifford_linear_backward(x, W, dy)):
        assert _rel(got, want) < 1e-5


@pytest.mark.parametrize("act,residual", [("gelu", False), ("sigmoid", True), ("relu", False)])
def test_moe_layer_backward_against_the_finite_difference_pinned_oracle(act, residual):
    g = np.random.default_rng(12)
    N, d, F, E, k = 30, 5, 9, 4, 2
    x = g.standard_normal((N, d, 8)).astype(np.float32)
    wu = (g.standard_normal((E, F, d, 8)) / 6).astype(np.float32)
    bu = (0.1 * g.standard_normal((E, F, 8))).astype(np.float32)
    wd = (g.standard_normal((E, d, F, 8)) / 8).astype(np.float32)
    bd = (0.1 * g.standard_normal((E, d, 8))).astype(np.float32)
    idx, w = moe.route_topk(moe.softmax(g.standard_normal((N, E)).astype(np.float32)), k)
    dout = g.standard_normal((N, d, 8)).astype(np.float32)
    dx, dWu, dbu, dWd, dbd = dense.moe_layer_backward(x, idx, w, wu, bu, wd, bd, dout, act, residual)
    dx_o, grads, _ = bw.moe_backward_reference(x, idx, w, [(wu[e], bu[e], wd[e], bd[e]) for e in range(E)], dout,
                                               act, residual)
    assert _rel(dx, dx_o) < 1e-5
    for j, got in enumerate((dWu, dbu, dWd, dbd)):
        assert _rel(got, np.stack([gr[j] for gr in grads])) < 1e-5, j
