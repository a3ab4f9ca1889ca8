"""CPU: the backward oracle pinned by finite differences and the algebra's adjoints.

The reference checks its backward passes with central finite differences
(``holograph/tests/test_backward_numerical.py:28-98``); the same check here
runs in float64 on the forward restatement, so it pins the oracle's analytic
gradients far below the fp32 tolerance the GPU is held to.
"""

import numpy as np
import pytest

from oracle import backward as bw
from oracle import moe
from oracle.cl3 import geom_prod_f64, reverse


def _fd(f, x, eps=1e-6):
    """Central differences of the scalar f at x (float64), all coordinates."""
    x = np.array(x, np.float64)
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        old = x[i]
        x[i] = old + eps
        fp = f(x)
        x[i] = old - eps
        fm = f(x)
        x[i] = old
        g[i] = (fp - fm) / (2 * eps)
    return g


def test_geometric_product_adjoints():
    """<a b, c> = <b, ~a c> = <a, c ~b> for the Euclidean component inner product."""
    g = np.random.default_rng(0)
    a, b, c = (g.standard_normal((50, 8)) for _ in range(3))
    lhs = np.sum(geom_prod_f64(a, b) * c, -1)
    assert np.allclose(lhs, np.sum(b * geom_prod_f64(reverse(a), c), -1), atol=1e-12)
    assert np.allclose(lhs, np.sum(a * geom_prod_f64(c, reverse(b)), -1), atol=1e-12)


def test_clifford_linear_backward_matches_finite_differences():
    g = np.random.default_rng(1)
    M, d_in, d_out = 3, 4, 5
    x = g.standard_normal((M, d_in, 8))
    W = g.standard_normal((d_out, d_in, 8)) / 4
    b = g.standard_normal((d_out, 8))
    c = g.standard_normal((M, d_out, 8))            # loss = <c, linear(x)>
    dx, dW, db = bw.clifford_linear_backward(x, W, c)
    loss = lambda xx=x, WW=W, bb=b: np.sum(c * bw.linear_f64(xx, WW, bb))
    assert np.allclose(dx, _fd(lambda v: loss(xx=v), x), atol=2e-5)
    assert np.allclose(dW, _fd(lambda v: loss(WW=v), W), atol=2e-5)
    assert np.allclose(db, _fd(lambda v: loss(bb=v), b), atol=2e-5)


@pytest.mark.parametrize("act", ["gelu", "sigmoid", "relu", "none"])
def test_activation_backward_matches_finite_differences(act):
    g = np.random.default_rng(2)
    h = g.standard_normal((6, 8)) * 1.5
    c = g.standard_normal((6, 8))
    got = bw.activation_backward(act, h.astype(np.float32), c.astype(np.float32))
    num = _fd(lambda v: np.sum(c * bw.activation_f64(act, v)), h)
    assert np.allclose(got, num, atol=5e-5), np.max(np.abs(got - num))
    # the float64 forward is the oracle's fp32 forward
    assert np.allclose(bw.activation_f64(act, h), moe.ACTIVATIONS[act](h.astype(np.float32)), atol=1e-6)


@pytest.mark.parametrize("act,residual", [("gelu", False), ("sigmoid", True), ("relu", False)])
def test_moe_backward_matches_finite_differences(act, residual):
    g = np.random.default_rng(3)
    N, d, F, E, k = 7, 3, 4, 3, 2
    x = g.standard_normal((N, d, 8))
    experts = [((g.standard_normal((F, d, 8)) / 3), 0.1 * g.standard_normal((F, 8)),
                (g.standard_normal((d, F, 8)) / 3), 0.1 * g.standard_normal((d, 8))) for _ in range(E)]
    idx = np.stack([g.permutation(E)[:k] for _ in range(N)]).astype(np.int32)
    w = g.uniform(0.1, 1.0, (N, k))
    c = g.standard_normal((N, d, 8))
    dx, grads, dw = bw.moe_backward_reference(x, idx, w, experts, c, act, residual)

    def loss(xx=x, ex=experts, ww=w):
        return np.sum(c * bw.moe_forward_fixed_routing_f64(xx, idx, ww, ex, act, residual))

    assert np.allclose(dx, _fd(lambda v: loss(xx=v), x), atol=1e-4)
    assert np.allclose(dw, _fd(lambda v: loss(ww=v), w), atol=1e-4)
    for e in range(E):
        for j in range(4):
            def f(v, e=e, j=j):
                ex = [list(t) for t in experts]
                ex[e][j] = v
                return loss(ex=[tuple(t) for t in ex])
            assert np.allclose(grads[e][j], _fd(f, experts[e][j]), atol=1e-4), (e, j)
