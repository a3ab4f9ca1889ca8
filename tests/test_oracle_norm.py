"""CPU: the pre-norm oracle (CliffordLayerNorm, normalization.py:44-67) pinned.

No reference fixture holds a forward of the norm, so the oracle is pinned by
what the mathematics fixes: NumPy's own sums (the order the device kernel
follows), the closed form for a scalar-1 gamma, the float64 geometric product
for a general gamma, invariance under x -> c x, and the eps term, which the
small-magnitude case makes visible.
"""

import numpy as np
import pytest

from oracle import moe
from oracle.cl3 import geom_prod_f64
from oracle.norm import block_ffn_reference, clifford_layer_norm, pairwise_sum_f32


@pytest.mark.parametrize("n", list(range(1, 140)) + [255, 256, 257, 300, 511, 1000, 1031, 2047, 4096])
def test_pairwise_sum_is_numpys_sum(n):
    g = np.random.default_rng(n)
    a = (g.standard_normal((6, n)) * g.uniform(0.01, 100.0, (6, 1))).astype(np.float32)
    assert np.array_equal(pairwise_sum_f32(a), np.sum(a, axis=-1))


def test_pairwise_order_differs_from_a_running_sum():
    """The order is observable: a running sum of long rows differs in the last bits."""
    a = np.random.default_rng(0).standard_normal((64, 1000)).astype(np.float32)
    seq = np.zeros(64, np.float32)
    for i in range(a.shape[1]):
        seq = seq + a[:, i]
    assert not np.array_equal(seq, pairwise_sum_f32(a))


def _literal(x, gamma, beta, eps=1e-6):
    """The reference's expression as NumPy evaluates it (normalization.py:54-62)."""
    from oracle.cl3 import geom_prod

    norm_sq = np.sum(x * x, axis=-1)
    rms = np.sqrt(np.mean(norm_sq, axis=-1, keepdims=True) + (2.0 * eps))
    return geom_prod(gamma, x / rms[..., np.newaxis]) + beta


@pytest.mark.parametrize("shape", [(2, 3, 4), (5, 64), (1, 7, 129), (3, 300), (2, 1000)])
def test_norm_matches_the_literal_numpy_expression(shape):
    g = np.random.default_rng(sum(shape))
    d = shape[-1]
    x = g.standard_normal((*shape, 8)).astype(np.float32)
    gamma = g.standard_normal((d, 8)).astype(np.float32)
    beta = g.standard_normal((d, 8)).astype(np.float32)
    assert np.array_equal(clifford_layer_norm(x, gamma, beta), _literal(x, gamma, beta))


def _rms64(x, eps):
    x = x.astype(np.float64)
    return np.sqrt(np.mean(np.sum(x * x, axis=-1), axis=-1) + 2.0 * eps)


def test_scalar_gamma_is_division_by_rms():
    g = np.random.default_rng(1)
    d = 48
    x = g.standard_normal((9, d, 8)).astype(np.float32)
    gamma = np.zeros((d, 8), np.float32)
    gamma[:, 0] = 1.0
    y = clifford_layer_norm(x, gamma, np.zeros((d, 8), np.float32))
    want = x.astype(np.float64) / _rms64(x, 1e-6)[:, None, None]
    assert np.max(np.abs(y - want)) < 4e-7 * np.max(np.abs(want))
    # unit RMS of the multivector norms after the norm (up to the eps term)
    assert np.allclose(np.sqrt(np.mean(np.sum(y.astype(np.float64) ** 2, -1), -1)), 1.0, atol=1e-5)


def test_general_gamma_is_the_left_geometric_product():
    g = np.random.default_rng(2)
    d = 16
    x = g.standard_normal((4, d, 8)).astype(np.float32)
    gamma = g.standard_normal((d, 8)).astype(np.float32)
    beta = g.standard_normal((d, 8)).astype(np.float32)
    y = clifford_layer_norm(x, gamma, beta)
    xh = x.astype(np.float64) / _rms64(x, 1e-6)[:, None, None]
    want = geom_prod_f64(gamma.astype(np.float64), xh) + beta
    assert np.max(np.abs(y - want)) < 1e-5
    # gamma on the right gives a different answer (the product does not commute)
    wrong = geom_prod_f64(xh, gamma.astype(np.float64)) + beta
    assert np.max(np.abs(y - wrong)) > 1e-2


def test_scale_invariance_and_the_eps_term():
    g = np.random.default_rng(3)
    d = 32
    x = g.standard_normal((3, d, 8)).astype(np.float32)
    gamma = g.standard_normal((d, 8)).astype(np.float32)
    beta = np.zeros((d, 8), np.float32)
    y1 = clifford_layer_norm(x, gamma, beta)
    y2 = clifford_layer_norm(np.float32(64.0) * x, gamma, beta)
    assert np.max(np.abs(y1 - y2)) < 1e-5
    # tiny inputs: the rms carries 2 eps, not eps and not zero
    tiny = (1e-4 * x).astype(np.float32)
    y = clifford_layer_norm(tiny, np.eye(1, 8, dtype=np.float32).repeat(d, 0), beta, eps=1e-6)
    for e2, ok in ((2e-6, True), (1e-6, False), (0.0, False)):
        r = np.sqrt(np.mean(np.sum(tiny.astype(np.float64) ** 2, -1), -1) + e2)
        close = np.max(np.abs(y - tiny / r[:, None, None])) < 1e-5
        assert close == ok, e2


def test_block_ffn_adds_the_residual_to_the_moe_of_the_normed_tokens():
    g = np.random.default_rng(4)
    B, T, d, F, E, k = 1, 12, 6, 10, 3, 2
    x = g.standard_normal((B, T, d, 8)).astype(np.float32)
    gamma = g.standard_normal((d, 8)).astype(np.float32)
    beta = (0.1 * g.standard_normal((d, 8))).astype(np.float32)
    experts = [tuple((0.3 * g.standard_normal(s)).astype(np.float32) for s in ((F, d, 8), (F, 8), (d, F, 8), (d, 8)))
               for _ in range(E)]
    rw = g.standard_normal((E, 4)).astype(np.float32)
    rb = np.zeros(E, np.float32)
    out, info = block_ffn_reference(x, gamma, beta, rw, rb, experts, k)
    xn = clifford_layer_norm(x, gamma, beta)
    moe_out, info2 = moe.moe_forward_reference(xn, rw, rb, experts, k)
    assert np.array_equal(out, x + moe_out)
    assert np.array_equal(info["idx"], info2["idx"])
    # the router saw the normed tokens, not x
    assert np.array_equal(info["logits"], moe.router_logits(xn.reshape(-1, d, 8), rw, rb)[0])
