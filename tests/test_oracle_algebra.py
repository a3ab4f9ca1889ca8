"""Pin the oracle's algebra against the reference's known answers and the mathematics.

Known answers re-derived from ``mjolnir/tests/test_multiplication_table.c:29-94``
and ``rune/tests/test_geometric_product.py:10-93``; the rest are closed forms,
invariants and float64 brute force chosen so that a wrong sign, index or
operand order fails at least one of them.
"""

import numpy as np
import pytest

from oracle import cl3, moe


def basis(i):
    v = np.zeros(8, np.float32)
    v[i] = 1
    return v


def test_all_64_basis_products_are_signed_basis_blades():
    for i in range(8):
        for j in range(8):
            r = cl3.geom_prod(basis(i), basis(j))
            exp = np.zeros(8, np.float32)
            exp[cl3.PRODUCT_IDX[i, j]] = cl3.PRODUCT_SIGN[i, j]
            assert np.array_equal(r, exp)


def test_named_products():
    # e_i^2 = +1 (signature (3,0)), e123^2 = -1, e1 e2 = e12, e2 e1 = -e12,
    # e12 e12 = -1, e1 e23 = e123, e3 e12 = e123, e2 e13 = -e123
    names = {n: i for i, n in enumerate(cl3.BLADE_NAMES)}

    def mul(a, b):
        return cl3.geom_prod(basis(names[a]), basis(names[b]))

    for v in ("e1", "e2", "e3"):
        assert np.array_equal(mul(v, v), basis(0))
    assert np.array_equal(mul("e123", "e123"), -basis(0))
    assert np.array_equal(mul("e1", "e2"), basis(names["e12"]))
    assert np.array_equal(mul("e2", "e1"), -basis(names["e12"]))
    assert np.array_equal(mul("e12", "e12"), -basis(0))
    assert np.array_equal(mul("e1", "e23"), basis(names["e123"]))
    assert np.array_equal(mul("e3", "e12"), basis(names["e123"]))
    assert np.array_equal(mul("e2", "e13"), -basis(names["e123"]))


def test_anticommutation_of_vectors():
    for i in range(1, 4):
        for j in range(i + 1, 4):
            s = cl3.geom_prod(basis(i), basis(j)) + cl3.geom_prod(basis(j), basis(i))
            assert np.array_equal(s, np.zeros(8, np.float32))


def test_identity_and_scalar_multiple():
    a = np.array([2, 3, -1, 0.5, 1.5, -0.5, 2, -1], np.float32)
    assert np.allclose(cl3.geom_prod(basis(0), a), a, atol=1e-5)
    b = np.arange(1, 9, dtype=np.float32)
    assert np.allclose(cl3.geom_prod(3 * basis(0), b), 3 * b, atol=1e-5)


@pytest.mark.parametrize("seed", [42, 123, 77])
def test_associativity_distributivity_reverse(seed):
    r = np.random.default_rng(seed)
    a, b, c = (r.standard_normal((50, 8)) for _ in range(3))
    gp = cl3.geom_prod_f64
    assert np.allclose(gp(gp(a, b), c), gp(a, gp(b, c)), atol=1e-10)
    assert np.allclose(gp(a, b + c), gp(a, b) + gp(a, c), atol=1e-10)
    rev = lambda v: v * cl3.REVERSE_SIGN
    assert np.allclose(rev(gp(a, b)), gp(rev(b), rev(a)), atol=1e-10)


def test_outer_product_of_e1_e2_is_e12():
    # for orthogonal vectors the geometric product is the outer product
    assert np.array_equal(cl3.geom_prod(basis(1), basis(2)), basis(4))


def test_fp32_product_matches_f64_truth():
    r = np.random.default_rng(5)
    a, b = r.standard_normal((2, 1000, 8)).astype(np.float32)
    assert np.allclose(cl3.geom_prod(a, b), cl3.geom_prod_f64(a, b), rtol=1e-5, atol=1e-5)


def test_left_multiplication_matrix():
    r = np.random.default_rng(6)
    w, x = r.standard_normal((2, 200, 8))
    L = cl3.left_mul_matrix(w)
    assert np.allclose(np.einsum("nrq,nq->nr", L, x), cl3.geom_prod_f64(w, x), atol=1e-12)
    # no structural zeros: every row and column of L(w) uses each w_p exactly once
    for rr in range(8):
        assert sorted(cl3.L_SRC[rr]) == list(range(8))
        assert sorted(cl3.L_SRC[:, rr]) == list(range(8))


def test_geom_matmul_against_f64_and_special_cases():
    r = np.random.default_rng(7)
    a = r.standard_normal((6, 9, 8)).astype(np.float32)
    b = r.standard_normal((9, 5, 8)).astype(np.float32)
    out = moe.geom_matmul(a, b)
    truth = moe.geom_matmul_f64(a, b)
    assert np.allclose(out, truth, rtol=1e-5, atol=1e-5)
    # brute force with the element-wise product
    brute = np.zeros((6, 5, 8))
    for m in range(6):
        for n in range(5):
            for k in range(9):
                brute[m, n] += cl3.geom_prod_f64(a[m, k], b[k, n])
    assert np.allclose(truth, brute, atol=1e-10)
    # scalar-only weights: every component is an ordinary matmul
    a_s = np.zeros_like(a)
    a_s[..., 0] = a[..., 0]
    out_s = moe.geom_matmul(a_s, b)
    for c in range(8):
        assert np.allclose(out_s[..., c], a[..., 0] @ b[..., c], rtol=1e-5, atol=1e-5)
    # scalar-only inputs: y[m, n] = sum_k W[m, k] * x_k
    b_s = np.zeros_like(b)
    b_s[..., 0] = b[..., 0]
    out_b = moe.geom_matmul(a, b_s)
    assert np.allclose(out_b, np.einsum("mkc,kn->mnc", a, b[..., 0]), rtol=1e-5, atol=1e-5)


def test_clifford_linear_weight_on_left():
    # W * x != x * W in general; the layer multiplies the weight on the left
    r = np.random.default_rng(8)
    w = r.standard_normal((1, 1, 8)).astype(np.float32)
    x = r.standard_normal((3, 1, 8)).astype(np.float32)
    y = moe.clifford_linear(x, w, None)
    assert np.allclose(y[:, 0], cl3.geom_prod_f64(w[0, 0], x[:, 0]), atol=1e-5)
    assert not np.allclose(y[:, 0], cl3.geom_prod_f64(x[:, 0], w[0, 0]), atol=1e-3)


def test_activation_closed_forms():
    r = np.random.default_rng(9)
    x = r.standard_normal((500, 8)).astype(np.float32) * 2
    g = moe.gelu(x)
    x64 = x.astype(np.float64)
    gel = lambda v: 0.5 * v * (1 + np.tanh(np.sqrt(2 / np.pi) * (v + 0.044715 * v ** 3)))
    assert np.allclose(g[:, 0], gel(x64[:, 0]), rtol=1e-6, atol=1e-7)
    assert np.allclose(g[:, 7], np.tanh(x64[:, 7]), rtol=1e-6, atol=1e-7)
    for sl in (slice(1, 4), slice(4, 7)):
        m = np.sqrt((x64[:, sl] ** 2).sum(-1, keepdims=True) + 1e-12)
        assert np.allclose(g[:, sl], x64[:, sl] / m * gel(m), rtol=1e-5, atol=1e-6)
    # scalar-only input: the textbook GELU on the scalar, zero elsewhere
    s = np.zeros_like(x)
    s[:, 0] = x[:, 0]
    gs = moe.gelu(s)
    assert np.allclose(gs[:, 1:7], 0, atol=1e-6) and np.array_equal(gs[:, 7], np.zeros(500, np.float32))
    rl = moe.relu(x)
    assert np.array_equal(rl[:, 0], np.maximum(x[:, 0], 0))
    assert np.allclose(rl[:, 1:4], x[:, 1:4], rtol=1e-5, atol=1e-6)  # zero threshold keeps vectors
    assert np.allclose(rl[:, 7], x[:, 7], atol=0)
    sg = moe.sigmoid(x)
    assert np.allclose(sg[:, 0], 1 / (1 + np.exp(-x64[:, 0])), rtol=1e-6)


def _pauli_matrix(w):
    p = moe.pauli_entries(w)
    return (p[..., 0::2] + 1j * p[..., 1::2]).reshape(p.shape[:-1] + (2, 2))


def test_pauli_entries_are_the_pauli_matrices():
    # scalar -> I, e1 -> sigma_x, e2 -> sigma_y, e3 -> sigma_z (the textbook matrices)
    sx = np.array([[0, 1], [1, 0]])
    sy = np.array([[0, -1j], [1j, 0]])
    sz = np.array([[1, 0], [0, -1]])
    for i, want in ((0, np.eye(2)), (1, sx), (2, sy), (3, sz), (4, sx @ sy), (5, sx @ sz), (6, sy @ sz),
                    (7, sx @ sy @ sz)):
        assert np.array_equal(_pauli_matrix(basis(i)), want), cl3.BLADE_NAMES[i]


def test_pauli_map_is_an_algebra_isomorphism():
    """The geometric product is the matrix product of the entries' matrices (float64), and
    from_pauli_entries inverts pauli_entries exactly on fp32 weights."""
    r = np.random.default_rng(31)
    a = r.standard_normal((50, 8))
    b = r.standard_normal((50, 8))
    ab = cl3.geom_prod_f64(a, b)
    assert np.allclose(_pauli_matrix(ab), _pauli_matrix(a) @ _pauli_matrix(b), rtol=0, atol=1e-12)
    # the weight on the left: W x differs from x W
    assert not np.allclose(_pauli_matrix(ab), _pauli_matrix(b) @ _pauli_matrix(a))
    a32 = a.astype(np.float32)  # weights are fp32: their entries (sums of two floats) are exact in float64
    assert np.array_equal(moe.from_pauli_entries(moe.pauli_entries(a32)), a32.astype(np.float64))
