"""Cl(3,0) algebra tables and the element-wise geometric product (oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Basis order (the reference's flat layout, ``rune/types/multivector.py:7``):
``1, e1, e2, e3, e12, e13, e23, e123``.

The tables are *derived* here from the defining relations of Cl(3,0)
(``e_i e_i = +1``, ``e_i e_j = -e_j e_i`` for ``i != j``) by sorting generator
words and counting transpositions, not copied.  The reference's tables are
``rune/types/multivector.py:16-58`` and ``mjolnir/include/cl3_tables.h:24-82``.

Pinning: ``tests/test_oracle_algebra.py`` checks the derived tables against
every known answer in ``mjolnir/tests/test_multiplication_table.c:29-94``
(all 64 basis products, vector squares, anticommutation, ``e123^2=-1``) and
``rune/tests/test_geometric_product.py:10-93`` (identity, scalar multiple,
associativity, distributivity, reverse anti-automorphism, ``e1^e2 = e12``),
and, where ``oracle/_ref`` is built, against the reference's own compiled
``cl3_geometric_product`` bit for bit.
"""

from __future__ import annotations

import numpy as np

# Blades as sorted tuples of generator indices, in the reference's order.
BLADES = ((), (1,), (2,), (3,), (1, 2), (1, 3), (2, 3), (1, 2, 3))
BLADE_NAMES = ("1", "e1", "e2", "e3", "e12", "e13", "e23", "e123")
_BLADE_INDEX = {b: i for i, b in enumerate(BLADES)}


def _blade_product(a: tuple, b: tuple) -> tuple[int, tuple]:
    """Product of two basis blades: returns (sign, blade).

    Concatenate the generator words, bubble-sort them counting adjacent
    transpositions (each flips the sign, by anticommutation), then cancel
    equal neighbours (``e_i e_i = +1`` in signature (3,0)).
    """
    word = list(a) + list(b)
    sign = 1
    n = len(word)
    for i in range(n):
        for j in range(n - 1 - i):
            if word[j] > word[j + 1]:
                word[j], word[j + 1] = word[j + 1], word[j]
                sign = -sign
    out = []
    for g in word:
        if out and out[-1] == g:
            out.pop()
        else:
            out.append(g)
    return sign, tuple(out)


def _build_tables():
    idx = np.zeros((8, 8), dtype=np.int32)
    sgn = np.zeros((8, 8), dtype=np.float32)
    for i, bi in enumerate(BLADES):
        for j, bj in enumerate(BLADES):
            s, blade = _blade_product(bi, bj)
            idx[i, j] = _BLADE_INDEX[blade]
            sgn[i, j] = s
    return idx, sgn


#: ``e_i * e_j = PRODUCT_SIGN[i, j] * e_{PRODUCT_IDX[i, j]}``
PRODUCT_IDX, PRODUCT_SIGN = _build_tables()
PRODUCT_IDX.setflags(write=False)
PRODUCT_SIGN.setflags(write=False)

BASIS_GRADE = np.array([len(b) for b in BLADES], dtype=np.int32)
#: grade slices in the flat 8-component layout
GRADE_SLICES = {0: slice(0, 1), 1: slice(1, 4), 2: slice(4, 7), 3: slice(7, 8)}
#: reverse: (-1)^(g(g-1)/2) per blade
REVERSE_SIGN = np.array([(-1) ** (g * (g - 1) // 2) for g in BASIS_GRADE], dtype=np.float32)


def geom_prod(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Element-wise geometric product ``a * b`` over the last axis (8).

    fp32 term order of the reference's NumPy path
    (``rune/ops/batched.py:72-82``): output component ``IDX[i, j]`` receives
    ``(SIGN[i, j] * a_i) * b_j`` for ``i = 0..7`` outer, ``j = 0..7`` inner,
    each product rounded to fp32 before it is added to a zero accumulator.
    """
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    shape = np.broadcast_shapes(a.shape, b.shape)
    out = np.zeros(shape, dtype=np.float32)
    for i in range(8):
        ai = a[..., i]
        for j in range(8):
            out[..., PRODUCT_IDX[i, j]] += float(PRODUCT_SIGN[i, j]) * ai * b[..., j]
    return out


def geom_prod_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Exact-ish float64 geometric product (for truth values in tests)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    out = np.zeros(np.broadcast_shapes(a.shape, b.shape), dtype=np.float64)
    for i in range(8):
        for j in range(8):
            out[..., PRODUCT_IDX[i, j]] += PRODUCT_SIGN[i, j] * a[..., i] * b[..., j]
    return out


def reverse(a: np.ndarray) -> np.ndarray:
    """Reversion ``~a`` (``rune/ops/batched.py:84-87``)."""
    return np.asarray(a, dtype=np.float32) * REVERSE_SIGN


def left_mul_matrix_table() -> tuple[np.ndarray, np.ndarray]:
    """Source component and sign of every entry of ``L(w)``.

    ``(w * x)_r = sum_q L(w)[r, q] x_q`` with ``L(w)[r, q] = sign[r, q] * w[src[r, q]]``.
    For a fixed column ``q`` the map ``p -> IDX[p, q]`` is a bijection, so
    every entry of ``L(w)`` is exactly one signed weight component (no
    structural zeros).  Reference precedent for the expansion:
    ``geoformer/hlm_v9_model_raw.py:62-100``.
    """
    src = np.full((8, 8), -1, dtype=np.int32)
    sgn = np.zeros((8, 8), dtype=np.float32)
    for p in range(8):
        for q in range(8):
            r = PRODUCT_IDX[p, q]
            assert src[r, q] == -1
            src[r, q] = p
            sgn[r, q] = PRODUCT_SIGN[p, q]
    assert (src >= 0).all()
    return src, sgn


L_SRC, L_SIGN = left_mul_matrix_table()


def left_mul_matrix(w: np.ndarray) -> np.ndarray:
    """``L(w)`` for ``w`` of shape ``(..., 8)`` -> ``(..., 8, 8)``."""
    w = np.asarray(w)
    return w[..., L_SRC] * L_SIGN.astype(w.dtype)
