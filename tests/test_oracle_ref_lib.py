"""Oracle against the reference's compiled CPU library (``oracle/_ref``).

``oracle/_ref/libmjolnir_cpu.so`` is built by ``oracle/Makefile`` from the
reference's own ``mjolnir/src/cpu`` sources; the reference's C known-answer
programs are built beside it and must pass.  Skipped where ``_ref`` is not
built (the GPU box has no reference tree, but carries the built files).
"""

import os
import subprocess

import numpy as np
import pytest

from oracle import cl3, moe, native

needs_ref = pytest.mark.skipif(native.ref_lib() is None, reason="oracle/_ref not built")
needs_c = pytest.mark.skipif(native.oracle_lib() is None, reason="oracle/_build not built")


@needs_ref
@pytest.mark.parametrize("shape", [(1, 1, 1), (3, 7, 5), (16, 40, 20), (64, 9, 33)])
def test_geom_matmul_bit_exact_vs_reference_c(shape):
    M, K, N = shape
    r = np.random.default_rng(M * 1000 + K * 10 + N)
    a = r.standard_normal((M, K, 8), dtype=np.float32)
    b = r.standard_normal((K, N, 8), dtype=np.float32)
    assert np.array_equal(moe.geom_matmul(a, b), native.ref_geom_matmul(a, b))


@needs_ref
def test_elementwise_product_bit_exact_vs_reference_c():
    r = np.random.default_rng(3)
    a, b = r.standard_normal((2, 4096, 8), dtype=np.float32)
    assert np.array_equal(cl3.geom_prod(a, b), native.ref_geom_prod(a, b))


@needs_ref
@pytest.mark.parametrize("prog", ["test_multiplication_table", "test_geometric_product", "test_associativity",
                                  "test_sandwich"])
def test_reference_known_answer_programs_pass(prog):
    path = os.path.join(os.path.dirname(native.REF_LIB), prog)
    if not os.path.exists(path):
        pytest.skip("reference test program not built")
    res = subprocess.run([path], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stdout[-2000:]


@needs_c
@pytest.mark.parametrize("shape", [(12, 30, 17), (1, 1, 1), (5, 0, 3), (7, 3, 1), (1, 64, 9)])
def test_c_restatement_tables_and_bits(shape):
    """The C restatement (tables, serial and OpenMP matmul, element-wise product) bit for bit
    against the NumPy restatement, on ragged shapes and an empty contraction (zeros)."""
    M, K, N = shape
    idx, sign = native.c_tables()
    assert np.array_equal(idx, cl3.PRODUCT_IDX) and np.array_equal(sign, cl3.PRODUCT_SIGN)
    r = np.random.default_rng(4 + M + K + N)
    a = r.standard_normal((M, K, 8), dtype=np.float32)
    b = r.standard_normal((K, N, 8), dtype=np.float32)
    ref = moe.geom_matmul(a, b) if K > 0 else np.zeros((M, N, 8), np.float32)
    assert np.array_equal(native.c_geom_matmul(a, b), ref)
    assert np.array_equal(native.c_geom_matmul(a, b, threads=4), ref)
    x, y = r.standard_normal((2, 3 * M + 1, 8), dtype=np.float32)
    assert np.array_equal(native.c_geom_prod(x, y), cl3.geom_prod(x, y))
