"""fp32-faithful NumPy restatement of the pre-norm around the MoE (oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

``clifford_layer_norm`` restates ``CliffordLayerNorm.forward``
(``holograph/layers/normalization.py:44-67``) and ``block_ffn_reference`` the
FFN half of ``HLMBlock.forward`` (``holograph/models/hlm_block.py:144-151``):
``x + moe(ffn_norm(x))``.

The device kernel follows the reduction order that NumPy uses for the two
sums, which ``pairwise_sum_f32`` spells out step by step (NumPy's pairwise
summation of a contiguous row: fewer than 8 values in order from zero; up to
128 values eight strided accumulators combined as a tree, then the remainder
in order; longer rows split at ``n/2`` rounded down to a multiple of 8).

Pinning summary (tests in ``tests/test_oracle_norm.py``):

* ``pairwise_sum_f32`` -- bit for bit against ``np.sum`` over the last axis for
  every row length 1..1100 and random data (the device kernel's sum order).
* ``clifford_layer_norm`` -- closed forms: with ``gamma`` the scalar 1 and
  ``beta`` zero the output is ``x / sqrt(mean_i |x_i|^2 + 2 eps)``, checked
  against a float64 evaluation; with a general ``gamma`` the output equals the
  float64 geometric product ``gamma x_hat`` plus ``beta`` (Cayley tables pinned
  separately); invariance under ``x -> c x`` when eps is negligible; bit-exact
  agreement with the literal NumPy expression of the reference on random data.
* ``block_ffn_reference`` -- composition of the pinned norm and
  ``moe.moe_forward_reference`` (reference goldens) with the residual add.
"""

from __future__ import annotations

import numpy as np

from .cl3 import geom_prod
from .moe import moe_forward_reference

F32 = np.float32

#: NumPy's pairwise-summation block (``PW_BLOCKSIZE``)
PW_BLOCK = 128


def pairwise_sum_f32(a: np.ndarray) -> np.ndarray:
    """Sum over the last axis in NumPy's pairwise order, spelled out (fp32)."""
    a = np.asarray(a, dtype=F32)
    n = a.shape[-1]
    if n < 8:
        res = np.zeros(a.shape[:-1], F32)
        for i in range(n):
            res = res + a[..., i]
        return res
    if n <= PW_BLOCK:
        r = [a[..., j].copy() for j in range(8)]
        n8 = n - n % 8
        for i in range(8, n8, 8):
            for j in range(8):
                r[j] = r[j] + a[..., i + j]
        res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]))
        for i in range(n8, n):
            res = res + a[..., i]
        return res
    n2 = n // 2
    n2 -= n2 % 8
    return pairwise_sum_f32(a[..., :n2]) + pairwise_sum_f32(a[..., n2:])


def clifford_layer_norm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """``CliffordLayerNorm.forward`` (``normalization.py:44-67``), fp32.

    ``x``: (..., d, 8); ``gamma``, ``beta``: (d, 8).  RMS of the multivector norms
    over d (``rms^2 = mean_i |x_i|^2 + 2 eps``), ``x_hat = x / rms``, then
    ``gamma x_hat`` (geometric product, gamma on the left) ``+ beta``.
    """
    x = np.asarray(x, dtype=F32)
    norm_sq = pairwise_sum_f32(x * x)                       # (..., d)
    mean = pairwise_sum_f32(norm_sq) / F32(norm_sq.shape[-1])
    rms = np.sqrt(mean + F32(2.0 * eps))[..., None]          # (..., 1)
    x_hat = x / rms[..., None]
    return geom_prod(np.asarray(gamma, F32), x_hat) + np.asarray(beta, F32)


def block_ffn_reference(x, gamma, beta, router_weight, router_bias, experts, k, activation="gelu", logits=None,
                        eps: float = 1e-6):
    """FFN half of ``HLMBlock.forward`` (``hlm_block.py:144-151``): ``x + moe(ffn_norm(x))``.

    ``x``: (B, T, d, 8).  The router sees the normed tokens, as in the reference
    (``_moe_forward`` receives ``x_norm``).  Returns ``(out, info)``.
    """
    x = np.asarray(x, dtype=F32)
    x_norm = clifford_layer_norm(x, gamma, beta, eps)
    ffn_out, info = moe_forward_reference(x_norm, router_weight, router_bias, experts, k, activation, logits)
    info["x_norm"] = x_norm
    return x + ffn_out, info
