"""Helpers shared by the GPU parity tests (no GPU needed to import)."""

from __future__ import annotations

import sys

import numpy as np

# Normwise relative error: max|got - ref| / max|ref|.  Element-wise relative
# error is ill-conditioned where outputs cancel to ~0, so the BASELINE bounds
# (1e-5 fp32, 2e-2 bf16 / int8 weights) are applied normwise.
TOL_F32 = 1e-5
TOL_BF16 = 2e-2


def normwise_err(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = np.abs(ref).max()
    return float(np.abs(got - ref).max() / (scale if scale > 0 else 1.0))


def say(msg: str) -> None:
    """Name the case before a GPU step (flushed, so a fault still shows it)."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def bf16_round(a: np.ndarray) -> np.ndarray:
    import _inputs

    return _inputs.bf16_round(a)


def moe_reference(x, idx, w, wu, bu, wd, bd, act, base=None, acc_dtype=np.float32):
    """The MoE layer from the oracle on a given routing (idx, w: (N, k)): each expert's FFN over all of
    its tokens in one call -- the oracle's operation order per element does not depend on how many rows
    a call holds -- then every token's slots added in ascending expert order, as the combine adds them,
    onto `base` (zeros when None)."""
    from oracle import moe

    x = np.asarray(x)
    out = np.zeros(x.shape, acc_dtype) if base is None else np.array(base, dtype=acc_dtype)
    rows = {}
    for e in np.unique(idx):
        ts = np.flatnonzero((idx == e).any(axis=1))
        y = moe.clifford_ffn(x[ts], wu[e], bu[e], wd[e], bd[e], act)
        rows[int(e)] = {int(t): y[i] for i, t in enumerate(ts)}
    for t in range(x.shape[0]):
        for s in np.argsort(idx[t]):
            out[t] += w[t, s] * rows[int(idx[t, s])][t]
    return out
