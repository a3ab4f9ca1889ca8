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
