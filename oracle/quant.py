"""NumPy restatement of grade-aware quantization and the checkpoint layouts (oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

``grade_quantize`` / ``grade_dequantize`` restate ``quantize_multivector`` /
``dequantize_multivector`` (``bifrost/quantization/grade_quantize.py:86-118,153-238``):
one scale (and, asymmetric, one zero point) per grade over the whole tensor,
computed in float64; codes ``clip(round(x / scale) + zp, qmin, qmax)`` with
NumPy's round-half-to-even; values ``(q - zp) * scale`` in float64.

``stratify`` / ``reconstruct`` restate the grade-stratified checkpoint layout
(``forge/training/checkpointing.py:22-64``): key
``param__<name>__grade_<k>`` holds ``data[..., GRADE_SLICES[k]]``, and a
parameter whose last axis is not 8 is stored whole under ``__raw``.

Pinning summary (``tests/test_oracle_quant.py``):

* quantization -- the reference test suite's properties
  (``bifrost/tests/test_quantization.py:54-102``: round-trip bounds on its own
  seeded inputs, 8-bit scalar at least as accurate as 4-bit trivector, payload
  bit count, shapes) and closed forms: values on the quantization grid come
  back exactly, every code lies in ``[qmin, qmax]``, in-range values move by at
  most half a step, the largest magnitude maps to ``qmax`` (symmetric) and the
  minimum to ``qmin`` (asymmetric, when it lies on the grid), and ties round to
  even.
* checkpoint layout -- round trip of the key scheme and the reconstruction
  rule (zeros where a grade key is missing).
"""

from __future__ import annotations

import numpy as np

GRADE_SLICES = {0: slice(0, 1), 1: slice(1, 4), 2: slice(4, 7), 3: slice(7, 8)}
DEFAULT_BITS = {0: 8, 1: 6, 2: 6, 3: 4}


def grade_quantize(mv: np.ndarray, grade_bits=None, symmetric: bool = True):
    """Returns ``(codes int64 (..., 8), scale float64 (4,), zero_point int64 (4,))``."""
    bits = DEFAULT_BITS if grade_bits is None else grade_bits
    mv = np.asarray(mv, dtype=np.float64)
    if mv.shape[-1] != 8:
        raise ValueError("last axis must be 8")
    codes = np.zeros(mv.shape, dtype=np.int64)
    scale = np.zeros(4, np.float64)
    zp = np.zeros(4, np.int64)
    for g, slc in GRADE_SLICES.items():
        b = bits[g]
        qmin, qmax = -(1 << (b - 1)), (1 << (b - 1)) - 1
        data = mv[..., slc]
        if symmetric:
            amax = max(np.max(np.abs(data)) if data.size else 1.0, 1e-12)
            s, z = amax / qmax, 0
        else:
            lo = np.min(data) if data.size else 0.0
            hi = np.max(data) if data.size else 1.0
            s = max(hi - lo, 1e-12) / (qmax - qmin)
            z = int(np.clip(np.round(qmin - lo / s), qmin, qmax))
        codes[..., slc] = np.clip(np.round(data / s) + z, qmin, qmax).astype(np.int64)
        scale[g], zp[g] = s, z
    return codes, scale, zp


def grade_dequantize(codes: np.ndarray, scale: np.ndarray, zp: np.ndarray) -> np.ndarray:
    """``(q - zp) * scale`` per grade, float64."""
    out = np.empty(codes.shape, np.float64)
    for g, slc in GRADE_SLICES.items():
        out[..., slc] = (codes[..., slc].astype(np.float64) - zp[g]) * scale[g]
    return out


def stratify(name: str, data: np.ndarray) -> dict:
    """The npz entries one parameter contributes to a grade-stratified checkpoint."""
    data = np.asarray(data)
    if data.shape and data.shape[-1] == 8:
        return {f"param__{name}__grade_{g}": data[..., slc].copy() for g, slc in GRADE_SLICES.items()}
    return {f"param__{name}__raw": data.copy()}


def reconstruct(entries: dict) -> dict:
    """``{name: array}`` from ``param__<name>__<grade_k | raw>`` entries."""
    groups: dict = {}
    for key, arr in entries.items():
        if not key.startswith("param__"):
            continue
        _, name, part = key.split("__")
        groups.setdefault(name, {})[part] = arr
    out = {}
    for name, parts in groups.items():
        if "raw" in parts:
            out[name] = parts["raw"].copy()
            continue
        data = np.zeros((*parts["grade_0"].shape[:-1], 8), np.float32)
        for g, slc in GRADE_SLICES.items():
            if f"grade_{g}" in parts:
                data[..., slc] = parts[f"grade_{g}"]
        out[name] = data
    return out
