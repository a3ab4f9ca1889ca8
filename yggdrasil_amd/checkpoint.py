"""Import of the reference's checkpoint layouts into the MI355X layer modules.

The reference stores parameters in ``.npz`` files in three layouts, all of
which ``holograph/model.py:56-82`` accepts:

* grade-stratified Forge checkpoints (``forge/training/checkpointing.py:22-64,128-160``):
  ``param__<name>__grade_<k>`` holds ``data[..., GRADE_SLICES[k]]`` for a
  multivector parameter, ``param__<name>__raw`` any other parameter;
* whole arrays under ``param__<name>``;
* serving exports: ``param_<i>`` in ``model.parameters()`` order.

A parameter's name is ``param_<i>``, its index in ``model.parameters()``
(``forge/param_utils.py:31-34``), unless the parameter is a dict with a name.
Files are opened with ``allow_pickle=False``: nothing in them is executed.

The arrays read here are fp32 host arrays; the modules' ``prepare()`` turns
them into the device layouts (bf16 / int8 / Pauli) on the GPU.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field

import numpy as np

#: component ranges of the grades in blade order (``rune/types/multivector.py``)
GRADE_SLICES = {0: slice(0, 1), 1: slice(1, 4), 2: slice(4, 7), 3: slice(7, 8)}


def resolve_checkpoint_path(path: str) -> str:
    """A file, or a directory's ``model.npz`` (else its first ``.npz``), as ``holograph/model.py:29-41``."""
    if os.path.isdir(path):
        cand = os.path.join(path, "model.npz")
        if os.path.exists(cand):
            return cand
        npz = sorted(os.path.join(path, n) for n in os.listdir(path) if n.endswith(".npz"))
        if not npz:
            raise FileNotFoundError(f"no .npz checkpoint in {path}")
        return npz[0]
    return path


def read_reference_checkpoint(path: str) -> dict[str, np.ndarray]:
    """``{parameter name: array}`` from any of the three layouts.

    Grade-stratified entries are reassembled as ``load_checkpoint`` does: an
    fp32 ``(..., 8)`` array of zeros with each stored grade written into its
    components.
    """
    with np.load(resolve_checkpoint_path(path), allow_pickle=False) as z:
        keys = list(z.files)
        if any(k.startswith("param__") and "__grade_" in k for k in keys):
            groups: dict[str, dict[str, np.ndarray]] = {}
            for k in keys:
                if k.startswith("param__"):
                    parts = k.split("__")
                    if len(parts) != 3:
                        raise ValueError(f"unexpected checkpoint key {k!r}")
                    groups.setdefault(parts[1], {})[parts[2]] = z[k]
            out = {}
            for name, g in groups.items():
                if "raw" in g:
                    out[name] = np.array(g["raw"])
                    continue
                if "grade_0" not in g:
                    raise ValueError(f"parameter {name!r} has no grade_0 entry")
                data = np.zeros((*g["grade_0"].shape[:-1], 8), np.float32)
                for grade, slc in GRADE_SLICES.items():
                    key = f"grade_{grade}"
                    if key in g:
                        data[..., slc] = g[key]
                out[name] = data
            return out
        if any(k.startswith("param__") for k in keys):
            return {k.split("param__", 1)[1]: np.array(z[k]) for k in keys if k.startswith("param__")}
        return {k: np.array(z[k]) for k in keys if k.startswith("param_")}


def hlm_block_ffn_state(state: dict[str, np.ndarray], first: int, n_experts: int) -> dict[str, np.ndarray]:
    """The FFN half of one ``HLMBlock`` from ``param_<i>`` entries.

    ``HLMBlock.parameters()`` (``hlm_block.py:230-241``) lists, after the
    attention half, ``ffn_norm.gamma, ffn_norm.beta`` (``normalization.py:105-107``),
    ``router.router_weight, router.router_bias`` (``clifford_router.py:119-120``)
    and for each expert ``up.weight, up.bias, down.weight, down.bias``
    (``hlm_block.py:89-90``, ``clifford_linear.py:169-173``).  ``first`` is the
    index of ``ffn_norm.gamma``.
    """
    def get(i):
        key = f"param_{i}"
        if key not in state:
            raise KeyError(f"checkpoint has no {key}")
        return np.asarray(state[key], dtype=np.float32)

    out = dict(gamma=get(first), beta=get(first + 1), router_weight=get(first + 2), router_bias=get(first + 3))
    ex = [[get(first + 4 + 4 * e + j) for j in range(4)] for e in range(n_experts)]
    out["w_up"] = np.stack([e[0] for e in ex])
    out["b_up"] = np.stack([e[1] for e in ex])
    out["w_down"] = np.stack([e[2] for e in ex])
    out["b_down"] = np.stack([e[3] for e in ex])
    E, F, d = out["w_up"].shape[:3]
    shapes = dict(gamma=(d, 8), beta=(d, 8), router_weight=(E, 4), router_bias=(E,), w_up=(E, F, d, 8),
                  b_up=(E, F, 8), w_down=(E, d, F, 8), b_down=(E, d, 8))
    for k, want in shapes.items():
        if out[k].shape != want:
            raise ValueError(f"{k}: shape {out[k].shape}, expected {want} (is param_{first} the ffn_norm gamma?)")
    return out


@dataclass
class GradeQuantConfig:
    """Per-grade bit widths of grade-aware quantization (``CliffordQuantConfig``,
    ``bifrost/quantization/grade_quantize.py:42-70``): default 8/6/6/4 bits for
    grades 0-3, symmetric."""

    grade_bits: dict = field(default_factory=lambda: {0: 8, 1: 6, 2: 6, 3: 4})
    symmetric: bool = True

    def __post_init__(self):
        for g in range(4):
            if g not in self.grade_bits:
                raise ValueError(f"missing bit width for grade {g}")
            if not 2 <= self.grade_bits[g] <= 16:
                raise ValueError(f"bit width for grade {g} must be in [2, 16], got {self.grade_bits[g]}")

    def bits(self) -> tuple:
        return tuple(self.grade_bits[g] for g in range(4))
