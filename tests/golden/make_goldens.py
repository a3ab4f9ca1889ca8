"""Write the golden fixtures by running the reference's own NumPy CPU path.

Run in the development container only (the reference tree is not on the GPU
box):  ``python tests/golden/make_goldens.py /root/reference``.

What is imported from the reference and executed (nothing is copied):

* ``rune.ops.batched.geom_matmul`` -- with no Mjolnir library built, the
  NumPy broadcast fallback (``rune/ops/batched.py:341-344``);
* ``holograph.models.hlm_block.HLMBlock._moe_forward`` with its
  ``CliffordRouter`` and ``CliffordFFN`` experts (``hlm_block.py:154-183``),
  parameters overwritten by the seeded arrays of ``_inputs.py``;
* ``holograph.layers.clifford_linear.CliffordLinear`` for the LM-head style
  logits (``holograph/models/hlm.py:109,141-145``);
* ``holograph.layers.clifford_router._softmax`` for route-from-logits cases.

For route-from-logits cases the layer's router is replaced by a stand-in that
applies the reference router's gating steps (``clifford_router.py:93-104``)
to the given logits; everything after the router is the reference's code.
Experts are wrapped to record the rows each one receives, which observes the
reference's dispatch order (the expert-grouped token permutation).

Each ``<case>.npz`` holds ``params`` (JSON), ``sha_<input>`` digests and the
reference outputs ``ref_*``.  NumPy's version is recorded: the reference's
fp32 rounding of the tanh-GELU depends on NumPy 2 promotion rules.
"""

from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.abspath(os.path.join(HERE, "..", "..")))

import _inputs  # noqa: E402

CASES = {
    "gm_small": dict(kind="geom_matmul", seed=1, M=8, K=16, N=12),
    "gm_rect": dict(kind="geom_matmul", seed=2, M=5, K=33, N=7),
    "c1_layer": dict(kind="layer", seed=101, B=2, T=128, d=64, E=8, k=2, F=256, act="gelu", logits=None),
    "c1_head": dict(kind="layer", seed=102, B=2, T=64, d=64, E=8, k=2, F=256, act="gelu", logits="clifford_head"),
    "small_gelu": dict(kind="layer", seed=201, B=2, T=12, d=8, E=4, k=2, F=16, act="gelu", logits=None,
                       bias_std=0.5, router_bias_std=0.3),
    "small_relu": dict(kind="layer", seed=202, B=2, T=12, d=8, E=4, k=2, F=16, act="relu", logits=None,
                       bias_std=0.5, router_bias_std=0.3),
    "small_sigmoid": dict(kind="layer", seed=203, B=2, T=12, d=8, E=4, k=3, F=16, act="sigmoid", logits=None,
                          bias_std=0.5, router_bias_std=0.3),
    "c2_route": dict(kind="route", seed=301, N=2048, E=16, k=2, d=8),
    "c3_small": dict(kind="layer", seed=401, B=1, T=256, d=16, E=8, k=4, F=64, act="gelu", logits="zipf", bf16=True),
    "c4_small": dict(kind="layer", seed=501, B=1, T=16, d=16, E=8, k=2, F=64, act="gelu", logits="normal",
                     bf16=True, int8=True),
    "c5_small": dict(kind="stack", seed=601, B=1, T=64, d=16, E=8, k=2, F=64, act="gelu", logits="normal_bias",
                     bf16=True, layers=2),
}


class _LogitsRouter:
    """Router stand-in: the reference gating steps applied to given logits."""

    def __init__(self, logits, k, softmax):
        self.logits, self.k, self.softmax = logits, k, softmax

    def forward(self, flat_x):
        probs = self.softmax(self.logits, axis=-1)
        idx = np.argsort(probs, axis=-1)[..., -self.k:]
        w = np.take_along_axis(probs, idx, axis=-1)
        w = w / (np.sum(w, axis=-1, keepdims=True) + 1e-12)
        return idx, w, None


class _Recorder:
    """Wraps an expert and records the rows it receives."""

    def __init__(self, inner, log, e):
        self.inner, self.log, self.e = inner, log, e

    def forward(self, x):
        self.log.append((self.e, np.array(x, copy=True)))
        return self.inner.forward(x) if self.inner is not None else np.array(x, copy=True)


def _tokens_of(rows, flat_x):
    """Token id of every recorded row (rows of random data are unique)."""
    keys = {flat_x[t].tobytes(): t for t in range(flat_x.shape[0])}
    return np.array([keys[r.tobytes()] for r in rows], dtype=np.int32)


def _run_layer(mods, p, inp, pre, x):
    """Run the reference ``_moe_forward`` once; returns (out, extras)."""
    HLMBlock = mods["HLMBlock"]
    E, k, d, F = p["E"], p["k"], p["d"], p["F"]
    block = HLMBlock(d, 1, F, activation=p["act"], use_moe=True, n_experts=E, moe_top_k=k)
    block.router.router_weight[...] = inp[pre + "router_w"]
    block.router.router_bias[...] = inp[pre + "router_b"]
    wu, bu, wd, bd = inp[pre + "w_up"], inp[pre + "b_up"], inp[pre + "w_down"], inp[pre + "b_down"]
    if p.get("int8"):
        from oracle.moe import quantize_int8, dequantize_int8
        wu = dequantize_int8(*quantize_int8(wu))
        wd = dequantize_int8(*quantize_int8(wd))
    for e, ex in enumerate(block.experts):
        ex.up.weight[...] = wu[e]
        ex.up.bias[...] = bu[e]
        ex.down.weight[...] = wd[e]
        ex.down.bias[...] = bd[e]
    N = x.shape[0] * x.shape[1]
    flat_x = x.reshape(N, d, 8)
    extras = {}
    lg = p.get("logits")
    if lg is None:
        idx, w, energy = block.router.forward(flat_x)
        extras["energy"] = energy
    else:
        if lg == "clifford_head":
            head = mods["CliffordLinear"](d, E, bias=False)
            head.weight[...] = inp[pre + "head_w"]
            logits = head.forward(flat_x)[..., 0]
        else:
            logits = inp[pre + "logits"]
        extras["logits"] = np.asarray(logits, dtype=np.float32)
        router = _LogitsRouter(extras["logits"], k, mods["_softmax"])
        idx, w, _ = router.forward(flat_x)
        block.router = router
    extras["idx"], extras["w"] = idx, w
    log = []
    block.experts = [_Recorder(ex, log, e) for e, ex in enumerate(block.experts)]
    out = block._moe_forward(x)
    extras["counts"] = np.bincount(idx.reshape(-1), minlength=E).astype(np.int32)
    extras["perm"] = np.concatenate([_tokens_of(rows, flat_x) for _, rows in log]) if log else np.zeros(0, np.int32)
    extras["perm_experts"] = np.array([e for e, _ in log], dtype=np.int32)
    return out, extras


def main(ref_root: str) -> None:
    sys.dont_write_bytecode = True  # the reference tree is read-only
    sys.path.insert(0, ref_root)
    from rune.ops.batched import geom_matmul, _native_available, _cuda_native_available
    from holograph.models.hlm_block import HLMBlock
    from holograph.layers.clifford_linear import CliffordLinear
    from holograph.layers.clifford_router import _softmax

    assert not _native_available() and not _cuda_native_available(), "expected the NumPy fallback"
    mods = dict(HLMBlock=HLMBlock, CliffordLinear=CliffordLinear, _softmax=_softmax)
    only = set(sys.argv[2:])
    for name, p in CASES.items():
        if only and name not in only:
            continue
        inp = _inputs.make_case(p)
        rec = {"params": json.dumps(p), "numpy_version": np.__version__}
        for key, arr in inp.items():
            rec["sha_" + key] = _inputs.digest(arr)
        if p["kind"] == "geom_matmul":
            rec["ref_out"] = geom_matmul(inp["a"], inp["b"])
        elif p["kind"] == "route":
            N, E, k, d = p["N"], p["E"], p["k"], p["d"]
            # identity experts: the output is the reference's weighted combine of x itself
            block = HLMBlock(d, 1, 1, use_moe=True, n_experts=E, moe_top_k=k)
            router = _LogitsRouter(inp["logits"], k, _softmax)
            idx, w, _ = router.forward(None)
            block.router = router
            log = []
            block.experts = [_Recorder(None, log, e) for e in range(E)]
            x = inp["x"].reshape(1, N, d, 8)
            rec["ref_out"] = block._moe_forward(x).reshape(N, d, 8)
            rec["ref_idx"], rec["ref_w"] = idx, w
            rec["ref_counts"] = np.bincount(idx.reshape(-1), minlength=E).astype(np.int32)
            rec["ref_perm"] = np.concatenate([_tokens_of(rows, inp["x"]) for _, rows in log])
            rec["ref_perm_experts"] = np.array([e for e, _ in log], dtype=np.int32)
            rec["ref_probs"] = _softmax(inp["logits"], axis=-1)
        else:
            x = inp["x"]
            layers = p.get("layers", 1)
            for li in range(layers):
                pre = f"l{li}_" if p["kind"] == "stack" else ""
                y, ex = _run_layer(mods, p, inp, pre, x)
                for kk, vv in ex.items():
                    rec[f"ref_{pre}{kk}"] = vv
                if p["kind"] == "stack":
                    x = (x + y).astype(np.float32)
                    rec[f"ref_{pre}out"] = x
                else:
                    x = y
            rec["ref_out"] = x
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **rec)
        print(f"{name}: {os.path.getsize(path) / 1024:.1f} KiB")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
