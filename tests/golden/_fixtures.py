"""Load a golden case: parameters, regenerated inputs (digest-checked), reference outputs."""

from __future__ import annotations

import json
import os

import numpy as np

import _inputs

HERE = os.path.dirname(os.path.abspath(__file__))

LAYER_CASES = ["small_gelu", "small_relu", "small_sigmoid", "c1_layer", "c1_head", "c3_small", "c4_small", "c5_small"]
ALL_CASES = ["gm_small", "gm_rect", "c2_route"] + LAYER_CASES


def load_case(name: str):
    z = np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False)
    params = json.loads(str(z["params"]))
    inputs = _inputs.make_case(params)
    for key, arr in inputs.items():
        want = str(z["sha_" + key])
        got = _inputs.digest(arr)
        if got != want:
            raise AssertionError(f"{name}: regenerated input {key!r} differs from the fixture's digest")
    ref = {k[4:]: z[k] for k in z.files if k.startswith("ref_")}
    return params, inputs, ref


def layer_weights(params, inputs, pre=""):
    """Per-layer weights as used by the reference run (int8 cases: dequantized masters)."""
    from oracle.moe import quantize_int8, dequantize_int8

    wu, wd = inputs[pre + "w_up"], inputs[pre + "w_down"]
    q = None
    if params.get("int8"):
        qu, su = quantize_int8(wu)
        qd, sd = quantize_int8(wd)
        q = (qu, su, qd, sd)
        wu, wd = dequantize_int8(qu, su), dequantize_int8(qd, sd)
    return wu, inputs[pre + "b_up"], wd, inputs[pre + "b_down"], q
