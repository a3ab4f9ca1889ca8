"""The oracle reproduces the reference's own outputs (goldens) bit for bit.

The goldens were written by ``tests/golden/make_goldens.py``, which runs the
reference's NumPy path.  Routing indices, weights, counts and permutation
and the layer outputs must be identical, not merely close.
"""

import numpy as np
import pytest

from _fixtures import LAYER_CASES, layer_weights, load_case
from oracle import moe


@pytest.mark.parametrize("name", ["gm_small", "gm_rect"])
def test_geom_matmul_golden(name):
    _, inp, ref = load_case(name)
    assert np.array_equal(moe.geom_matmul(inp["a"], inp["b"]), ref["out"])


def test_route_golden():
    p, inp, ref = load_case("c2_route")
    probs = moe.softmax(inp["logits"])
    assert np.array_equal(probs, ref["probs"])
    idx_r, w_r = moe.topk_reference(probs, p["k"])
    assert np.array_equal(idx_r, ref["idx"]) and np.array_equal(w_r, ref["w"])
    # build rule: descending slots; on tie-free input it is the reference's selection reversed,
    # and the weights are bit-identical because the renormalising sum keeps the reference's order
    idx, w = moe.route_topk(probs, p["k"])
    assert np.array_equal(idx, ref["idx"][:, ::-1]) and np.array_equal(w, ref["w"][:, ::-1])
    counts, offsets, perm, slot_pos = moe.dispatch_plan(idx, p["E"])
    assert np.array_equal(counts, ref["counts"])
    assert np.array_equal(perm, ref["perm"])
    assert np.array_equal(ref["perm_experts"], np.nonzero(counts)[0])  # experts visited in ascending order
    out = moe.combine(inp["x"][perm], idx, w, slot_pos)
    assert np.array_equal(out, ref["out"])


def _run_case(p, inp, ref):
    x = inp["x"]
    for li in range(p.get("layers", 1)):
        pre = f"l{li}_" if p["kind"] == "stack" else ""
        wu, bu, wd, bd, _ = layer_weights(p, inp, pre)
        experts = [(wu[e], bu[e], wd[e], bd[e]) for e in range(p["E"])]
        logits = None
        if p.get("logits") == "clifford_head":
            N = x.shape[0] * x.shape[1]
            logits = moe.clifford_linear(x.reshape(N, p["d"], 8), inp[pre + "head_w"], None)[..., 0]
        elif p.get("logits"):
            logits = inp[pre + "logits"]
        y, info = moe.moe_forward_reference(x, inp[pre + "router_w"], inp[pre + "router_b"], experts, p["k"],
                                            p["act"], logits=logits)
        assert np.array_equal(info["idx"], ref[pre + "idx"])
        assert np.array_equal(info["w"], ref[pre + "w"])
        assert np.array_equal(info["counts"], ref[pre + "counts"])
        assert np.array_equal(info["perm"], ref[pre + "perm"])
        if info["energy"] is not None:
            assert np.array_equal(info["energy"], ref[pre + "energy"])
        # the build's counting sort gives the reference's dispatch order
        idx_b, _ = moe.route_topk(info["probs"], p["k"])
        _, _, perm_b, _ = moe.dispatch_plan(idx_b, p["E"])
        assert np.array_equal(perm_b, ref[pre + "perm"])
        x = (x + y).astype(np.float32) if p["kind"] == "stack" else y
    return x


@pytest.mark.parametrize("name", LAYER_CASES)
def test_layer_golden(name):
    p, inp, ref = load_case(name)
    out = _run_case(p, inp, ref)
    assert np.array_equal(out, ref["out"])
