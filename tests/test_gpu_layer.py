"""GPU parity: expert products and the whole MoE-HLM layer against the reference.

Reference goldens (``tests/golden``, written by the reference's own NumPy
path) and the oracle.  Routing is compared bit-exactly; outputs normwise
(fp32 <= 1e-5, bf16 / int8 weights <= 2e-2; see ``_gpu_helpers``).
"""

import numpy as np
import pytest
import torch

import _inputs
from _fixtures import LAYER_CASES, load_case
from _gpu_helpers import TOL_BF16, TOL_F32, moe_reference, normwise_err, say
from oracle import moe

pytestmark = pytest.mark.gpu


def _mods():
    import yggdrasil_amd
    from yggdrasil_amd import ops

    return yggdrasil_amd, ops


@pytest.mark.parametrize("name", ["gm_small", "gm_rect"])
def test_geom_matmul_operator(name):
    _, ops = _mods()
    _, inp, ref = load_case(name)
    say(f"geom_matmul {name}")
    out = ops.geom_matmul(torch.from_numpy(inp["a"]).cuda(), torch.from_numpy(inp["b"]).cuda()).cpu().numpy()
    assert normwise_err(out, ref["out"]) < TOL_F32


@pytest.mark.parametrize("fmt,act,d_in,d_out,E,P", [
    ("f32", "none", 8, 16, 3, 50), ("f32", "gelu", 64, 256, 8, 512), ("f32", "relu", 7, 5, 2, 33),
    ("bf16", "none", 16, 64, 4, 200), ("bf16", "gelu", 128, 512, 3, 300), ("bf16", "sigmoid", 9, 40, 5, 77),
    ("int8", "gelu", 32, 64, 4, 100), ("int8", "none", 128, 96, 2, 70),
    # at most 16 rows per expert on average: the decode-shape (weight-streaming) kernel
    ("int8", "gelu", 128, 512, 8, 60), ("int8", "sigmoid", 10, 40, 5, 30), ("int8", "none", 64, 130, 4, 50),
    # decode shape with d_in above one 128-input chunk (the chunk walk), odd d_in tails
    ("int8", "gelu", 300, 72, 4, 60), ("int8", "relu", 129, 33, 2, 30)])
def test_grouped_clifford_linear(fmt, act, d_in, d_out, E, P):
    _, ops = _mods()
    g = np.random.default_rng(d_in * 7 + d_out + E)
    W = (g.standard_normal((E, d_out, d_in, 8), dtype=np.float32) / np.sqrt(8 * d_in)).astype(np.float32)
    b = (0.3 * g.standard_normal((E, d_out, 8))).astype(np.float32)
    x = g.standard_normal((P, d_in, 8), dtype=np.float32)
    counts = np.bincount(g.integers(0, E, P), minlength=E)
    counts[0] = 0 if E > 2 else counts[0]  # an empty expert
    counts[-1] += P - counts.sum()
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    Wref = W
    if fmt in ("bf16", "int8"):
        x = _inputs.bf16_round(x)
    if fmt == "bf16":
        Wref = _inputs.bf16_round(W)
    if fmt == "int8":
        q, s = moe.quantize_int8(W)
        Wref = moe.dequantize_int8(q, s)
    dt = torch.float32 if fmt == "f32" else torch.bfloat16
    say(f"grouped_clifford_linear fmt={fmt} act={act} d_in={d_in} d_out={d_out} E={E} P={P}")
    pw = ops.prepare_weights(torch.from_numpy(W).cuda(), fmt)
    pb = ops.prepare_bias(torch.from_numpy(b).cuda())
    xs = ops.to_mask_order(torch.from_numpy(x).cuda().to(dt))
    y = ops.grouped_clifford_linear(xs, pw, torch.from_numpy(offsets).cuda(), pb, act, out_dtype=torch.float32)
    y = y.cpu().numpy()
    if fmt == "int8":
        assert np.array_equal(pw.scales.cpu().numpy(), s)
    for e in range(E):
        rows = slice(offsets[e], offsets[e + 1])
        if offsets[e] == offsets[e + 1]:
            continue
        ref = moe.ACTIVATIONS[act](moe.clifford_linear(x[rows], Wref[e], b[e]))
        tol = TOL_F32 if fmt == "f32" else 5e-3
        assert normwise_err(y[rows], ref) < tol, e


def _run_layer_case(name, fmt_override=None):
    yggdrasil_amd, ops = _mods()
    p, inp, ref = load_case(name)
    bf16 = bool(p.get("bf16"))
    dt = torch.bfloat16 if bf16 else torch.float32
    fmt = fmt_override or ("int8" if p.get("int8") else ("bf16" if bf16 else "f32"))
    router = {None: "energy", "clifford_head": "clifford_head"}.get(p.get("logits"), "logits")
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=p["d"], d_ff=p["F"], n_experts=p["E"], top_k=p["k"],
                                     activation=p["act"], dtype=dt, weight_format=fmt, router=router)
    x = torch.from_numpy(inp["x"]).cuda().to(dt)
    for li in range(p.get("layers", 1)):
        pre = f"l{li}_" if p["kind"] == "stack" else ""
        layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
        layer.load_reference_weights(router_weight=inp[pre + "router_w"], router_bias=inp[pre + "router_b"],
                                     w_up=inp[pre + "w_up"], b_up=inp[pre + "b_up"], w_down=inp[pre + "w_down"],
                                     b_down=inp[pre + "b_down"], head_weight=inp.get(pre + "head_w"))
        logits = torch.from_numpy(inp[pre + "logits"]).cuda() if router == "logits" else None
        say(f"layer {name} {pre} N={x.shape[0] * x.shape[1]} d={p['d']} E={p['E']} k={p['k']} F={p['F']} {fmt}")
        y = layer.moe_forward(x, logits=logits, residual=x if p["kind"] == "stack" else None)
        torch.cuda.synchronize()
        rt = layer.last_routing
        assert np.array_equal(rt["topk_idx"].cpu().numpy(), ref[pre + "idx"][:, ::-1]), "routing indices"
        assert np.array_equal(rt["counts"].cpu().numpy(), ref[pre + "counts"]), "expert counts"
        assert np.allclose(rt["topk_w"].cpu().numpy(), ref[pre + "w"][:, ::-1], rtol=1e-5, atol=1e-6)
        x = y
    got = x.detach().float().cpu().numpy()
    err = normwise_err(got, ref["out"])
    tol = TOL_BF16 if bf16 else TOL_F32
    assert err < tol, f"{name}: normwise error {err:.3e} >= {tol}"
    return err


@pytest.mark.parametrize("name", LAYER_CASES)
def test_layer_against_reference_golden(name):
    _run_layer_case(name)


@pytest.mark.parametrize("name", ["c3_small", "c5_small"])
def test_layer_pauli_weights_against_reference_golden(name):
    """The bf16 goldens again, with the expert products on Pauli (complex 2x2) weights."""
    _run_layer_case(name, fmt_override="pauli")


def test_geoformer_interface_flat_input():
    yggdrasil_amd, _ = _mods()
    p, inp, ref = load_case("c1_layer")
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=p["d"], d_ff=p["F"], n_experts=p["E"], top_k=p["k"])
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(router_weight=inp["router_w"], router_bias=inp["router_b"], w_up=inp["w_up"],
                                 b_up=inp["b_up"], w_down=inp["w_down"], b_down=inp["b_down"])
    B, T = p["B"], p["T"]
    xf = torch.from_numpy(inp["x"]).cuda().reshape(B, T, 8 * p["d"])
    say("geoformer flat interface c1")
    out, aux = layer(xf)
    assert out.shape == xf.shape and aux.dim() == 0
    assert out.requires_grad  # fp32 Pauli layers are autograd nodes
    assert normwise_err(out.detach().cpu().numpy().reshape(ref["out"].shape), ref["out"]) < TOL_F32
    c = ref["counts"].astype(np.float64)
    f = c / c.sum()
    assert abs(aux.item() - ((f - 1 / p["E"]) ** 2).sum()) < 1e-6


def _sampled_layer_check(N, d, F, E, k, fmt, logits, seed, n_sample=12):
    """Full-size layer on the GPU; the oracle recomputes a sample of tokens."""
    yggdrasil_amd, _ = _mods()
    g = np.random.default_rng(seed)
    x = _inputs.bf16_round(g.standard_normal((N, d, 8), dtype=np.float32))
    wu, bu, wd, bd = _inputs.expert_weights(g, E, d, F)
    wu, wd = _inputs.bf16_round(wu), _inputs.bf16_round(wd)
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, dtype=torch.bfloat16,
                                     weight_format=fmt, router="logits")
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    xt = torch.from_numpy(x).cuda().bfloat16().reshape(1, N, d, 8)
    lt = torch.from_numpy(logits).cuda()
    say(f"full layer N={N} d={d} F={F} E={E} k={k} {fmt}")
    y = layer.moe_forward(xt, logits=lt).float().cpu().numpy().reshape(N, d, 8)
    rt = layer.last_routing
    idx = rt["topk_idx"].cpu().numpy()
    w = rt["topk_w"].cpu().numpy()
    idx_o, w_o = moe.route_topk(moe.softmax(logits), k)
    assert np.array_equal(idx, idx_o)
    if fmt == "int8":
        wu = moe.dequantize_int8(*moe.quantize_int8(wu))
        wd = moe.dequantize_int8(*moe.quantize_int8(wd))
    sample = g.choice(N, size=n_sample, replace=False)
    errs = []
    for t in sample:
        ref = np.zeros((d, 8), np.float32)
        for s in np.argsort(idx[t]):
            e = idx[t, s]
            ye = moe.clifford_ffn(x[t][None], wu[e], bu[e], wd[e], bd[e], "gelu")[0]
            ref = ref + w_o[t, s] * ye
        errs.append(normwise_err(y[t], ref))
    assert max(errs) < TOL_BF16, max(errs)
    # token permutation equivariance: every row is computed independently of its tile position
    pi = g.permutation(N)
    say(f"full layer permuted N={N}")
    y2 = layer.moe_forward(xt[:, pi], logits=lt[pi]).float().cpu().numpy().reshape(N, d, 8)
    assert np.array_equal(y2, y[pi])
    return max(errs)


@pytest.mark.parametrize("fmt", ["bf16", "pauli"])
def test_full_c3_prefill_bf16_sampled(fmt):
    g = np.random.default_rng(303)
    logits = _inputs.zipf_logits(g, 8192, 32, 4)
    _sampled_layer_check(8192, 128, 512, 32, 4, fmt, logits, 33)


def test_full_c5_layer_bf16_sampled():
    """One layer of BASELINE config 5 at full size (N=4096, d=256, F=1024, E=64, k=2):
    logits N(0,1) plus a per-expert bias N(0, 0.5), as the config draws them."""
    g = np.random.default_rng(505)
    logits = (g.standard_normal((4096, 64), dtype=np.float32)
              + (0.5 * g.standard_normal(64)).astype(np.float32)[None, :])
    _sampled_layer_check(4096, 256, 1024, 64, 2, "pauli", logits, 55, n_sample=8)


def test_full_layer_max_experts_and_top_k_sampled():
    """E = 64 and k = 8 (the maxima) through the multi-block routing (N > 1024) and the Pauli products."""
    g = np.random.default_rng(707)
    logits = g.standard_normal((2048, 64), dtype=np.float32)
    _sampled_layer_check(2048, 32, 64, 64, 8, "pauli", logits, 77)


def test_full_c4_decode_int8_sampled():
    g = np.random.default_rng(404)
    logits = g.standard_normal((64, 32), dtype=np.float32)
    _sampled_layer_check(64, 128, 512, 32, 2, "int8", logits, 44, n_sample=16)


def test_decode_int8_skewed_layer():
    """Decode-shape int8 layer: one expert gets more than 16 rows (row-block loop), F = 302
    gives three K splits of the down product with a tail, bias on both products."""
    yggdrasil_amd, _ = _mods()
    g = np.random.default_rng(606)
    N, d, F, E, k = 64, 96, 302, 8, 2
    x = _inputs.bf16_round(g.standard_normal((N, d, 8), dtype=np.float32))
    wu, bu, wd, bd = _inputs.expert_weights(g, E, d, F, bias_std=0.3)
    logits = g.standard_normal((N, E), dtype=np.float32)
    logits[:40, 0] += 6.0  # expert 0 takes 40 tokens
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, dtype=torch.bfloat16,
                                     weight_format="int8", router="logits")
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    say(f"decode int8 skewed N={N} d={d} F={F} E={E} k={k}")
    y = layer.moe_forward(torch.from_numpy(x).cuda().bfloat16().reshape(1, N, d, 8),
                          logits=torch.from_numpy(logits).cuda()).float().cpu().numpy().reshape(N, d, 8)
    idx = layer.last_routing["topk_idx"].cpu().numpy()
    assert layer.last_routing["counts"].cpu().numpy()[0] >= 40
    idx_o, w_o = moe.route_topk(moe.softmax(logits), k)
    assert np.array_equal(idx, idx_o)
    wu_q = moe.dequantize_int8(*moe.quantize_int8(wu))
    wd_q = moe.dequantize_int8(*moe.quantize_int8(wd))
    ref = moe_reference(x.reshape(N, d, 8), idx, w_o, wu_q, bu, wd_q, bd, "gelu")
    assert normwise_err(y, ref) < TOL_BF16


def test_module_rejects_cpu_tensors():
    yggdrasil_amd, _ = _mods()
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=8, d_ff=16, n_experts=4, top_k=2)
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    with pytest.raises(ValueError):
        layer.moe_forward(torch.zeros(1, 4, 8, 8))


@pytest.mark.parametrize("N,d,F,E,k,act", [(64, 128, 512, 32, 2, "gelu"), (1, 16, 32, 4, 1, "relu"),
                                           (128, 64, 96, 64, 2, "sigmoid"), (37, 40, 72, 9, 3, "gelu"),
                                           (100, 32, 64, 16, 2, "relu")])
def test_decode_routing_inside_up_product(N, d, F, E, k, act):
    """Decode layers given logits route inside the up product: the routing arrays equal
    ygg_route's bit for bit (ties included), the output is the oracle's at the int8 bound."""
    yggdrasil_amd, ops = _mods()
    g = np.random.default_rng(N * 3 + E)
    x = _inputs.bf16_round(g.standard_normal((N, d, 8), dtype=np.float32))
    wu, bu, wd, bd = _inputs.expert_weights(g, E, d, F, bias_std=0.2)
    logits = np.round(g.standard_normal((N, E)), 1).astype(np.float32)  # many exact ties
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, activation=act,
                                     dtype=torch.bfloat16, weight_format="int8", router="logits")
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    lt = torch.from_numpy(logits).cuda()
    say(f"decode routed up N={N} d={d} F={F} E={E} k={k} {act}")
    y = layer.moe_forward(torch.from_numpy(x).cuda().bfloat16().reshape(1, N, d, 8), logits=lt)
    y = y.float().cpu().numpy().reshape(N, d, 8)
    r = ops.route(lt, k)
    for key in ("topk_idx", "topk_w", "counts", "offsets"):
        assert torch.equal(layer.last_routing[key], getattr(r, key)), key
    idx, w = r.topk_idx.cpu().numpy(), r.topk_w.cpu().numpy()
    wu_q = moe.dequantize_int8(*moe.quantize_int8(wu))
    wd_q = moe.dequantize_int8(*moe.quantize_int8(wd))
    ref = moe_reference(x.reshape(N, d, 8), idx, w, wu_q, bu, wd_q, bd, act)
    assert normwise_err(y, ref) < TOL_BF16


@pytest.mark.parametrize("fmt,router", [("pauli_f32", "energy"), ("f32", "logits"), ("pauli", "logits"),
                                        ("bf16", "clifford_head"), ("int8", "logits")])
def test_layer_with_no_tokens(fmt, router):
    """An empty batch (the reference's _moe_forward on zero tokens): an empty output, every
    expert's count and offset zero; the fp32 Pauli layer's weight gradients are zero."""
    yggdrasil_amd, _ = _mods()
    g = np.random.default_rng(11)
    d, F, E, k = 16, 32, 4, 2
    dt = torch.float32 if fmt in ("f32", "pauli_f32") else torch.bfloat16
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, dtype=dt, weight_format=fmt,
                                     router=router)
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    wu, bu, wd, bd = _inputs.expert_weights(g, E, d, F, bias_std=0.1)
    layer.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    x = torch.zeros((1, 0, d, 8), device="cuda", dtype=dt, requires_grad=fmt == "pauli_f32")
    lg = torch.zeros((0, E), device="cuda") if router == "logits" else None
    say(f"empty batch {fmt} {router}")
    y = layer.moe_forward(x, logits=lg)
    torch.cuda.synchronize()
    assert tuple(y.shape) == (1, 0, d, 8)
    assert layer.last_routing["counts"].cpu().tolist() == [0] * E
    assert layer.last_routing["offsets"].cpu().tolist() == [0] * (E + 1)
    if fmt == "pauli_f32":
        y.sum().backward()
        torch.cuda.synchronize()
        for name in ("w_up", "b_up", "w_down", "b_down"):
            grad = getattr(layer, name).grad
            assert grad is not None and not grad.any(), name
