"""GPU parity at BASELINE's full sizes, on every row, against the float64 BLAS oracle.

``oracle/dense.py`` recomputes the whole layer -- every token of config 3, every
token of one config 5 layer, a 12-layer config 5 stack on a token set that holds
every expert of every layer, and the config 3 training step's gradients -- in
seconds, so nothing here is sampled.  The oracle is pinned against the
reference's goldens, its reference-order restatement and finite differences
(``tests/test_oracle_dense.py``).

Bounds (written here, as in ``_gpu_helpers``): routing indices bit-exact; bf16
outputs within 2e-2 of the float64 truth *per token* (each token's max error over
its own max magnitude), which is stricter than the normwise bound over the whole
output; fp32 gradients within 3e-5 normwise per tensor.
"""

import numpy as np
import pytest
import torch

import _inputs
from _gpu_helpers import TOL_BF16, normwise_err, say
from oracle import dense, moe

pytestmark = pytest.mark.gpu

TOL_BW = 3e-5


def _ops():
    from yggdrasil_amd import ops

    return ops


def _per_token_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max(axis=(1, 2)) / np.abs(ref).max(axis=(1, 2))


def _device_weights(seed, E, d, F, dtype):
    """Expert weights ~ N(0, 1/sqrt(8 fan_in)) drawn on the device (the C5 weights are 6.4 GB over 12 layers),
    rounded to bf16 for bf16 layers; biases ~ N(0, 0.1).  Returns device fp32 tensors and host copies."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen, device="cuda", dtype=torch.float32)
    wu = rn(E, F, d, 8) / (8.0 * d) ** 0.5
    wd = rn(E, d, F, 8) / (8.0 * F) ** 0.5
    if dtype == torch.bfloat16:
        wu, wd = wu.bfloat16().float(), wd.bfloat16().float()
    bu, bd = 0.1 * rn(E, F, 8), 0.1 * rn(E, d, 8)
    dev = dict(w_up=wu, w_down=wd, b_up=bu, b_down=bd)
    host = {k: v.cpu().numpy() for k, v in dev.items()}
    return dev, host


def _every(n, what):
    """Progress of a long oracle computation: one line every n experts."""
    return lambda e: say(f"{what}: expert {e}") if e % n == n - 1 else None


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).bfloat16().float().numpy()


def _layer(ops, dev, fmt):
    return dict(w_up=ops.prepare_weights(dev["w_up"], fmt), w_down=ops.prepare_weights(dev["w_down"], fmt),
                b_up=ops.prepare_bias(dev["b_up"]), b_down=ops.prepare_bias(dev["b_down"]))


def _check_routing(rt, logits, k):
    idx_o, w_o = moe.route_topk(moe.softmax(logits), k)
    assert np.array_equal(rt["topk_idx"].cpu().numpy(), idx_o)
    counts_o = np.bincount(idx_o.reshape(-1), minlength=logits.shape[1])
    assert np.array_equal(rt["counts"].cpu().numpy(), counts_o)
    return idx_o, w_o


# ---- config 3: every token ------------------------------------------------------------


@pytest.fixture(scope="module")
def c3_case():
    N, d, E, k, F = 8192, 128, 32, 4, 512
    g = np.random.default_rng(3030)
    logits = _inputs.zipf_logits(g, N, E, k)
    x = _bf16(g.standard_normal((N, d, 8), dtype=np.float32))
    dev, host = _device_weights(3031, E, d, F, torch.bfloat16)
    idx, w = moe.route_topk(moe.softmax(logits), k)
    say("c3 float64 oracle, every token")
    ref = dense.moe_layer(x, idx, w, host["w_up"], host["b_up"], host["w_down"], host["b_down"], "gelu",
                          progress=_every(8, "c3 oracle"))
    return dict(N=N, d=d, E=E, k=k, F=F, logits=logits, x=x, dev=dev, ref=ref)


@pytest.mark.parametrize("fmt", ["pauli", "bf16"])
def test_c3_every_token(c3_case, fmt):
    c = c3_case
    ops = _ops()
    P = _layer(ops, c["dev"], fmt)
    xt = torch.from_numpy(c["x"]).cuda().bfloat16()
    say(f"c3 full layer {fmt}, N={c['N']}")
    out, rt = ops.moe_forward(xt, c["k"], P["w_up"], P["w_down"], P["b_up"], P["b_down"], "gelu",
                              logits=torch.from_numpy(c["logits"]).cuda())
    _check_routing(rt, c["logits"], c["k"])
    err = _per_token_err(out.float().cpu().numpy(), c["ref"])
    say(f"c3 {fmt}: worst token error {err.max():.3e}, median {np.median(err):.3e}")
    assert err.max() < TOL_BF16, (int(err.argmax()), float(err.max()))


@pytest.mark.parametrize("N", [40960, 73728])
def test_c3_shape_prefill_beyond_32k_tokens(N):
    """Prefill at the config 3 shape with more tokens than a 32-bit offset over whole operands allows:
    at N = 73728 the hidden rows h (P = 294912 rows of 8 KiB) span 2.4 GB, so the down product reads,
    and the up product writes, rows past 2 GiB.  Routing indices and expert counts are bit-exact; the
    outputs of a sample of tokens -- 512 random ones and every token of the last two experts in row
    order, whose rows sit at the end of h -- are within the bf16 bound of the float64 oracle per
    token; and the layer is token-permutation equivariant bit for bit (reversed order, every token)."""
    d, E, k, F = 128, 32, 4, 512
    ops = _ops()
    g = np.random.default_rng(3090 + N)
    logits = _inputs.normal(g, (N, E), 1.0)
    logits[:, :4] += 1.5  # a skewed load, the first four experts heaviest
    x = _bf16(g.standard_normal((N, d, 8), dtype=np.float32))
    dev, host = _device_weights(3091, E, d, F, torch.bfloat16)
    P = _layer(ops, dev, "pauli")
    del dev
    xt = torch.from_numpy(x).cuda().bfloat16()
    lt = torch.from_numpy(logits).cuda()
    say(f"c3-shape prefill N={N} (P={N * k} rows, h {N * k * F * 16 / 2**30:.2f} GiB)")
    out, rt = ops.moe_forward(xt, k, P["w_up"], P["w_down"], P["b_up"], P["b_down"], "gelu", logits=lt)
    idx, w = _check_routing(rt, logits, k)
    got = out.float().cpu().numpy()
    last = np.flatnonzero((idx >= E - 2).any(axis=1))
    sample = np.union1d(g.choice(N, size=512, replace=False), last)
    say(f"c3-shape prefill N={N}: float64 oracle on {sample.size} tokens")
    ref = dense.moe_layer(x[sample], idx[sample], w[sample], host["w_up"], host["b_up"], host["w_down"],
                          host["b_down"], "gelu")
    err = _per_token_err(got[sample], ref)
    say(f"c3-shape prefill N={N}: worst token error {err.max():.3e}, median {np.median(err):.3e}")
    assert err.max() < TOL_BF16, (int(sample[err.argmax()]), float(err.max()))
    say(f"c3-shape prefill N={N}: reversed token order")
    out_r, _ = ops.moe_forward(torch.flip(xt, [0]).contiguous(), k, P["w_up"], P["w_down"], P["b_up"],
                               P["b_down"], "gelu", logits=torch.flip(lt, [0]).contiguous())
    assert torch.equal(torch.flip(out_r, [0]), out)


@pytest.mark.parametrize("fmt", ["int8", "int8_pauli"])
def test_c4_decode_every_token(fmt):
    """BASELINE config 4 (N=64, d=128, F=512, E=32, k=2, int8 weights) against the float64 layer on the
    dequantized weights the int8 format holds (blade codes, or the codes of the weights' matrix entries)."""
    N, d, E, k, F = 64, 128, 32, 2, 512
    ops = _ops()
    g = np.random.default_rng(4040)
    logits = g.standard_normal((N, E), dtype=np.float32)
    x = _bf16(g.standard_normal((N, d, 8), dtype=np.float32))
    dev, host = _device_weights(4041, E, d, F, torch.float32)
    P = _layer(ops, dev, fmt)
    say(f"c4 full layer {fmt}, N={N}")
    out, rt = ops.moe_forward(torch.from_numpy(x).cuda().bfloat16(), k, P["w_up"], P["w_down"], P["b_up"],
                              P["b_down"], "gelu", logits=torch.from_numpy(logits).cuda())
    idx, w = _check_routing(rt, logits, k)
    if fmt == "int8":
        wu = moe.dequantize_int8(*moe.quantize_int8(host["w_up"]))
        wd = moe.dequantize_int8(*moe.quantize_int8(host["w_down"]))
    else:
        wu = moe.dequantize_int8_pauli(*moe.quantize_int8_pauli(host["w_up"]))
        wd = moe.dequantize_int8_pauli(*moe.quantize_int8_pauli(host["w_down"]))
    ref = dense.moe_layer(x, idx, w, wu, host["b_up"], wd, host["b_down"], "gelu")
    err = _per_token_err(out.float().cpu().numpy(), ref)
    say(f"c4 {fmt}: worst token error {err.max():.3e}, median {np.median(err):.3e}")
    assert err.max() < TOL_BF16, (int(err.argmax()), float(err.max()))


def test_c4_quantization_error_against_fp32_masters():
    """BASELINE config 4 quantizes its expert weights to int8 from fp32 masters.  Both int8 formats run
    the full layer and are compared with the float64 layer on those masters, so the error includes the
    quantization itself.  Format 2 holds per-output-channel codes of the blade coefficients (the
    reference quantizer's scheme, bifrost/quantization/grade_quantize.py); format 5 holds codes of the
    Pauli matrix entries, sums of two blade coefficients, whose per-coefficient bound is about sqrt(2)
    coarser.  At the layer's output the two measure alike (the float64 oracle on the dequantized weights
    gives 1.2 % RMS for both at this shape); the bounds: normwise 2e-2, per token 3e-2, and format 5
    within 1.5 times format 2."""
    N, d, E, k, F = 64, 128, 32, 2, 512
    ops = _ops()
    g = np.random.default_rng(4040)
    logits = g.standard_normal((N, E), dtype=np.float32)
    x = _bf16(g.standard_normal((N, d, 8), dtype=np.float32))
    dev, host = _device_weights(4041, E, d, F, torch.float32)
    idx, w = moe.route_topk(moe.softmax(logits), k)
    ref = dense.moe_layer(x, idx, w, host["w_up"], host["b_up"], host["w_down"], host["b_down"], "gelu")
    errs = {}
    for fmt in ("int8", "int8_pauli"):
        P = _layer(ops, dev, fmt)
        say(f"c4 {fmt} against the fp32 masters, N={N}")
        out, rt = ops.moe_forward(torch.from_numpy(x).cuda().bfloat16(), k, P["w_up"], P["w_down"], P["b_up"],
                                  P["b_down"], "gelu", logits=torch.from_numpy(logits).cuda())
        _check_routing(rt, logits, k)
        got = out.float().cpu().numpy()
        errs[fmt] = (normwise_err(got, ref), float(_per_token_err(got, ref).max()))
        say(f"c4 {fmt}: normwise {errs[fmt][0]:.3e}, worst token {errs[fmt][1]:.3e} against the fp32 masters")
    for fmt, (nw, tok) in errs.items():
        assert nw < 2e-2 and tok < 3e-2, (fmt, nw, tok)
    assert errs["int8_pauli"][0] < 1.5 * errs["int8"][0], errs


# ---- config 5: one layer, every token; the 12-layer stack ---------------------------------


def _c5_logits(g, N, E):
    return (g.standard_normal((N, E), dtype=np.float32) + (0.5 * g.standard_normal(E)).astype(np.float32)[None, :])


def test_c5_layer_every_token():
    N, d, E, k, F = 4096, 256, 64, 2, 1024
    ops = _ops()
    g = np.random.default_rng(5050)
    logits = _c5_logits(g, N, E)
    x = _bf16(g.standard_normal((N, d, 8), dtype=np.float32))
    dev, host = _device_weights(5051, E, d, F, torch.bfloat16)
    P = _layer(ops, dev, "pauli")
    del dev
    say(f"c5 full layer, N={N}")
    out, rt = ops.moe_forward(torch.from_numpy(x).cuda().bfloat16(), k, P["w_up"], P["w_down"], P["b_up"],
                              P["b_down"], "gelu", logits=torch.from_numpy(logits).cuda())
    idx, w = _check_routing(rt, logits, k)
    assert int((rt["counts"] > 0).sum()) == E
    ref = dense.moe_layer(x, idx, w, host["w_up"], host["b_up"], host["w_down"], host["b_down"], "gelu",
                          progress=_every(16, "c5 oracle"))
    err = _per_token_err(out.float().cpu().numpy(), ref)
    say(f"c5 layer: worst token error {err.max():.3e}, median {np.median(err):.3e}")
    assert err.max() < TOL_BF16, (int(err.argmax()), float(err.max()))


def _covering_tokens(idx_layers, extra, g):
    """A token set that holds every expert of every layer that any token selects (greedy), plus `extra`
    random tokens."""
    N = idx_layers[0].shape[0]
    holds = [set((li, int(e)) for li in range(len(idx_layers)) for e in idx_layers[li][t]) for t in range(N)]
    need = set().union(*holds)
    chosen = set()
    while need:
        t = max(range(N), key=lambda t: len(holds[t] & need))
        chosen.add(t)
        need -= holds[t]
    chosen |= set(g.choice(N, size=extra, replace=False).tolist())
    return np.array(sorted(chosen))


def test_c5_stack_12_layers():
    """BASELINE config 5 as the bench runs it: 12 layers, x <- x + moe(x) in bf16 between layers.  The
    logits of each layer are given, so a token's path through the stack depends on that token alone: the
    oracle chains the 12 layers on a token set that holds every expert of every layer, rounding x to bf16
    after each layer as the GPU stores it."""
    N, d, E, k, F, n_layers = 4096, 256, 64, 2, 1024, 12
    ops = _ops()
    g = np.random.default_rng(5151)
    logits = [_c5_logits(g, N, E) for _ in range(n_layers)]
    routing = [moe.route_topk(moe.softmax(lg), k) for lg in logits]
    subset = _covering_tokens([r[0] for r in routing], extra=128, g=g)
    say(f"c5 stack: {len(subset)} tokens hold all {sum(len(np.unique(r[0])) for r in routing)} (layer, expert) pairs")
    x0 = _bf16(g.standard_normal((N, d, 8), dtype=np.float32))
    cur = torch.from_numpy(x0).cuda().bfloat16()
    xs = x0[subset].astype(np.float64)
    for li in range(n_layers):
        dev, host = _device_weights(5200 + li, E, d, F, torch.bfloat16)
        P = _layer(ops, dev, "pauli")
        del dev
        say(f"c5 stack layer {li}")
        cur, rt = ops.moe_forward(cur, k, P["w_up"], P["w_down"], P["b_up"], P["b_down"], "gelu",
                                  logits=torch.from_numpy(logits[li]).cuda(), residual=cur)
        _check_routing(rt, logits[li], k)
        idx, w = routing[li]
        xs = dense.moe_layer(xs, idx[subset], w[subset], host["w_up"], host["b_up"], host["w_down"],
                             host["b_down"], "gelu", residual=xs)
        xs = _bf16(xs).astype(np.float64)
        del P, host
    got = cur.float().cpu().numpy()[subset]
    err = _per_token_err(got, xs)
    say(f"c5 stack: {len(subset)} tokens, worst token error {err.max():.3e}, median {np.median(err):.3e}")
    assert err.max() < TOL_BF16, (int(subset[err.argmax()]), float(err.max()))


# ---- config 3 shape, fp32 training step: every gradient ----------------------------------


def test_c3t_gradients_every_element():
    """The fp32 training step at the config 3 shape (d=128, F=512, E=32, k=4, N=8192): the MFMA weight
    gradient from Pauli rows in 384-row chunks, the adjoint products and the activation backward, all
    against the float64 oracle backward on the GPU's own routing."""
    import yggdrasil_amd

    N, d, E, k, F = 8192, 128, 32, 4, 512
    g = np.random.default_rng(3300)
    logits = _inputs.zipf_logits(g, N, E, k)
    x = g.standard_normal((N, d, 8), dtype=np.float32)
    c = g.standard_normal((N, d, 8), dtype=np.float32)
    dev, host = _device_weights(3301, E, d, F, torch.float32)
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, router="logits")
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(w_up=dev["w_up"], b_up=dev["b_up"], w_down=dev["w_down"], b_down=dev["b_down"])
    del dev
    xt = torch.from_numpy(x).cuda().reshape(1, N, d, 8).requires_grad_(True)
    say(f"c3t autograd N={N}")
    out = layer.moe_forward(xt, logits=torch.from_numpy(logits).cuda())
    out.backward(torch.from_numpy(c).cuda().reshape(1, N, d, 8))
    torch.cuda.synchronize()
    idx, w = _check_routing(layer.last_routing, logits, k)
    say("c3t float64 oracle backward")
    ref_out = dense.moe_layer(x, idx, w, host["w_up"], host["b_up"], host["w_down"], host["b_down"], "gelu",
                              progress=_every(8, "c3t forward oracle"))
    assert normwise_err(out.detach().cpu().numpy()[0], ref_out) < 1e-5
    dx, dWu, dbu, dWd, dbd = dense.moe_layer_backward(x, idx, w, host["w_up"], host["b_up"], host["w_down"],
                                                      host["b_down"], c, "gelu",
                                                      progress=_every(4, "c3t backward oracle"))
    errs = dict(x=normwise_err(xt.grad.cpu().numpy()[0], dx),
                w_up=normwise_err(layer.w_up.grad.cpu().numpy(), dWu),
                b_up=normwise_err(layer.b_up.grad.cpu().numpy(), dbu),
                w_down=normwise_err(layer.w_down.grad.cpu().numpy(), dWd),
                b_down=normwise_err(layer.b_down.grad.cpu().numpy(), dbd))
    say("c3t gradient errors " + ", ".join(f"{k}={v:.2e}" for k, v in errs.items()))
    for name, e in errs.items():
        assert e < TOL_BW, (name, e)
