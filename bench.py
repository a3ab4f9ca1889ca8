"""Benchmark of the MoE-HLM expert layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c3,c1,c2,c4,c5,c3b,c3ep,c1t,c3t] [--no-cpu-baseline]

A step is one forward pass of the layer over one batch of synthetic input
(inputs resident in HBM before timing starts).  The headline workload is
the bf16 prefill-shape layer, N=8192 tokens, d=128
multivectors, E=32 experts, top-4, expert FFN 128 -> 512 -> 128 with the
grade-wise GELU, Zipf(1.2) expert load.  Configs 1, 2, 4 and 5 are timed in
the same run and reported under "configs", with "c3b": config 3 inside the
FFN half of the block, x + moe(ffn_norm(x)) (CliffordLayerNorm in front, the
residual added in the combine), and "c1t" / "c3t": a training step (forward and
backward, fp32) at the config 1 and 3 shapes.

One JSON line is printed.  ``roofline`` covers the dominant kernel, the
grouped CliffordLinear MFMA kernel (both expert products), from HIP events
around its launches on the stream it runs on.  Its ``achieved`` and ``frac`` count
the MFMA work the kernel issues (for the Pauli form 32 multiply-adds per
multivector pair), so ``frac`` is a fraction of the hardware peak;
``dense_equiv_tflops`` is the rate in the reference's arithmetic (64 multiply-adds
per pair, the dense 8x8 L(w) block), an effective rate and no fraction of any peak.
HBM traffic / MFMA-busy counters appear only when ``profiles/pins.json`` holds them
for the current sources of the kernel.
``cpu_baseline`` (per BASELINE config under "configs", the headline's at the
top) times the reference's own compiled CPU geometric matmul (``oracle/_ref``,
built from the reference sources) -- or the C restatement if that is absent --
plus the NumPy restatement of routing / dispatch / combine, on every row where
that takes seconds and on a sample extrapolated linearly in FLOPs otherwise,
with the reference's NumPy broadcast fallback and an OpenMP port beside it.
The decode config (4) reports the fused layer's bytes per step against HBM, timed as
HIP graph replay of the steps (a Python loop of such short steps is host-bound; its
figure is reported beside it as ms_per_step_eager).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16 = 2.5e15  # dense bf16 MFMA, FLOP/s
PEAK_F32 = 157.3e12  # fp32 MFMA
PEAK_HBM = 8.0e12  # bytes/s
# counter figures (HBM traffic, MFMA-busy) measured by rocprofv3 for a kernel build: each entry
# names the sources it was measured on and their SHA-256, and is used only while they match
PINS = os.path.join(ROOT, "profiles", "pins.json")
WGRAD_MFMA_ROWS_PER_EXPERT = 256  # as ygg_moe_backward: mean rows per expert from which it uses the MFMA kernel
SEEDS = {"c1": 1, "c1e": 1, "c1l": 1, "c1t": 1, "c2": 2, "c3": 3, "c3l": 3, "c3b": 3, "c3ep": 3, "c3t": 3, "c4": 4,
         "c4l": 4, "c5": 5, "gm": 6}

CONFIGS = {
    # name: N, d, E, k, F, dtype, weight format, logits kind, layers
    # config 1: the router is CliffordLinear(d -> E) then the scalar part (the step computes it)
    "c1": dict(N=256, d=64, E=8, k=2, F=256, dtype="f32", fmt="pauli_f32", logits="head", layers=1),
    # config 1 with CliffordRouter's grade-energy router, and with the fp32 8x8 L(w)-block products
    # on the vector units (comparisons)
    "c1e": dict(N=256, d=64, E=8, k=2, F=256, dtype="f32", fmt="pauli_f32", logits="energy", layers=1),
    "c1l": dict(N=256, d=64, E=8, k=2, F=256, dtype="f32", fmt="f32", logits="energy", layers=1),
    "c2": dict(N=16384, d=128, E=16, k=2, F=0, dtype="f32", fmt=None, logits="normal", layers=1),
    "c3": dict(N=8192, d=128, E=32, k=4, F=512, dtype="bf16", fmt="pauli", logits="zipf", layers=1),
    # config 3 again with the 8x8 L(w)-block expert products (comparison; not in the default set)
    "c3l": dict(N=8192, d=128, E=32, k=4, F=512, dtype="bf16", fmt="bf16", logits="zipf", layers=1),
    # decode: each step runs the layer with the next of 10 weight sets (335 MB, more than the 256 MB
    # Infinity Cache), so the weights stream from HBM as in a multi-layer decode step
    # (int8 Pauli weights: the one-launch decode layer); "c4l" the same with int8 L(w)-block weights
    "c4": dict(N=64, d=128, E=32, k=2, F=512, dtype="bf16", fmt="int8_pauli", logits="normal", layers=1, rotate=10),
    "c4l": dict(N=64, d=128, E=32, k=2, F=512, dtype="bf16", fmt="int8", logits="normal", layers=1, rotate=10),
    "c5": dict(N=4096, d=256, E=64, k=2, F=1024, dtype="bf16", fmt="pauli", logits="normal_bias", layers=12),
    # training step (forward + backward, fp32 Pauli weights) at the config 1 and config 3 shapes
    "c1t": dict(N=256, d=64, E=8, k=2, F=256, dtype="f32", fmt="pauli_f32", logits="energy", layers=1, train=True),
    "c3t": dict(N=8192, d=128, E=32, k=4, F=512, dtype="f32", fmt="pauli_f32", logits="zipf", layers=1, train=True),
    # config 3 at one GPU's expert-parallel share (8 GPUs x 4 experts): the GPU holding the most
    # rows under the Zipf load, its rows delivered contiguously (the all-to-all is not on one GPU)
    "c3ep": dict(N=8192, d=128, E=32, k=4, F=512, dtype="bf16", fmt="pauli", logits="zipf", layers=1, ep=8),
    # the FFN half of the block around config 3: x + moe(ffn_norm(x)) (pre-norm, residual)
    "c3b": dict(N=8192, d=128, E=32, k=4, F=512, dtype="bf16", fmt="pauli", logits="zipf", layers=1, block=True),
    # the operator boundary geom_matmul (fp32) at CliffordLinear's config 3 shapes: the up
    # projection W (512, 128) on 8192 token columns, and the down projection (128, 512)
    "gm": dict(N=8192, d=128, E=1, k=1, F=512, dtype="f32", fmt=None, logits=None, layers=1, gm=True),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--configs", default="c3,c1,c2,c4,c5,c3b,c3ep,c1t,c3t,gm")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-rows", type=int, default=256)
    # a plain device copy of this many MiB, run (3 times) before the configs: the reference
    # point that scales the FETCH_SIZE / WRITE_SIZE counters of a --pmc profile
    ap.add_argument("--calib-copy-mb", type=int, default=0)
    # library GEMM rates (hipBLASLt through torch.matmul) on random bf16 operands at the dense
    # shapes the C3 Pauli products issue: the practical reference for the MFMA roofline
    ap.add_argument("--calibrate", action="store_true")
    # record counter figures measured by rocprofv3 for the current build of a kernel, e.g.
    # --pin '{"key": "pauli_gemm_dma_kernel_c3", "sources": ["yggdrasil_amd/csrc/pauli_gemm.hip"],
    #         "traffic_bytes_per_launch": 4.1e8, "mfma_busy": 0.36, "profile": "profiles/....md"}'
    ap.add_argument("--pin", default=None)
    return ap.parse_args()


def write_pin(spec):
    """Store a kernel's counter figures with the SHA-256 of the sources they were measured on."""
    import hashlib

    entry = json.loads(spec)
    key = entry.pop("key")
    h = hashlib.sha256()
    for rel in entry["sources"]:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    entry["sha256"] = h.hexdigest()
    try:
        with open(PINS) as f:
            pins = json.load(f)
    except (OSError, ValueError):
        pins = {}
    pins[key] = entry
    with open(PINS, "w") as f:
        json.dump(pins, f, indent=1, sort_keys=True)
        f.write("\n")


# ---------------------------------------------------------------------------
# synthetic inputs (on the device, seeded)
# ---------------------------------------------------------------------------


def make_inputs(torch, c, seed=0):
    dev = "cuda"
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    N, d, E, k, F = c["N"], c["d"], c["E"], c["k"], c["F"]
    dt = torch.float32 if c["dtype"] == "f32" else torch.bfloat16
    rn = lambda *s: torch.randn(*s, generator=g, device=dev, dtype=torch.float32)
    x = rn(N, d, 8).to(dt)
    layers = []
    for _ in range(c["layers"]):
        L = {}
        if F:
            L["w_up"] = rn(E, F, d, 8) / (8.0 * d) ** 0.5
            L["w_down"] = rn(E, d, F, 8) / (8.0 * F) ** 0.5
            if dt == torch.bfloat16:
                L["w_up"] = L["w_up"].bfloat16().float()
                L["w_down"] = L["w_down"].bfloat16().float()
        if c["logits"] == "normal":
            L["logits"] = rn(N, E)
        elif c["logits"] == "normal_bias":
            L["logits"] = rn(N, E) + 0.5 * rn(E)[None, :]
        elif c["logits"] == "zipf":
            ranking = torch.randperm(E, generator=g, device=dev)
            p = torch.arange(1, E + 1, device=dev, dtype=torch.float64) ** -1.2
            chosen = torch.multinomial((p / p.sum()).float().expand(N, E), k, replacement=False, generator=g)
            lg = 0.1 * rn(N, E)
            bonus = (k - torch.arange(k, device=dev, dtype=torch.float32)).expand(N, k)
            lg.scatter_add_(1, ranking[chosen], bonus)
            L["logits"] = lg.contiguous()
        elif c["logits"] == "head":  # CliffordLinear(d -> E) weights; logits = scalar part of its output
            L["head_w"] = rn(1, E, d, 8) / (8.0 * d) ** 0.5
        else:  # energy router
            L["router_w"] = 0.1 * rn(E, 4)
            L["router_b"] = torch.zeros(E, device=dev)
        layers.append(L)
    return x, layers


# ---------------------------------------------------------------------------
# GPU timing
# ---------------------------------------------------------------------------


# Warm-up runs at least this long as well as at least W steps: a config that starts on an idle GPU
# otherwise times its first steps before the clocks have settled (5 steps of config 3 take 2 ms)
WARMUP_MIN_S = 0.3


def time_fn(torch, fn, steps, warmup):
    t0 = time.perf_counter()
    n = 0
    while n < warmup or time.perf_counter() - t0 < WARMUP_MIN_S:
        fn()
        n += 1
        if n >= warmup and n % 8 == 0:
            torch.cuda.synchronize()  # so the wall clock follows the device
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps  # ms


def pinned(key):
    """The counter figures measured for kernel `key` if its sources are unchanged since, else None."""
    import hashlib

    try:
        with open(PINS) as f:
            entry = json.load(f)[key]
    except (OSError, KeyError, ValueError):
        return None
    h = hashlib.sha256()
    for rel in entry["sources"]:
        try:
            with open(os.path.join(ROOT, rel), "rb") as f:
                h.update(f.read())
        except OSError:
            return None
    if h.hexdigest() != entry["sha256"]:
        return None
    return entry


def run_layer_config(torch, ops, name, c, steps, warmup):
    rot = c.get("rotate", 0)
    x, layers = make_inputs(torch, dict(c, layers=rot) if rot else c, seed=SEEDS[name])
    N, d, E, k, F = c["N"], c["d"], c["E"], c["k"], c["F"]
    qerr = None
    if rot and c["fmt"] in ("int8", "int8_pauli"):
        # the int8 formats' error against the fp32 masters they are quantized from, on weight set 0:
        # the same layer with fp32 activations and the master weights (format 4) as the reference
        L0 = layers[0]
        ref, _ = ops.moe_forward(x.float(), k, ops.prepare_weights(L0["w_up"], "pauli_f32"),
                                 ops.prepare_weights(L0["w_down"], "pauli_f32"), None, None, "gelu",
                                 logits=L0["logits"])
        qerr = {}
        for f in ("int8", "int8_pauli"):
            o, _ = ops.moe_forward(x, k, ops.prepare_weights(L0["w_up"], f), ops.prepare_weights(L0["w_down"], f),
                                   None, None, "gelu", logits=L0["logits"])
            qerr[f] = float(((o.float() - ref).abs().max() / ref.abs().max()).item())
        del ref, o
    prepared = []
    for L in layers:
        prepared.append(dict(
            w_up=ops.prepare_weights(L["w_up"], c["fmt"]), w_down=ops.prepare_weights(L["w_down"], c["fmt"]),
            logits=L.get("logits"), router_w=L.get("router_w"), router_b=L.get("router_b"),
            head=L["head_w"][0].contiguous() if "head_w" in L else None))
        del L["w_up"], L["w_down"]

    def head_logits(cur, P):
        # the layer's CliffordLinear head (CliffordMoELayer._head_logits): scalar part of W_h x
        return ops.router_head_logits(cur, P["head"])
    torch.cuda.synchronize()
    ws = torch.empty(ops.moe_workspace_bytes(N, d, F, E, k, x.dtype, c["fmt"]), device="cuda", dtype=torch.uint8)
    bufs = [torch.empty_like(x), torch.empty_like(x)]
    resid = c["layers"] > 1
    info = {}

    def step():
        cur = x
        for li, P in enumerate(prepared):
            out = bufs[li % 2]
            lg = head_logits(cur, P) if P["head"] is not None else P["logits"]
            _, rt = ops.moe_forward(cur, k, P["w_up"], P["w_down"], None, None, "gelu", logits=lg,
                                    router_weight=P["router_w"], router_bias=P["router_b"],
                                    residual=cur if resid else None, workspace=ws, out=out)
            cur = out
        info["rt"] = rt

    all_sets = prepared
    if rot:  # one layer per step with weight set i mod rot; the warm figure reuses set 0 every step
        def layer(P):
            _, rt = ops.moe_forward(x, k, P["w_up"], P["w_down"], None, None, "gelu", logits=P["logits"],
                                    workspace=ws, out=bufs[0])
            info["rt"] = rt

        def graph_of(sets):
            # a decode loop as serving runs it: the steps captured once in a HIP graph and replayed,
            # so the host's per-call cost (Python, argument checks, launches) is outside the figure
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for P in sets:
                    layer(P)
            torch.cuda.current_stream().wait_stream(side)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for P in sets:
                    layer(P)
            return g

        reps = max(1, steps // rot)
        g_rot, g_warm = graph_of(all_sets), graph_of([all_sets[0]] * rot)
        ms = time_fn(torch, g_rot.replay, reps, max(1, warmup // rot)) / rot
        ms_warm = time_fn(torch, g_warm.replay, reps, max(1, warmup // rot)) / rot
        counter = [0]

        def step_rot():
            P = all_sets[counter[0] % rot]
            counter[0] += 1
            layer(P)

        ms_eager = time_fn(torch, step_rot, steps, warmup)
        info["ms_eager"] = ms_eager
    else:
        ms = time_fn(torch, step, steps, warmup)
    counts = info["rt"]["counts"].cpu()
    P = N * k
    es = 4 if c["dtype"] == "f32" else 2
    R = d * 8 * es
    n_touched = int((counts > 0).sum())
    wbytes_expert = {"bf16": 2 * 2 * 8 * d * F, "pauli": 2 * 2 * 8 * d * F, "int8": 2 * 8 * d * F + 4 * (d + F),
                     "int8_pauli": 2 * 8 * d * F + 4 * (d + F),
                     "f32": 2 * 4 * 8 * d * F, "pauli_f32": 2 * 4 * 8 * d * F}[c["fmt"]]
    res = dict(
        workload=name, N=N, d=d, E=E, k=k, F=F, dtype=c["dtype"], weights=c["fmt"], layers=c["layers"],
        ms_per_step=ms, tokens_per_s=N / (ms * 1e-3), layer_tflops=c["layers"] * 256.0 * d * F * P / (ms * 1e-3) / 1e12,
        expert_counts_max=int(counts.max()), expert_counts_min=int(counts.min()), experts_touched=n_touched)
    if rot:  # the decode layer: one fused kernel (routing and both products) and the combine
        # bytes the step must move: the touched experts' weights (codes and scales), x in,
        # the logits, and the output written
        moved = n_touched * wbytes_expert + 2 * N * R + 4 * N * E
        res.update(weight_sets=rot, decode_bytes=moved, decode_hbm_frac=moved / (ms * 1e-3) / PEAK_HBM,
                   timing="HIP graph replay of the layer steps (launch cost on the device only)",
                   # one weight set, resident in the Infinity Cache after the first step
                   ms_per_step_warm=ms_warm, decode_hbm_frac_warm=moved / (ms_warm * 1e-3) / PEAK_HBM,
                   # the same steps launched one by one from Python (host-bound at this size)
                   ms_per_step_eager=info["ms_eager"])
        if qerr is not None:
            res.update(quant_error_vs_fp32=dict(
                qerr, measured=c["fmt"],
                basis="max |y_int8 - y_fp32| / max |y_fp32| over the layer's output, weight set 0; y_fp32 the "
                      "same layer with fp32 activations and the fp32 master weights (format 4)"))
        return res
    # the dominant kernel: both grouped expert products of layer 0, timed alone
    P0 = prepared[0]
    if P0["head"] is not None:
        logits = head_logits(x, P0)
    else:
        logits = P0["logits"] if P0["logits"] is not None else ops.router_energy_logits(x, P0["router_w"],
                                                                                         P0["router_b"])
    r = ops.route(logits, k)
    fmt_code = ops.WFORMAT_CODE[c["fmt"]]
    L = ops.lib()
    st = ops.stream_handle()
    dt_code = ops.DTYPE_CODE[x.dtype]
    ys = torch.empty((N * k, d, 8), device="cuda", dtype=x.dtype)
    if c["fmt"] == "pauli":
        # x -> Pauli half-rows once; up: those rows gathered through perm inside the
        # product, h in Pauli half-rows; down: h -> blade rows
        xp = ops.pauli_rows_from_blade(x)
        h = torch.empty((N * k, 2, F, 4), device="cuda", dtype=x.dtype)

        def up():
            ops.check(L.ygg_pauli_grouped_linear(xp.data_ptr(), 1, N, r.perm.data_ptr(), N * k,
                                                 P0["w_up"].data.data_ptr(), None, r.offsets.data_ptr(), E, d, F, 1,
                                                 h.data_ptr(), 0, dt_code, st))

        def down():
            ops.check(L.ygg_pauli_grouped_linear(h.data_ptr(), 1, N * k, None, N * k, P0["w_down"].data.data_ptr(), None,
                                                 r.offsets.data_ptr(), E, F, d, 0, ys.data_ptr(), 1, dt_code, st))
    elif c["fmt"] == "pauli_f32":
        # as above in fp32 split rows; the layer's down product splits its contraction
        # into partial planes, the exported entry timed here writes blade rows directly
        xp = ops.pauli_rows_from_blade_f32(x)
        h = torch.empty((N * k, F, 2, 2, 2), device="cuda", dtype=x.dtype)

        def up():
            ops.check(L.ygg_pauli_grouped_linear_f32(xp.data_ptr(), r.perm.data_ptr(), N * k,
                                                     P0["w_up"].data.data_ptr(), None, r.offsets.data_ptr(), E, d,
                                                     F, 1, h.data_ptr(), 0, st))

        def down():
            ops.check(L.ygg_pauli_grouped_linear_f32(h.data_ptr(), None, N * k, P0["w_down"].data.data_ptr(), None,
                                                     r.offsets.data_ptr(), E, F, d, 0, ys.data_ptr(), 1, st))
    else:
        xs = ops.dispatch(x, r, mask_order=True)
        h = torch.empty((N * k, F, 8), device="cuda", dtype=x.dtype)

        def up():
            ops.check(L.ygg_grouped_clifford_linear(xs.data_ptr(), N * k, P0["w_up"].data.data_ptr(), fmt_code,
                                                    ops.ptr(P0["w_up"].scales), None, r.offsets.data_ptr(), E, d, F,
                                                    1, h.data_ptr(), dt_code, 0, st))

        def down():
            ops.check(L.ygg_grouped_clifford_linear(h.data_ptr(), N * k, P0["w_down"].data.data_ptr(), fmt_code,
                                                    ops.ptr(P0["w_down"].scales), None, r.offsets.data_ptr(), E, F,
                                                    d, 0, ys.data_ptr(), dt_code, 1, st))

    ms_up = time_fn(torch, up, steps, warmup)
    ms_down = time_fn(torch, down, steps, warmup)
    ms_route = time_route(torch, ops, logits, k, steps, warmup)
    if c["fmt"] == "pauli":  # the only pass over x before the products: the Pauli conversion
        ms_disp = time_fn(torch, lambda: ops.pauli_rows_from_blade(x), steps, warmup)
    elif c["fmt"] == "pauli_f32":
        ms_disp = time_fn(torch, lambda: ops.pauli_rows_from_blade_f32(x), steps, warmup)
    else:
        xs_t = ops.dispatch(x, r, mask_order=True)
        ms_disp = time_fn(torch, lambda: ops.dispatch(x, r, mask_order=True, out=xs_t), steps, warmup)
    out_t = torch.empty_like(x)
    ms_comb = time_fn(torch, lambda: ops.combine(ys, r, out=out_t), steps, warmup)
    ms_route_conv = None
    if c["fmt"] in ("pauli", "pauli_f32") and logits is not None:
        # what the layer runs first: the routing with the conversion of x to Pauli rows in the
        # same launches (ygg_route_pauli_rows), buffers reused
        r_rc, xp_rc = ops.route_pauli_rows(logits, k, x)
        ws_rc = torch.empty((max(L.ygg_route_workspace_bytes(N, E, k), 1),), device="cuda", dtype=torch.uint8)
        ms_route_conv = time_fn(torch, lambda: ops.route_pauli_rows(logits, k, x, out=r_rc, x_pauli=xp_rc,
                                                                    workspace=ws_rc), steps, warmup)

    flops_proj = 128.0 * d * F * P  # per projection in the reference's arithmetic (64 multiply-adds per pair)
    # what the MFMA units execute: the Pauli (complex 2x2) form issues 32 of the 64 multiply-adds
    issued_proj = flops_proj / 2 if c["fmt"] in ("pauli", "pauli_f32") else flops_proj
    peak = PEAK_F32 if c["dtype"] == "f32" else PEAK_BF16
    # bytes each timed kernel moves itself.  route: logits in; top-k indices and weights,
    # slot positions, the permutation and the counts / offsets out.  The pass over x before
    # the products: for the Pauli formats the conversion to Pauli rows (x in, rows out; the
    # gather by expert happens inside the up product, whose time counts as FLOPs), else the
    # dispatch (x rows gathered in, sorted rows out, the permutation read).  combine: the
    # expert outputs and the slots' routing in, the tokens' outputs out.
    b_route = 4 * N * E + 12 * P + 4 * P + 8 * E
    b_pass = 2 * N * R if c["fmt"] in ("pauli", "pauli_f32") else P * R + P * R + 4 * P
    b_comb = P * R + 12 * P + N * R
    # the layer's route / dispatch / combine time: for the Pauli formats the routing launches that
    # also convert x (as the layer runs them), else the routing and the dispatch copy
    ms_rdc = (ms_route_conv if ms_route_conv is not None else ms_route + ms_disp) + ms_comb
    res.update(
        kernels_ms=dict(route=ms_route, dispatch=ms_disp, expert_up=ms_up, expert_down=ms_down, combine=ms_comb,
                        **({} if ms_route_conv is None else {"route_with_conversion": ms_route_conv})),
        expert_tflops=2 * issued_proj / ((ms_up + ms_down) * 1e-3) / 1e12,
        expert_mfma_frac=2 * issued_proj / ((ms_up + ms_down) * 1e-3) / peak,
        expert_dense_equiv_tflops=2 * flops_proj / ((ms_up + ms_down) * 1e-3) / 1e12,
        kernel_bytes=dict(route=b_route, dispatch=b_pass, combine=b_comb),
        kernel_hbm_frac=dict(route=b_route / (ms_route * 1e-3) / PEAK_HBM, dispatch=b_pass / (ms_disp * 1e-3) / PEAK_HBM,
                             combine=b_comb / (ms_comb * 1e-3) / PEAK_HBM),
        route_dispatch_combine_ms=ms_rdc,
        route_dispatch_combine_hbm_frac=(b_route + b_pass + b_comb) / (ms_rdc * 1e-3) / PEAK_HBM)
    res["_flops_per_launch"] = issued_proj
    res["_dense_flops_per_launch"] = flops_proj
    res["_ms_per_launch"] = (ms_up + ms_down) / 2
    return res


def run_ep_config(torch, ops, name, c, steps, warmup):
    """One GPU's share of config 3 under expert parallelism: its experts' rows, Pauli products."""
    x, layers = make_inputs(torch, c, seed=SEEDS[name])
    N, d, E, k, F = c["N"], c["d"], c["E"], c["k"], c["F"]
    G = c["ep"]
    L0 = layers[0]
    r = ops.route(L0["logits"], k)
    off = r.offsets.cpu()
    per = E // G
    rows = [int(off[(g + 1) * per] - off[g * per]) for g in range(G)]
    g = max(range(G), key=lambda i: rows[i])
    e0, beg, end = g * per, int(off[g * per]), int(off[(g + 1) * per])
    x_local = x[r.perm[beg:end].long()].contiguous()  # the rows the all-to-all delivers, expert-grouped
    offs = (r.offsets[e0:e0 + per + 1] - r.offsets[e0]).contiguous()
    pu = ops.prepare_weights(L0["w_up"][e0:e0 + per].contiguous(), c["fmt"])
    pd = ops.prepare_weights(L0["w_down"][e0:e0 + per].contiguous(), c["fmt"])
    del L0["w_up"], L0["w_down"]
    P = end - beg
    Lb, st, dt = ops.lib(), ops.stream_handle(), ops.DTYPE_CODE[x.dtype]
    xp = torch.empty((P, 2, d, 4), device="cuda", dtype=x.dtype)
    h = torch.empty((P, 2, F, 4), device="cuda", dtype=x.dtype)
    y = torch.empty((P, d, 8), device="cuda", dtype=x.dtype)

    def step():
        ops.check(Lb.ygg_pauli_rows_from_blade(x_local.data_ptr(), P, d, xp.data_ptr(), st))
        ops.check(Lb.ygg_pauli_grouped_linear(xp.data_ptr(), 1, P, None, P, pu.data.data_ptr(), None, offs.data_ptr(),
                                              per, d, F, 1, h.data_ptr(), 0, dt, st))
        ops.check(Lb.ygg_pauli_grouped_linear(h.data_ptr(), 1, P, None, P, pd.data.data_ptr(), None, offs.data_ptr(),
                                              per, F, d, 0, y.data_ptr(), 1, dt, st))

    ms = time_fn(torch, step, steps, warmup)
    flops = 2 * 128.0 * d * F * P  # both products, the reference's 64 multiply-adds per pair
    issued = flops / 2  # the Pauli form's 32
    return dict(workload=name, gpus_modelled=G, experts_here=list(range(e0, e0 + per)), rows_here=P,
                rows_per_gpu=rows, straggler_ratio=P / (N * k / G), ms_per_step=ms,
                rows_per_s=P / (ms * 1e-3), expert_tflops=issued / (ms * 1e-3) / 1e12,
                expert_mfma_frac=issued / (ms * 1e-3) / PEAK_BF16,
                expert_dense_equiv_tflops=flops / (ms * 1e-3) / 1e12)


def run_block_config(torch, ops, name, c, steps, warmup):
    """x + moe(ffn_norm(x)) through ygg_moe_block_ffn; the norm kernel also timed alone."""
    x, layers = make_inputs(torch, c, seed=SEEDS[name])
    N, d, E, k, F = c["N"], c["d"], c["E"], c["k"], c["F"]
    L0 = layers[0]
    wu, wd = ops.prepare_weights(L0.pop("w_up"), c["fmt"]), ops.prepare_weights(L0.pop("w_down"), c["fmt"])
    g = torch.Generator(device="cuda")
    g.manual_seed(SEEDS[name] + 100)
    gamma = torch.zeros(d, 8, device="cuda")
    gamma[:, 0] = 1.0
    gamma += 0.1 * torch.randn(d, 8, generator=g, device="cuda")
    beta = 0.1 * torch.randn(d, 8, generator=g, device="cuda")
    ws = torch.empty(ops.moe_block_ffn_workspace_bytes(N, d, F, E, k, x.dtype, c["fmt"]), device="cuda",
                     dtype=torch.uint8)
    out = torch.empty_like(x)
    logits = L0.get("logits")

    def step():
        ops.moe_block_ffn(x, k, gamma, beta, wu, wd, None, None, "gelu", logits=logits,
                          router_weight=L0.get("router_w"), router_bias=L0.get("router_b"), workspace=ws, out=out)

    ms = time_fn(torch, step, steps, warmup)
    xn = torch.empty_like(x)
    Lb = ops.lib()
    args = (x.data_ptr(), ops.DTYPE_CODE[x.dtype], N, d, gamma.data_ptr(), beta.data_ptr(), 1e-6, xn.data_ptr(),
            ops.DTYPE_CODE[x.dtype], ops.stream_handle())
    ms_norm = time_fn(torch, lambda: ops.check(Lb.ygg_clifford_layer_norm(*args)), steps, warmup)
    R = d * 8 * x.element_size()
    norm_bytes = 2 * N * R + 2 * d * 32  # x in, x_norm out, gamma and beta
    # weight import: grade-aware quantization of this config's up weights (E fp32 tensors),
    # codes and fp32 values written; the weights are read twice (extrema, then codes)
    w = torch.randn(E, F, d, 8, generator=g, device="cuda")
    ms_gq = time_fn(torch, lambda: ops.grade_quantize(w, (8, 6, 6, 4), True), steps, warmup)
    gq_bytes = w.numel() * (4 + 4 + 2 + 4)
    return dict(workload=name, N=N, d=d, E=E, k=k, F=F, dtype=c["dtype"], weights=c["fmt"],
                ms_per_step=ms, tokens_per_s=N / (ms * 1e-3), kernels_ms=dict(norm=ms_norm, grade_quantize=ms_gq),
                norm_bytes=norm_bytes, norm_hbm_frac=norm_bytes / (ms_norm * 1e-3) / PEAK_HBM,
                grade_quantize_bytes=gq_bytes, grade_quantize_hbm_frac=gq_bytes / (ms_gq * 1e-3) / PEAK_HBM)


def run_train_config(torch, ops, name, c, steps, warmup):
    """Forward + backward of the layer (fp32 Pauli weights), as autograd runs it (no routing-weight
    gradient); the weight-gradient kernel timed alone."""
    x, layers = make_inputs(torch, c, seed=SEEDS[name])
    N, d, E, k, F = c["N"], c["d"], c["E"], c["k"], c["F"]
    L0 = layers[0]
    w_up, w_down = L0.pop("w_up"), L0.pop("w_down")
    pu, pd = ops.prepare_weights(w_up, c["fmt"]), ops.prepare_weights(w_down, c["fmt"])
    au = ops.prepare_weights(ops.adjoint_weights(w_up), c["fmt"])
    ad = ops.prepare_weights(ops.adjoint_weights(w_down), c["fmt"])
    del w_up, w_down
    g = torch.Generator(device="cuda")
    g.manual_seed(SEEDS[name] + 200)
    dout = torch.randn(x.shape, generator=g, device="cuda")
    logits, rw, rb = L0.get("logits"), L0.get("router_w"), L0.get("router_b")
    ws_f = torch.empty(ops.moe_workspace_bytes(N, d, F, E, k, x.dtype, c["fmt"]), device="cuda", dtype=torch.uint8)
    ws_b = torch.empty(ops.lib().ygg_moe_backward_workspace_bytes(N, d, F, E, k), device="cuda", dtype=torch.uint8)

    def step():  # as the autograd node runs it: the forward keeps h before the activation
        _, _, h_pre = ops.moe_forward_train(x, k, pu, pd, None, None, "gelu", logits=logits, router_weight=rw,
                                            router_bias=rb, workspace=ws_f)
        ops.moe_backward(x, k, pu, au, pd, ad, dout, None, None, "gelu", logits=logits, router_weight=rw,
                         router_bias=rb, workspace=ws_b, routing_grad=False, h_pre=h_pre)

    ms = time_fn(torch, step, steps, warmup)
    # the weight gradients alone: up (rows of x through perm, F outputs) and down (h rows, d outputs)
    r = ops.route(logits if logits is not None else ops.router_energy_logits(x, rw, rb), k)
    P = N * k
    dh = torch.randn(P, F, 8, generator=g, device="cuda")
    dy = torch.randn(P, d, 8, generator=g, device="cuda")
    h = torch.randn(P, F, 8, generator=g, device="cuda")
    if P >= WGRAD_MFMA_ROWS_PER_EXPERT * E:  # the backward's choice: MFMA on Pauli rows
        wg_kind = "mfma"
        dhp, xp = ops.pauli_rows_from_blade_f32(dh), ops.pauli_rows_from_blade_f32(x.reshape(N, d, 8))
        dyp, hp = ops.pauli_rows_from_blade_f32(dy), ops.pauli_rows_from_blade_f32(h)
        ws_w = torch.empty(ops.lib().ygg_grouped_weight_grad_pauli_f32_workspace_bytes(P, E, d, F), device="cuda",
                           dtype=torch.uint8)
        ms_wg_up = time_fn(torch, lambda: ops.grouped_weight_grad_pauli(dhp, xp, r.offsets, E, gather=r.perm,
                                                                        workspace=ws_w), steps, warmup)
        ms_wg_down = time_fn(torch, lambda: ops.grouped_weight_grad_pauli(dyp, hp, r.offsets, E, workspace=ws_w),
                             steps, warmup)
    else:  # vector ALUs on blade rows
        wg_kind = "valu"
        ms_wg_up = time_fn(torch, lambda: ops.grouped_weight_grad(dh, x, r.offsets, E, gather=r.perm), steps, warmup)
        ms_wg_down = time_fn(torch, lambda: ops.grouped_weight_grad(dy, h, r.offsets, E), steps, warmup)
    flops_proj = 128.0 * d * F * P
    return dict(workload=name, N=N, d=d, E=E, k=k, F=F, dtype="f32", weights=c["fmt"],
                ms_per_step=ms, tokens_per_s=N / (ms * 1e-3), weight_grad_kernel=wg_kind,
                kernels_ms=dict(weight_grad_up=ms_wg_up, weight_grad_down=ms_wg_down),
                step_tflops=6 * flops_proj / (ms * 1e-3) / 1e12,
                # the reference's arithmetic (64 multiply-adds per multivector pair): an effective rate
                weight_grad_dense_equiv_tflops=2 * flops_proj / ((ms_wg_up + ms_wg_down) * 1e-3) / 1e12,
                # the MFMA work issued (the Pauli form's 32 multiply-adds per pair) against the fp32 peak
                weight_grad_mfma_frac_f32=(flops_proj / ((ms_wg_up + ms_wg_down) * 1e-3) / PEAK_F32
                                           if wg_kind == "mfma" else None))


def run_gm(torch, ops, name, c, steps, warmup):
    """geom_matmul at CliffordLinear's shapes, buffers reused across calls (the workspace entry)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(SEEDS[name])
    N, d, F = c["N"], c["d"], c["F"]
    res = dict(workload=name, dtype="f32", kernels=["pauli_f32_prep_kernel", "pauli_f32_rows_t_kernel",
                                                    "pauli_f32_kernel"],
               frac_basis="MFMA work issued (the Pauli form's 32 multiply-adds per multivector pair) against "
                          "the fp32 MFMA peak; dense_equiv_tflops counts the reference's 64 (an effective rate)")
    for tag, M, K in (("up", F, d), ("down", d, F)):
        a = torch.randn(M, K, 8, generator=g, device="cuda") / (8.0 * K) ** 0.5
        b = torch.randn(K, N, 8, generator=g, device="cuda")
        ws = torch.empty(ops.geom_matmul_workspace_bytes(M, K, N), device="cuda", dtype=torch.uint8)
        out = torch.empty((M, N, 8), device="cuda")
        ms = time_fn(torch, lambda: ops.geom_matmul(a, b, workspace=ws, out=out), steps, warmup)
        flops = 128.0 * M * K * N  # the reference's arithmetic: 64 multiply-adds per multivector pair
        res[tag] = dict(M=M, K=K, N=N, ms=ms, tflops=flops / 2 / (ms * 1e-3) / 1e12,
                        mfma_frac_f32=flops / 2 / (ms * 1e-3) / PEAK_F32,
                        dense_equiv_tflops=flops / (ms * 1e-3) / 1e12)
        del a, b, ws, out
    return res


def calibrate_gemm(torch):
    """hipBLASLt (torch.matmul) bf16 GEMM rates on N(0,1) operands, two timed passes per shape."""
    out = []
    for (M, K, N) in [(16384, 16384, 16384), (8192, 8192, 8192), (65536, 512, 2048), (65536, 2048, 512)]:
        a = torch.randn(M, K, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(K, N, device="cuda", dtype=torch.bfloat16)
        for _ in range(2):
            ms = time_fn(torch, lambda: a @ b, 20, 5)
            out.append(dict(M=M, K=K, N=N, us=ms * 1e3, tflops=2.0 * M * K * N / (ms * 1e-3) / 1e12))
            print(f"[calibrate] {out[-1]}", file=sys.stderr, flush=True)
        del a, b
    return out


def time_route(torch, ops, logits, k, steps, warmup):
    """ygg_route alone, through the C ABI with preallocated outputs (no per-call allocation)."""
    N, E = logits.shape
    r = ops.route(logits, k)
    L = ops.lib()
    ws_bytes = L.ygg_route_workspace_bytes(N, E, k)
    ws = torch.empty((max(ws_bytes, 1),), device="cuda", dtype=torch.uint8)
    args = (logits.data_ptr(), N, E, k, r.topk_idx.data_ptr(), r.topk_w.data_ptr(), r.counts.data_ptr(),
            r.offsets.data_ptr(), r.perm.data_ptr(), r.slot_pos.data_ptr(), ws.data_ptr(), ws_bytes,
            ops.stream_handle())
    return time_fn(torch, lambda: L.ygg_route(*args), steps, warmup)


def run_c2(torch, ops, c, steps, warmup):
    x, layers = make_inputs(torch, c, seed=2)
    logits = layers[0]["logits"]
    N, E, k, d = c["N"], c["E"], c["k"], c["d"]
    # buffers allocated once, as a caller of the path would: the step is route -> dispatch -> combine
    r = ops.route(logits, k)
    ws = torch.empty((max(ops.lib().ygg_route_workspace_bytes(N, E, k), 1),), device="cuda", dtype=torch.uint8)
    xs = ops.dispatch(x, r)
    out = torch.empty_like(x)

    def step():
        ops.route(logits, k, out=r, workspace=ws)
        ops.dispatch(x, r, out=xs)
        ops.combine(xs, r, out=out)

    ms = time_fn(torch, step, steps, warmup)
    ms_route = time_route(torch, ops, logits, k, steps, warmup)
    ms_disp = time_fn(torch, lambda: ops.dispatch(x, r, out=xs), steps, warmup)
    ms_comb = time_fn(torch, lambda: ops.combine(xs, r, out=out), steps, warmup)
    R = d * 8 * 4
    P = N * k
    b_route = 4 * N * E + 8 * N * k + 4 * N * k
    b_disp = N * R + P * R + 4 * P
    b_comb = P * R + 8 * P + N * R
    return dict(workload="c2", N=N, E=E, k=k, d=d, ms_per_step=ms, tokens_per_s=N / (ms * 1e-3),
                kernels_ms=dict(route=ms_route, dispatch=ms_disp, combine=ms_comb),
                bytes=b_route + b_disp + b_comb,
                hbm_frac_step=(b_route + b_disp + b_comb) / (ms * 1e-3) / PEAK_HBM,
                dispatch_hbm_frac=b_disp / (ms_disp * 1e-3) / PEAK_HBM,
                combine_hbm_frac=b_comb / (ms_comb * 1e-3) / PEAK_HBM)


# ---------------------------------------------------------------------------
# CPU baseline (bounded sample)
# ---------------------------------------------------------------------------


def cpu_baseline(name, c, sample_rows):
    """The reference's CPU path for config c, timed on this host (fp32, as the reference's CPU
    path computes): routing / dispatch / combine in NumPy over all tokens, the expert FFNs through
    the reference's compiled geometric matmul (``oracle/_ref``; the C restatement if that is
    absent) on every token-expert row when they take at most a few seconds, else on a sample
    extrapolated linearly in FLOPs; a multi-layer step is its layers' sum.  Two flavours beside
    it: the NumPy broadcast fallback the reference falls back to without its native library
    (``rune/ops/batched.py:341-344``), on a few rows, and the C restatement with OpenMP."""
    import numpy as np

    from oracle import moe, native
    from oracle.cl3 import geom_prod

    g = np.random.default_rng(11)
    N, d, E, k, F = c["N"], c["d"], c["E"], c["k"], c["F"]
    layers = c["layers"]
    logits = g.standard_normal((N, E), dtype=np.float32)
    x = g.standard_normal((N, d, 8), dtype=np.float32)
    # routing + dispatch + combine over all tokens (NumPy restatement of the reference)
    t0 = time.perf_counter()
    probs = moe.softmax(logits)
    idx, w = moe.topk_reference(probs, k)
    flat = idx.reshape(-1)
    tok = np.repeat(np.arange(N), k)
    out = np.zeros_like(x)
    for e in range(E):
        m = flat == e
        if m.any():
            rows = x[tok[m]]
            np.add.at(out, tok[m], w.reshape(-1)[m][:, None, None] * rows)
    t_rdc = time.perf_counter() - t0
    host = dict(nproc=os.cpu_count(), affinity=len(os.sched_getaffinity(0)), cpu=_cpu_model())
    if not F:
        return dict(value=N / t_rdc, unit="tokens/s", cores=1, kind="port", dtype="f32",
                    sample=f"{config_label(c)} config, computed in fp32: NumPy routing / dispatch / combine over "
                           f"all {N} tokens, "
                           f"measured {t_rdc:.2f} s", host=host)
    P = N * k
    flops_row = 2 * 128.0 * d * F  # both expert products of one token-expert row
    full = P * flops_row <= 8e9    # about 2-4 s through the reference C on one core
    # else a sample of about 4 GFLOP (sample_rows at the config 3 shape)
    rows = P if full else min(P, max(16, int(sample_rows * (2 * 128.0 * 128 * 512) / flops_row)))
    wu = (g.standard_normal((F, d, 8)) / np.sqrt(8 * d)).astype(np.float32)
    wd = (g.standard_normal((d, F, 8)) / np.sqrt(8 * F)).astype(np.float32)
    xs = np.resize(x, (rows, d, 8))
    if native.ref_lib() is not None:
        gm, kind, what = native.ref_geom_matmul, "reference", "oracle/_ref cl3_geom_matmul_flat (reference C, 1 thread)"
    else:
        gm, kind, what = native.c_geom_matmul, "port", "oracle C restatement of cl3_batch_geom_matmul (1 thread)"

    def ffn(gmm, xr, **kw):
        h = np.transpose(gmm(wu, np.ascontiguousarray(np.transpose(xr, (1, 0, 2))), **kw), (1, 0, 2))
        h = moe.gelu(h)
        return gmm(wd, np.ascontiguousarray(np.transpose(h, (1, 0, 2))), **kw)

    t0 = time.perf_counter()
    ffn(gm, xs)
    t_ffn = time.perf_counter() - t0
    t_layer = t_rdc + t_ffn / rows * P
    how = (f"the expert FFN on all {P} token-expert rows" if full else
           f"the expert FFN on {rows} of {P} token-expert rows, extrapolated linearly in FLOPs")
    res = dict(value=N / (layers * t_layer), unit="tokens/s", cores=1, kind=kind, dtype="f32",
               sample=(f"{config_label(c)} config, computed in fp32: {how} via {what}, measured {t_ffn:.2f} s; "
                       f"NumPy routing / dispatch / "
                       f"combine over all {N} tokens ({t_rdc:.2f} s)"
                       + (f"; one layer timed, the {layers}-layer step is {layers} x that" if layers > 1 else "")),
               host=host)

    # the NumPy broadcast fallback: per CliffordLinear, the pairwise geometric product over a
    # broadcast (d_out, d_in, rows, 8) then the sum over d_in, a few rows at a time
    def gm_broadcast(a, b):
        return np.stack([geom_prod(a[:, :, None, :], b[None, :, j:j + 1, :]).sum(axis=1)[:, 0]
                         for j in range(b.shape[1])], axis=1)

    rows_np = 2
    t0 = time.perf_counter()
    ffn(gm_broadcast, xs[:rows_np])
    t_np = time.perf_counter() - t0
    res["numpy_fallback"] = dict(
        value=N / (layers * (t_rdc + t_np / rows_np * P)), unit="tokens/s", cores=1, kind="port", dtype="f32",
        sample=(f"the reference's NumPy fallback (broadcast pairwise geometric product, then sum over d_in; "
                f"rune/ops/batched.py:341-344) on {rows_np} rows, measured {t_np:.2f} s, same extrapolation"))
    # the C restatement with OpenMP on every host core this process may use
    threads = host["affinity"]
    rows_p = min(8 * rows, P)
    t0 = time.perf_counter()
    ffn(native.c_geom_matmul, np.resize(x, (rows_p, d, 8)), threads=threads)
    t_par = time.perf_counter() - t0
    res["parallel"] = dict(value=N / (layers * (t_rdc + t_par / rows_p * P)), unit="tokens/s", cores=threads,
                           kind="port", dtype="f32",
                           sample=(f"oracle C restatement of cl3_batch_geom_matmul with OpenMP on {threads} "
                                   f"threads, {rows_p} rows, measured {t_par:.2f} s, same extrapolation"))
    return res


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def config_label(c):
    return f"N={c['N']} d={c['d']} E={c['E']} k={c['k']} F={c['F']} {c['dtype']}"


def main():
    args = parse()
    if args.pin:
        write_pin(args.pin)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (multi-GPU is design-only: "
                                   "tokens shard with no exchange, experts with one all-to-all each way)"}))
        sys.exit(2)
    import torch

    from yggdrasil_amd import ops

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU"}))
        sys.exit(1)
    if args.calibrate:
        print(json.dumps({"calibration": calibrate_gemm(torch)}))
        return
    names = [s.strip() for s in args.configs.split(",") if s.strip()]
    if args.calib_copy_mb:
        n = args.calib_copy_mb << 18  # fp32 elements
        src = torch.ones(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    results = {}
    for name in names:
        c = CONFIGS[name]
        print(f"[bench] {name} {config_label(c)}", file=sys.stderr, flush=True)
        if name == "c2":
            results[name] = run_c2(torch, ops, c, args.steps, args.warmup)
        elif c.get("gm"):
            results[name] = run_gm(torch, ops, name, c, args.steps, args.warmup)
        elif c.get("ep"):
            results[name] = run_ep_config(torch, ops, name, c, args.steps, args.warmup)
        elif c.get("train"):
            results[name] = run_train_config(torch, ops, name, c, args.steps, args.warmup)
        elif c.get("block"):
            results[name] = run_block_config(torch, ops, name, c, args.steps, args.warmup)
        else:
            results[name] = run_layer_config(torch, ops, name, c, args.steps, args.warmup)
        torch.cuda.empty_cache()
    # the headline: config 3 when it ran, else the first config that has a token rate
    head_name = "c3" if "c3" in results else next((n for n in names if "tokens_per_s" in results[n]), names[0])
    head = results[head_name]
    cpu = None
    if not args.no_cpu_baseline:
        # the reference CPU path for every BASELINE config in this run (the training, block and
        # expert-parallel variants have none)
        for name in names:
            if name in ("c1", "c2", "c3", "c4", "c5"):
                print(f"[bench] cpu baseline {name}", file=sys.stderr, flush=True)
                results[name]["cpu_baseline"] = cpu_baseline(name, CONFIGS[name], args.cpu_sample_rows)
        cpu = results[head_name].get("cpu_baseline")
    roof = None
    if "_flops_per_launch" in head:
        ach = head["_flops_per_launch"] / (head["_ms_per_launch"] * 1e-3)
        peak = PEAK_F32 if CONFIGS[head_name]["dtype"] == "f32" else PEAK_BF16
        pauli = CONFIGS[head_name]["fmt"] == "pauli"
        kern = "pauli_gemm_dma_kernel" if pauli else "grouped_cl_mfma"
        roof = dict(bound="mfma", kernel=f"{kern} (mean of the up and down expert products)",
                    achieved=ach / 1e12, peak=peak / 1e12, unit="TFLOP/s", frac=ach / peak, traffic=None)
        dense = head["_dense_flops_per_launch"] / (head["_ms_per_launch"] * 1e-3)
        if pauli:
            # achieved and frac count the MFMA work issued: the complex (Pauli) form's 32
            # multiply-adds per multivector pair; the reference's arithmetic (64, the dense L(w)
            # block) is reported as an effective rate beside it
            roof["frac_basis"] = ("MFMA work issued: 32 multiply-adds per multivector pair (Pauli form), "
                                  "against the dense bf16 peak")
        roof["dense_equiv_tflops"] = dense / 1e12
        pin = pinned(f"{kern}_{head_name}")
        if pin is not None:
            # HBM bytes per launch (mean of the two products, rocprofv3 FETCH_SIZE / WRITE_SIZE scaled by
            # a device copy) and SQ_VALU_MFMA_BUSY_CYCLES, measured on this kernel build
            roof["traffic"] = pin["traffic_bytes_per_launch"]
            roof["traffic_unit"] = "bytes per launch"
            if "mfma_busy" in pin:
                roof["mfma_busy_counter"] = pin["mfma_busy"]
            roof["counters_from"] = pin["profile"]
    for r in results.values():
        r.pop("_flops_per_launch", None)
        r.pop("_dense_flops_per_launch", None)
        r.pop("_ms_per_launch", None)
    c = CONFIGS[head_name]
    line = {
        "metric": "MoE-HLM layer tokens/sec (prefill+decode) at 1 GPU; % of MFMA/HBM roofline",
        "value": head.get("tokens_per_s"),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_min_s": WARMUP_MIN_S,
        "ms_per_step": head.get("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if c["dtype"] == "bf16" else "f32",
        "data": "synthetic (seeded; random-init weights ~N(0, 1/sqrt(8 fan_in)))",
        "config": {"workload": (f"BASELINE config {head_name[1]}: MoE-HLM layer, " + config_label(c)
                                + (", Zipf(1.2) expert load" if c["logits"] == "zipf" else ""))
                   if head_name in ("c1", "c2", "c3", "c4", "c5") else f"{head_name}: " + config_label(c),
                   "tokens": c["N"], "d": c["d"], "experts": c["E"], "top_k": c["k"], "d_ff": c["F"],
                   "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "configs": results,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
