"""GPU parity: the Pauli (complex 2x2) grouped CliffordLinear against the oracle.

The kernel rounds its operands to bf16 in Pauli coordinates.  Each product is
pinned three ways:

* the linear part (``act='none'``, fp32 output) against the oracle run on the
  operands rounded exactly as the kernel rounds them (``pauli_round``), to 1e-4
  normwise -- this leaves only the fp32 summation order;
* the fused activation against the oracle's activation applied to the
  kernel's own pre-activation output, to 2e-5 normwise;
* the whole product against the oracle on the exact fp32 weights, to the
  bf16 bound (the sigmoid's magnitude gate is excluded there: for vectors of
  small norm it amplifies any rounding of the direction).
"""

import numpy as np
import pytest
import torch

import _inputs
from _gpu_helpers import TOL_BF16, moe_reference, normwise_err, say
from oracle import moe

pytestmark = pytest.mark.gpu

TOL_LINEAR_SAME_OPERANDS = 1e-4
TOL_EPILOGUE = 2e-5
TOL_BF16_LINEAR = 1e-2


def _ops():
    from yggdrasil_amd import ops

    return ops


def _bf16(a):
    return _inputs.bf16_round(np.asarray(a, np.float32))


def pauli_round(x, scale=1.0):
    """Blade fp32 -> Pauli coordinates (fp32 sums) -> bf16 -> back to blade (exact).

    ``scale`` = 0.5 reproduces the prepared weights, which hold W/2 (a power of
    two: it does not change the rounding).
    """
    x = np.asarray(x, np.float32) * np.float32(scale)
    s, v1, v2, v3, b12, b13, b23, t = [x[..., i] for i in range(8)]
    P = [s + v3, t + b12, v1 + b13, b23 + v2, v1 - b13, b23 - v2, s - v3, t - b12]
    m00r, m00i, m10r, m10i, m01r, m01i, m11r, m11i = [_bf16(p).astype(np.float64) for p in P]
    out = np.stack([(m00r + m11r) / 2, (m10r + m01r) / 2, (m10i - m01i) / 2, (m00r - m11r) / 2,
                    (m00i - m11i) / 2, (m10r - m01r) / 2, (m10i + m01i) / 2, (m00i + m11i) / 2], -1)
    return (out / scale).astype(np.float32)


def _offsets(g, E, P, empty_first=True):
    counts = np.bincount(g.integers(0, E, P), minlength=E)
    if empty_first and E > 2:
        counts[-1] += counts[0]
        counts[0] = 0
    counts[-1] += P - counts.sum()
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


def _per_expert(offsets, fn):
    errs = []
    for e in range(len(offsets) - 1):
        rows = slice(offsets[e], offsets[e + 1])
        if offsets[e] < offsets[e + 1]:
            errs.append(fn(e, rows))
    return max(errs)


@pytest.mark.parametrize("act,d_in,d_out,E,P,N,x_layout", [
    ("none", 16, 64, 4, 200, 90, "blade"), ("gelu", 128, 512, 3, 300, 120, "pauli"),
    ("sigmoid", 10, 40, 5, 77, 77, "blade"), ("relu", 2, 6, 2, 33, 20, "pauli"),
    ("gelu", 64, 130, 2, 129, 64, "blade"), ("none", 512, 128, 4, 260, 100, "pauli"),
    ("gelu", 128, 512, 32, 3000, 1000, "pauli")])
def test_pauli_product(act, d_in, d_out, E, P, N, x_layout):
    ops = _ops()
    g = np.random.default_rng(d_in * 13 + d_out + E)
    W = (g.standard_normal((E, d_out, d_in, 8), dtype=np.float32) / np.sqrt(8 * d_in)).astype(np.float32)
    b = (0.3 * g.standard_normal((E, d_out, 8))).astype(np.float32)
    x = _bf16(g.standard_normal((N, d_in, 8), dtype=np.float32))
    gather = g.integers(0, N, P).astype(np.int32)
    offsets = _offsets(g, E, P)
    say(f"pauli product act={act} d_in={d_in} d_out={d_out} E={E} P={P} N={N} x={x_layout}")
    pw = ops.prepare_weights(torch.from_numpy(W).cuda(), "pauli")
    pb = ops.prepare_bias(torch.from_numpy(b).cuda())
    xt = torch.from_numpy(x).cuda().bfloat16()
    if x_layout == "pauli":
        xt = ops.pauli_rows_from_blade(xt)
    off = torch.from_numpy(offsets).cuda()
    gt = torch.from_numpy(gather).cuda()

    def run(a, y_layout="blade"):
        return ops.pauli_grouped_linear(xt, pw, off, pb, a, x_layout=x_layout, gather=gt, y_layout=y_layout,
                                        out_dtype=torch.float32)

    pre = run("none").cpu().numpy()
    xr, Wr = pauli_round(x), pauli_round(W, 0.5)
    err = _per_expert(offsets, lambda e, rows: normwise_err(pre[rows], moe.clifford_linear(xr[gather[rows]], Wr[e], b[e])))
    assert err < TOL_LINEAR_SAME_OPERANDS, err
    y = run(act).cpu().numpy() if act != "none" else pre
    assert normwise_err(y, moe.ACTIVATIONS[act](pre)) < TOL_EPILOGUE
    if act != "sigmoid":
        err = _per_expert(offsets, lambda e, rows: normwise_err(
            y[rows], moe.ACTIVATIONS[act](moe.clifford_linear(x[gather[rows]], W[e], b[e]))))
        assert err < TOL_BF16_LINEAR, err
    if d_out % 2 == 0:
        # the Pauli half-row output holds the same values, rounded to bf16
        yp = run(act, "pauli")
        back = ops.pauli_grouped_linear(yp, ops.prepare_weights(_identity_weights(d_out), "pauli"),
                                        torch.tensor([0, P], device="cuda", dtype=torch.int32), None, "none",
                                        x_layout="pauli", y_layout="blade", out_dtype=torch.float32)
        assert normwise_err(back.cpu().numpy(), y) < 8e-3


def _identity_weights(d):
    w = torch.zeros(1, d, d, 8)
    w[0, torch.arange(d), torch.arange(d), 0] = 1.0
    return w.cuda()


def test_pauli_rows_roundtrip_exact_for_representable_values():
    """Blade -> Pauli is exact when every pairwise sum is a bf16 value (small integers)."""
    ops = _ops()
    g = np.random.default_rng(3)
    x = g.integers(-8, 9, size=(37, 6, 8)).astype(np.float32)
    say("pauli rows roundtrip")
    xp = ops.pauli_rows_from_blade(torch.from_numpy(x).cuda().bfloat16()).float().cpu().numpy()
    s, v1, v2, v3, b12, b13, b23, t = [x[..., i] for i in range(8)]
    col0 = np.stack([s + v3, t + b12, v1 + b13, b23 + v2], -1)
    col1 = np.stack([v1 - b13, b23 - v2, s - v3, t - b12], -1)
    assert np.array_equal(xp[:, 0], col0) and np.array_equal(xp[:, 1], col1)


@pytest.mark.parametrize("rows,d", [(300, 130), (5, 2), (1, 128)])
def test_pauli_rows_random_against_numpy(rows, d):
    """Random bf16 rows: every Pauli coordinate is the fp32 pairwise sum rounded to nearest even bf16."""
    ops = _ops()
    g = np.random.default_rng(rows + d)
    x = _inputs.bf16_round(g.standard_normal((rows, d, 8), dtype=np.float32))
    say(f"pauli rows random rows={rows} d={d}")
    xp = ops.pauli_rows_from_blade(torch.from_numpy(x).cuda().bfloat16()).float().cpu().numpy()
    s, v1, v2, v3, b12, b13, b23, t = [x[..., i] for i in range(8)]
    col0 = _inputs.bf16_round(np.stack([s + v3, t + b12, v1 + b13, b23 + v2], -1))
    col1 = _inputs.bf16_round(np.stack([v1 - b13, b23 - v2, s - v3, t - b12], -1))
    assert xp.shape == (rows, 2, d, 4)
    assert np.array_equal(xp[:, 0], col0) and np.array_equal(xp[:, 1], col1)


@pytest.mark.parametrize("E,d_in,d_out,P,N,x_layout,biased", [
    (2, 8, 6, 40, 40, "blade", False), (3, 42, 70, 300, 120, "pauli", True),
    (5, 2, 64, 200, 64, "pauli", True), (4, 522, 34, 410, 90, "pauli", False)])
def test_pauli_small_integer_product_is_exact(E, d_in, d_out, P, N, x_layout, biased):
    """Integer operands whose Pauli coordinates and sums stay exact in bf16/fp32 give exact results:
    every staged piece (gathered rows, K tails, ragged column tiles, the bias) lands where it belongs."""
    ops = _ops()
    g = np.random.default_rng(4 + d_in)
    W = g.integers(-2, 3, size=(E, d_out, d_in, 8)).astype(np.float32)
    x = g.integers(-2, 3, size=(N, d_in, 8)).astype(np.float32)
    b = g.integers(-3, 4, size=(E, d_out, 8)).astype(np.float32) if biased else None
    gather = g.integers(0, N, P).astype(np.int32) if N != P else np.arange(P, dtype=np.int32)
    offsets = _offsets(g, E, P)
    say(f"pauli integer product E={E} d_in={d_in} d_out={d_out} P={P} x={x_layout} bias={biased}")
    xt = torch.from_numpy(x).cuda().bfloat16()
    if x_layout == "pauli":
        xt = ops.pauli_rows_from_blade(xt)
    pb = ops.prepare_bias(torch.from_numpy(b).cuda()) if biased else None
    y = ops.pauli_grouped_linear(xt, ops.prepare_weights(torch.from_numpy(W).cuda(), "pauli"),
                                 torch.from_numpy(offsets).cuda(), pb, "none", x_layout=x_layout,
                                 gather=torch.from_numpy(gather).cuda() if N != P else None,
                                 y_layout="blade", out_dtype=torch.float32).cpu().numpy()
    for e in range(E):
        rows = slice(offsets[e], offsets[e + 1])
        ref = moe.clifford_linear(x[gather[rows]], W[e], b[e] if biased else None)
        assert np.array_equal(y[rows], ref), e


@pytest.mark.parametrize("E,d_in,d_out,P,N", [(2, 512, 512, 3000, 1000), (3, 128, 512, 6000, 2000)])
def test_pauli_integer_product_exact_at_full_load(E, d_in, d_out, P, N):
    """Exact integer products with every CU busy (hundreds of tiles): staged chunks that a
    wait let through before they landed would show as whole wrong tiles.  The reference is
    the dense L(W) product in float64 (``oracle.dense.linear``)."""
    from oracle import dense
    ops = _ops()
    g = np.random.default_rng(d_in + P)
    W = g.integers(-2, 3, size=(E, d_out, d_in, 8)).astype(np.float32)
    x = g.integers(-2, 3, size=(N, d_in, 8)).astype(np.float32)
    b = g.integers(-3, 4, size=(E, d_out, 8)).astype(np.float32)
    gather = g.integers(0, N, P).astype(np.int32)
    offsets = _offsets(g, E, P, empty_first=False)
    say(f"pauli integer product at full load E={E} d_in={d_in} d_out={d_out} P={P}")
    xt = ops.pauli_rows_from_blade(torch.from_numpy(x).cuda().bfloat16())
    y = ops.pauli_grouped_linear(xt, ops.prepare_weights(torch.from_numpy(W).cuda(), "pauli"),
                                 torch.from_numpy(offsets).cuda(), ops.prepare_bias(torch.from_numpy(b).cuda()),
                                 "none", x_layout="pauli", gather=torch.from_numpy(gather).cuda(),
                                 y_layout="blade", out_dtype=torch.float32).cpu().numpy()
    for e in range(E):
        rows = slice(offsets[e], offsets[e + 1])
        ref = dense.linear(x[gather[rows]], W[e], b[e])
        bad = np.nonzero(np.any(y[rows] != ref, axis=-1))
        assert bad[0].size == 0, (e, bad[0][:8], bad[1][:8])


def test_pauli_rejects_bad_arguments():
    ops = _ops()
    with pytest.raises(ValueError):
        ops.prepare_weights(torch.zeros(1, 4, 3, 8, device="cuda"), "pauli")
    L = ops.lib()
    assert L.ygg_pauli_grouped_linear(None, 0, 4, None, 4, None, None, None, 65, 4, 4, 0, None, 1, 1, None) == -1
    assert b"E <= 64" in L.ygg_last_error()


@pytest.mark.parametrize("fmt", ["bf16", "pauli"])
def test_layer_formats_against_oracle(fmt):
    """Whole layer with 'pauli' and with 'bf16' (8x8 L(w) blocks) weights against the oracle on exact weights."""
    import yggdrasil_amd

    g = np.random.default_rng(12)
    N, d, F, E, k = 500, 32, 96, 6, 2
    x = _bf16(g.standard_normal((1, N, d, 8), dtype=np.float32))
    wu, bu, wd, bd = _inputs.expert_weights(g, E, d, F, bias_std=0.2)
    logits_np = g.standard_normal((N, E), dtype=np.float32)
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, dtype=torch.bfloat16,
                                     weight_format=fmt, router="logits")
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    say(f"layer fmt={fmt} N={N} d={d} F={F} E={E} k={k}")
    out = layer.moe_forward(torch.from_numpy(x).cuda().bfloat16(), logits=torch.from_numpy(logits_np).cuda())
    out = out.float().cpu().numpy().reshape(N, d, 8)
    idx = layer.last_routing["topk_idx"].cpu().numpy()
    idx_o, w = moe.route_topk(moe.softmax(logits_np), k)
    assert np.array_equal(idx, idx_o)
    ref = moe_reference(x[0], idx, w, wu, bu, wd, bd, "gelu")
    assert normwise_err(out, ref) < TOL_BF16


@pytest.mark.parametrize("d_in,d_out,gathered,y_layout", [(64, 96, True, "pauli"), (96, 64, False, "blade"),
                                                          (256, 1024, True, "pauli"), (1024, 256, False, "blade")])
def test_pauli_integer_product_exact_with_compact_tiles(d_in, d_out, gathered, y_layout):
    """Experts whose last row tile holds at most 32 rows run it as a compact tile (half the
    MFMAs, its rows staged at the token slots of one row block per wave): counts 1, 16, 17,
    31, 32 and 64 k + those, next to counts of 33, 63, 64 and 65 rows that stay whole, an
    empty expert, and enough tiles for a half-tile remainder.  Exact integer products, every
    row, against the float64 dense oracle, in both output layouts."""
    from oracle import dense
    ops = _ops()
    g = np.random.default_rng(d_in * 3 + d_out)
    counts = np.array([1, 16, 17, 31, 32, 33, 0, 63, 64, 65, 96, 97, 128 + 5, 320 + 32, 2, 200], np.int64)
    E, P = counts.size, int(counts.sum())
    N = 700
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    W = g.integers(-2, 3, size=(E, d_out, d_in, 8)).astype(np.float32)
    x = g.integers(-2, 3, size=(N if gathered else P, d_in, 8)).astype(np.float32)
    b = g.integers(-3, 4, size=(E, d_out, 8)).astype(np.float32)
    gather = g.integers(0, N, P).astype(np.int32) if gathered else None
    say(f"pauli integer product with compact tiles d_in={d_in} d_out={d_out} gathered={gathered} y={y_layout}")
    xt = ops.pauli_rows_from_blade(torch.from_numpy(x).cuda().bfloat16())
    y = ops.pauli_grouped_linear(xt, ops.prepare_weights(torch.from_numpy(W).cuda(), "pauli"),
                                 torch.from_numpy(offsets).cuda(), ops.prepare_bias(torch.from_numpy(b).cuda()),
                                 "none", x_layout="pauli", gather=None if gather is None else torch.from_numpy(gather).cuda(),
                                 y_layout=y_layout, out_dtype=torch.float32 if y_layout == "blade" else torch.bfloat16)
    y = y.float().cpu().numpy()
    for e in range(E):
        rows = slice(offsets[e], offsets[e + 1])
        if counts[e] == 0:
            continue
        xe = x[gather[rows]] if gathered else x[rows]
        ref = dense.linear(xe, W[e], b[e])
        if y_layout == "pauli":
            # the exact integer result's Pauli half-rows, rounded to bf16 as the kernel stores them
            ref = _bf16(_blade_to_pauli_rows(ref))
        bad = np.nonzero(np.any((y[rows] != ref).reshape(ref.shape[0], -1), axis=-1))
        assert bad[0].size == 0, (e, int(counts[e]), bad[0][:8])


@pytest.mark.parametrize("d_in,d_out", [(128, 512), (512, 128)])
def test_pauli_integer_product_exact_items_after_partial_round(d_in, d_out):
    """Config 3's expert-parallel share: 4 experts of about 1930 rows, three of them ending in
    compact tiles.  The whole tiles end in a partial round that is not cut into halves (up
    shape, 512 workgroups over 8 XCDs) or fill fewer workgroups than the grid holds (down shape,
    one XCD range), so the compact items go to the workgroups that run one whole tile fewer.
    Exact integer products, every row, against the float64 dense oracle."""
    from oracle import dense
    ops = _ops()
    g = np.random.default_rng(d_in + d_out + 7)
    counts = np.array([1930, 1950, 1900, 1937], np.int64)
    E, P = counts.size, int(counts.sum())
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    W = g.integers(-2, 3, size=(E, d_out, d_in, 8)).astype(np.float32)
    x = g.integers(-2, 3, size=(P, d_in, 8)).astype(np.float32)
    b = g.integers(-3, 4, size=(E, d_out, 8)).astype(np.float32)
    say(f"pauli integer product, items after a partial round d_in={d_in} d_out={d_out} P={P}")
    xt = ops.pauli_rows_from_blade(torch.from_numpy(x).cuda().bfloat16())
    y = ops.pauli_grouped_linear(xt, ops.prepare_weights(torch.from_numpy(W).cuda(), "pauli"),
                                 torch.from_numpy(offsets).cuda(), ops.prepare_bias(torch.from_numpy(b).cuda()),
                                 "none", x_layout="pauli", y_layout="blade", out_dtype=torch.float32)
    y = y.cpu().numpy()
    for e in range(E):
        rows = slice(offsets[e], offsets[e + 1])
        ref = dense.linear(x[rows], W[e], b[e])
        bad = np.nonzero(np.any(y[rows] != ref, axis=-1))
        assert bad[0].size == 0, (e, int(counts[e]), bad[0][:8])


def _blade_to_pauli_rows(y):
    """(rows, d, 8) blade order -> (rows, 2, d, 4) Pauli half-rows: half b holds column b of each
    multivector's 2x2 complex matrix as (row 0 re, row 0 im, row 1 re, row 1 im)."""
    s, v1, v2, v3, b12, b13, b23, t = (y[..., i] for i in range(8))
    m00 = (s + v3, t + b12)
    m01 = (v1 - b13, b23 - v2)
    m10 = (v1 + b13, b23 + v2)
    m11 = (s - v3, t - b12)
    h0 = np.stack([m00[0], m00[1], m10[0], m10[1]], axis=-1)
    h1 = np.stack([m01[0], m01[1], m11[0], m11[1]], axis=-1)
    return np.stack([h0, h1], axis=1)
