"""GPU parity: the fp32 Pauli (complex 2x2) grouped CliffordLinear against the oracle.

Every operand stays fp32, so each product is compared with the oracle on the
exact weights at the fp32 bound (1e-5 normwise): only the summation order and
the Pauli coordinate sums differ.  The Pauli row conversion is a set of single
fp32 additions and is compared bit for bit with NumPy's fp32 additions.
"""

import numpy as np
import pytest
import torch

from _fixtures import load_case
from _gpu_helpers import TOL_F32, moe_reference, normwise_err, say
from oracle import moe

pytestmark = pytest.mark.gpu


def _ops():
    from yggdrasil_amd import ops

    return ops


def _offsets(g, E, P):
    counts = np.bincount(g.integers(0, E, P), minlength=E)
    if E > 2:  # an empty expert in front
        counts[-1] += counts[0]
        counts[0] = 0
    counts[-1] += P - counts.sum()
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


def pauli_split_rows(x):
    """(rows, d, 8) blade order -> (rows, d, 2, 2, 2): [b][re / im][c] of the 2x2 matrix X[c][b]."""
    s, v1, v2, v3, b12, b13, b23, t = [x[..., i] for i in range(8)]
    m00 = (s + v3, t + b12)
    m10 = (v1 + b13, b23 + v2)
    m01 = (v1 - b13, b23 - v2)
    m11 = (s - v3, t - b12)
    col0 = np.stack([np.stack([m00[k], m10[k]], -1) for k in range(2)], -2)  # [k][c]
    col1 = np.stack([np.stack([m01[k], m11[k]], -1) for k in range(2)], -2)
    return np.stack([col0, col1], -3)


def test_pauli_rows_from_blade_f32_bit_exact():
    ops = _ops()
    g = np.random.default_rng(21)
    x = g.standard_normal((45, 7, 8), dtype=np.float32)
    say("pauli f32 rows from blade")
    got = ops.pauli_rows_from_blade_f32(torch.from_numpy(x).cuda()).cpu().numpy()
    assert got.shape == (45, 7, 2, 2, 2)
    assert np.array_equal(got, pauli_split_rows(x))


@pytest.mark.parametrize("act,d_in,d_out,E,P,N", [
    ("none", 8, 16, 3, 50, 40), ("gelu", 64, 256, 8, 512, 300), ("relu", 7, 5, 2, 33, 33),
    ("sigmoid", 9, 40, 5, 77, 60), ("gelu", 128, 512, 4, 700, 256), ("none", 256, 64, 2, 129, 64),
    ("gelu", 1, 33, 3, 17, 17),
    # enough tiles for the wide-tile kernel (32 tokens x 64 columns per workgroup)
    ("gelu", 8, 1024, 3, 2000, 1500), ("none", 5, 1100, 2, 1900, 700),
    # 32-token tiles on a small grid (they keep one workgroup per CU), ragged d_in and d_out
    ("relu", 9, 70, 7, 1500, 900)])
def test_pauli_f32_product(act, d_in, d_out, E, P, N):
    ops = _ops()
    g = np.random.default_rng(d_in * 5 + d_out + E)
    W = (g.standard_normal((E, d_out, d_in, 8), dtype=np.float32) / np.sqrt(8 * d_in)).astype(np.float32)
    b = (0.3 * g.standard_normal((E, d_out, 8))).astype(np.float32)
    x = g.standard_normal((N, d_in, 8), dtype=np.float32)
    gather = g.integers(0, N, P).astype(np.int32)
    offsets = _offsets(g, E, P)
    say(f"pauli f32 product act={act} d_in={d_in} d_out={d_out} E={E} P={P} N={N}")
    pw = ops.prepare_weights(torch.from_numpy(W).cuda(), "pauli_f32")
    pb = ops.prepare_bias(torch.from_numpy(b).cuda())
    xp = ops.pauli_rows_from_blade_f32(torch.from_numpy(x).cuda())
    off = torch.from_numpy(offsets).cuda()
    gt = torch.from_numpy(gather).cuda()
    y = ops.pauli_grouped_linear_f32(xp, pw, off, pb, act, gather=gt).cpu().numpy()
    for e in range(E):
        rows = slice(offsets[e], offsets[e + 1])
        if offsets[e] == offsets[e + 1]:
            continue
        ref = moe.ACTIVATIONS[act](moe.clifford_linear(x[gather[rows]], W[e], b[e]))
        assert normwise_err(y[rows], ref) < TOL_F32, e
    # the Pauli split-row output holds the same values in Pauli coordinates
    yp = ops.pauli_grouped_linear_f32(xp, pw, off, pb, act, gather=gt, y_layout="pauli").cpu().numpy()
    assert normwise_err(yp, pauli_split_rows(y)) < 1e-6


def test_pauli_f32_small_integer_product_is_exact():
    """Integer operands: every Pauli coordinate, product and partial sum is an exact fp32 value."""
    ops = _ops()
    g = np.random.default_rng(5)
    E, d_in, d_out, P = 2, 9, 6, 40
    W = g.integers(-3, 4, size=(E, d_out, d_in, 8)).astype(np.float32)
    x = g.integers(-3, 4, size=(P, d_in, 8)).astype(np.float32)
    offsets = np.array([0, 23, P], np.int32)
    say("pauli f32 integer product")
    y = ops.pauli_grouped_linear_f32(ops.pauli_rows_from_blade_f32(torch.from_numpy(x).cuda()),
                                     ops.prepare_weights(torch.from_numpy(W).cuda(), "pauli_f32"),
                                     torch.from_numpy(offsets).cuda()).cpu().numpy()
    for e in range(E):
        rows = slice(offsets[e], offsets[e + 1])
        assert np.array_equal(y[rows], moe.clifford_linear(x[rows], W[e], None))


def test_pauli_f32_rejects_bad_arguments():
    ops = _ops()
    L = ops.lib()
    assert L.ygg_pauli_grouped_linear_f32(None, None, 4, None, None, None, 65, 4, 4, 0, None, 1, None) == -1
    assert L.ygg_pauli_grouped_linear_f32(None, None, 4, None, None, None, 2, 4, 4, 0, None, 2, None) == -1
    assert L.ygg_pauli_rows_from_blade_f32(None, 3, 0, None, None) == -1
    with pytest.raises(ValueError):
        ops.pauli_grouped_linear_f32(torch.zeros(4, 3, 2, 2, 2, device="cuda"),
                                     ops.prepare_weights(torch.zeros(1, 4, 3, 8, device="cuda"), "f32"),
                                     torch.tensor([0, 4], device="cuda", dtype=torch.int32))


@pytest.mark.parametrize("name", ["small_gelu", "small_relu", "small_sigmoid", "c1_layer", "c1_head"])
def test_layer_pauli_f32_against_reference_golden(name):
    """The fp32 goldens with the expert products on fp32 Pauli weights (the fp32 default)."""
    from test_gpu_layer import _run_layer_case

    p, _, _ = load_case(name)
    assert not p.get("bf16")
    _run_layer_case(name, fmt_override="pauli_f32")


@pytest.mark.parametrize("N,k", [(96, 2), (96, 1), (96, 3), (180, 3)])
def test_layer_pauli_f32_large_down_splits(N, k):
    """F = 1024 over few rows: the down product splits its contraction over several partial planes,
    written at slot rows t k + s.  (96, 2): 8 planes, the two-slot combine; (96, 1), (96, 3): 13 and 6
    planes, the general plane combine; (180, 3): 4 planes, the half-multivector combine sorting three
    slots by expert."""
    import yggdrasil_amd

    g = np.random.default_rng(77 + N + k)
    d, F, E = 64, 1024, 4
    x = g.standard_normal((1, N, d, 8), dtype=np.float32)
    wu = (g.standard_normal((E, F, d, 8), dtype=np.float32) / np.sqrt(8 * d)).astype(np.float32)
    wd = (g.standard_normal((E, d, F, 8), dtype=np.float32) / np.sqrt(8 * F)).astype(np.float32)
    bu = (0.1 * g.standard_normal((E, F, 8))).astype(np.float32)
    bd = (0.1 * g.standard_normal((E, d, 8))).astype(np.float32)
    logits_np = g.standard_normal((N, E), dtype=np.float32)
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, router="logits")
    assert cfg.weight_format == "pauli_f32"
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    say(f"layer pauli_f32 N={N} d={d} F={F} E={E} k={k}")
    xt = torch.from_numpy(x).cuda()
    out = layer.moe_forward(xt, logits=torch.from_numpy(logits_np).cuda(), residual=xt)
    out = out.detach().cpu().numpy().reshape(N, d, 8)
    idx = layer.last_routing["topk_idx"].cpu().numpy()
    idx_o, w = moe.route_topk(moe.softmax(logits_np), k)
    assert np.array_equal(idx, idx_o)
    ref = moe_reference(x[0], idx, w, wu, bu, wd, bd, "gelu", base=x[0])
    assert normwise_err(out, ref) < TOL_F32


@pytest.mark.parametrize("N,E,k,d", [(256, 8, 2, 16), (1, 4, 1, 16), (77, 32, 4, 16), (256, 32, 8, 16),
                                     (200, 16, 3, 16), (257, 8, 2, 16), (33, 1, 1, 5), (96, 8, 2, 64)])
def test_layer_pauli_f32_routed_up_product(N, E, k, d):
    """Batches of at most 256 tokens with logits route inside the fp32 up product (no routing launch)
    and stage x's rows in LDS: the routing arrays equal ygg_route's bit for bit, and the layer matches
    the float64 oracle.  (257, 8, 2) takes the routing launch instead, for contrast; (200, 16, 3) leaves
    some experts without tokens (logits shifted away from them); rows 2 and 3 hold ties; (96, 8, 2, 64)
    stages rows of the largest routed width and has a NaN logit in token 5 (its routing still equals
    ygg_route's; its output is left out of the comparison)."""
    ops = _ops()
    g = np.random.default_rng(1000 + N + E + k + d)
    F = 48
    x = g.standard_normal((N, d, 8), dtype=np.float32)
    wu = (g.standard_normal((E, F, d, 8), dtype=np.float32) / np.sqrt(8 * d)).astype(np.float32)
    wd = (g.standard_normal((E, d, F, 8), dtype=np.float32) / np.sqrt(8 * F)).astype(np.float32)
    bu = (0.1 * g.standard_normal((E, F, 8))).astype(np.float32)
    bd = (0.1 * g.standard_normal((E, d, 8))).astype(np.float32)
    logits_np = g.standard_normal((N, E), dtype=np.float32)
    if N > 3:
        logits_np[3, :] = 0.25  # a row of ties: the lowest indices win
        logits_np[2, 1::2] = logits_np[2, 0]  # ties with the row's first logit
    if N == 200:
        logits_np[:, [1, 5, 6]] -= 40.0  # experts 1, 5, 6 are never chosen
    keep = np.ones(N, dtype=bool)
    if d == 64:
        logits_np[5, 2] = np.nan
        keep[5] = False
    say(f"routed fp32 up product N={N} E={E} k={k} d={d}")
    xt, lt = torch.from_numpy(x).cuda(), torch.from_numpy(logits_np).cuda()
    pu = ops.prepare_weights(torch.from_numpy(wu).cuda(), "pauli_f32")
    pd = ops.prepare_weights(torch.from_numpy(wd).cuda(), "pauli_f32")
    out, r = ops.moe_forward(xt, k, pu, pd, b_up=ops.prepare_bias(torch.from_numpy(bu).cuda()),
                             b_down=ops.prepare_bias(torch.from_numpy(bd).cuda()), act="gelu", logits=lt)
    rr = ops.route(lt, k)
    torch.cuda.synchronize()
    for key in ("topk_idx", "topk_w", "counts", "offsets"):
        a, b = r[key].cpu().numpy(), getattr(rr, key).cpu().numpy()
        assert np.array_equal(a.view(np.int32), b.view(np.int32)), key
    if N == 200:
        assert (r["counts"].cpu().numpy()[[1, 5, 6]] == 0).all()
    idx, w = r["topk_idx"].cpu().numpy(), r["topk_w"].cpu().numpy()
    ref = moe_reference(x, idx, w, wu, bu, wd, bd, "gelu")
    assert normwise_err(out.cpu().numpy()[keep], ref[keep]) < TOL_F32
