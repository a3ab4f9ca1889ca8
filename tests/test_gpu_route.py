"""GPU parity: routing (softmax / top-k / counting sort), dispatch and combine.

Integer outputs (indices, counts, offsets, permutation, slot rows) must be
bit-exact against the reference goldens and the oracle; the combine must be
bit-exact given the same routing weights (same order, no fused multiply-add).
"""

import numpy as np
import pytest
import torch

from _fixtures import load_case
from _gpu_helpers import normwise_err, say
from oracle import moe

pytestmark = pytest.mark.gpu


def _ops():
    from yggdrasil_amd import ops

    return ops


def _check_route(logits_np, k, E, tag):
    ops = _ops()
    say(f"route {tag} N={logits_np.shape[0]} E={E} k={k}")
    r = ops.route(torch.from_numpy(logits_np).cuda(), k)
    torch.cuda.synchronize()
    probs = moe.softmax(logits_np)
    idx_o, w_o = moe.route_topk(probs, k)
    counts_o, offsets_o, perm_o, slot_o = moe.dispatch_plan(idx_o, E)
    assert np.array_equal(r.topk_idx.cpu().numpy(), idx_o)
    assert np.array_equal(r.counts.cpu().numpy(), counts_o)
    assert np.array_equal(r.offsets.cpu().numpy(), offsets_o)
    assert np.array_equal(r.perm.cpu().numpy(), perm_o)
    assert np.array_equal(r.slot_pos.cpu().numpy(), slot_o)
    w = r.topk_w.cpu().numpy()
    assert np.allclose(w, w_o, rtol=2e-6, atol=1e-7)
    return r


def test_route_dispatch_combine_against_reference_golden():
    ops = _ops()
    p, inp, ref = load_case("c2_route")
    r = _check_route(inp["logits"], p["k"], p["E"], "c2 golden")
    # reference selection, reversed to the build's descending order
    assert np.array_equal(r.topk_idx.cpu().numpy(), ref["idx"][:, ::-1])
    assert np.array_equal(r.counts.cpu().numpy(), ref["counts"])
    assert np.array_equal(r.perm.cpu().numpy(), ref["perm"])
    assert np.allclose(r.topk_w.cpu().numpy(), ref["w"][:, ::-1], rtol=2e-6, atol=1e-7)
    x = torch.from_numpy(inp["x"]).cuda()
    say("dispatch c2 golden")
    xs = ops.dispatch(x, r)
    assert np.array_equal(xs.cpu().numpy(), inp["x"][ref["perm"]])
    xm = ops.dispatch(x, r, mask_order=True)
    assert np.array_equal(xm.cpu().numpy(), inp["x"][ref["perm"]][..., [0, 1, 2, 4, 3, 5, 6, 7]])
    say("combine c2 golden (identity experts)")
    out = ops.combine(xs, r).cpu().numpy()
    assert normwise_err(out, ref["out"]) < 1e-6
    # bit-exact against the oracle's combine given the GPU's own weights
    o2 = moe.combine(inp["x"][ref["perm"]], r.topk_idx.cpu().numpy(), r.topk_w.cpu().numpy(),
                     r.slot_pos.cpu().numpy())
    assert np.array_equal(out, o2)
    out_m = ops.combine(xm, r, y_mask_order=True).cpu().numpy()
    assert np.array_equal(out_m, out)


@pytest.mark.parametrize("N,E,k,seed", [(1, 4, 1, 0), (255, 8, 2, 1), (257, 16, 4, 2), (1000, 64, 8, 3),
                                        (16384, 16, 2, 4), (8192, 32, 4, 5), (4096, 64, 2, 6),
                                        # either side of the one-workgroup path's limit (1024 tokens)
                                        (64, 32, 2, 7), (1024, 64, 8, 8), (1025, 33, 3, 9)])
def test_route_random_sizes(N, E, k, seed):
    r = np.random.default_rng(seed)
    _check_route(r.standard_normal((N, E), dtype=np.float32), k, E, f"random seed={seed}")


@pytest.mark.parametrize("E,k", [(4, 2), (16, 2), (32, 4), (64, 8)])
def test_route_ties_lowest_index_wins(E, k):
    r = np.random.default_rng(E + k)
    logits = r.integers(0, 3, size=(700, E)).astype(np.float32)  # exact ties everywhere
    _check_route(logits, k, E, f"ties E={E} k={k}")


@pytest.mark.parametrize("E,k", [(1, 1), (3, 2), (5, 5), (7, 3), (9, 4), (12, 2), (20, 6), (33, 8), (63, 2)])
def test_route_expert_counts_off_the_lane_grid(E, k):
    """E below 8 and E not a multiple of 8 take the other branches of the pairwise row sum."""
    r = np.random.default_rng(100 + E * 8 + k)
    _check_route(r.standard_normal((613, E), dtype=np.float32) * 3, k, E, f"E={E} k={k}")


def test_route_nan_rows_stay_in_range():
    """NaN logits leave the weights unspecified but every slot still names a distinct valid expert."""
    ops = _ops()
    r = np.random.default_rng(77)
    N, E, k = 300, 24, 4
    logits = r.standard_normal((N, E), dtype=np.float32)
    logits[::7, 3] = np.nan
    logits[::11] = np.nan
    say("route NaN rows")
    rt = ops.route(torch.from_numpy(logits).cuda(), k)
    idx = rt.topk_idx.cpu().numpy()
    assert idx.min() >= 0 and idx.max() < E
    assert all(len(set(row)) == k for row in idx)
    assert rt.counts.cpu().numpy().sum() == N * k
    perm = rt.perm.cpu().numpy()
    assert np.array_equal(np.sort(perm), np.repeat(np.arange(N), k))
    clean = ~np.isnan(logits).any(axis=1)
    idx_o, _ = moe.route_topk(moe.softmax(logits[clean]), k)
    assert np.array_equal(idx[clean], idx_o)


def test_route_zipf_skew_and_empty_experts():
    r = np.random.default_rng(9)
    N, E, k = 3000, 32, 4
    logits = np.full((N, E), -30.0, np.float32)
    logits[:, :4] = r.standard_normal((N, 4), dtype=np.float32)  # only experts 0..3 ever chosen
    rt = _check_route(logits, k, E, "empty experts")
    c = rt.counts.cpu().numpy()
    assert c[4:].sum() == 0 and c[:4].sum() == N * k


def test_full_c2_route_dispatch_combine():
    """BASELINE C2: N=16384, E=16, k=2, d=128 fp32; identity expert."""
    ops = _ops()
    g = np.random.default_rng(2024)
    N, E, k, d = 16384, 16, 2, 128
    logits = g.standard_normal((N, E), dtype=np.float32)
    x = g.standard_normal((N, d, 8), dtype=np.float32)
    r = _check_route(logits, k, E, "C2 full")
    xt = torch.from_numpy(x).cuda()
    say("dispatch C2 full")
    xs = ops.dispatch(xt, r)
    perm = r.perm.cpu().numpy()
    assert np.array_equal(xs.cpu().numpy(), x[perm])
    say("combine C2 full")
    out = ops.combine(xs, r).cpu().numpy()
    o2 = moe.combine(x[perm], r.topk_idx.cpu().numpy(), r.topk_w.cpu().numpy(), r.slot_pos.cpu().numpy())
    assert np.array_equal(out, o2)
    # identity experts with renormalised weights return the token itself
    assert normwise_err(out, x) < 1e-6


def test_combine_residual_and_bf16():
    ops = _ops()
    g = np.random.default_rng(5)
    N, E, k, d = 300, 8, 3, 16
    r = ops.route(torch.from_numpy(g.standard_normal((N, E), dtype=np.float32)).cuda(), k)
    y = torch.from_numpy(g.standard_normal((N * k, d, 8), dtype=np.float32)).cuda()
    res = torch.from_numpy(g.standard_normal((N, d, 8), dtype=np.float32)).cuda()
    say("combine residual fp32")
    out = ops.combine(y, r, residual=res).cpu().numpy()
    ref = moe.combine(y.cpu().numpy(), r.topk_idx.cpu().numpy(), r.topk_w.cpu().numpy(), r.slot_pos.cpu().numpy())
    assert np.array_equal(out, (res.cpu().numpy() + ref).astype(np.float32))
    say("combine bf16")
    outb = ops.combine(y.bfloat16(), r).float().cpu().numpy()
    refb = moe.combine(y.bfloat16().float().cpu().numpy(), r.topk_idx.cpu().numpy(), r.topk_w.cpu().numpy(),
                       r.slot_pos.cpu().numpy())
    assert normwise_err(outb, refb) < 8e-3


@pytest.mark.parametrize("k", [1, 2, 3, 4, 5, 8])
def test_combine_slot_order_every_k(k):
    """The combine puts a token's slots in ascending expert order by a sorting network for 2, 4
    or 8 slots: fp32 rows bit-exact against the oracle's order for every slot bound, bf16 rows
    within bf16 rounding."""
    ops = _ops()
    g = np.random.default_rng(40 + k)
    N, E, d = 300, 16, 16
    r = ops.route(torch.from_numpy(g.standard_normal((N, E), dtype=np.float32) * 3).cuda(), k)
    y = torch.from_numpy(g.standard_normal((N * k, d, 8), dtype=np.float32)).cuda()
    say(f"combine slot order k={k}")
    idx, w, sp = r.topk_idx.cpu().numpy(), r.topk_w.cpu().numpy(), r.slot_pos.cpu().numpy()
    out = ops.combine(y, r).cpu().numpy()
    assert np.array_equal(out, moe.combine(y.cpu().numpy(), idx, w, sp))
    outb = ops.combine(y.bfloat16(), r).float().cpu().numpy()
    refb = moe.combine(y.bfloat16().float().cpu().numpy(), idx, w, sp)
    assert normwise_err(outb, refb) < 8e-3


def test_route_rejects_bad_arguments():
    ops = _ops()
    from yggdrasil_amd._native import NativeLibraryError

    with pytest.raises(NativeLibraryError):
        ops.route(torch.zeros((4, 65), device="cuda"), 2)  # E > 64
    with pytest.raises(NativeLibraryError):
        ops.route(torch.zeros((4, 8), device="cuda"), 9)  # k > 8


def test_route_dispatch_combine_reuse_out_buffers():
    """out= / workspace= buffers are filled in place and give the same results as fresh ones."""
    ops = _ops()
    r = np.random.default_rng(31)
    N, E, k, d = 300, 16, 2, 5
    logits = torch.from_numpy(r.standard_normal((N, E), dtype=np.float32)).cuda()
    x = torch.from_numpy(r.standard_normal((N, d, 8), dtype=np.float32)).cuda()
    say("route/dispatch/combine out= buffers")
    fresh = ops.route(logits, k)
    xs_f = ops.dispatch(x, fresh)
    out_f = ops.combine(xs_f, fresh)
    reuse = ops.route(torch.zeros_like(logits), k)  # filled with other values first
    ws = torch.empty(ops.lib().ygg_route_workspace_bytes(N, E, k), device="cuda", dtype=torch.uint8)
    xs = torch.full_like(xs_f, 7.0)
    out = torch.full_like(out_f, 7.0)
    got = ops.route(logits, k, out=reuse, workspace=ws)
    assert got is reuse
    assert ops.dispatch(x, got, out=xs) is xs
    assert ops.combine(xs, got, out=out) is out
    for a, b in [(got.topk_idx, fresh.topk_idx), (got.perm, fresh.perm), (got.slot_pos, fresh.slot_pos),
                 (got.counts, fresh.counts), (got.offsets, fresh.offsets), (xs, xs_f), (out, out_f)]:
        assert torch.equal(a, b)
    with pytest.raises(ValueError):
        ops.dispatch(x, got, out=torch.empty(N, d, 8, device="cuda"))


@pytest.mark.parametrize("N,d,E,k,dtype", [(256, 64, 8, 2, "f32"), (1024, 16, 64, 8, "f32"), (37, 9, 5, 3, "bf16"),
                                           (1500, 32, 16, 2, "f32"), (700, 128, 32, 4, "bf16")])
def test_route_energy_fused_against_oracle(N, d, E, k, dtype):
    """CliffordRouter.forward in one call: indices exact, weights to 1e-5 against the oracle's
    energy logits; up to 1024 tokens the logits are computed inside the routing kernel."""
    ops = _ops()
    r = np.random.default_rng(N + d + E)
    x = r.standard_normal((N, d, 8), dtype=np.float32) * r.uniform(0.2, 3.0, size=(1, 1, 8)).astype(np.float32)
    rw = (0.5 * r.standard_normal((E, 4))).astype(np.float32)
    rb = (0.1 * r.standard_normal(E)).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    if dtype == "bf16":
        xt = xt.bfloat16()
        x = xt.float().cpu().numpy()
    say(f"route_energy N={N} d={d} E={E} k={k} {dtype}")
    got = ops.route_energy(xt, torch.from_numpy(rw).cuda(), torch.from_numpy(rb).cuda(), k)
    logits, _ = moe.router_logits(x, rw, rb)
    idx_o, w_o = moe.route_topk(moe.softmax(logits), k)
    assert np.array_equal(got.topk_idx.cpu().numpy(), idx_o)
    assert np.allclose(got.topk_w.cpu().numpy(), w_o, rtol=1e-5, atol=1e-7)
    # the counting sort matches the one run on the oracle's logits through ygg_route
    ref = ops.route(torch.from_numpy(logits.astype(np.float32)).cuda(), k)
    for a, b in [(got.perm, ref.perm), (got.slot_pos, ref.slot_pos), (got.counts, ref.counts),
                 (got.offsets, ref.offsets)]:
        assert torch.equal(a, b)


@pytest.mark.parametrize("N,d,E,dtype", [(256, 64, 8, "f32"), (33, 7, 5, "f32"), (100, 16, 64, "bf16"),
                                         (3000, 32, 16, "f32"), (5, 130, 70, "f32"), (61, 128, 32, "bf16")])
def test_router_head_logits_bit_exact(N, d, E, dtype):
    """The CliffordLinear(d -> E) head's scalar part in the reference's fp32 order, bit for bit."""
    ops = _ops()
    g = np.random.default_rng(N + d + E)
    x = g.standard_normal((N, d, 8), dtype=np.float32)
    W = (g.standard_normal((E, d, 8)) / np.sqrt(8 * d)).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    if dtype == "bf16":
        xt = xt.bfloat16()
        x = xt.float().cpu().numpy()
    say(f"router head logits N={N} d={d} E={E} {dtype}")
    got = ops.router_head_logits(xt, torch.from_numpy(W).cuda()).cpu().numpy()
    assert np.array_equal(got, moe.clifford_linear(x, W, None)[..., 0])


@pytest.mark.parametrize("N,d,E,k,dtype", [(8192, 128, 32, 4, torch.bfloat16), (4096, 256, 64, 2, torch.bfloat16),
                                           (1500, 40, 16, 2, torch.float32), (700, 64, 8, 2, torch.bfloat16),
                                           (1030, 6, 5, 3, torch.float32)])
def test_route_pauli_rows_equals_route_and_conversion(N, d, E, k, dtype):
    """The layer's first launches -- the routing with the conversion of x to Pauli rows split over
    both of its launches (one launch up to 1024 tokens) -- give ygg_route's routing and
    ygg_pauli_rows_from_blade(_f32)'s rows bit for bit, and the routing matches the oracle."""
    ops = _ops()
    g = np.random.default_rng(N + d + E)
    logits = g.standard_normal((N, E), dtype=np.float32)
    x = torch.from_numpy(g.standard_normal((N, d, 8), dtype=np.float32)).cuda().to(dtype)
    lt = torch.from_numpy(logits).cuda()
    say(f"route_pauli_rows N={N} d={d} E={E} k={k} {dtype}")
    r, xp = ops.route_pauli_rows(lt, k, x)
    r0 = ops.route(lt, k)
    want = ops.pauli_rows_from_blade(x) if dtype == torch.bfloat16 else ops.pauli_rows_from_blade_f32(x)
    torch.cuda.synchronize()
    for key in ("topk_idx", "topk_w", "counts", "offsets", "perm", "slot_pos"):
        assert torch.equal(getattr(r, key), getattr(r0, key)), key
    assert torch.equal(xp.reshape(-1), want.reshape(-1))
    idx_o, _ = moe.route_topk(moe.softmax(logits), k)
    assert np.array_equal(r.topk_idx.cpu().numpy(), idx_o)
