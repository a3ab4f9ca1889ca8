"""GPU parity: the expert-FFN backward (fp32) against the finite-difference-pinned oracle.

Every gradient is compared with ``oracle/backward.py`` on the same routing at
the fp32 bound (1e-5 normwise; 3e-5 where two products and the activation's
derivative compose).  The adjoint weights are exact (a sign flip and a
transpose).
"""

import numpy as np
import pytest
import torch

from _gpu_helpers import TOL_F32, normwise_err, say
from oracle import backward as bw
from oracle import moe
from oracle.cl3 import reverse

pytestmark = pytest.mark.gpu

TOL_BW = 3e-5


def _ops():
    from yggdrasil_amd import ops

    return ops


def _offsets(g, E, P):
    counts = np.bincount(g.integers(0, E, P), minlength=E)
    if E > 2:
        counts[-1] += counts[0]
        counts[0] = 0
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


def test_adjoint_weights_exact():
    ops = _ops()
    g = np.random.default_rng(0)
    W = g.standard_normal((3, 5, 7, 8)).astype(np.float32)
    say("adjoint weights")
    got = ops.adjoint_weights(torch.from_numpy(W).cuda()).cpu().numpy()
    assert np.array_equal(got, np.transpose(reverse(W), (0, 2, 1, 3)))


@pytest.mark.parametrize("act", ["gelu", "sigmoid", "relu", "none"])
def test_activation_backward(act):
    ops = _ops()
    g = np.random.default_rng(1)
    h = (1.5 * g.standard_normal((3000, 8))).astype(np.float32)
    h[:10, 1:4] = 0.0  # zero vector part: the magnitude's eps regime
    gr = g.standard_normal((3000, 8)).astype(np.float32)
    say(f"activation backward {act}")
    got = ops.activation_backward(torch.from_numpy(h).cuda(), torch.from_numpy(gr).cuda(), act).cpu().numpy()
    assert normwise_err(got, bw.activation_backward(act, h, gr)) < TOL_F32


@pytest.mark.parametrize("E,d_in,d_out,P,gathered", [(3, 8, 16, 50, False), (4, 64, 128, 700, True),
                                                     (2, 7, 33, 129, True), (5, 40, 9, 300, False)])
def test_grouped_weight_grad(E, d_in, d_out, P, gathered):
    ops = _ops()
    g = np.random.default_rng(E * 10 + d_in)
    dy = g.standard_normal((P, d_out, 8)).astype(np.float32)
    nsrc = P + 17
    a = g.standard_normal((nsrc if gathered else P, d_in, 8)).astype(np.float32)
    gather = g.integers(0, nsrc, P).astype(np.int32) if gathered else None
    offsets = _offsets(g, E, P)
    say(f"weight grad E={E} d_in={d_in} d_out={d_out} P={P} gathered={gathered}")
    dW, db = ops.grouped_weight_grad(torch.from_numpy(dy).cuda(), torch.from_numpy(a).cuda(),
                                     torch.from_numpy(offsets).cuda(), E,
                                     gather=torch.from_numpy(gather).cuda() if gathered else None)
    dW, db = dW.cpu().numpy(), db.cpu().numpy()
    rows_a = a[gather] if gathered else a
    for e in range(E):
        sl = slice(offsets[e], offsets[e + 1])
        if offsets[e] == offsets[e + 1]:
            assert not dW[e].any() and not db[e].any()
            continue
        _, dW_o, db_o = bw.clifford_linear_backward(rows_a[sl], np.zeros((d_out, d_in, 8), np.float32), dy[sl])
        assert normwise_err(dW[e], dW_o) < TOL_F32, e
        assert normwise_err(db[e], db_o) < TOL_F32, e


@pytest.mark.parametrize("E,d_in,d_out,P,gathered", [(3, 8, 16, 50, False), (2, 40, 70, 2300, True),
                                                     (4, 64, 128, 700, True), (1, 7, 33, 1029, False),
                                                     (5, 16, 9, 3000, True)])
def test_grouped_weight_grad_pauli(E, d_in, d_out, P, gathered):
    """The MFMA weight gradient from Pauli rows: per-chunk partial sums (384 rows) added in order."""
    ops = _ops()
    g = np.random.default_rng(E * 7 + d_in + P)
    dy = g.standard_normal((P, d_out, 8)).astype(np.float32)
    nsrc = P + 17
    a = g.standard_normal((nsrc if gathered else P, d_in, 8)).astype(np.float32)
    gather = g.integers(0, nsrc, P).astype(np.int32) if gathered else None
    offsets = _offsets(g, E, P)
    say(f"weight grad (MFMA) E={E} d_in={d_in} d_out={d_out} P={P} gathered={gathered}")
    dyp = ops.pauli_rows_from_blade_f32(torch.from_numpy(dy).cuda())
    ap = ops.pauli_rows_from_blade_f32(torch.from_numpy(a).cuda())
    dW, db = ops.grouped_weight_grad_pauli(dyp, ap, torch.from_numpy(offsets).cuda(), E,
                                           gather=torch.from_numpy(gather).cuda() if gathered else None)
    dW, db = dW.cpu().numpy(), db.cpu().numpy()
    rows_a = a[gather] if gathered else a
    for e in range(E):
        sl = slice(offsets[e], offsets[e + 1])
        if offsets[e] == offsets[e + 1]:
            assert not dW[e].any() and not db[e].any()
            continue
        _, dW_o, db_o = bw.clifford_linear_backward(rows_a[sl], np.zeros((d_out, d_in, 8), np.float32), dy[sl])
        assert normwise_err(dW[e], dW_o) < TOL_F32, e
        assert normwise_err(db[e], db_o) < TOL_F32, e


def _layer_case(g, N, d, F, E, k, act, router):
    import yggdrasil_amd

    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, activation=act, router=router)
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    wu = (g.standard_normal((E, F, d, 8)) / np.sqrt(8 * d)).astype(np.float32)
    wd = (g.standard_normal((E, d, F, 8)) / np.sqrt(8 * F)).astype(np.float32)
    bu = (0.1 * g.standard_normal((E, F, 8))).astype(np.float32)
    bd = (0.1 * g.standard_normal((E, d, 8))).astype(np.float32)
    rw = g.standard_normal((E, 4)).astype(np.float32)
    layer.load_reference_weights(router_weight=rw, router_bias=np.zeros(E, np.float32), w_up=wu, b_up=bu,
                                 w_down=wd, b_down=bd)
    return layer, [(wu[e], bu[e], wd[e], bd[e]) for e in range(E)]


@pytest.mark.parametrize("N,d,F,E,k,act,router,residual", [
    (64, 16, 32, 4, 2, "gelu", "logits", False),
    (300, 32, 64, 8, 2, "sigmoid", "energy", True),
    (130, 8, 24, 5, 3, "relu", "logits", True),
    (1200, 16, 32, 8, 2, "gelu", "energy", False),
    (2600, 8, 24, 2, 2, "gelu", "logits", True),  # 2600 rows per expert: the weight gradient's row chunks
    # d_model > d_ff with the MFMA weight gradient (512 rows per expert): the down product's
    # partial sums (d-wide bias planes) are the larger use of the shared workspace region
    (1024, 32, 16, 4, 2, "gelu", "logits", False),
])
def test_layer_autograd_against_oracle(N, d, F, E, k, act, router, residual):
    g = np.random.default_rng(N + d + F)
    layer, experts = _layer_case(g, N, d, F, E, k, act, router)
    x = g.standard_normal((1, N, d, 8)).astype(np.float32)
    c = g.standard_normal((1, N, d, 8)).astype(np.float32)
    logits = g.standard_normal((N, E)).astype(np.float32) if router == "logits" else None
    xt = torch.from_numpy(x).cuda().requires_grad_(True)
    say(f"layer autograd N={N} d={d} F={F} E={E} k={k} {act} {router} residual={residual}")
    out = layer.moe_forward(xt, logits=torch.from_numpy(logits).cuda() if logits is not None else None,
                            residual=xt if residual else None)
    out.backward(torch.from_numpy(c).cuda())
    torch.cuda.synchronize()
    idx = layer.last_routing["topk_idx"].cpu().numpy()
    w = layer.last_routing["topk_w"].cpu().numpy()
    dx_o, grads, _ = bw.moe_backward_reference(x[0], idx, w, experts, c[0], act, residual)
    assert normwise_err(xt.grad.cpu().numpy()[0], dx_o) < TOL_BW
    for name, j in (("w_up", 0), ("b_up", 1), ("w_down", 2), ("b_down", 3)):
        got = getattr(layer, name).grad.cpu().numpy()
        want = np.stack([gr[j] for gr in grads])
        assert normwise_err(got, want) < TOL_BW, name
    assert layer.router_weight.grad is None


def test_moe_backward_routing_weight_gradient():
    """dtopk_w = <dout_t, y_slot>: the gradient a caller chains into its own router."""
    ops = _ops()
    g = np.random.default_rng(9)
    N, d, F, E, k = 200, 16, 48, 6, 2
    layer, experts = _layer_case(g, N, d, F, E, k, "gelu", "logits")
    x = g.standard_normal((N, d, 8)).astype(np.float32)
    c = g.standard_normal((N, d, 8)).astype(np.float32)
    logits = g.standard_normal((N, E)).astype(np.float32)
    prep, adj = layer._get_prepared(), layer._get_adjoint()
    xt, ct, lt = (torch.from_numpy(a).cuda() for a in (x, c, logits))
    say("moe backward dtopk_w")
    dx, dWu, dbu, dWd, dbd, dtw = ops.moe_backward(xt, k, prep["w_up"], adj["w_up"], prep["w_down"], adj["w_down"],
                                                   ct, prep["b_up"], prep["b_down"], "gelu", logits=lt)
    r = ops.route(lt, k)
    idx, w = r.topk_idx.cpu().numpy(), r.topk_w.cpu().numpy()
    dx_o, grads, dw_o = bw.moe_backward_reference(x, idx, w, experts, c, "gelu")
    assert normwise_err(dtw.cpu().numpy(), dw_o) < TOL_BW
    assert normwise_err(dx.cpu().numpy(), dx_o) < TOL_BW
    # the forward it differentiates: out = sum_s w y, so <dout, out> = sum dw * w
    out, _ = ops.moe_forward(xt, k, prep["w_up"], prep["w_down"], prep["b_up"], prep["b_down"], "gelu", logits=lt)
    assert abs(float((out * ct).sum()) - float((dtw * r.topk_w).sum())) < 1e-3 * float((out * ct).abs().sum())


def test_forward_train_keeps_what_the_backward_would_recompute():
    """moe_forward_train's output is moe_forward's, and a backward given its h_pre equals the
    recomputing backward bit for bit."""
    ops = _ops()
    g = np.random.default_rng(10)
    N, d, F, E, k = 300, 16, 40, 6, 2
    layer, _ = _layer_case(g, N, d, F, E, k, "gelu", "logits")
    prep, adj = layer._get_prepared(), layer._get_adjoint()
    xt = torch.from_numpy(g.standard_normal((N, d, 8)).astype(np.float32)).cuda()
    ct = torch.from_numpy(g.standard_normal((N, d, 8)).astype(np.float32)).cuda()
    lt = torch.from_numpy(g.standard_normal((N, E)).astype(np.float32)).cuda()
    say("forward_train h_pre")
    args = (xt, k, prep["w_up"], prep["w_down"], prep["b_up"], prep["b_down"], "gelu")
    out, rt, h_pre = ops.moe_forward_train(*args, logits=lt)
    ref, rt2 = ops.moe_forward(*args, logits=lt)
    assert torch.equal(out, ref) and torch.equal(rt["topk_idx"], rt2["topk_idx"])
    bargs = (xt, k, prep["w_up"], adj["w_up"], prep["w_down"], adj["w_down"], ct, prep["b_up"], prep["b_down"], "gelu")
    g1 = ops.moe_backward(*bargs, logits=lt, h_pre=h_pre)
    g2 = ops.moe_backward(*bargs, logits=lt)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)
