"""GPU parity: the pre-norm (CliffordLayerNorm) and the FFN half of HLMBlock.forward.

The norm follows NumPy's reduction order and IEEE divide / square root with no
multiply-add contraction, so fp32 outputs are compared bit for bit with the
oracle; bf16 outputs are the oracle's fp32 values rounded to nearest even,
also bit for bit.  The whole sub-layer ``x + moe(ffn_norm(x))`` is compared
with the oracle at the layer bounds (1e-5 fp32, 2e-2 bf16, normwise).
"""

import numpy as np
import pytest
import torch

from _gpu_helpers import TOL_BF16, TOL_F32, bf16_round, normwise_err, say
from oracle import moe
from oracle.norm import block_ffn_reference, clifford_layer_norm

pytestmark = pytest.mark.gpu


def _ops():
    from yggdrasil_amd import ops

    return ops


def _params(g, d, default=False):
    gamma = np.zeros((d, 8), np.float32)
    gamma[:, 0] = 1.0
    beta = np.zeros((d, 8), np.float32)
    if not default:
        gamma = (gamma + 0.5 * g.standard_normal((d, 8))).astype(np.float32)
        beta = (0.2 * g.standard_normal((d, 8))).astype(np.float32)
    return gamma, beta


@pytest.mark.parametrize("N,d,default", [(1, 1, False), (5, 7, False), (64, 64, True), (300, 128, False),
                                         (33, 129, False), (17, 300, False), (9, 1000, False), (3, 4096, False),
                                         (4099, 32, False)])
def test_layer_norm_f32_bit_exact(N, d, default):
    ops = _ops()
    g = np.random.default_rng(N * 7 + d)
    x = (g.standard_normal((N, d, 8)) * g.uniform(0.05, 20.0, (N, 1, 1))).astype(np.float32)
    gamma, beta = _params(g, d, default)
    say(f"layer norm f32 N={N} d={d}")
    got = ops.clifford_layer_norm(torch.from_numpy(x).cuda(), torch.from_numpy(gamma).cuda(),
                                  torch.from_numpy(beta).cuda()).cpu().numpy()
    assert np.array_equal(got, clifford_layer_norm(x, gamma, beta))


@pytest.mark.parametrize("N,d", [(40, 64), (7, 300)])
def test_layer_norm_bf16_bit_exact(N, d):
    ops = _ops()
    g = np.random.default_rng(N + d)
    x = bf16_round(g.standard_normal((N, d, 8)).astype(np.float32))
    gamma, beta = _params(g, d)
    ref = clifford_layer_norm(x, gamma, beta)
    xt = torch.from_numpy(x).cuda().bfloat16()
    gt, bt = torch.from_numpy(gamma).cuda(), torch.from_numpy(beta).cuda()
    say(f"layer norm bf16 N={N} d={d}")
    y32 = ops.clifford_layer_norm(xt, gt, bt, out_dtype=torch.float32).cpu().numpy()
    assert np.array_equal(y32, ref)
    y16 = ops.clifford_layer_norm(xt, gt, bt).float().cpu().numpy()
    assert np.array_equal(y16, bf16_round(ref))


def test_layer_norm_eps_and_batch_shape():
    """A (B, T, d, 8) batch, a non-default eps, and tiny inputs where eps matters."""
    ops = _ops()
    g = np.random.default_rng(9)
    x = (1e-4 * g.standard_normal((2, 3, 16, 8))).astype(np.float32)
    gamma, beta = _params(g, 16)
    say("layer norm eps batch")
    for eps in (1e-6, 1e-3, 0.0):
        got = ops.clifford_layer_norm(torch.from_numpy(x).cuda(), torch.from_numpy(gamma).cuda(),
                                      torch.from_numpy(beta).cuda(), eps=eps).cpu().numpy()
        assert got.shape == x.shape
        assert np.array_equal(got, clifford_layer_norm(x, gamma, beta, eps)), eps


def test_layer_norm_rejects_bad_arguments():
    ops = _ops()
    x = torch.zeros(4, 8, 8, device="cuda")
    with pytest.raises(ValueError):
        ops.clifford_layer_norm(x, torch.zeros(7, 8, device="cuda"), torch.zeros(8, 8, device="cuda"))
    with pytest.raises(RuntimeError):
        ops.clifford_layer_norm(x, torch.zeros(8, 8, device="cuda"), torch.zeros(8, 8, device="cuda"), eps=-1.0)
    big = torch.zeros(1, 4097, 8, device="cuda")
    with pytest.raises(RuntimeError):
        ops.clifford_layer_norm(big, torch.zeros(4097, 8, device="cuda"), torch.zeros(4097, 8, device="cuda"))


def _experts(g, E, d, F):
    wu = (g.standard_normal((E, F, d, 8)) / np.sqrt(8 * d)).astype(np.float32)
    wd = (g.standard_normal((E, d, F, 8)) / np.sqrt(8 * F)).astype(np.float32)
    bu = (0.1 * g.standard_normal((E, F, 8))).astype(np.float32)
    bd = (0.1 * g.standard_normal((E, d, 8))).astype(np.float32)
    return wu, bu, wd, bd


@pytest.mark.parametrize("N,d,F,E,k,dtype,fmt,router", [
    (48, 16, 32, 4, 2, "f32", "pauli_f32", "energy"),
    (300, 64, 256, 8, 2, "f32", "f32", "energy"),
    (1500, 32, 64, 8, 2, "f32", "pauli_f32", "energy"),
    (256, 64, 128, 8, 2, "bf16", "pauli", "logits"),
    (200, 32, 64, 16, 4, "bf16", "bf16", "logits"),
    (64, 128, 512, 32, 2, "bf16", "int8", "logits"),
])
def test_block_ffn_against_oracle(N, d, F, E, k, dtype, fmt, router):
    import yggdrasil_amd

    g = np.random.default_rng(N + d + F + E)
    x = g.standard_normal((1, N, d, 8)).astype(np.float32)
    if dtype == "bf16":
        x = bf16_round(x)
    wu, bu, wd, bd = _experts(g, E, d, F)
    rw = g.standard_normal((E, 4)).astype(np.float32)
    rb = (0.1 * g.standard_normal(E)).astype(np.float32)
    logits = g.standard_normal((N, E)).astype(np.float32) if router == "logits" else None
    dt = torch.float32 if dtype == "f32" else torch.bfloat16
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, dtype=dt, weight_format=fmt,
                                     router=router)
    block = yggdrasil_amd.CliffordMoEBlockFFN(cfg, device="cuda")
    gamma, beta = _params(g, d)
    with torch.no_grad():
        block.ffn_norm.gamma.copy_(torch.from_numpy(gamma))
        block.ffn_norm.beta.copy_(torch.from_numpy(beta))
    block.moe.load_reference_weights(router_weight=rw, router_bias=rb, w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    if fmt == "int8":  # the oracle runs on the dequantized weights the layer holds
        qu, su = moe.quantize_int8(wu)
        qd, sd = moe.quantize_int8(wd)
        wu, wd = moe.dequantize_int8(qu, su), moe.dequantize_int8(qd, sd)
    experts = [(wu[e], bu[e], wd[e], bd[e]) for e in range(E)]
    say(f"block ffn N={N} d={d} F={F} E={E} k={k} {dtype} {fmt} {router}")
    xt = torch.from_numpy(x).cuda().to(dt)
    lt = torch.from_numpy(logits).cuda() if logits is not None else None
    out = block(xt, logits=lt)
    torch.cuda.synchronize()
    ref, info = block_ffn_reference(x, gamma, beta, rw, rb, experts, k, logits=logits)
    assert np.array_equal(block.moe.last_routing["topk_idx"].cpu().numpy(), info["idx"][:, ::-1])
    err = normwise_err(out.float().cpu().numpy(), ref)
    assert err < (TOL_F32 if dtype == "f32" else TOL_BF16), err


def test_block_ffn_clifford_head_router():
    """The CliffordLinear -> grade-0 head reads the normed tokens too."""
    import yggdrasil_amd

    g = np.random.default_rng(12)
    N, d, F, E, k = 40, 8, 16, 4, 2
    x = g.standard_normal((1, N, d, 8)).astype(np.float32)
    wu, bu, wd, bd = _experts(g, E, d, F)
    head = (g.standard_normal((E, d, 8)) / np.sqrt(8 * d)).astype(np.float32)
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, router="clifford_head")
    block = yggdrasil_amd.CliffordMoEBlockFFN(cfg, device="cuda")
    gamma, beta = _params(g, d)
    with torch.no_grad():
        block.ffn_norm.gamma.copy_(torch.from_numpy(gamma))
        block.ffn_norm.beta.copy_(torch.from_numpy(beta))
    block.moe.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd, head_weight=head)
    say("block ffn clifford head")
    out = block(torch.from_numpy(x).cuda()).cpu().numpy()
    xn = clifford_layer_norm(x, gamma, beta)
    logits = moe.clifford_linear(xn.reshape(N, d, 8), head, None)[..., 0]
    ref, _ = block_ffn_reference(x, gamma, beta, None, None, [(wu[e], bu[e], wd[e], bd[e]) for e in range(E)], k,
                                 logits=logits)
    assert normwise_err(out, ref) < TOL_F32
