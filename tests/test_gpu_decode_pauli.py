"""GPU parity of the int8 Pauli decode layer (weight format 5, ``csrc/decode_pauli.hip``).

* Weight preparation: the codes and scales ``ygg_prepare_weights(format=5)`` writes are
  the oracle's ``quantize_int8_pauli`` bit for bit, read back through the documented
  layout.
* The layer (routing, both products and the activation in one launch, then the plane
  combine): the routing arrays equal ``ygg_route``'s bit for bit (ties included), and
  the output is the reference layer's (``oracle.moe``) on the dequantized weights the
  format holds, within the int8 bound 2e-2 normwise (``_gpu_helpers``).  The products
  carry the activations as 16-bit fixed point per token, so the error stays far below
  the bound; it is printed.
"""

import numpy as np
import pytest
import torch

import _inputs
from _gpu_helpers import TOL_BF16, moe_reference, normwise_err, say
from oracle import moe

pytestmark = pytest.mark.gpu


def _mods():
    import yggdrasil_amd
    from yggdrasil_amd import ops

    return yggdrasil_amd, ops


def _unpack_format5(data: np.ndarray, E: int, d_out: int, d_in: int) -> np.ndarray:
    """Prepared bytes -> codes (E, d_out, d_in, 8) in entry order [U00, V00, U01, V01, U10, V10, U11, V11].

    Layout per expert: [jb][ks][U, V][g 4][n 16][16 bytes], channel j = 8 jb + n // 2, row a = n % 2,
    input i = 32 ks + 8 g + m, byte 2 m + c holds entry (a, c) of U or V."""
    JB, KS = (d_out + 7) // 8, (d_in + 31) // 32
    b = data.view(np.int8).reshape(E, JB, KS, 2, 4, 16, 8, 2)  # e jb ks uv g n m c
    q = np.zeros((E, JB * 8, KS * 32, 8), np.int8)
    for uv in range(2):
        for a in range(2):
            for c in range(2):
                blk = b[:, :, :, uv, :, a::2, :, c]  # e jb ks g jj m
                q[..., 4 * a + 2 * c + uv] = blk.transpose(0, 1, 4, 2, 3, 5).reshape(E, JB * 8, KS * 32)
    return q[:, :d_out, :d_in]


@pytest.mark.parametrize("E,d_out,d_in", [(2, 16, 32), (3, 13, 45), (1, 512, 128), (2, 8, 1)])
def test_prepare_int8_pauli_weights_bit_exact(E, d_out, d_in):
    _, ops = _mods()
    g = np.random.default_rng(E * 1000 + d_out + d_in)
    w = g.standard_normal((E, d_out, d_in, 8)).astype(np.float32)
    w[0, min(3, d_out - 1)] = 0  # an all-zero channel: scale 1e-12 / 127, codes zero
    say(f"prepare int8_pauli E={E} d_out={d_out} d_in={d_in}")
    pw = ops.prepare_weights(torch.from_numpy(w).cuda(), "int8_pauli")
    torch.cuda.synchronize()
    q_ref, s_ref = moe.quantize_int8_pauli(w)
    assert np.array_equal(pw.scales.cpu().numpy(), s_ref)
    data = pw.data.cpu().numpy()
    assert data.size == E * ((d_out + 7) // 8) * ((d_in + 31) // 32) * 2048
    assert np.array_equal(_unpack_format5(data, E, d_out, d_in), q_ref)
    # padding channels and inputs hold zero codes
    JB, KS = (d_out + 7) // 8, (d_in + 31) // 32
    full = np.zeros((E, JB * 8, KS * 32, 8), np.int8)
    full[:, :d_out, :d_in] = q_ref
    assert np.count_nonzero(data.view(np.int8)) == np.count_nonzero(full)


def _layer_ref(x, idx, w, wu, bu, wd, bd, act):
    return moe_reference(x, idx, w, wu.astype(np.float32), bu, wd.astype(np.float32), bd, act,
                         acc_dtype=np.float64)


@pytest.mark.parametrize("N,d,F,E,k,act", [(64, 128, 512, 32, 2, "gelu"), (1, 16, 32, 4, 1, "relu"),
                                           (128, 64, 96, 64, 2, "sigmoid"), (37, 40, 72, 9, 3, "gelu"),
                                           (100, 32, 64, 16, 2, "relu"), (64, 128, 130, 32, 2, "gelu")])
def test_decode_pauli_layer(N, d, F, E, k, act):
    """The one-launch layer: routing arrays equal ygg_route's bit for bit (exact logit ties
    included), output within the int8 bound of the oracle on the format's dequantized weights."""
    yggdrasil_amd, ops = _mods()
    g = np.random.default_rng(N * 7 + E + d)
    x = _inputs.bf16_round(g.standard_normal((N, d, 8), dtype=np.float32))
    wu, bu, wd, bd = _inputs.expert_weights(g, E, d, F, bias_std=0.2)
    logits = np.round(g.standard_normal((N, E)), 1).astype(np.float32)  # many exact ties
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, activation=act,
                                     dtype=torch.bfloat16, weight_format="int8_pauli", router="logits")
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    lt = torch.from_numpy(logits).cuda()
    say(f"decode pauli N={N} d={d} F={F} E={E} k={k} {act}")
    y = layer.moe_forward(torch.from_numpy(x).cuda().bfloat16().reshape(1, N, d, 8), logits=lt)
    y = y.float().cpu().numpy().reshape(N, d, 8)
    r = ops.route(lt, k)
    for key in ("topk_idx", "topk_w", "counts", "offsets"):
        assert torch.equal(layer.last_routing[key], getattr(r, key)), key
    idx, w = r.topk_idx.cpu().numpy(), r.topk_w.cpu().numpy()
    wu_q = moe.dequantize_int8_pauli(*moe.quantize_int8_pauli(wu))
    wd_q = moe.dequantize_int8_pauli(*moe.quantize_int8_pauli(wd))
    ref = _layer_ref(x, idx, w, wu_q, bu, wd_q, bd, act)
    err = normwise_err(y, ref)
    say(f"decode pauli normwise error {err:.3e}")
    assert err < TOL_BF16


def test_decode_pauli_skewed_batches():
    """One expert takes 40 of 64 tokens (three 16-token batches, the last ragged); F = 302
    leaves a partial hidden chunk and a partial column block; biases on both products."""
    yggdrasil_amd, ops = _mods()
    g = np.random.default_rng(616)
    N, d, F, E, k = 64, 96, 302, 8, 2
    x = _inputs.bf16_round(g.standard_normal((N, d, 8), dtype=np.float32))
    wu, bu, wd, bd = _inputs.expert_weights(g, E, d, F, bias_std=0.3)
    logits = g.standard_normal((N, E), dtype=np.float32)
    logits[:40, 0] += 6.0
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, dtype=torch.bfloat16,
                                     weight_format="int8_pauli", router="logits")
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    say(f"decode pauli skewed N={N} d={d} F={F} E={E} k={k}")
    y = layer.moe_forward(torch.from_numpy(x).cuda().bfloat16().reshape(1, N, d, 8),
                          logits=torch.from_numpy(logits).cuda()).float().cpu().numpy().reshape(N, d, 8)
    assert layer.last_routing["counts"].cpu().numpy()[0] >= 40
    idx, w = moe.route_topk(moe.softmax(logits), k)
    assert np.array_equal(layer.last_routing["topk_idx"].cpu().numpy(), idx)
    wu_q = moe.dequantize_int8_pauli(*moe.quantize_int8_pauli(wu))
    wd_q = moe.dequantize_int8_pauli(*moe.quantize_int8_pauli(wd))
    err = normwise_err(y, _layer_ref(x, idx, w, wu_q, bu, wd_q, bd, "gelu"))
    say(f"decode pauli skewed normwise error {err:.3e}")
    assert err < TOL_BF16


def test_decode_pauli_energy_router_and_residual():
    """The reference router (grade-energy logits computed first) and the residual add of
    the block (x + moe(x)) on the int8 Pauli layer."""
    yggdrasil_amd, ops = _mods()
    g = np.random.default_rng(818)
    N, d, F, E, k = 48, 64, 128, 8, 2
    x = _inputs.bf16_round(g.standard_normal((N, d, 8), dtype=np.float32))
    wu, bu, wd, bd = _inputs.expert_weights(g, E, d, F, bias_std=0.1)
    rw = (0.5 * g.standard_normal((E, 4))).astype(np.float32)
    rb = (0.2 * g.standard_normal(E)).astype(np.float32)
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, dtype=torch.bfloat16,
                                     weight_format="int8_pauli", router="energy")
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(router_weight=rw, router_bias=rb, w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    xt = torch.from_numpy(x).cuda().bfloat16().reshape(1, N, d, 8)
    say(f"decode pauli energy router N={N} d={d} F={F} E={E} k={k}")
    y = layer.moe_forward(xt, residual=xt).float().cpu().numpy().reshape(N, d, 8)
    lg, _ = moe.router_logits(x, rw, rb)
    idx_o, _ = moe.route_topk(moe.softmax(lg), k)
    idx = layer.last_routing["topk_idx"].cpu().numpy()
    assert np.array_equal(idx, idx_o)
    w = layer.last_routing["topk_w"].cpu().numpy()
    wu_q = moe.dequantize_int8_pauli(*moe.quantize_int8_pauli(wu))
    wd_q = moe.dequantize_int8_pauli(*moe.quantize_int8_pauli(wd))
    ref = x + _layer_ref(x, idx, w, wu_q, bu, wd_q, bd, "gelu")
    err = normwise_err(y, ref)
    say(f"decode pauli energy router normwise error {err:.3e}")
    assert err < TOL_BF16


@pytest.mark.parametrize("fmt", ["int8_pauli", "int8"])
def test_decode_tiny_and_nonfinite_tokens(fmt):
    """Both int8 decode layers scale each token's row (and hidden row) by a power of two
    before the integer or fp16 products.  Rows whose largest entry lies far below 2^-112
    take the largest normal shift and quantize to (nearly) zero codes, so their outputs
    stay the oracle's (the biases' image) instead of overflowing the scale; an all-zero
    token gives the biases' image too.  A token holding a NaN or an Inf gives a non-finite
    output row, as the reference's arithmetic does, and leaves every other token exact to
    the int8 bound."""
    yggdrasil_amd, ops = _mods()
    g = np.random.default_rng(4242)
    N, d, F, E, k = 32, 64, 128, 8, 2
    x = _inputs.bf16_round(g.standard_normal((N, d, 8), dtype=np.float32))
    x[0:4] *= np.float32(2.0 ** -120)   # near zero, representable in bf16 (2^-133 and up)
    x[4] *= np.float32(2.0 ** -130)     # subnormal in bf16 and fp32
    x[5] = 0.0
    x[6, 3, 2] = np.nan
    x[7, 10, 5] = np.inf
    x = _inputs.bf16_round(x)
    wu, bu, wd, bd = _inputs.expert_weights(g, E, d, F, bias_std=0.2)
    logits = g.standard_normal((N, E), dtype=np.float32)
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k, dtype=torch.bfloat16,
                                     weight_format=fmt, router="logits")
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    say(f"decode {fmt} tiny and non-finite tokens N={N} d={d} F={F} E={E} k={k}")
    y = layer.moe_forward(torch.from_numpy(x).cuda().bfloat16().reshape(1, N, d, 8),
                          logits=torch.from_numpy(logits).cuda()).float().cpu().numpy().reshape(N, d, 8)
    idx, w = moe.route_topk(moe.softmax(logits), k)
    assert np.array_equal(layer.last_routing["topk_idx"].cpu().numpy(), idx)
    if fmt == "int8_pauli":
        wu_q = moe.dequantize_int8_pauli(*moe.quantize_int8_pauli(wu))
        wd_q = moe.dequantize_int8_pauli(*moe.quantize_int8_pauli(wd))
    else:
        wu_q, wd_q = moe.dequantize_int8(*moe.quantize_int8(wu)), moe.dequantize_int8(*moe.quantize_int8(wd))
    bad = [6, 7]
    good = [t for t in range(N) if t not in bad]
    ref = _layer_ref(x[good], idx[good], w[good], wu_q, bu, wd_q, bd, "gelu")
    assert np.isfinite(y[good]).all()
    err = normwise_err(y[good], ref)
    # the near-zero and zero tokens on their own: their outputs are the biases' image
    err_tiny = normwise_err(y[:6], ref[:6])
    say(f"decode {fmt} finite tokens normwise error {err:.3e}, near-zero tokens {err_tiny:.3e}")
    assert err < TOL_BF16 and err_tiny < TOL_BF16
    for t in bad:
        assert not np.isfinite(y[t]).any(), f"token {t}: a non-finite input gave finite outputs"
