"""GPU parity of the grouped-expert boundary ``ops.grouped_experts`` and
``CliffordMoELayer.experts`` -- geoformer's ``FusedMoEExperts.forward(x_sorted,
expert_offsets, expert_counts) -> y_sorted``
(``geoformer/triton_kernels/fused_expert.py:306-331``) over this layer's expert,
``CliffordFFN.forward`` (``holograph/models/hlm_block.py:55-61``).

Every weight format runs both products on rows the caller has already grouped
(an empty expert included); each expert's rows are compared with the oracle's
CliffordFFN (``oracle.moe.clifford_ffn``, pinned by the reference goldens) on the
same operands: the bf16-rounded inputs / weights, the int8 codes dequantized.
Normwise error <= 1e-5 for the fp32 formats, <= 2e-2 (TOL_BF16) otherwise.
"""

import numpy as np
import pytest
import torch

import _inputs
from _gpu_helpers import TOL_BF16, TOL_F32, normwise_err, say
from oracle import moe

pytestmark = pytest.mark.gpu


def _case(fmt, E, d, F, P, seed):
    g = np.random.default_rng(seed)
    wu, bu, wd, bd = _inputs.expert_weights(g, E, d, F, bias_std=0.2)
    x = g.standard_normal((P, d, 8), dtype=np.float32)
    counts = np.bincount(g.integers(0, E, P), minlength=E)
    counts[1] += counts[0]
    counts[0] = 0  # an empty expert
    offsets = np.concatenate([[0], np.cumsum(counts)[:-1]]).astype(np.int32)
    ref_w = (wu, wd)
    if fmt in ("bf16", "int8", "pauli"):
        x = _inputs.bf16_round(x)
    if fmt in ("bf16", "pauli"):
        ref_w = (_inputs.bf16_round(wu), _inputs.bf16_round(wd))
    if fmt == "int8":
        ref_w = tuple(moe.dequantize_int8(*moe.quantize_int8(w)) for w in (wu, wd))
    return x, (wu, bu, wd, bd), ref_w, offsets, counts.astype(np.int32)


@pytest.mark.parametrize("fmt,act,E,d,F,P", [
    ("pauli", "gelu", 6, 32, 64, 300), ("pauli_f32", "gelu", 5, 16, 48, 200), ("bf16", "sigmoid", 4, 24, 40, 150),
    ("int8", "relu", 5, 32, 96, 120), ("f32", "none", 3, 8, 16, 77), ("pauli", "gelu", 8, 128, 512, 2048)])
def test_grouped_experts_against_oracle(fmt, act, E, d, F, P):
    from yggdrasil_amd import ops

    x, (wu, bu, wd, bd), (wu_r, wd_r), offsets, counts = _case(fmt, E, d, F, P, seed=E * 100 + d + F)
    dt = torch.float32 if fmt in ("f32", "pauli_f32") else torch.bfloat16
    say(f"grouped experts fmt={fmt} act={act} E={E} d={d} F={F} P={P}")
    dev = "cuda"
    y = ops.grouped_experts(torch.from_numpy(x).to(dev, dt), torch.from_numpy(offsets).to(dev),
                            torch.from_numpy(counts).to(dev), ops.prepare_weights(torch.from_numpy(wu).to(dev), fmt),
                            ops.prepare_weights(torch.from_numpy(wd).to(dev), fmt),
                            ops.prepare_bias(torch.from_numpy(bu).to(dev)), ops.prepare_bias(torch.from_numpy(bd).to(dev)),
                            act, validate=True)
    assert y.shape == (P, d, 8) and y.dtype == dt
    y = y.float().cpu().numpy()
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    for e in range(E):
        rows = slice(offsets[e], offsets[e] + counts[e])
        if counts[e] == 0:
            continue
        ref = moe.clifford_ffn(x[rows], wu_r[e], bu[e], wd_r[e], bd[e], act)
        assert normwise_err(y[rows], ref) < tol, e


def test_layer_experts_flat_rows_and_range_check():
    """The layer's method takes geoformer's flat (P, 8 d) rows and returns them flat; ranges
    that do not tile the rows are refused when validated."""
    import yggdrasil_amd
    from yggdrasil_amd import ops

    E, d, F, P = 4, 16, 32, 90
    x, (wu, bu, wd, bd), _, offsets, counts = _case("pauli_f32", E, d, F, P, seed=3)
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=2, dtype=torch.float32,
                                     weight_format="pauli_f32")
    layer = yggdrasil_amd.CliffordMoELayer(cfg, device="cuda")
    layer.load_reference_weights(w_up=wu, b_up=bu, w_down=wd, b_down=bd)
    say("layer.experts flat rows")
    xt = torch.from_numpy(x).cuda()
    off_t, cnt_t = torch.from_numpy(offsets).cuda(), torch.from_numpy(counts).cuda()
    y_flat = layer.experts(xt.reshape(P, 8 * d), off_t, cnt_t)
    assert y_flat.shape == (P, 8 * d)
    y = layer.experts(xt, off_t, cnt_t)
    assert torch.equal(y_flat.reshape(P, d, 8), y)
    for e in range(E):
        rows = slice(offsets[e], offsets[e] + counts[e])
        if counts[e]:
            ref = moe.clifford_ffn(x[rows], wu[e], bu[e], wd[e], bd[e], "gelu")
            assert normwise_err(y[rows].cpu().numpy(), ref) < TOL_F32, e
    prep = layer._get_prepared()
    bad = cnt_t.clone()
    bad[-1] += 1  # the last range runs past the rows
    with pytest.raises(ValueError):
        ops.grouped_experts(xt, off_t, bad, prep["w_up"], prep["w_down"], validate=True)


@pytest.mark.parametrize("fmt", ["pauli", "pauli_f32", "bf16"])
def test_grouped_experts_unvalidated_ranges_are_clamped(fmt):
    """Without validation the ranges are clamped on the device into ascending bounds within
    the rows: counts that sum past P (the last range running 50 rows past the end), or an
    offset beyond P, reach the products as ranges inside [0, P].  The first gives exactly
    the valid call's rows; in the second every expert from the bad offset on is empty and
    the rows before it are the valid call's."""
    from yggdrasil_amd import ops

    E, d, F, P = 5, 32, 64, 240
    x, (wu, bu, wd, bd), _, offsets, counts = _case(fmt, E, d, F, P, seed=77)
    dt = torch.float32 if fmt == "pauli_f32" else torch.bfloat16
    dev = "cuda"
    xt = torch.from_numpy(x).to(dev, dt)
    pu, pd = (ops.prepare_weights(torch.from_numpy(w).to(dev), fmt) for w in (wu, wd))
    bup, bdn = ops.prepare_bias(torch.from_numpy(bu).to(dev)), ops.prepare_bias(torch.from_numpy(bd).to(dev))
    off_t, cnt_t = torch.from_numpy(offsets).to(dev), torch.from_numpy(counts).to(dev)
    say(f"grouped experts clamped ranges fmt={fmt} E={E} d={d} F={F} P={P}")
    y = ops.grouped_experts(xt, off_t, cnt_t, pu, pd, bup, bdn, "gelu", validate=True)
    long_last = cnt_t.clone()
    long_last[-1] += 50
    y_long = ops.grouped_experts(xt, off_t, long_last, pu, pd, bup, bdn, "gelu")
    assert torch.equal(y_long, y)
    far = off_t.clone()
    far[3] = P + 100  # experts 3 and 4 become empty; expert 2's range runs to P
    y_far = ops.grouped_experts(xt, far, cnt_t, pu, pd, bup, bdn, "gelu")
    torch.cuda.synchronize()
    assert torch.equal(y_far[:offsets[2]], y[:offsets[2]])
    assert bool(torch.isfinite(y_far.float()).all())
