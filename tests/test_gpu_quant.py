"""GPU parity: grade-aware quantization and checkpoint import into the layer.

``ygg_grade_quantize`` computes in float64 like the reference, so codes,
scales, zero points and the fp32-rounded values are compared bit for bit with
the oracle.  A block loaded from a grade-stratified checkpoint, with and
without grade quantization, is compared with the oracle's block on the same
weights at the fp32 bound.
"""

import numpy as np
import pytest
import torch

from _gpu_helpers import TOL_F32, normwise_err, say
from oracle import quant
from oracle.norm import block_ffn_reference

pytestmark = pytest.mark.gpu


def _ops():
    from yggdrasil_amd import ops

    return ops


@pytest.mark.parametrize("T,shape,bits,symmetric", [
    (1, (10,), (8, 6, 6, 4), True), (4, (16, 12), (8, 6, 6, 4), True), (3, (5, 7), (8, 6, 6, 4), False),
    (2, (33, 9), (2, 3, 16, 5), True), (5, (8, 8), (4, 4, 4, 4), False), (2, (1,), (16, 16, 16, 16), False)])
def test_grade_quantize_bit_exact(T, shape, bits, symmetric):
    ops = _ops()
    g = np.random.default_rng(T * 100 + sum(bits) + symmetric)
    w = (g.standard_normal((T, *shape, 8)) * g.uniform(0.05, 4.0, 8) + (0 if symmetric else 1.5)).astype(np.float32)
    say(f"grade quantize T={T} shape={shape} bits={bits} symmetric={symmetric}")
    deq, codes, sc, zp = ops.grade_quantize(torch.from_numpy(w).cuda(), bits, symmetric)
    for t in range(T):
        c_o, s_o, z_o = quant.grade_quantize(w[t], dict(enumerate(bits)), symmetric)
        assert np.array_equal(sc[t].cpu().numpy(), s_o), t
        assert np.array_equal(zp[t].cpu().numpy(), z_o.astype(np.int32)), t
        assert np.array_equal(codes[t].cpu().numpy().astype(np.int64), c_o), t
        want = quant.grade_dequantize(c_o, s_o, z_o).astype(np.float32)
        assert np.array_equal(deq[t].cpu().numpy(), want), t


def test_grade_quantize_ties_and_zero_tensor():
    ops = _ops()
    w = np.zeros((2, 6, 8), np.float32)
    w[0, :, 0] = [7.0, 0.5, 1.5, 2.5, -0.5, -1.5]  # 4-bit scalar grade, scale exactly 1
    say("grade quantize ties")
    deq, codes, sc, zp = ops.grade_quantize(torch.from_numpy(w).cuda(), (4, 8, 8, 8), True)
    assert sc[0, 0].item() == 1.0
    assert codes[0, :, 0].tolist() == [7, 0, 2, 2, 0, -2]
    # an all-zero tensor: scale from the 1e-12 floor, all codes zero
    assert torch.all(codes[1] == 0) and sc[1, 0].item() == 1e-12 / 7


def _write_block_checkpoint(path, g, d, F, E):
    ps = [g.standard_normal((d, 8)).astype(np.float32) for _ in range(2)]  # attn_norm
    ps += [g.standard_normal((d, d, 8)).astype(np.float32)]                # an attention weight stand-in
    first = len(ps)
    gamma = np.zeros((d, 8), np.float32)
    gamma[:, 0] = 1.0
    gamma += (0.2 * g.standard_normal((d, 8))).astype(np.float32)
    ps += [gamma, (0.1 * g.standard_normal((d, 8))).astype(np.float32)]
    ps += [g.standard_normal((E, 4)).astype(np.float32), (0.1 * g.standard_normal(E)).astype(np.float32)]
    for _ in range(E):
        ps += [(g.standard_normal((F, d, 8)) / np.sqrt(8 * d)).astype(np.float32),
               (0.1 * g.standard_normal((F, 8))).astype(np.float32),
               (g.standard_normal((d, F, 8)) / np.sqrt(8 * F)).astype(np.float32),
               (0.1 * g.standard_normal((d, 8))).astype(np.float32)]
    entries = {"step": np.array(1, np.int64)}
    for i, p in enumerate(ps):
        entries.update(quant.stratify(f"param_{i}", p))
    np.savez_compressed(path, **entries)
    return ps, first


@pytest.mark.parametrize("grade_quant", [False, True])
def test_block_from_stratified_checkpoint(tmp_path, grade_quant):
    import yggdrasil_amd
    from yggdrasil_amd.checkpoint import GradeQuantConfig

    g = np.random.default_rng(5 + grade_quant)
    N, d, F, E, k = 96, 16, 32, 4, 2
    ps, first = _write_block_checkpoint(tmp_path / "ckpt.npz", g, d, F, E)
    cfg = yggdrasil_amd.MoEHLMConfig(d_model=d, d_ff=F, n_experts=E, top_k=k)
    block = yggdrasil_amd.CliffordMoEBlockFFN(cfg, device="cuda")
    gq = GradeQuantConfig() if grade_quant else None
    say(f"block from checkpoint grade_quant={grade_quant}")
    block.load_reference_checkpoint(str(tmp_path / "ckpt.npz"), first, grade_quant=gq)
    x = g.standard_normal((1, N, d, 8)).astype(np.float32)
    out = block(torch.from_numpy(x).cuda()).cpu().numpy()
    experts = []
    for e in range(E):
        wu, bu, wd, bd = ps[first + 4 + 4 * e: first + 8 + 4 * e]
        if grade_quant:  # the reference's mixed-precision weights: per-tensor grade quantization
            wu = quant.grade_dequantize(*quant.grade_quantize(wu)).astype(np.float32)
            wd = quant.grade_dequantize(*quant.grade_quantize(wd)).astype(np.float32)
        experts.append((wu, bu, wd, bd))
    ref, info = block_ffn_reference(x, ps[first], ps[first + 1], ps[first + 2], ps[first + 3], experts, k)
    assert np.array_equal(block.moe.last_routing["topk_idx"].cpu().numpy(), info["idx"][:, ::-1])
    assert normwise_err(out, ref) < TOL_F32
