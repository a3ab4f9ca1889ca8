"""CPU: grade-aware quantization oracle and the checkpoint reader.

The quantization oracle (``oracle/quant.py``) is pinned by the properties the
reference's own suite asserts (``bifrost/tests/test_quantization.py:54-102``,
on the same seeded inputs) and by closed forms.  The checkpoint reader
(``yggdrasil_amd/checkpoint.py``, host code of the product) is checked on
files written in each of the reference's three layouts.
"""

import os

import numpy as np
import pytest

from oracle import quant


def _rt_err(mv, **kw):
    codes, s, z = quant.grade_quantize(mv, **kw)
    return np.max(np.abs(mv - quant.grade_dequantize(codes, s, z)))


def test_reference_suite_properties():
    # test_roundtrip_symmetric_default / _asymmetric / high_precision_scalar
    assert _rt_err(np.random.RandomState(42).randn(10, 8)) < 0.5
    assert _rt_err(np.random.RandomState(7).randn(5, 8) + 2.0, symmetric=False) < 1.0
    mv = np.random.RandomState(99).randn(100, 8)
    codes, s, z = quant.grade_quantize(mv)
    rec = quant.grade_dequantize(codes, s, z)
    assert np.max(np.abs(mv[:, 0] - rec[:, 0])) <= np.max(np.abs(mv[:, 7] - rec[:, 7])) + 1e-9
    # test_quantized_bits_count: payload bits of 4 multivectors
    codes, _, _ = quant.grade_quantize(np.ones((4, 8)))
    assert sum(codes[..., sl].size * b for (g, sl), b in zip(quant.GRADE_SLICES.items(), (8, 6, 6, 4))) == \
        4 * (8 + 18 + 18 + 4)
    # test_batch_shape_preserved / test_bad_last_axis_raises
    c, s, z = quant.grade_quantize(np.zeros((3, 5, 8)))
    assert quant.grade_dequantize(c, s, z).shape == (3, 5, 8)
    with pytest.raises(ValueError):
        quant.grade_quantize(np.zeros((4, 7)))


@pytest.mark.parametrize("bits,symmetric", [((8, 6, 6, 4), True), ((8, 6, 6, 4), False), ((2, 3, 16, 5), True),
                                            ((4, 4, 4, 4), False)])
def test_closed_forms(bits, symmetric):
    g = np.random.default_rng(sum(bits) + symmetric)
    bd = dict(enumerate(bits))
    mv = g.standard_normal((7, 9, 8)) * g.uniform(0.1, 5.0, 8)
    codes, s, z = quant.grade_quantize(mv, bd, symmetric)
    for gr, sl in quant.GRADE_SLICES.items():
        qmin, qmax = -(1 << (bits[gr] - 1)), (1 << (bits[gr] - 1)) - 1
        q = codes[..., sl]
        assert q.min() >= qmin and q.max() <= qmax
        rec = (q - z[gr]) * s[gr]
        # in range: at most half a step from the value
        assert np.all(np.abs(rec - mv[..., sl]) <= s[gr] / 2 * (1 + 1e-12))
        if symmetric:
            assert z[gr] == 0 and np.max(np.abs(q)) == qmax
            assert s[gr] == np.max(np.abs(mv[..., sl])) / qmax
        else:
            assert s[gr] == (mv[..., sl].max() - mv[..., sl].min()) / (qmax - qmin)
    if symmetric:  # values on the grid come back exactly
        on_grid = quant.grade_dequantize(codes, s, z)
        c2, s2, z2 = quant.grade_quantize(on_grid, bd, symmetric)
        assert np.array_equal(quant.grade_dequantize(c2, s2, z2), on_grid)


def test_ties_round_to_even():
    # grade 0 with 4 bits, scale 1: values k + 0.5 round to the even neighbour
    mv = np.zeros((6, 8))
    mv[:, 0] = [7.0, 0.5, 1.5, 2.5, -0.5, -1.5]
    codes, s, _ = quant.grade_quantize(mv, {0: 4, 1: 8, 2: 8, 3: 8})
    assert s[0] == 1.0
    assert list(codes[:, 0]) == [7, 0, 2, 2, 0, -2]


def _block_params(g, d, F, E, n_attn=3):
    """A parameter list in HLMBlock.parameters() order with a few attention stand-ins in front."""
    ps = [g.standard_normal((d, 8)).astype(np.float32) for _ in range(2)]          # attn_norm
    ps += [g.standard_normal((d, d, 8)).astype(np.float32) for _ in range(n_attn)]  # attention
    first = len(ps)
    ps += [g.standard_normal((d, 8)).astype(np.float32), g.standard_normal((d, 8)).astype(np.float32)]
    ps += [g.standard_normal((E, 4)).astype(np.float32), g.standard_normal(E).astype(np.float32)]
    for _ in range(E):
        ps += [g.standard_normal((F, d, 8)).astype(np.float32), g.standard_normal((F, 8)).astype(np.float32),
               g.standard_normal((d, F, 8)).astype(np.float32), g.standard_normal((d, 8)).astype(np.float32)]
    return ps, first


@pytest.mark.parametrize("layout", ["stratified", "whole", "serving", "directory"])
def test_checkpoint_reader_all_layouts(tmp_path, layout):
    from yggdrasil_amd.checkpoint import hlm_block_ffn_state, read_reference_checkpoint

    g = np.random.default_rng(3)
    d, F, E = 4, 6, 3
    ps, first = _block_params(g, d, F, E)
    entries = {"step": np.array(7, np.int64), "opt__t": np.array(7, np.int64)}
    for i, p in enumerate(ps):
        if layout in ("stratified", "directory"):
            entries.update(quant.stratify(f"param_{i}", p))
        elif layout == "whole":
            entries[f"param__param_{i}"] = p
        else:
            entries[f"param_{i}"] = p
    path = tmp_path / "ckpt.npz"
    if layout == "directory":
        os.makedirs(tmp_path / "run")
        path = tmp_path / "run" / "model.npz"
    np.savez_compressed(path, **entries)
    state = read_reference_checkpoint(str(tmp_path / "run") if layout == "directory" else str(path))
    assert len(state) == len(ps)
    for i, p in enumerate(ps):
        assert np.array_equal(state[f"param_{i}"], p), i
    st = hlm_block_ffn_state(state, first, E)
    assert np.array_equal(st["gamma"], ps[first]) and np.array_equal(st["router_bias"], ps[first + 3])
    for e in range(E):
        b = first + 4 + 4 * e
        assert np.array_equal(st["w_up"][e], ps[b]) and np.array_equal(st["b_down"][e], ps[b + 3])
    with pytest.raises((ValueError, KeyError)):
        hlm_block_ffn_state(state, first + 1, E)  # off by one: shapes do not fit, or past the end
    with pytest.raises(ValueError):
        hlm_block_ffn_state(state, first - 1, E)


def test_stratified_reconstruction_fills_missing_grades_with_zero(tmp_path):
    from yggdrasil_amd.checkpoint import read_reference_checkpoint

    g = np.random.default_rng(4)
    p = g.standard_normal((5, 8)).astype(np.float32)
    entries = quant.stratify("param_0", p)
    entries.update(quant.stratify("param_1", np.arange(6, dtype=np.float32)))  # not a multivector: raw
    del entries["param__param_0__grade_2"]
    want = p.copy()
    want[:, 4:7] = 0
    assert np.array_equal(quant.reconstruct(entries)["param_0"], want)
    np.savez(tmp_path / "c.npz", **entries)
    got = read_reference_checkpoint(str(tmp_path / "c.npz"))
    assert np.array_equal(got["param_0"], want)
    assert np.array_equal(got["param_1"], np.arange(6, dtype=np.float32))


def test_grade_quant_config_validation():
    from yggdrasil_amd.checkpoint import GradeQuantConfig

    assert GradeQuantConfig().bits() == (8, 6, 6, 4)
    with pytest.raises(ValueError):
        GradeQuantConfig(grade_bits={0: 8, 1: 6, 2: 6})
    with pytest.raises(ValueError):
        GradeQuantConfig(grade_bits={0: 1, 1: 6, 2: 6, 3: 4})
