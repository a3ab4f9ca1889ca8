"""GPU: ygg_moe_forward_noalloc (scratch in the library's per-GPU device array) against
ygg_moe_forward (caller's workspace), both called through the C ABI.

The two entry points run the same kernels on the same inputs, so every output --
routing indices, weights, counts, offsets and the layer output -- must be
bit-identical.  Each case makes two calls in a row, the second on fewer tokens,
so the second runs over scratch the first left behind.
"""

import numpy as np
import pytest
import torch

from _gpu_helpers import say

pytestmark = pytest.mark.gpu


def _ops():
    from yggdrasil_amd import ops

    return ops


def _weights(g, ops, E, d, F, fmt):
    wu = torch.from_numpy((g.standard_normal((E, F, d, 8)) / np.sqrt(8 * d)).astype(np.float32)).cuda()
    wd = torch.from_numpy((g.standard_normal((E, d, F, 8)) / np.sqrt(8 * F)).astype(np.float32)).cuda()
    bu = torch.from_numpy((0.1 * g.standard_normal((E, F, 8))).astype(np.float32)).cuda()
    bd = torch.from_numpy((0.1 * g.standard_normal((E, d, 8))).astype(np.float32)).cuda()
    return (ops.prepare_weights(wu, fmt), ops.prepare_weights(wd, fmt), ops.prepare_bias(bu),
            ops.prepare_bias(bd))


def _call(ops, noalloc, x, k, pu, pd, bu, bd, act, logits, rw, rb, residual):
    L = ops.lib()
    Nt, d = x.shape[0], x.shape[1]
    E, F = pu.E, pu.d_out
    dev = x.device
    out = torch.full_like(x, float("nan"))
    i32 = dict(device=dev, dtype=torch.int32)
    idx = torch.full((Nt, k), -7, **i32)
    tw = torch.full((Nt, k), float("nan"), device=dev, dtype=torch.float32)
    counts = torch.full((E,), -7, **i32)
    offsets = torch.full((E + 1,), -7, **i32)
    p = ops.ptr
    common = (p(x), ops.DTYPE_CODE[x.dtype], Nt, d, F, E, k, ops.ACT_CODE[act], p(logits), p(rw), p(rb),
              p(pu.data), p(pu.scales), p(bu), p(pd.data), p(pd.scales), p(bd), ops.WFORMAT_CODE[pu.fmt],
              p(residual), p(out), p(idx), p(tw), p(counts), p(offsets))
    st = ops.stream_handle(dev)
    if noalloc:
        ops.check(L.ygg_moe_forward_noalloc(*common, st), "moe_forward_noalloc")
    else:
        nb = L.ygg_moe_workspace_bytes(Nt, d, F, E, k, ops.DTYPE_CODE[x.dtype], ops.WFORMAT_CODE[pu.fmt])
        ws = torch.empty((max(nb, 1),), device=dev, dtype=torch.uint8)
        ops.check(L.ygg_moe_forward(*common, p(ws), nb, st), "moe_forward")
    torch.cuda.synchronize()
    return out, idx, tw, counts, offsets


CASES = [
    # (name, dtype, fmt, N first, N second, d, F, E, k, router, residual)
    ("int8 decode, routed in the up product", torch.bfloat16, "int8", 64, 16, 128, 512, 32, 2, "logits", False),
    ("int8 Pauli decode layer", torch.bfloat16, "int8_pauli", 64, 16, 128, 512, 32, 2, "logits", False),
    ("int8 Pauli decode, grade-energy router", torch.bfloat16, "int8_pauli", 48, 20, 64, 128, 8, 2, "energy", True),
    ("bf16 Pauli", torch.bfloat16, "pauli", 512, 96, 32, 64, 8, 2, "logits", True),
    ("fp32 Pauli, grade-energy router", torch.float32, "pauli_f32", 300, 33, 16, 32, 6, 2, "energy", False),
    ("fp32 Pauli, routed in the up product", torch.float32, "pauli_f32", 200, 37, 32, 64, 8, 2, "logits", True),
    ("bf16 L(w) blocks", torch.bfloat16, "bf16", 200, 40, 16, 32, 4, 3, "logits", False),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_workspace_entry(case):
    name, dtype, fmt, n1, n2, d, F, E, k, router, residual = case
    ops = _ops()
    g = np.random.default_rng(n1 + d + F)
    pu, pd, bu, bd = _weights(g, ops, E, d, F, fmt)
    rw = torch.from_numpy((0.5 * g.standard_normal((E, 4))).astype(np.float32)).cuda()
    rb = torch.from_numpy((0.2 * g.standard_normal(E)).astype(np.float32)).cuda()
    for Nt in (n1, n2):
        x = torch.from_numpy(g.standard_normal((Nt, d, 8)).astype(np.float32)).cuda().to(dtype)
        logits = torch.from_numpy(g.standard_normal((Nt, E)).astype(np.float32)).cuda() if router == "logits" else None
        res = torch.from_numpy(g.standard_normal((Nt, d, 8)).astype(np.float32)).cuda().to(dtype) if residual else None
        args = (x, k, pu, pd, bu, bd, "gelu", logits, None if logits is not None else rw,
                None if logits is not None else rb, res)
        say(f"noalloc {name} N={Nt} d={d} F={F} E={E} k={k}")
        want = _call(ops, False, *args)
        got = _call(ops, True, *args)
        for a, b, what in zip(got, want, ("out", "topk_idx", "topk_w", "counts", "offsets")):
            assert torch.equal(a, b), f"{name} N={Nt}: {what} differs from ygg_moe_forward"
        assert torch.isfinite(got[0].float()).all()
        assert int(got[3].sum()) == Nt * k


def test_noalloc_rejects_calls_beyond_its_scratch():
    ops = _ops()
    L = ops.lib()
    limit = 64 << 20
    # BASELINE config 3's shape needs hundreds of MiB: refused with a message, nothing launched
    assert L.ygg_moe_workspace_bytes(8192, 128, 512, 32, 4, 1, 3) > limit
    rc = L.ygg_moe_forward_noalloc(1, 1, 8192, 128, 512, 32, 4, 1, 1, None, None, 1, None, None, 1, None, None, 3,
                                   None, 1, 1, 1, 1, 1, ops.stream_handle())
    assert rc == -1 and b"ygg_moe_forward with a workspace" in L.ygg_last_error()
