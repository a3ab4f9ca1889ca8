"""GPU parity of the operator boundary ``geom_matmul`` (one fp32 Pauli MFMA product).

``out[m, n] = sum_k gp(a[m, k], b[k, n])`` -- ``rune/ops/batched.py:320-344``,
``mjolnir/src/cuda/batch_ops.cu:264-339,389-401`` -- against the float64 dense
oracle (``oracle.dense.linear``: the contraction with L(a), whose equivalence to
the reference's geometric matmul is pinned in ``test_oracle_algebra``) at the
CliffordLinear shapes of config 3 (W (512, 128) on 8192 token columns, and the
down projection's transpose), on ragged and degenerate sizes, and through both
entry points (caller's workspace, and the reference signature that takes its
scratch from the stream-ordered pool).  fp32 operands, fp32 accumulation:
normwise error <= 1e-5 (TOL_F32).
"""

import numpy as np
import pytest
import torch

from _gpu_helpers import TOL_F32, normwise_err, say
from oracle import dense

pytestmark = pytest.mark.gpu


def _ops():
    from yggdrasil_amd import ops

    return ops


def _operands(M, K, N, seed):
    g = np.random.default_rng(seed)
    a = (g.standard_normal((M, K, 8)) / np.sqrt(8 * K)).astype(np.float32)
    b = g.standard_normal((K, N, 8)).astype(np.float32)
    return a, b


def _truth(a, b):
    # out[m, n] = sum_k a[m, k] b[k, n]: a CliffordLinear with weight a on the rows b[:, n]
    y = dense.linear(np.transpose(b, (1, 0, 2)), a)  # (N, M, 8) float64
    return np.transpose(y, (1, 0, 2))


@pytest.mark.parametrize("M,K,N", [(512, 128, 8192), (128, 512, 8192)])
def test_clifford_linear_sizes_against_dense_oracle(M, K, N):
    ops = _ops()
    a, b = _operands(M, K, N, seed=M + K)
    say(f"geom_matmul M={M} K={K} N={N}")
    out = ops.geom_matmul(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()).cpu().numpy()
    assert normwise_err(out, _truth(a, b)) < TOL_F32


@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (33, 7, 65), (5, 300, 3), (64, 16, 31), (40, 1, 1000)])
def test_ragged_sizes_and_both_entry_points(M, K, N):
    """Sizes off every tile edge; the reference-signature entry (pool scratch) and the
    workspace entry run the same kernels, so they agree bit for bit."""
    ops = _ops()
    from yggdrasil_amd._native import check, lib, ptr, stream_handle

    a, b = _operands(M, K, N, seed=M * 7 + K * 3 + N)
    say(f"geom_matmul ragged M={M} K={K} N={N}")
    at, bt = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    out = ops.geom_matmul(at, bt)
    assert normwise_err(out.cpu().numpy(), _truth(a, b)) < TOL_F32
    out2 = torch.full_like(out, float("nan"))
    check(lib().ygg_geom_matmul_f32(ptr(at), ptr(bt), ptr(out2), M, K, N, stream_handle(at.device)), "geom_matmul")
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_reused_buffers_and_empty_sum():
    ops = _ops()
    M, K, N = 96, 40, 257
    ws = torch.empty(ops.geom_matmul_workspace_bytes(M, K, N), device="cuda", dtype=torch.uint8)
    out = torch.empty((M, N, 8), device="cuda")
    say("geom_matmul reused workspace, then K = 0")
    for seed in (1, 2):  # the second call overwrites every output element of the first
        a, b = _operands(M, K, N, seed)
        ops.geom_matmul(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), workspace=ws, out=out)
        assert normwise_err(out.cpu().numpy(), _truth(a, b)) < TOL_F32
    z = ops.geom_matmul(torch.zeros((3, 0, 8), device="cuda"), torch.zeros((0, 5, 8), device="cuda"))
    assert z.shape == (3, 5, 8) and not z.any()
