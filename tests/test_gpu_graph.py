"""GPU: the layer step captured in a HIP graph (through torch) replays bit for bit.

The library allocates nothing and clears nothing with memsets, so a caller may
capture a whole layer step.  Each graph is replayed several times with eager work
and synchronisation between the replays, and every replay is compared with the
eager result.
"""

import numpy as np
import pytest
import torch

from _gpu_helpers import say

pytestmark = pytest.mark.gpu


def _layer(fmt, dtype, N, d, F, E, k, seed):
    import yggdrasil_amd
    from yggdrasil_amd import ops

    g = np.random.default_rng(seed)
    wu = (g.standard_normal((E, F, d, 8)) / np.sqrt(8 * d)).astype(np.float32)
    wd = (g.standard_normal((E, d, F, 8)) / np.sqrt(8 * F)).astype(np.float32)
    pu = ops.prepare_weights(torch.from_numpy(wu).cuda(), fmt)
    pd = ops.prepare_weights(torch.from_numpy(wd).cuda(), fmt)
    x = torch.from_numpy(g.standard_normal((N, d, 8)).astype(np.float32)).cuda().to(dtype)
    logits = torch.from_numpy(g.standard_normal((N, E)).astype(np.float32)).cuda()
    ws = torch.empty(ops.moe_workspace_bytes(N, d, F, E, k, dtype, fmt), device="cuda", dtype=torch.uint8)
    out = torch.empty_like(x)

    def step():
        y, _ = ops.moe_forward(x, k, pu, pd, None, None, "gelu", logits=logits, workspace=ws, out=out)
        return y

    return step


@pytest.mark.parametrize("fmt,dtype,N,d,F,E,k", [("pauli_f32", torch.float32, 256, 64, 256, 8, 2),
                                                 ("pauli", torch.bfloat16, 2048, 32, 64, 16, 2),
                                                 ("int8", torch.bfloat16, 64, 32, 64, 8, 2),
                                                 ("int8_pauli", torch.bfloat16, 64, 128, 512, 32, 2)])
def test_layer_step_graph_replays_match_eager(fmt, dtype, N, d, F, E, k):
    step = _layer(fmt, dtype, N, d, F, E, k, seed=N + E)
    say(f"graph capture {fmt} N={N} d={d} F={F} E={E} k={k}")
    ref = step().clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on a side stream, as torch asks before capture
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gout = step()
    for r in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gout, ref), f"replay {r}"
        eager = step()  # the program's own work between replays
        torch.cuda.synchronize()
        assert torch.equal(eager, ref)
