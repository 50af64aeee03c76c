"""The kernels under HIP graph capture (the decode step of engine/cuda_graphs.py
is captured and replayed): every replay, with eager work and host
synchronisation between replays, must equal the eager result bit for bit."""

from __future__ import annotations

import pytest
import torch

from helpers import activations, bf16_gpu, weights
from pageserve_amd import quantization as Q

pytestmark = pytest.mark.gpu


def _w(gpu, seed, n, k):
    return Q.QuantizedWeight(torch.from_numpy(weights(seed, n, k)).to(gpu))


@pytest.mark.parametrize("m", [1, 512])
def test_graph_replays_equal_eager(gpu, m):
    k, inter = 2048, 11008
    wq, wk, wv, wo = _w(gpu, 1, 2048, k), _w(gpu, 2, 256, k), _w(gpu, 3, 256, k), _w(gpu, 4, 2048, 2048)
    wg, wu, wd = _w(gpu, 5, inter, k), _w(gpu, 6, inter, k), _w(gpu, 7, k, inter)
    x = bf16_gpu(activations(8, m, k), gpu)

    def step(inp):
        q, kk, v = Q.linear_group(inp, [wq, wk, wv])
        o = wo.linear(q)
        act = Q.swiglu(o, wg, wu)
        return wd.linear(act), kk, v

    eager = step(x)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(x)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured = step(x)
    for i in range(4):
        junk = torch.randn(1 << 20, device=gpu).sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(captured, eager):
            assert torch.equal(a, b), f"replay {i} differs from eager"
        del junk
