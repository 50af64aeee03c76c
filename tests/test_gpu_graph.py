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


@pytest.mark.parametrize("m", [1, 3, 16])
def test_graph_fused_layer_chain(gpu, m):
    """One decoder layer with its neighbours fused (rms_norm inside q|k|v and
    gate|up, RoPE of q and k in place, residual adds in the epilogues); at 16
    tokens the norm runs as its own kernel into the workspace."""
    H, I, KV, hd = 2048, 11008, 256, 128
    wq, wk, wv, wo = _w(gpu, 11, H, H), _w(gpu, 12, KV, H), _w(gpu, 13, KV, H), _w(gpu, 14, H, H)
    wg, wu, wd = _w(gpu, 15, I, H), _w(gpu, 16, I, H), _w(gpu, 17, H, I)
    ln1 = (1 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(18))).to(torch.bfloat16).to(gpu)
    ln2 = (1 + 0.1 * torch.randn(H, generator=torch.Generator().manual_seed(19))).to(torch.bfloat16).to(gpu)
    pos = torch.arange(7, 7 + m, device=gpu).float()
    inv = 1.0 / (1e6 ** (torch.arange(0, hd, 2, device=gpu).float() / hd))
    emb = torch.cat((torch.outer(pos, inv),) * 2, dim=-1)
    cos, sin = emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)
    x = bf16_gpu(activations(20, m, H), gpu)
    attn = bf16_gpu(activations(21, m, H), gpu)

    def step(inp):
        q, kk, v = Q.rmsnorm_linear_group(inp, ln1, 1e-6, [wq, wk, wv])
        Q.rope_qk(q.view(m, H // hd, hd), kk.view(m, KV // hd, hd), cos, sin, inplace=True)
        x1 = wo.linear(attn, residual=inp)
        return Q.rmsnorm_mlp(x1, ln2, 1e-6, wg, wu, wd, residual=x1), q, kk, v

    eager = step(x)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(x)  # warm-up on the capture stream (allocates its workspace)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured = step(x)
    for i in range(4):
        junk = torch.randn(1 << 20, device=gpu).sum()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(captured, eager):
            assert torch.equal(a, b), f"replay {i} differs from eager"
        del junk
