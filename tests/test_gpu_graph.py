"""The kernels under HIP graph capture (the decode step of engine/cuda_graphs.py
is captured and replayed): every replay, with eager work and host
synchronisation between replays, must equal the eager result bit for bit, and
every stage of a captured layer chain must match the oracle; graphs that
share a memory pool keep correct workspaces."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import activations, bf16_gpu, report, to_np, weights
from oracle import quantization_oracle as O
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


# ---------------------------------------------------------------------------
# captured outputs against the oracle (engine/cuda_graphs.py:49-69 replays a
# captured forward_step): every stage of a captured layer chain, on the
# replay's own inputs, against the oracle; no warm-up before the capture, so
# the capture itself allocates and zero-fills its workspace
# ---------------------------------------------------------------------------

def _oracle_weights(gpu, seed, n, k):
    w = weights(seed, n, k)
    return Q.QuantizedWeight(torch.from_numpy(w).to(gpu)), O.quantize_per_channel(w)


@pytest.mark.parametrize("m", [1, 512])
def test_captured_layer_chain_matches_oracle(gpu, m):
    H, I, KV, hd = 2048, 11008, 256, 128
    (wq, oq), (wk, ok), (wv, ov) = (_oracle_weights(gpu, 61 + j, n, H) for j, n in enumerate((H, KV, KV)))
    wo, oo = _oracle_weights(gpu, 64, H, H)
    (wg, og), (wu, ou) = (_oracle_weights(gpu, 65 + j, I, H) for j in range(2))
    wd, od = _oracle_weights(gpu, 67, H, I)
    rng = np.random.default_rng(68)
    ln1 = O.round_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    ln2 = O.round_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    bq, bk, bv = (O.round_to_bf16(rng.standard_normal(n).astype(np.float32)) for n in (H, KV, KV))
    pos = np.arange(5, 5 + m, dtype=np.float64)
    inv = 1.0 / (1e6 ** (np.arange(0, hd, 2) / hd))
    emb = np.concatenate([np.outer(pos, inv)] * 2, axis=-1)
    cos, sin = O.round_to_bf16(np.cos(emb).astype(np.float32)), O.round_to_bf16(np.sin(emb).astype(np.float32))
    x, attn = activations(69, m, H), activations(70, m, H)
    xt, at = bf16_gpu(x, gpu), bf16_gpu(attn, gpu)
    l1, l2, ct, st = (bf16_gpu(v, gpu) for v in (ln1, ln2, cos, sin))
    bts = [bf16_gpu(b, gpu) for b in (bq, bk, bv)]

    def step():
        q, kk, v = Q.rmsnorm_linear_group(xt, l1, 1e-6, [wq, wk, wv], bts)
        qr, kr = Q.rope_qk(q.view(m, H // hd, hd), kk.view(m, KV // hd, hd), ct, st)
        x1 = wo.linear(at, residual=xt)
        act = Q.rmsnorm_swiglu(x1, l2, 1e-6, wg, wu)
        x2 = wd.linear(act, residual=x1)
        return q, kk, v, qr, kr, x1, act, x2

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        cap = step()
    torch.cuda.current_stream().wait_stream(s)
    rows = np.arange(m) if m <= 8 else np.sort(rng.choice(m, 24, replace=False))
    for rep in range(3):
        junk = torch.randn(1 << 20, device=gpu).sum()  # eager work between replays
        step()  # the same calls eagerly, on their own workspace
        g.replay()
        torch.cuda.synchronize()
        q, kk, v, qr, kr, x1, act, x2 = (to_np(t) for t in cap)
        what = f"replay {rep} m={m}"
        h, dh = O.rmsnorm(x[rows], ln1, 1e-6), O.rmsnorm_dx(x[rows], ln1, 1e-6)
        for y, (qq, ss), b, nm in ((q, oq, bq, "q"), (kk, ok, bk, "k"), (v, ov, bv, "v")):
            report(y[rows], O.linear(h, qq, ss, b), H, f"{what} {nm}", acc=O.acc_bound(h, qq, ss, b, dx=dh))
        np.testing.assert_array_equal(qr.reshape(m, -1)[rows],
                                      O.rope(q.reshape(m, -1, hd)[rows], cos[rows], sin[rows]).reshape(len(rows), -1))
        np.testing.assert_array_equal(kr.reshape(m, -1)[rows],
                                      O.rope(kk.reshape(m, -1, hd)[rows], cos[rows], sin[rows]).reshape(len(rows), -1))
        report(x1[rows], O.linear_residual(attn[rows], *oo, x[rows]), H, f"{what} o + residual",
               ulp_of=O.linear_residual_intermediate(attn[rows], *oo))
        h2, dh2 = O.rmsnorm(x1[rows], ln2, 1e-6), O.rmsnorm_dx(x1[rows], ln2, 1e-6)
        report(act[rows], O.swiglu(h2, *og, *ou), H, f"{what} gate|up", acc=O.swiglu_acc(h2, *og, *ou, dx=dh2))
        report(x2[rows], O.linear_residual(act[rows], *od, x1[rows]), I, f"{what} down + residual",
               ulp_of=O.linear_residual_intermediate(act[rows], *od))
        del junk


def test_graphs_sharing_a_pool_keep_their_workspaces(gpu):
    """Two graphs captured on one memory pool without warm-up, each with K
    splits that need a workspace (pair slots at 9 tokens, split-K partials
    for down_proj at 200 tokens), replayed alternately with eager calls of
    other shapes in between on the capture stream: every replay matches the
    oracle."""
    (wo, oo), (wd, od) = _oracle_weights(gpu, 81, 2048, 2048), _oracle_weights(gpu, 82, 2048, 11008)
    x9o, x9d = activations(83, 9, 2048), activations(84, 9, 11008)
    x200 = activations(85, 200, 11008)
    t9o, t9d, t200 = bf16_gpu(x9o, gpu), bf16_gpu(x9d, gpu), bf16_gpu(x200, gpu)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g1, g2 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1, stream=s):
        y1 = (wo.linear(t9o), wd.linear(t9d))
    with torch.cuda.graph(g2, stream=s, pool=g1.pool()):
        y2 = (wd.linear(t200), wo.linear(t9o))
    torch.cuda.current_stream().wait_stream(s)
    refs1 = [(O.linear(x9o, *oo), O.acc_bound(x9o, *oo), 2048), (O.linear(x9d, *od), O.acc_bound(x9d, *od), 11008)]
    rows = np.arange(0, 200, 9)
    refs2 = [(O.linear(x200[rows], *od), O.acc_bound(x200[rows], *od), 11008),
             (O.linear(x9o, *oo), O.acc_bound(x9o, *oo), 2048)]
    x12 = bf16_gpu(activations(86, 12, 11008), gpu)
    for rep in range(3):
        for g, ys, refs, sel in ((g1, y1, refs1, (slice(None), slice(None))), (g2, y2, refs2, (rows, slice(None)))):
            with torch.cuda.stream(s):
                wd.linear(x12)  # an eager paired split on the capture stream's own workspace
                wo.linear(t9o)
                g.replay()
            torch.cuda.synchronize()
            for j, (y, (ref, acc, k)) in enumerate(zip(ys, refs)):
                yy = to_np(y)
                yy = yy[sel] if y.shape[0] == 200 else yy
                report(yy, ref, k, f"rep {rep} graph output {j}", acc=acc)
