"""Drop-in check: a decoder layer written the way engine/model.py:158-190
writes it -- ``F.linear(h, _resolve(W), b)`` on ``QuantizedWeight`` objects --
runs the fused W8A16 kernels unchanged, and matches the same layer computed
by the oracle in fp32.

The layer here is this test's own minimal Qwen2-style block (RMSNorm, q/k/v
with bias, causal attention over the chunk, o, SwiGLU MLP, residuals) with
synthetic weights; only the linear call sites are the subject.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import activations, bf16_gpu, to_np, weights
from oracle import quantization_oracle as O
from pageserve_amd import quantization as Q

pytestmark = pytest.mark.gpu

HIDDEN, HEADS, KV_HEADS, HEAD_DIM, INTER = 2048, 16, 2, 128, 11008


def _resolve(w):  # engine/model.py:25-26
    return w.get() if isinstance(w, Q.QuantizedWeight) else w


def rms_norm(x, weight, eps=1e-6):  # same math as engine/model.py:29-34
    dtype = x.dtype
    x = x.float()
    x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return weight * x.to(dtype)


def attention(q, k, v):
    """Causal GQA attention over one chunk, fp32 math (not the subject)."""
    m = q.shape[0]
    rep = HEADS // KV_HEADS
    qf = q.float().transpose(0, 1)                                      # [H, m, d]
    kf = k.float().repeat_interleave(rep, dim=1).transpose(0, 1)
    vf = v.float().repeat_interleave(rep, dim=1).transpose(0, 1)
    s = torch.matmul(qf, kf.transpose(1, 2).contiguous()) / HEAD_DIM ** 0.5
    mask = torch.triu(torch.ones(m, m, dtype=torch.bool, device=q.device), 1)
    p = torch.softmax(s.masked_fill(mask, float("-inf")), dim=-1)
    return torch.matmul(p, vf).transpose(0, 1).reshape(m, HEADS * HEAD_DIM).to(q.dtype)


def layer_forward(x, L):
    """engine/model.py:162-190 call structure."""
    m = x.shape[0]
    residual = x
    h = rms_norm(x, L["input_ln"])
    q = F.linear(h, _resolve(L["q_w"]), L["q_b"]).view(m, HEADS, HEAD_DIM)
    k = F.linear(h, _resolve(L["k_w"]), L["k_b"]).view(m, KV_HEADS, HEAD_DIM)
    v = F.linear(h, _resolve(L["v_w"]), L["v_b"]).view(m, KV_HEADS, HEAD_DIM)
    attn_out = attention(q, k, v)
    x = residual + F.linear(attn_out, _resolve(L["o_w"]))
    residual = x
    h = rms_norm(x, L["post_ln"])
    gate = F.linear(h, _resolve(L["gate_w"]))
    up = F.linear(h, _resolve(L["up_w"]))
    return residual + F.linear(F.silu(gate) * up, _resolve(L["down_w"]))


def _layer(gpu, seed):
    shapes = {"q_w": (HEADS * HEAD_DIM, HIDDEN), "k_w": (KV_HEADS * HEAD_DIM, HIDDEN),
              "v_w": (KV_HEADS * HEAD_DIM, HIDDEN), "o_w": (HIDDEN, HEADS * HEAD_DIM),
              "gate_w": (INTER, HIDDEN), "up_w": (INTER, HIDDEN), "down_w": (HIDDEN, INTER)}
    L, ref = {}, {}
    for j, (name, shape) in enumerate(shapes.items()):
        w = weights(seed + j, *shape)
        L[name] = Q.QuantizedWeight(torch.from_numpy(w).to(gpu).to(torch.bfloat16))
        wq = L[name]
        q, s = O.quantize_per_channel(O.f32_to_bf16_bits(w), bf16_bits=True)
        assert torch.equal(wq.q.cpu(), torch.from_numpy(q))
        ref[name] = torch.from_numpy(O.dequantize(q, s, "f32")).to(gpu)   # fp32 dense oracle weight
    for name, n in (("q_b", HEADS * HEAD_DIM), ("k_b", KV_HEADS * HEAD_DIM), ("v_b", KV_HEADS * HEAD_DIM)):
        b = O.round_to_bf16(np.random.default_rng(seed + 50 + n).standard_normal(n).astype(np.float32) * 0.1)
        L[name] = bf16_gpu(b, gpu)
        ref[name] = L[name].float()
    for name in ("input_ln", "post_ln"):
        g = O.round_to_bf16(1.0 + 0.1 * np.random.default_rng(seed + 99).standard_normal(HIDDEN).astype(np.float32))
        L[name] = bf16_gpu(g, gpu)
        ref[name] = L[name].float()
    return L, ref


@pytest.mark.parametrize("m", [1, 7, 64])
def test_unchanged_model_code_runs_the_fused_kernels(gpu, m, monkeypatch):
    L, ref = _layer(gpu, 31337)
    x = bf16_gpu(activations(12 + m, m, HIDDEN), gpu)

    # the weight must never be materialised on this path
    def no_dense(self):
        raise AssertionError("dense weight materialised: F.linear did not take the W8A16 kernel")

    with monkeypatch.context() as mp:
        mp.setattr(Q.QuantizedWeight, "dense", no_dense)
        with torch.no_grad():
            out = layer_forward(x, L)
    assert out.dtype == torch.bfloat16 and out.shape == (m, HIDDEN)

    with torch.no_grad():
        expect = layer_forward(x.float(), ref)  # same layer, fp32 dense oracle weights
    r = O.compare(to_np(out), to_np(expect), INTER)
    assert r["ok"], r


def test_other_ops_see_the_dense_weight(gpu):
    w = torch.randn(64, 128, device=gpu, dtype=torch.bfloat16)
    qw = Q.QuantizedWeight(w)
    g = qw.get()
    assert isinstance(g, Q.W8A16Weight) and g.shape == (64, 128) and g.dtype == torch.bfloat16
    dense = Q.dequantize(qw.q, qw.scale, torch.bfloat16)
    assert torch.equal(g + 0, dense)
    assert torch.equal(g.T.contiguous(), dense.T.contiguous())
    # fp32 activations are not the W8A16 path: F.linear sees the dense weight
    wf = Q.QuantizedWeight(w.float())
    x = torch.randn(3, 128, device=gpu)
    assert torch.equal(F.linear(x, wf.get()), F.linear(x, Q.dequantize(wf.q, wf.scale, torch.float32)))
