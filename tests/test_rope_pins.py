"""Pins of the oracle's RoPE (engine/model.py:53-56, rotate_half :37-39) on
the CPU: closed forms (the identity at cos = 1, sin = 0; an exact
rotate_half at cos = 0, sin = 1), agreement with torch's own bf16 CPU
arithmetic running the reference's expression on a real cache (an
independent implementation of the three roundings), and planted mistakes
that must be caught."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quantization_oracle as O


def _bf16(a: np.ndarray) -> np.ndarray:
    return O.round_to_bf16(np.asarray(a, np.float32))


def _cache(max_len: int, head_dim: int, theta: float = 1e6):
    # the reference's cache construction (engine/model.py:42-47), in torch on the CPU
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    t = torch.arange(max_len).float()
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


def _torch_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    x1, x2 = x.chunk(2, dim=-1)
    rot = torch.cat((-x2, x1), dim=-1)
    return x * cos.unsqueeze(1) + rot * sin.unsqueeze(1)


def _x(rng, m, heads, hd, scale=3.0):
    return _bf16(rng.standard_normal((m, heads, hd)).astype(np.float32) * np.float32(scale))


def test_identity_at_position_zero():
    rng = np.random.default_rng(1)
    x = _x(rng, 4, 3, 64)
    c = np.ones((4, 64), np.float32)
    s = np.zeros((4, 64), np.float32)
    assert np.array_equal(O.rope(x, c, s), x)


def test_quarter_turn_is_rotate_half():
    rng = np.random.default_rng(2)
    x = _x(rng, 3, 2, 16)
    c = np.zeros((3, 16), np.float32)
    s = np.ones((3, 16), np.float32)
    expect = np.concatenate([-x[..., 8:], x[..., :8]], axis=-1)
    assert np.array_equal(O.rope(x, c, s), expect)


@pytest.mark.parametrize("m,heads,hd,start", [(5, 4, 128, 0), (9, 2, 64, 1000), (3, 1, 24, 77)])
def test_matches_torch_bf16_expression(m, heads, hd, start):
    rng = np.random.default_rng(m * 7 + hd)
    cos_t, sin_t = _cache(start + m, hd)
    cos_t, sin_t = cos_t[start:start + m], sin_t[start:start + m]
    x = _x(rng, m, heads, hd)
    xt = torch.from_numpy(x).to(torch.bfloat16)
    want = _torch_rope(xt, cos_t, sin_t).float().numpy()
    got = O.rope(x, cos_t.float().numpy(), sin_t.float().numpy())
    assert np.array_equal(got, want)


def test_planted_mistakes_are_caught():
    rng = np.random.default_rng(5)
    m, heads, hd = 6, 3, 32
    cos_t, sin_t = _cache(200, hd)
    cos_t, sin_t = cos_t[150:156], sin_t[150:156]
    c, s = cos_t.float().numpy(), sin_t.float().numpy()
    x = _x(rng, m, heads, hd)
    good = O.rope(x, c, s)
    h = hd // 2
    # rotation the other way round
    bad = O.round_to_bf16(O.round_to_bf16(x * c[:, None]) +
                          O.round_to_bf16(np.concatenate([x[..., h:], -x[..., :h]], -1) * s[:, None]))
    assert not np.array_equal(bad, good)
    # one rounding at the end instead of three
    bad = O.round_to_bf16(x * c[:, None] + np.concatenate([-x[..., h:], x[..., :h]], -1) * s[:, None])
    assert not np.array_equal(bad, good)
    # positions off by one (cache rows start + 1 ..)
    cos_n, sin_n = _cache(200, hd)
    assert not np.array_equal(O.rope(x, cos_n[151:157].float().numpy(), sin_n[151:157].float().numpy()), good)
    # cos and sin exchanged
    assert not np.array_equal(O.rope(x, s, c), good)
