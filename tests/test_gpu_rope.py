"""RoPE of q and k on the GPU (engine/model.py:53-56 at :172-173) against the
oracle: bit-exact on every element (the same three bf16 roundings), for the
vector path (head_dim / 2 a multiple of 8) and the scalar path, q with and
without k, in place and out of place, on a real rotary cache."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import bf16_gpu, to_np
from oracle import quantization_oracle as O
from pageserve_amd import quantization as Q

pytestmark = pytest.mark.gpu


def _cache(max_len: int, head_dim: int, theta: float = 1e6):
    # the reference's cache construction (engine/model.py:42-47), on the CPU
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    t = torch.arange(max_len).float()
    emb = torch.cat((torch.outer(t, inv_freq),) * 2, dim=-1)
    return emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16)


def _case(gpu, m, qh, kh, hd, start, seed):
    rng = np.random.default_rng(seed)
    q = O.round_to_bf16(rng.standard_normal((m, qh, hd)).astype(np.float32) * np.float32(4.0))
    k = O.round_to_bf16(rng.standard_normal((m, kh, hd)).astype(np.float32) * np.float32(4.0)) if kh else None
    c, s = _cache(start + m, hd)
    c, s = c[start:start + m], s[start:start + m]
    return q, k, c, s


@pytest.mark.parametrize("m,qh,kh,hd,start", [
    (1, 16, 2, 128, 0), (1, 16, 2, 128, 4095), (7, 16, 2, 128, 33), (512, 16, 2, 128, 100),
    (3, 4, 0, 64, 9), (5, 3, 1, 24, 2), (2, 2, 2, 16, 1), (4, 14, 2, 64, 17)])
def test_rope_bit_exact(gpu, m, qh, kh, hd, start):
    q, k, c, s = _case(gpu, m, qh, kh, hd, start, m * 131 + hd)
    qt = bf16_gpu(q, gpu)
    kt = bf16_gpu(k, gpu) if k is not None else None
    ct, st = c.to(gpu), s.to(gpu)
    qo, ko = Q.rope_qk(qt, kt, ct, st)
    cf, sf = c.float().numpy(), s.float().numpy()
    assert np.array_equal(to_np(qo), O.rope(q, cf, sf))
    if k is not None:
        assert np.array_equal(to_np(ko), O.rope(k, cf, sf))
    else:
        assert ko is None
    # inputs untouched out of place; in place gives the same bits
    assert np.array_equal(to_np(qt), q)
    q2 = qt.clone()
    k2 = kt.clone() if kt is not None else None
    qi, ki = Q.rope_qk(q2, k2, ct, st, inplace=True)
    assert qi.data_ptr() == q2.data_ptr() and torch.equal(qi, qo)
    if k2 is not None:
        assert torch.equal(ki, ko)


def test_apply_rope_single_tensor_and_views(gpu):
    q, _, c, s = _case(gpu, 6, 8, 0, 128, 50, 7)
    qt = bf16_gpu(q, gpu)
    ct, st = c.to(gpu), s.to(gpu)
    want = O.rope(q, c.float().numpy(), s.float().numpy())
    assert np.array_equal(to_np(Q.apply_rope(qt, ct, st)), want)
    # a non-contiguous view of the same values (heads-major storage)
    qv = qt.transpose(0, 1).contiguous().transpose(0, 1)
    assert not qv.is_contiguous()
    assert np.array_equal(to_np(Q.apply_rope(qv, ct, st)), want)


def test_rope_errors(gpu):
    q = torch.zeros(2, 2, 10, dtype=torch.bfloat16, device=gpu)
    c = torch.ones(2, 10, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        Q.rope_qk(torch.zeros(2, 2, 9, dtype=torch.bfloat16, device=gpu), None, c[:, :9], c[:, :9])
    with pytest.raises(TypeError):
        Q.rope_qk(q.float(), None, c, c)
    with pytest.raises(ValueError):
        Q.rope_qk(q, None, c[:1], c[:1])
    with pytest.raises(ValueError):
        Q.rope_qk(q, torch.zeros(3, 2, 10, dtype=torch.bfloat16, device=gpu), c, c)


# seeded random soak: token counts, head counts, head_dim (even, vector and
# scalar paths), positions and theta
ROPE_CASES = int(__import__("os").environ.get("PGS_RANDOM_ROPE_CASES", "16"))


@pytest.mark.parametrize("i", range(ROPE_CASES))
def test_random_rope_bit_exact(gpu, i):
    rng = np.random.default_rng(50_000 + i)
    m, qh = int(rng.integers(1, 300)), int(rng.integers(1, 33))
    kh = int(rng.integers(0, qh + 1))
    hd = 2 * int(rng.integers(1, 129))
    start = int(rng.integers(0, 8192))
    theta = float(rng.choice([1e4, 1e6]))
    q = O.round_to_bf16(rng.standard_normal((m, qh, hd)).astype(np.float32) * np.float32(4.0))
    k = O.round_to_bf16(rng.standard_normal((m, kh, hd)).astype(np.float32) * np.float32(4.0)) if kh else None
    c, s = _cache(start + m, hd, theta)
    c, s = c[start:start + m], s[start:start + m]
    qo, ko = Q.rope_qk(bf16_gpu(q, gpu), bf16_gpu(k, gpu) if k is not None else None, c.to(gpu), s.to(gpu))
    cf, sf = c.float().numpy(), s.float().numpy()
    what = f"case {i}: m={m} qh={qh} kh={kh} hd={hd} start={start}"
    assert np.array_equal(to_np(qo), O.rope(q, cf, sf)), what
    if k is not None:
        assert np.array_equal(to_np(ko), O.rope(k, cf, sf)), what
