"""The linears' neighbours on the GPU: the RMSNorm kernel (engine/model.py:29-34)
and the residual add in the linear epilogue (engine/model.py:184, 190),
against the oracle.

RMSNorm: every element inside the oracle's bracket (the formula evaluated
at every r within 4 fp32 ulps of the correctly rounded r: the fp32 sum of
squares is reduced in another order than the oracle's correctly rounded mean),
almost all equal to the oracle, and repeat calls identical.  Residual linear: within the linear tolerance of the oracle's
residual + bf16(linear); equal to the unfused kernel output plus a bf16 add
(same roundings).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import activations, bf16_gpu, report, to_np, weights
from oracle import quantization_oracle as O
from pageserve_amd import quantization as Q

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,k", [(1, 2048), (16, 2048), (512, 2048), (7, 896), (3, 100), (2, 11008), (1, 8)])
def test_rmsnorm_matches_oracle(gpu, m, k):
    rng = np.random.default_rng(m * 100 + k)
    x = O.round_to_bf16(rng.standard_normal((m, k), dtype=np.float32) * np.float32(2.0))
    w = O.round_to_bf16((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    xt, wt = bf16_gpu(x, gpu), bf16_gpu(w, gpu)
    h = Q.rmsnorm(xt, wt, 1e-6)
    assert h.dtype == torch.bfloat16 and h.shape == (m, k)
    ref = O.rmsnorm(x, w, 1e-6)
    got = to_np(h)
    lo, hi = O.rmsnorm_bracket(x, w, 1e-6)
    assert np.all((lo <= got) & (got <= hi)), f"outside the bracket at {np.argwhere((got < lo) | (got > hi))[:5]}"
    assert np.mean(got != ref) < 1e-3
    assert torch.equal(h, Q.rmsnorm(xt, wt, 1e-6))


def test_rmsnorm_leading_dims_and_zero_rows(gpu):
    x = np.zeros((2, 3, 64), np.float32)
    x[1, 2] = O.round_to_bf16(np.linspace(-3, 3, 64).astype(np.float32))
    w = np.ones(64, np.float32)
    h = Q.rmsnorm(bf16_gpu(x, gpu), bf16_gpu(w, gpu), 1e-5)
    assert h.shape == (2, 3, 64)
    got = to_np(h).reshape(6, 64)
    assert np.all(got[:5] == 0)
    np.testing.assert_array_equal(got[5], O.rmsnorm(x.reshape(6, 64)[5:], w, 1e-5)[0])


@pytest.mark.parametrize("m,n,k", [(1, 2048, 2048), (1, 2048, 11008), (3, 1000, 1040), (16, 2048, 2048),
                                   (40, 2048, 2048), (512, 2048, 11008), (100, 300, 208)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_linear_residual_matches_oracle(gpu, m, n, k, with_bias):
    seed = m + n + k + with_bias
    w = weights(seed, n, k)
    x = activations(seed + 1, m, k)
    r = O.round_to_bf16(np.random.default_rng(seed + 2).standard_normal((m, n)).astype(np.float32))
    b = O.round_to_bf16(np.random.default_rng(seed + 3).standard_normal(n).astype(np.float32)) if with_bias else None
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    q, s = O.quantize_per_channel(w)
    xt, rt = bf16_gpu(x, gpu), bf16_gpu(r, gpu)
    bt = bf16_gpu(b, gpu) if with_bias else None
    y = qw.linear(xt, bt, residual=rt)
    report(to_np(y), O.linear_residual(x, q, s, r, b), k, f"residual linear m={m} n={n} k={k}",
           ulp_of=O.linear_residual_intermediate(x, q, s, b))
    # same roundings as the unfused kernel followed by a bf16 add
    unfused = (qw.linear(xt, bt).float() + rt.float()).to(torch.bfloat16)
    assert torch.equal(y, unfused)


def test_linear_residual_in_place_and_fp32(gpu):
    m, n, k = 8, 2048, 2048
    w = weights(11, n, k)
    x = activations(12, m, k)
    r = O.round_to_bf16(np.random.default_rng(13).standard_normal((m, n)).astype(np.float32))
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    q, s = O.quantize_per_channel(w)
    xt = bf16_gpu(x, gpu)
    buf = bf16_gpu(r, gpu)
    out = qw.linear(xt, residual=buf, out=buf)  # x = residual + linear, in place
    assert out.data_ptr() == buf.data_ptr()
    report(to_np(buf), O.linear_residual(x, q, s, r), k, "in-place residual",
           ulp_of=O.linear_residual_intermediate(x, q, s))
    y32 = qw.linear(xt, residual=bf16_gpu(r, gpu), out_dtype=torch.float32)
    report(to_np(y32), O.linear_residual(x, q, s, r, bf16_out=False), k, "fp32 residual", bf16_out=False)


def test_decode_layer_neighbours_chain(gpu):
    """One decoder layer's linears with their neighbours, fused as the explicit
    API offers them: h = rmsnorm(x); q|k|v; x1 = x + o(a); h2 = rmsnorm(x1);
    x2 = x1 + down(swiglu(h2)) -- against the oracle chain (attention output
    a is an input here)."""
    H, I, KV, m = 512, 1408, 64, 2
    rng = np.random.default_rng(77)
    x = O.round_to_bf16(rng.standard_normal((m, H)).astype(np.float32))
    a = O.round_to_bf16(rng.standard_normal((m, H)).astype(np.float32))
    ln1 = O.round_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    ln2 = O.round_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    ws = {nm: weights(200 + j, n, kk) for j, (nm, n, kk) in enumerate(
        [("q", H, H), ("k", KV, H), ("v", KV, H), ("o", H, H), ("g", I, H), ("u", I, H), ("d", H, I)])}
    qs = {nm: O.quantize_per_channel(w) for nm, w in ws.items()}
    qw = {nm: Q.QuantizedWeight(torch.from_numpy(w).to(gpu)) for nm, w in ws.items()}
    xt = bf16_gpu(x, gpu)
    h = Q.rmsnorm(xt, bf16_gpu(ln1, gpu), 1e-6)
    qkv = Q.linear_group(h, [qw["q"], qw["k"], qw["v"]])
    x1 = qw["o"].linear(bf16_gpu(a, gpu), residual=xt)
    h2 = Q.rmsnorm(x1, bf16_gpu(ln2, gpu), 1e-6)
    x2 = Q.mlp(h2, qw["g"], qw["u"], qw["d"], residual=x1)
    # oracle chain (fed with the kernel's own intermediate where rounding
    # boundaries could otherwise diverge by one ulp)
    for j, nm in enumerate("qkv"):
        report(to_np(qkv[j]), O.linear(to_np(h), *qs[nm]), H, f"layer {nm}", acc=O.acc_bound(to_np(h), *qs[nm]))
    lo, hi = O.rmsnorm_bracket(x, ln1, 1e-6)
    assert ((lo <= to_np(h)) & (to_np(h) <= hi)).all(), "layer rmsnorm 1 outside the oracle's bracket"
    report(to_np(x1), O.linear_residual(a, *qs["o"], x), H, "layer o + residual",
           ulp_of=O.linear_residual_intermediate(a, *qs["o"]))
    lo, hi = O.rmsnorm_bracket(to_np(x1), ln2, 1e-6)
    assert ((lo <= to_np(h2)) & (to_np(h2) <= hi)).all(), "layer rmsnorm 2 outside the oracle's bracket"
    act = O.swiglu(to_np(h2), *qs["g"], *qs["u"])
    report(to_np(x2), O.linear_residual(O.round_to_bf16(act), *qs["d"], to_np(x1)), I, "layer down + residual",
           ulp_of=O.linear_residual_intermediate(O.round_to_bf16(act), *qs["d"]))


# seeded random soak of the RMSNorm kernel: rows, widths (vector and scalar
# paths), magnitudes and eps
NORM_CASES = int(__import__("os").environ.get("PGS_RANDOM_RMSNORM_CASES", "16"))


@pytest.mark.parametrize("i", range(NORM_CASES))
def test_random_rmsnorm(gpu, i):
    rng = np.random.default_rng(60_000 + i)
    m, k = int(rng.integers(1, 400)), int(rng.integers(1, 9000))
    scale = np.float32(10.0 ** rng.uniform(-3, 3))
    x = O.round_to_bf16(rng.standard_normal((m, k), dtype=np.float32) * scale)
    w = O.round_to_bf16((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    eps = float(rng.choice([1e-6, 1e-5, 0.0]))
    got = to_np(Q.rmsnorm(bf16_gpu(x, gpu), bf16_gpu(w, gpu), eps))
    ref = O.rmsnorm(x, w, eps)
    lo, hi = O.rmsnorm_bracket(x, w, eps)
    what = f"case {i}: m={m} k={k} scale={scale:.3g} eps={eps}"
    out = np.argwhere((got < lo) | (got > hi))
    assert out.size == 0, f"{what}: outside the bracket at {out[:5].tolist()}"
    assert np.mean(got != ref) < 1e-2, what
