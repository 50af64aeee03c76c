"""Pins of the oracle's restatement of the linears' neighbours
(engine/model.py:29-34 rms_norm; :184, :190 residual adds), on the CPU.

rms_norm is checked against torch running the reference's own op sequence
on the CPU (x.float(), pow(2).mean(-1), rsqrt, cast back, multiply by the
weight) -- an independent implementation of the same formula -- plus closed
forms and planted mistakes that must fail.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quantization_oracle as O


def _torch_rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """The reference's op sequence, run by torch on the CPU in bf16."""
    xt = torch.from_numpy(O.f32_to_bf16_bits(x).view(np.int16).copy()).view(torch.bfloat16)
    wt = torch.from_numpy(O.f32_to_bf16_bits(w).view(np.int16).copy()).view(torch.bfloat16)
    dtype = xt.dtype
    xf = xt.float()
    variance = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(variance + eps)
    return (wt * xf.to(dtype)).float().numpy()


def _inputs(seed, m, k):
    rng = np.random.default_rng(seed)
    x = O.round_to_bf16(rng.standard_normal((m, k), dtype=np.float32) * np.float32(3.0))
    w = O.round_to_bf16((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    return x, w


@pytest.mark.parametrize("m,k", [(1, 2048), (7, 896), (16, 2048), (3, 100)])
def test_rmsnorm_matches_torch_running_the_reference_ops(m, k):
    x, w = _inputs(m + k, m, k)
    h = O.rmsnorm(x, w, 1e-6)
    ref = _torch_rms_norm(x, w, 1e-6)
    diff = np.abs(h - ref)
    # the fp32 reductions differ in order: at most one bf16 ulp, and rarely
    assert np.all(diff <= O.bf16_ulp(ref) + 0.0), diff.max()
    assert np.mean(diff > 0) < 1e-3


def test_rmsnorm_closed_forms():
    k = 64
    ones = np.ones((1, k), np.float32)
    # constant row c: var = c^2, x * r = 1/sqrt(1 + eps/c^2) -> 1.0 in bf16
    for c in (1.0, -2.5, 1024.0):
        h = O.rmsnorm(ones * np.float32(c), ones, 1e-6)
        assert np.all(h == np.float32(np.sign(c)))
    # zero row: rsqrt(eps) * 0 = 0
    assert np.all(O.rmsnorm(np.zeros((1, k), np.float32), ones, 1e-6) == 0)
    # the weight multiplies elementwise
    w = O.round_to_bf16(np.linspace(-2, 2, k).astype(np.float32))
    assert np.array_equal(O.rmsnorm(ones, w, 0.0)[0], w)


@pytest.mark.parametrize("mutant", ["no_inner_rounding", "no_eps", "sum_not_mean", "sqrt_not_rsqrt"])
def test_rmsnorm_planted_mistakes_fail(mutant):
    x, w = _inputs(5, 4, 256)
    eps = 1e-1  # large enough that dropping it shows
    ref = _torch_rms_norm(x, w, eps)
    xf = x.astype(np.float64)
    var = np.mean(xf ** 2, axis=-1, keepdims=True)
    if mutant == "no_inner_rounding":
        h = O.round_to_bf16((w * (x * (1 / np.sqrt(var + eps))).astype(np.float32)).astype(np.float32))
    elif mutant == "no_eps":
        h = O.round_to_bf16((w * O.round_to_bf16((x / np.sqrt(var)).astype(np.float32))).astype(np.float32))
    elif mutant == "sum_not_mean":
        s = np.sum(xf ** 2, axis=-1, keepdims=True)
        h = O.round_to_bf16((w * O.round_to_bf16((x / np.sqrt(s + eps)).astype(np.float32))).astype(np.float32))
    else:
        h = O.round_to_bf16((w * O.round_to_bf16((x * np.sqrt(var + eps)).astype(np.float32))).astype(np.float32))
    assert np.mean(h != ref) > 1e-3


def test_linear_residual_closed_forms():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((32, 64)) * 0.02).astype(np.float32)
    q, s = O.quantize_per_channel(w)
    x = O.round_to_bf16(rng.standard_normal((2, 64)).astype(np.float32))
    zero = np.zeros((2, 32), np.float32)
    # zero residual: the bf16-rounded linear
    assert np.array_equal(O.linear_residual(x, q, s, zero), O.round_to_bf16(O.linear(x, q, s)))
    # zero input: the residual itself
    r = O.round_to_bf16(rng.standard_normal((2, 32)).astype(np.float32))
    assert np.array_equal(O.linear_residual(np.zeros_like(x), q, s, r), r)
    # fp32 output: plain sum
    np.testing.assert_array_equal(O.linear_residual(x, q, s, r, bf16_out=False), O.linear(x, q, s) + r)


def test_rmsnorm_bracket_holds_torch_and_the_oracle():
    """The bracket of r within 4 fp32 ulps contains the oracle itself and
    torch's CPU rms_norm (another reduction order) on every element, and is
    tight: a planted mistake (no inner rounding) leaves it."""
    for seed, (m, k) in enumerate([(64, 2048), (33, 896), (8, 11008), (100, 100)]):
        x, w = _inputs(700 + seed, m, k)
        lo, hi = O.rmsnorm_bracket(x, w, 1e-6)
        for h in (O.rmsnorm(x, w, 1e-6), _torch_rms_norm(x, w, 1e-6)):
            assert np.all((lo <= h) & (h <= hi))
        assert np.mean(lo == hi) > 0.95
        xf = np.asarray(x, np.float32)
        var = np.mean(xf.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
        r = (1.0 / np.sqrt((var + np.float32(1e-6)).astype(np.float64))).astype(np.float32)
        mutant = O.round_to_bf16((w * (xf * r)).astype(np.float32))  # no inner bf16 rounding
        assert not np.all((lo <= mutant) & (mutant <= hi))
