"""Seeded random shapes through every launch plan, against the oracle.

The plan picks kernels and tilings by token count m, output rows n and K
(skinny / paired split / K groups / tile sizes / split K / K-tail pointer
kernel); hand-picked shapes cover each branch once, this sweep covers their
combinations: ragged m and n, K a multiple of 16 (half of them of 64; up to
8304, so the long-K split plans are drawn too), bias
on and off, single linears, q|k|v-style groups, the SwiGLU pair and the
residual epilogue.  Sizes are capped so the float64 oracle stays fast.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from helpers import activations, bf16_gpu, report, to_np, weights
from oracle import quantization_oracle as O
from pageserve_amd import quantization as Q

pytestmark = pytest.mark.gpu

# PGS_RANDOM_CASES raises the count for a longer soak of the launch plans;
# PGS_RANDOM_START moves the window of seeded cases
CASES = int(os.environ.get("PGS_RANDOM_CASES", "40"))
START = int(os.environ.get("PGS_RANDOM_START", "0"))
MAX_WORK = 1.2e8  # m * n * k of the oracle's float64 product


def _case(i: int):
    rng = np.random.default_rng(10_000 + i)
    band = i % 4
    m = int(rng.integers(1, 17) if band == 0 else rng.integers(17, 129) if band == 1 else rng.integers(129, 700)
            if band == 2 else rng.integers(1, 700))
    k = 16 * int(rng.integers(1, 520))  # up to 8304: long-K split plans too
    if i % 2 == 0:
        k = 64 * max(1, k // 64)
    n = int(rng.integers(1, 3200))
    while m * n * k > MAX_WORK:
        n = max(1, n // 2)
        if n == 1 and m * k > MAX_WORK:
            k = max(16, k // 2)
    kind = ["linear", "group", "swiglu", "residual"][int(rng.integers(0, 4))]
    return m, n, k, kind, bool(rng.integers(0, 2))


@pytest.mark.parametrize("i", range(START, START + CASES))
def test_random_shape(gpu, i):
    m, n, k, kind, bias = _case(i)
    what = f"case {i}: {kind} m={m} n={n} k={k} bias={bias}"
    x = activations(20_000 + i, m, k)
    xt = bf16_gpu(x, gpu)
    if kind == "group":
        ns = [n, max(1, n // 3), max(1, (2 * n) // 5)]
        ws = [weights(21_000 + 10 * i + j, nn, k) for j, nn in enumerate(ns)]
        bs = [O.round_to_bf16(np.random.default_rng(22_000 + 10 * i + j).standard_normal(nn).astype(np.float32))
              if bias else None for j, nn in enumerate(ns)]
        qws = [Q.QuantizedWeight(torch.from_numpy(w).to(gpu)) for w in ws]
        ys = Q.linear_group(xt, qws, [bf16_gpu(b, gpu) if b is not None else None for b in bs])
        for j, (w, b, y) in enumerate(zip(ws, bs, ys)):
            report(to_np(y), O.linear(x, *O.quantize_per_channel(w), b), k, f"{what} member {j}", acc=O.acc_bound(x, *O.quantize_per_channel(w), b))
        return
    w = weights(23_000 + i, n, k)
    q, s = O.quantize_per_channel(w)
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    if kind == "swiglu":
        w2 = weights(24_000 + i, n, k)
        act = Q.swiglu(xt, qw, Q.QuantizedWeight(torch.from_numpy(w2).to(gpu)))
        report(to_np(act), O.swiglu(x, q, s, *O.quantize_per_channel(w2)), k, what, acc=O.swiglu_acc(x, q, s, *O.quantize_per_channel(w2)))
        return
    b = O.round_to_bf16(np.random.default_rng(25_000 + i).standard_normal(n).astype(np.float32)) if bias else None
    bt = bf16_gpu(b, gpu) if bias else None
    if kind == "residual":
        r = O.round_to_bf16(np.random.default_rng(26_000 + i).standard_normal((m, n)).astype(np.float32))
        y = qw.linear(xt, bt, residual=bf16_gpu(r, gpu))
        report(to_np(y), O.linear_residual(x, q, s, r, b), k, what, ulp_of=O.linear_residual_intermediate(x, q, s, b))
    else:
        y = qw.linear(xt, bt)
        report(to_np(y), O.linear(x, q, s, b), k, what, acc=O.acc_bound(x, q, s, b))


# rms_norm fused into the projections (engine/model.py:166-170, 187-189):
# random token counts around the fused / unfused boundary (4 tokens), K with
# and without K % 64 == 0, groups and the SwiGLU pair
NORM_CASES = int(os.environ.get("PGS_RANDOM_NORM_CASES", "24"))


def _norm_case(i: int):
    rng = np.random.default_rng(30_000 + i)
    m = int(rng.integers(1, 9) if i % 2 == 0 else rng.integers(1, 40))
    k = 64 * int(rng.integers(1, 80)) if i % 3 else 16 * int(rng.integers(1, 300))
    n = int(rng.integers(1, 3000))
    while m * n * k > MAX_WORK:
        n = max(1, n // 2)
    return m, n, k, ["group", "swiglu"][int(rng.integers(0, 2))], float(rng.choice([1e-6, 1e-5, 0.0]))


@pytest.mark.parametrize("i", range(NORM_CASES))
def test_random_fused_norm(gpu, i):
    m, n, k, kind, eps = _norm_case(i)
    what = f"norm case {i}: {kind} m={m} n={n} k={k} eps={eps}"
    rng = np.random.default_rng(31_000 + i)
    x = O.round_to_bf16(rng.standard_normal((m, k), dtype=np.float32) * np.float32(2.0))
    w = O.round_to_bf16((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))
    # entries whose squares sum exactly in fp32 in any order: fused == unfused bit for bit
    xe = rng.choice(np.array([0.5, -0.5, 1.0, -1.0, 2.0, -2.0], np.float32), size=(m, k))
    xt, xet, wt = bf16_gpu(x, gpu), bf16_gpu(xe, gpu), bf16_gpu(w, gpu)
    h, dh = O.rmsnorm(x, w, eps), O.rmsnorm_dx(x, w, eps)
    if kind == "group":
        ns = [n, max(1, n // 4)]
        ws = [weights(32_000 + 10 * i + j, nn, k) for j, nn in enumerate(ns)]
        qws = [Q.QuantizedWeight(torch.from_numpy(v).to(gpu)) for v in ws]
        bs = [O.round_to_bf16(rng.standard_normal(nn).astype(np.float32)) for nn in ns] if i % 4 < 2 else [None] * 2
        bts = [bf16_gpu(b, gpu) if b is not None else None for b in bs]
        ys = Q.rmsnorm_linear_group(xt, wt, eps, qws, bts)
        for j, (v, b, y) in enumerate(zip(ws, bs, ys)):
            q, s = O.quantize_per_channel(v)
            report(to_np(y), O.linear(h, q, s, b), k, f"{what} output {j}", acc=O.acc_bound(h, q, s, b, dx=dh))
        fused = Q.rmsnorm_linear_group(xet, wt, eps, qws, bts)
        plain = Q.linear_group(Q.rmsnorm(xet, wt, eps), qws, bts)
        assert all(torch.equal(a, b) for a, b in zip(fused, plain)), what
    else:
        wg, wu = weights(33_000 + i, n, k), weights(34_000 + i, n, k)
        g, u = Q.QuantizedWeight(torch.from_numpy(wg).to(gpu)), Q.QuantizedWeight(torch.from_numpy(wu).to(gpu))
        act = Q.rmsnorm_swiglu(xt, wt, eps, g, u)
        qg, qu = O.quantize_per_channel(wg), O.quantize_per_channel(wu)
        report(to_np(act), O.swiglu(h, *qg, *qu), k, what, acc=O.swiglu_acc(h, *qg, *qu, dx=dh))
        assert torch.equal(Q.rmsnorm_swiglu(xet, wt, eps, g, u), Q.swiglu(Q.rmsnorm(xet, wt, eps), g, u)), what


# the fused row argmax of the lm_head (server.py:51 after engine/model.py:193):
# random token counts over every skinny plan it rides on (1..32), ragged
# vocabularies, K with and without K % 64 == 0, bias on and off.  The checks
# hold for any summation order (O.acc_bound bounds every fp32 evaluation):
# the returned maximum lies within the bound of the exact logit at the
# returned index, that index can be the maximum of some evaluation within
# the bounds, and where the winner is decided it is the oracle's argmax.
ARGMAX_CASES = int(os.environ.get("PGS_RANDOM_ARGMAX_CASES", "16"))


def _argmax_case(i: int):
    rng = np.random.default_rng(40_000 + i)
    m = int(rng.integers(1, 33))
    k = 16 * int(rng.integers(1, 200))
    if i % 2 == 0:
        k = 64 * max(1, k // 64)
    n = int(rng.integers(1, 9000))
    while m * n * k > MAX_WORK:
        n = max(1, n // 2)
    return m, n, k, bool(rng.integers(0, 2))


@pytest.mark.parametrize("i", range(ARGMAX_CASES))
def test_random_argmax(gpu, i):
    m, n, k, bias = _argmax_case(i)
    what = f"argmax case {i}: m={m} n={n} k={k} bias={bias}"
    rng = np.random.default_rng(41_000 + i)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    b = O.round_to_bf16(rng.standard_normal(n).astype(np.float32)) if bias else None
    x = activations(42_000 + i, m, k)
    q, s = O.quantize_per_channel(w)
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    idx, vmax = Q.linear_argmax(bf16_gpu(x, gpu), qw, bf16_gpu(b, gpu) if bias else None, return_values=True)
    idx, vmax = idx.cpu().numpy(), vmax.cpu().numpy().astype(np.float64)
    exact = np.asarray(x, np.float64) @ O.dequantize(q, s, "f32").astype(np.float64).T
    if bias:
        exact = exact + np.asarray(b, np.float64).reshape(1, -1)
    acc = O.acc_bound(x, q, s, b)
    rows = np.arange(m)
    assert idx.shape == (m,) and np.all((idx >= 0) & (idx < n)), what
    assert np.all(np.abs(vmax - exact[rows, idx]) <= acc[rows, idx]), what
    assert np.all(exact[rows, idx] + acc[rows, idx] >= (exact - acc).max(axis=1)), what
    best = O.argmax_rows(exact)
    lo = exact[rows, best] - acc[rows, best]
    others = np.where(np.arange(n)[None, :] == best[:, None], -np.inf, exact + acc)
    decided = lo > others.max(axis=1) if n > 1 else np.ones(m, bool)
    np.testing.assert_array_equal(idx[decided], best[decided], err_msg=what)
