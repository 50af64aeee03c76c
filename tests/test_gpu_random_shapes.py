"""Seeded random shapes through every launch plan, against the oracle.

The plan picks kernels and tilings by token count m, output rows n and K
(skinny / paired split / K groups / tile sizes / split K / K-tail pointer
kernel); hand-picked shapes cover each branch once, this sweep covers their
combinations: ragged m and n, K a multiple of 16 (half of them of 64), bias
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

# PGS_RANDOM_CASES raises the count for a longer soak of the launch plans
CASES = int(os.environ.get("PGS_RANDOM_CASES", "40"))
MAX_WORK = 1.2e8  # m * n * k of the oracle's float64 product


def _case(i: int):
    rng = np.random.default_rng(10_000 + i)
    band = i % 4
    m = int(rng.integers(1, 17) if band == 0 else rng.integers(17, 129) if band == 1 else rng.integers(129, 700)
            if band == 2 else rng.integers(1, 700))
    k = 16 * int(rng.integers(1, 260))
    if i % 2 == 0:
        k = 64 * max(1, k // 64)
    n = int(rng.integers(1, 3200))
    while m * n * k > MAX_WORK:
        n = max(1, n // 2)
        if n == 1 and m * k > MAX_WORK:
            k = max(16, k // 2)
    kind = ["linear", "group", "swiglu", "residual"][int(rng.integers(0, 4))]
    return m, n, k, kind, bool(rng.integers(0, 2))


@pytest.mark.parametrize("i", range(CASES))
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
            report(to_np(y), O.linear(x, *O.quantize_per_channel(w), b), k, f"{what} member {j}")
        return
    w = weights(23_000 + i, n, k)
    q, s = O.quantize_per_channel(w)
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    if kind == "swiglu":
        w2 = weights(24_000 + i, n, k)
        act = Q.swiglu(xt, qw, Q.QuantizedWeight(torch.from_numpy(w2).to(gpu)))
        report(to_np(act), O.swiglu(x, q, s, *O.quantize_per_channel(w2)), k, what)
        return
    b = O.round_to_bf16(np.random.default_rng(25_000 + i).standard_normal(n).astype(np.float32)) if bias else None
    bt = bf16_gpu(b, gpu) if bias else None
    if kind == "residual":
        r = O.round_to_bf16(np.random.default_rng(26_000 + i).standard_normal((m, n)).astype(np.float32))
        y = qw.linear(xt, bt, residual=bf16_gpu(r, gpu))
        report(to_np(y), O.linear_residual(x, q, s, r, b), k, what, ulp_of=O.linear_residual_intermediate(x, q, s, b))
    else:
        y = qw.linear(xt, bt)
        report(to_np(y), O.linear(x, q, s, b), k, what)
