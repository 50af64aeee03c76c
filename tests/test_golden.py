"""The committed 4864x896 gate_proj fixture (tests/golden/gate_proj_4864x896.npz, made by
tests/golden/make_golden.py): W fp32 [4864, 896] ~ N(0, 0.02), x bf16 [1, 896].

CPU: the oracle regenerates the fixture from its seeds (full q and scale by
SHA-256, sampled rows element for element, y within fp32 rounding), and the
sampled rows agree with the exact-arithmetic restatement.
GPU: the quantizer kernel reproduces the fixture's q and scale bit for bit,
the packed storage unpacks to it, and the fused linear matches y within the
specification's tolerance.
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import exact  # noqa: E402
import make_golden as G  # noqa: E402
from helpers import report  # noqa: E402
from oracle import quantization_oracle as O  # noqa: E402


@pytest.fixture(scope="module")
def fixture():
    with np.load(G.PATH, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _sha(a: np.ndarray) -> np.ndarray:
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), dtype=np.uint8)


def test_fixture_describes_the_4864x896_linear(fixture):
    assert tuple(fixture["shape"]) == (G.N, G.K, G.M) == (4864, 896, 1)
    assert tuple(fixture["seeds"]) == (G.W_SEED, G.X_SEED, G.ROW_SEED)
    assert np.array_equal(fixture["rows"], G.sample_rows())


def test_oracle_reproduces_the_fixture(fixture):
    w, x = G.inputs()
    q, s = O.quantize_per_channel(w)
    assert np.array_equal(_sha(q), fixture["q_sha256"]) and np.array_equal(_sha(s), fixture["scale_sha256"])
    rows = fixture["rows"]
    assert np.array_equal(q[rows], fixture["q_rows"])
    assert np.array_equal(s[rows].view(np.uint32), fixture["scale_rows"].view(np.uint32))
    y = O.linear(x, q, s)
    np.testing.assert_allclose(y, fixture["y"], rtol=1e-6, atol=1e-7)


def test_fixture_rows_match_exact_arithmetic(fixture):
    w, _ = G.inputs()
    for i, r in enumerate(fixture["rows"][:12]):
        q_ex, s_ex = exact.quantize_row(w[r])
        assert np.array_equal(np.asarray(q_ex, dtype=np.int8), fixture["q_rows"][i])
        assert np.float32(s_ex).view(np.uint32) == fixture["scale_rows"][i, 0].view(np.uint32)


@pytest.mark.gpu
def test_gpu_reproduces_the_fixture(gpu, fixture):
    from pageserve_amd import quantization as Q

    w, x = G.inputs()
    q, s = Q.quantize_per_channel(torch.from_numpy(w).to(gpu))
    q, s = q.cpu().numpy(), s.cpu().numpy()
    assert np.array_equal(_sha(q), fixture["q_sha256"]), "kernel q differs from the fixture"
    assert np.array_equal(_sha(s), fixture["scale_sha256"]), "kernel scale differs from the fixture"
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    assert np.array_equal(_sha(qw.q.cpu().numpy()), fixture["q_sha256"])
    xt = torch.from_numpy(O.f32_to_bf16_bits(x).view(np.int16).copy()).view(torch.bfloat16).to(gpu)
    y = qw.linear(xt)
    report(y.float().cpu().numpy(), fixture["y"], G.K, "4864x896 linear vs fixture",
           acc=O.acc_bound(x, *O.quantize_per_channel(w)))
