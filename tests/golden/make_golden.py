"""Writes tests/golden/gate_proj_4864x896.npz: a fixture for the single-linear
case (Qwen2.5-0.5B gate_proj shape): W fp32 [4864, 896] ~ N(0, 0.02), x bf16
[1, 896] ~ N(0, 1), quantized per output row and y = x (q s)^T.

The reference ships no golden vectors for engine/quantization.py, so this
fixture is built here from seeded inputs and the oracle, and every stored
quantizer row is checked first against the exact-arithmetic restatement in
tests/exact.py (rational quotient, IEEE rounding to fp32, round half to
even), independent of numpy's arithmetic.  Stored: the seeds and shapes, the
SHA-256 of the full q (int8 bytes) and scale (fp32 bytes), 48 sampled rows of
q and scale, and the fp32 y (float64 accumulation, rounded once).

Usage: python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from oracle import quantization_oracle as O  # noqa: E402
import exact  # noqa: E402

N, K, M = 4864, 896, 1
W_SEED, X_SEED, ROW_SEED = 20240, 20241, 20242
PATH = os.path.join(HERE, "gate_proj_4864x896.npz")


def inputs():
    w = (np.random.default_rng(W_SEED).standard_normal((N, K), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = O.round_to_bf16(np.random.default_rng(X_SEED).standard_normal((M, K), dtype=np.float32))
    return w, x


def sample_rows():
    rng = np.random.default_rng(ROW_SEED)
    return np.sort(np.concatenate([[0, 1, N - 1], rng.choice(np.arange(2, N - 1), 45, replace=False)]))


def sha(a: np.ndarray) -> np.ndarray:
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), dtype=np.uint8)


def main():
    w, x = inputs()
    q, s = O.quantize_per_channel(w)
    rows = sample_rows()
    for r in rows:
        q_ex, s_ex = exact.quantize_row(w[r])
        assert np.array_equal(np.asarray(q_ex, dtype=np.int8), q[r]), f"row {r}: q differs from the exact restatement"
        assert np.float32(s_ex).view(np.uint32) == s[r, 0].view(np.uint32), f"row {r}: scale differs"
    y = O.linear(x, q, s)
    np.savez_compressed(PATH, shape=np.array([N, K, M]), seeds=np.array([W_SEED, X_SEED, ROW_SEED]),
                        q_sha256=sha(q), scale_sha256=sha(s), rows=rows, q_rows=q[rows], scale_rows=s[rows],
                        y=y.astype(np.float32))
    print(f"wrote {PATH} ({os.path.getsize(PATH)} bytes); {len(rows)} rows checked against the exact restatement")


if __name__ == "__main__":
    main()
