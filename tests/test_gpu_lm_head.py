"""INT8 lm_head (engine/model.py:193 with the quantizer applied to its weight):
W [151936, 2048], x [m, 2048] at m = 1, 8, 256, fp32 logits; the argmax of
every row must equal the oracle's exactly (server.py:47-51 consumes it)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import activations, bf16_gpu, report, to_np
from oracle import quantization_oracle as O
from pageserve_amd import quantization as Q

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN = 151936, 2048


@pytest.fixture(scope="module")
def lm_head(gpu):
    rng = np.random.default_rng(151936)
    w = (rng.standard_normal((VOCAB, HIDDEN), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    q, s = O.quantize_per_channel(w)
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    assert torch.equal(qw.q.cpu(), torch.from_numpy(q)) and torch.equal(qw.scale.cpu(), torch.from_numpy(s))
    del w
    return qw, q, s


def _oracle_blocked(x: np.ndarray, q: np.ndarray, s: np.ndarray, block: int = 16384) -> np.ndarray:
    """O.linear over the vocabulary in blocks of rows (the float64 dequantized
    weight of one block at a time stays a few hundred MB)."""
    return np.concatenate([O.linear(x, q[i:i + block], s[i:i + block]) for i in range(0, q.shape[0], block)], axis=1)


@pytest.mark.parametrize("m", [1, 8, 256])
def test_lm_head_logits_and_argmax(gpu, lm_head, m):
    """Every row: fp32 logits within the tolerance of the oracle's, and the
    argmax (server.py:51 takes it) equal to the oracle's; rows whose top two
    oracle logits are too close to decide are reported, not skipped."""
    qw, q, s = lm_head
    x = activations(77 + m, m, HIDDEN)
    logits = qw.linear(bf16_gpu(x, gpu), out_dtype=torch.float32)
    assert logits.dtype == torch.float32 and logits.shape == (m, VOCAB)
    got = to_np(logits)
    ref = _oracle_blocked(x, q, s)
    report(got, ref, HIDDEN, f"lm_head m={m}", bf16_out=False)
    gap = O.top2_gap(ref)
    # the kernel's fp32 logits sit within the accumulation bound of the exact
    # ones: a gap above twice the largest bound decides the argmax
    worst = float(np.abs(got - ref).max())
    assert (gap > 2 * worst).all(), f"near-tie in the oracle: gap {gap.min()} vs error {worst}"
    np.testing.assert_array_equal(O.argmax_rows(got), O.argmax_rows(ref))
    # and through torch's own argmax on the GPU, as the serving loop takes it
    np.testing.assert_array_equal(logits.argmax(dim=-1).cpu().numpy(), O.argmax_rows(ref))
