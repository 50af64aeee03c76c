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


@pytest.mark.parametrize("m", [1, 8, 256])
def test_lm_head_logits_and_argmax(gpu, lm_head, m):
    qw, q, s = lm_head
    x = activations(77 + m, m, HIDDEN)
    logits = qw.linear(bf16_gpu(x, gpu), out_dtype=torch.float32)
    assert logits.dtype == torch.float32 and logits.shape == (m, VOCAB)
    got = to_np(logits)
    rows = np.arange(m) if m <= 8 else np.random.default_rng(m).choice(m, 24, replace=False)
    ref = O.linear(x[rows], q, s)
    report(got[rows], ref, HIDDEN, f"lm_head m={m}", bf16_out=False)
    gap = O.top2_gap(ref)
    assert (gap > 1e-4).all(), f"near-tie in the oracle, argmax not decidable: {gap.min()}"
    np.testing.assert_array_equal(O.argmax_rows(got[rows]), O.argmax_rows(ref))
    # every row's argmax via the GPU's own argmax as the serving loop takes it
    assert torch.equal(logits.argmax(dim=-1).cpu(), torch.from_numpy(O.argmax_rows(got)))
