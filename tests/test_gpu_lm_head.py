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


@pytest.mark.parametrize("m", [1, 8])
def test_fused_argmax_lm_head(gpu, lm_head, m):
    """Q.linear_argmax (the argmax reduced inside the projection, no logits
    written) on the full lm_head: every row's index equals the oracle's
    argmax (decided: top-2 gap above twice the kernel's logit error) and
    torch's argmax of the fp32 logits of Q.linear, and the returned maximum
    is bit-equal to that logit."""
    qw, q, s = lm_head
    x = activations(177 + m, m, HIDDEN)
    xs = bf16_gpu(x, gpu)
    idx, vmax = Q.linear_argmax(xs, qw, return_values=True)
    assert idx.dtype == torch.int64 and idx.shape == (m,) and vmax.dtype == torch.float32
    logits = qw.linear(xs, out_dtype=torch.float32)
    ref = _oracle_blocked(x, q, s)
    worst = float(np.abs(to_np(logits) - ref).max())
    assert (O.top2_gap(ref) > 2 * worst).all()
    np.testing.assert_array_equal(idx.cpu().numpy(), O.argmax_rows(ref))
    np.testing.assert_array_equal(idx.cpu().numpy(), logits.argmax(dim=-1).cpu().numpy())
    picked = logits.gather(1, idx.view(-1, 1)).view(-1)
    assert torch.equal(vmax.view(torch.int32), picked.view(torch.int32))


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 12, 16, 17, 24, 32])
def test_fused_argmax_every_plan(gpu, m):
    """Every skinny plan the argmax rides on (folded at 1..2 tokens, staged
    3..8 and 9..16, two token blocks 17..32), with a bias and a ragged
    vocabulary: indices equal torch's argmax of the same kernel's fp32
    logits, maxima bit-equal, and both equal the oracle's where decided."""
    n, k = 5000 + 8, 2048
    rng = np.random.default_rng(4242 + m)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    b = O.round_to_bf16(rng.standard_normal(n).astype(np.float32))
    q, s = O.quantize_per_channel(w)
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    x = activations(500 + m, m, k)
    xs, bt = bf16_gpu(x, gpu), bf16_gpu(b, gpu)
    idx, vmax = Q.linear_argmax(xs, qw, bt, return_values=True)
    logits = qw.linear(xs, bt, out_dtype=torch.float32)
    np.testing.assert_array_equal(idx.cpu().numpy(), logits.argmax(dim=-1).cpu().numpy())
    assert torch.equal(vmax.view(torch.int32), logits.gather(1, idx.view(-1, 1)).view(-1).view(torch.int32))
    ref = O.linear(x, q, s, b)
    decided = O.top2_gap(ref) > 2 * float(np.abs(to_np(logits) - ref).max())
    np.testing.assert_array_equal(idx.cpu().numpy()[decided], O.argmax_rows(ref)[decided])


def test_fused_argmax_ties_and_nan(gpu):
    """torch.argmax's choices: duplicated weight rows give equal logits and
    the first index wins; a token whose activations hold a NaN has all-NaN
    logits and gets index 0 (NaN counts as the maximum); other tokens are
    unaffected."""
    n, k = 700, 1024
    rng = np.random.default_rng(99)
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    # rows 611 and 613 copy row 600, whose scale is then the largest
    w[600] *= 4.0
    w[611] = w[600]
    w[613] = w[600]
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    x = np.zeros((3, k), dtype=np.float32)
    x[0] = O.round_to_bf16(np.sign(w[600]).astype(np.float32))  # aligns with row 600 (and its copies)
    x[1] = x[0]
    x[1, 5] = np.nan
    x[2] = -x[0]
    xs = bf16_gpu(x, gpu)
    idx, vmax = Q.linear_argmax(xs, qw, return_values=True)
    logits = qw.linear(xs, out_dtype=torch.float32)
    assert int(idx[0]) == 600 and float(logits[0, 611]) == float(logits[0, 600])
    assert int(idx[1]) == 0 and torch.isnan(vmax[1])
    assert int(idx[2]) == int(logits[2].argmax())
    np.testing.assert_array_equal(idx.cpu().numpy()[[0, 2]], logits.argmax(dim=-1).cpu().numpy()[[0, 2]])


def test_fused_argmax_rejects_too_many_rows(gpu, lm_head):
    qw, _, _ = lm_head
    with pytest.raises(ValueError, match="1..32"):
        Q.linear_argmax(bf16_gpu(activations(3, 33, HIDDEN), gpu), qw)
