"""Routing logic of ``QuantizedWeight.get()``'s tensor view, on the CPU.

``F.linear(x_bf16, w.get(), b)`` (engine/model.py:168-190 through _resolve,
engine/model.py:25-26) must reach the fused linear entry point; metadata reads
must not materialise anything; every other op must see the dense weight.
The kernels are stubbed here: this checks host dispatch only.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import quantization_oracle as O
from pageserve_amd.quantization import W8A16Weight


class FakeQW:
    """Stands in for a GPU QuantizedWeight: records calls, no kernels."""

    def __init__(self, dtype=torch.bfloat16):
        self.q = torch.randint(-127, 128, (6, 16), dtype=torch.int8)
        self.qp = self.q  # only its device is read by the view
        self.shape = self.q.shape
        self.scale = torch.rand(6, 1) * 0.01
        self.dtype = dtype
        self.calls = []

    def dense(self):
        self.calls.append("dense")
        return (self.q.float() * self.scale).to(self.dtype)

    def linear(self, x, bias=None):
        self.calls.append("linear")
        return F.linear(x, self.dense(), bias)


def test_f_linear_reaches_the_fused_entry_point():
    qw = FakeQW()
    w = W8A16Weight(qw)
    assert w.shape == (6, 16) and w.dtype == torch.bfloat16 and w.device.type == "cpu"
    assert qw.calls == []  # metadata only
    x = torch.randn(3, 16).to(torch.bfloat16)
    b = torch.randn(6).to(torch.bfloat16)
    y = F.linear(x, w, b)
    assert qw.calls[0] == "linear"
    assert type(y) is torch.Tensor and y.shape == (3, 6)
    qw.calls.clear()
    F.linear(x, w)
    F.linear(input=x, weight=w, bias=b)
    assert qw.calls.count("linear") == 2


def test_other_ops_get_the_dense_weight():
    qw = FakeQW()
    w = W8A16Weight(qw)
    dense = (qw.q.float() * qw.scale).to(torch.bfloat16)
    assert torch.equal(w + 0, dense)
    assert torch.equal(w.t().contiguous(), dense.t().contiguous())
    assert type(w.float()) is torch.Tensor
    assert "linear" not in qw.calls and "dense" in qw.calls


def test_non_bf16_activations_use_the_dense_weight():
    qw = FakeQW(dtype=torch.float32)
    w = W8A16Weight(qw)
    x = torch.randn(2, 16)
    y = F.linear(x, w)
    assert "linear" not in qw.calls
    torch.testing.assert_close(y, x @ (qw.q.float() * qw.scale).T)


def test_metadata_reads_do_not_materialise():
    qw = FakeQW()
    w = W8A16Weight(qw)
    _ = (w.shape, w.dtype, w.device, w.dim(), w.size(0), w.ndim, w.is_cuda, w.requires_grad, repr(w))
    assert qw.calls == []


def test_compare_floors_bf16_outputs_at_half_an_ulp():
    ref = np.array([10.0, 0.5, -3.0], dtype=np.float32)
    # half a bf16 ulp at 10.0 is 0.03125 > 2e-2*sqrt(2): allowed only for a bf16 output
    y = ref + np.array([0.03125, 0.0, 0.0], dtype=np.float32)
    assert not O.compare(y, ref, 2048)["ok"]
    assert O.compare(y, ref, 2048, bf16_out=True, acc=0.0)["ok"]
    # a whole ulp is a wrong rounding, not a rounding of the right value
    y1 = ref + np.array([0.0625, 0.0, 0.0], dtype=np.float32)
    assert not O.compare(y1, ref, 2048, bf16_out=True, acc=0.0)["ok"]
    # the accumulation bound widens the floor elementwise, and only by itself
    y2 = ref + np.array([0.04, 0.0, 0.0], dtype=np.float32)
    assert O.compare(y2, ref, 2048, bf16_out=True, acc=np.array([0.01, 0.0, 0.0]))["ok"]
    assert not O.compare(y2, ref, 2048, bf16_out=True, acc=np.array([0.005, 0.0, 0.0]))["ok"]
    # small values keep the specification's absolute bound
    y3 = ref + np.array([0.0, 0.03, 0.0], dtype=np.float32)
    assert not O.compare(y3, ref, 2048, bf16_out=True, acc=0.0)["ok"]
    # a single-rounding bf16 comparison must state its accumulation bound
    with pytest.raises(ValueError, match="accumulation bound"):
        O.compare(y, ref, 2048, bf16_out=True)


def test_compare_floor_across_a_power_of_two_and_for_a_rounded_intermediate():
    # reference just below 8.0 (bf16 spacing 2^-5 there), result 8.0 (the fp32
    # sum landed on the other side of the midpoint): a quarter ulp of the upper
    # binade apart, which a K = 16 bound (0.005) cannot resolve; the next bf16
    # value above 8 is a wrong rounding
    ref = np.array([8 - 2 ** -6, 0.25], dtype=np.float32)
    assert O.compare(np.array([8.0, 0.25], np.float32), ref, 16, bf16_out=True, acc=0.0)["ok"]
    assert not O.compare(np.array([8.0625, 0.25], np.float32), ref, 16, bf16_out=True, acc=0.0)["ok"]
    # residual + bf16(linear) cancelling to a small sum: a one-ulp step of the
    # intermediate (3.0 -> ulp 2^-6) is allowed only when the intermediate is given
    # (a second element of typical size keeps the relative bound, max|dy| / max|ref|, out of the way)
    ref2 = np.array([0.1015625, 4.0], dtype=np.float32)
    inter = np.array([3.0, 1.0])
    step = np.array([2 ** -6, 0.0], dtype=np.float32)
    assert not O.compare(ref2 + step, ref2, 128, bf16_out=True, acc=0.0)["ok"]
    assert O.compare(ref2 + step, ref2, 128, bf16_out=True, ulp_of=inter)["ok"]
    assert not O.compare(ref2 + 2 * step, ref2, 128, bf16_out=True, ulp_of=inter)["ok"]
    # intermediate and result of similar size: the flip and the final rounding add up
    ref3 = np.array([1.5, 4.0], dtype=np.float32)
    inter3 = np.array([1.25, 1.0])
    step3 = np.array([2 ** -6, 0.0], dtype=np.float32)   # = ulp(1.25) + ulp(1.5)
    assert not O.compare(ref3 + step3, ref3, 48, bf16_out=True, acc=0.0)["ok"]
    assert O.compare(ref3 + step3, ref3, 48, bf16_out=True, ulp_of=inter3)["ok"]
    assert not O.compare(ref3 + 2 * step3, ref3, 48, bf16_out=True, ulp_of=inter3)["ok"]


@pytest.mark.parametrize("v,ulp", [(1.0, 2 ** -7), (10.0, 2 ** -4), (0.5, 2 ** -8), (-3.0, 2 ** -6)])
def test_bf16_ulp(v, ulp):
    assert O.bf16_ulp(np.array([v]))[0] == ulp
