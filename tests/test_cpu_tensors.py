"""CPU-resident tensors keep the reference's math (engine/quantization.py:16-50)
evaluated by torch on the CPU: bit-exact against the oracle, with no tensor
on any other device and no call into the native library along the way.  The
fused entry points take GPU tensors only and refuse CPU ones."""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch.utils._python_dispatch import TorchDispatchMode
from torch.utils._pytree import tree_flatten

from oracle import quantization_oracle as O
from pageserve_amd import _native
from pageserve_amd import quantization as Q
from helpers import weights
from test_oracle_pins import adversarial_rows, kat_rows, random_matrix


class _Devices(TorchDispatchMode):
    """Records the device of every tensor that any torch op takes or makes."""

    def __init__(self):
        super().__init__()
        self.seen: set[str] = set()

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        out = func(*args, **(kwargs or {}))
        for t in tree_flatten((args, kwargs or {}, out))[0]:
            if isinstance(t, torch.Tensor):
                self.seen.add(t.device.type)
        return out


@pytest.fixture
def no_native(monkeypatch):
    """Any call into the HIP library (or its host module) fails the test."""
    def boom(*a, **k):
        raise AssertionError("the CPU path called into the native library")

    monkeypatch.setattr(_native, "load", boom)
    monkeypatch.setattr(_native, "load_host", boom)


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
def test_cpu_quantizer_is_the_reference_closed_form(no_native, dtype):
    for w in (random_matrix(12, 33, 130), weights(13, 5, 7), adversarial_rows(rows=16, per_row=48)):
        wt = torch.from_numpy(w).to(dtype)
        mode = _Devices()
        with mode:
            q, s = Q.quantize_per_channel(wt)
        assert mode.seen == {"cpu"}
        assert q.dtype == torch.int8 and s.dtype == torch.float32 and s.shape == (w.shape[0], 1)
        q_ref, s_ref = O.quantize_per_channel(wt.float().numpy())
        np.testing.assert_array_equal(q.numpy(), q_ref)
        np.testing.assert_array_equal(_bits(s.numpy()), _bits(s_ref))


def test_cpu_quantizer_known_answers(no_native):
    """Hand-derived q and scale: ties to even, the 1e-8 floor, +-absmax."""
    w, q_exp, s_exp = kat_rows()
    q, s = Q.quantize_per_channel(torch.from_numpy(w))
    np.testing.assert_array_equal(q.numpy(), q_exp)
    np.testing.assert_array_equal(_bits(s.numpy()), _bits(s_exp))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
def test_cpu_dequantize_bit_exact(no_native, dtype):
    q_ref, s_ref = O.quantize_per_channel(random_matrix(14, 17, 100))
    mode = _Devices()
    with mode:
        out = Q.dequantize(torch.from_numpy(q_ref), torch.from_numpy(s_ref), dtype)
    assert mode.seen == {"cpu"} and out.dtype == dtype and out.device.type == "cpu"
    if dtype == torch.bfloat16:
        np.testing.assert_array_equal(out.view(torch.int16).numpy().view(np.uint16), O.dequantize(q_ref, s_ref, "bf16"))
    elif dtype == torch.float16:
        np.testing.assert_array_equal(_bits(out.numpy()), _bits(O.dequantize(q_ref, s_ref, "f16")))
    else:
        np.testing.assert_array_equal(out.numpy(), O.dequantize(q_ref, s_ref, "f32").astype(np.float64))


@pytest.mark.parametrize("n,k", [(1, 1), (3, 7), (17, 100), (16, 64), (40, 200)])
def test_cpu_pack_layout_matches_the_oracle(no_native, n, k):
    q = torch.from_numpy(weights(15 + n, n, k).astype(np.int8) if n < 4 else
                         O.quantize_per_channel(random_matrix(15 + n, n, k))[0])
    qp = Q.pack(q)
    assert qp.numel() == Q.packed_numel(n, k)
    np.testing.assert_array_equal(qp.numpy(), O.pack_tiles(q.numpy()))
    np.testing.assert_array_equal(Q.unpack(qp, n, k).numpy(), q.numpy())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cpu_weight_get_makes_no_device_copy(no_native, dtype):
    """QuantizedWeight on a CPU weight: quantized, stored, unpacked and
    dequantized on the CPU.  get() is the reference's dequantized tensor."""
    w = torch.from_numpy(random_matrix(16, 40, 200)).to(dtype)
    mode = _Devices()
    with mode:
        qw = Q.QuantizedWeight(w)
        dense = qw.get()
        again = qw.get()
        q = qw.q
    assert mode.seen == {"cpu"}
    assert qw.device.type == "cpu" and qw.dtype == dtype
    assert type(dense) is torch.Tensor and dense.dtype == dtype and dense.shape == (40, 200)
    q_ref, s_ref = O.quantize_per_channel(w.float().numpy())
    np.testing.assert_array_equal(q.numpy(), q_ref)
    np.testing.assert_array_equal(qw.qp.numpy(), O.pack_tiles(q_ref))
    name = "bf16" if dtype == torch.bfloat16 else "f32"
    ref = O.dequantize(q_ref, s_ref, name)
    got = dense.view(torch.int16).numpy().view(np.uint16) if dtype == torch.bfloat16 else dense.numpy()
    np.testing.assert_array_equal(got, ref)
    assert torch.equal(dense, again)
    # assigning q repacks on the CPU
    with mode:
        qw.q = torch.from_numpy(q_ref[::-1].copy())
    assert mode.seen == {"cpu"}
    np.testing.assert_array_equal(qw.qp.numpy(), O.pack_tiles(q_ref[::-1]))


def test_reference_contract_on_the_cpu(no_native):
    """tests/test_quantization.py:14-46 of the reference, on CPU weights."""
    torch.manual_seed(0)
    w = torch.randn(64, 128, dtype=torch.float32)
    qw = Q.QuantizedWeight(w)
    assert qw.q.dtype == torch.int8 and qw.scale.shape == (64, 1) and qw.dtype == torch.float32
    err = (w - qw.get()).abs().max().item()
    step = (w.abs().amax(dim=1, keepdim=True) / 127.0).max().item()
    assert err <= step
    big = Q.QuantizedWeight(torch.randn(2048, 2048))
    assert big.storage_bytes < 2048 * 2048 * 4 / 3
    torch.manual_seed(1)
    x = torch.randn(8, 128)
    wt = torch.randn(64, 128)
    exp = x @ wt.T
    act = x @ Q.QuantizedWeight(wt).get().T
    assert (exp - act).abs().max().item() / exp.abs().max().item() < 0.05


def test_cpu_state_round_trip(no_native, tmp_path):
    w = torch.from_numpy(random_matrix(17, 24, 70)).to(torch.bfloat16)
    qw = Q.QuantizedWeight(w)
    path = str(tmp_path / "w.safetensors")
    Q.save_quantized(path, {"layer.w": qw})
    back = Q.load_quantized(path)["layer.w"]
    assert back.device.type == "cpu" and back.dtype == torch.bfloat16
    assert torch.equal(back.qp, qw.qp) and torch.equal(back.scale, qw.scale)
    assert torch.equal(back.get(), qw.get())


def test_fused_entry_points_refuse_cpu_tensors(no_native):
    """The fused linears are the HIP path only: a CPU weight is refused, never
    computed on the CPU."""
    qw = Q.QuantizedWeight(torch.randn(32, 64))
    x = torch.zeros(1, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        Q.linear(x, qw)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        qw.linear(x)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        Q.linear_group(x, [qw, qw])
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        Q.swiglu(x, qw, qw)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        Q.linear_argmax(x, qw)
