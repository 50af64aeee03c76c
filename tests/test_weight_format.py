"""The stored form of QuantizedWeight (the reference
re-quantizes every weight at load, engine/model.py:101-112; the packed form
loads as a copy).  CPU: state round trips, validation, the safetensors file,
and the packed size against the library's own; GPU: a reloaded weight holds
the oracle's q and scale and its outputs match the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quantization_oracle as O
from pageserve_amd import quantization as Q


def _cpu_weight(seed, n, k, dtype=torch.bfloat16):
    w = (np.random.default_rng(seed).standard_normal((n, k)) * 0.02).astype(np.float32)
    q, s = O.quantize_per_channel(w)
    meta = torch.tensor([n, k, {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[dtype]])
    qw = Q.QuantizedWeight.from_state({"qp": torch.from_numpy(O.pack_tiles(q)), "scale": torch.from_numpy(s),
                                       "meta": meta})
    return qw, q, s


def test_state_round_trip_on_cpu():
    qw, q, s = _cpu_weight(1, 40, 200)
    assert qw.shape == (40, 200) and qw.dtype == torch.bfloat16 and qw.device.type == "cpu"
    again = Q.QuantizedWeight.from_state(qw.state())
    assert torch.equal(again.qp, qw.qp) and torch.equal(again.scale, qw.scale) and again.shape == qw.shape
    assert qw.storage_bytes == Q.packed_numel(40, 200) + 40 * 4


def test_safetensors_file_round_trip(tmp_path):
    ws = {f"layers.{i}.{nm}": _cpu_weight(10 * i + j, n, k, dt)[0]
          for i in range(2) for j, (nm, n, k, dt) in enumerate([("q_w", 64, 128, torch.bfloat16),
                                                               ("down_w", 48, 100, torch.float32)])}
    path = str(tmp_path / "w8.safetensors")
    Q.save_quantized(path, ws)
    back = Q.load_quantized(path)
    assert set(back) == set(ws)
    for name, w in ws.items():
        b = back[name]
        assert torch.equal(b.qp, w.qp) and torch.equal(b.scale, w.scale)
        assert b.shape == w.shape and b.dtype == w.dtype


def test_bad_states_are_rejected(tmp_path):
    qw, _, _ = _cpu_weight(2, 16, 64)
    st = qw.state()
    with pytest.raises(ValueError, match="lacks"):
        Q.QuantizedWeight.from_state({"qp": st["qp"], "scale": st["scale"]})
    with pytest.raises(ValueError, match="packed weight"):
        Q.QuantizedWeight.from_state({**st, "qp": st["qp"][:-1]})
    with pytest.raises(ValueError, match="scale"):
        Q.QuantizedWeight.from_state({**st, "scale": st["scale"].double()})
    with pytest.raises(ValueError, match="meta"):
        Q.QuantizedWeight.from_state({**st, "meta": torch.tensor([16, 64, 9])})
    from safetensors.torch import save_file

    other = str(tmp_path / "other.safetensors")
    save_file({"x": torch.zeros(3)}, other)
    with pytest.raises(ValueError, match="not a pageserve_amd"):
        Q.load_quantized(other)


@pytest.mark.parametrize("n,k", [(1, 1), (16, 64), (17, 65), (4864, 896), (151936, 2048)])
def test_packed_size_matches_the_library(native_lib, n, k):
    assert Q.packed_numel(n, k) == native_lib.pgs_packed_bytes(n, k)


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", [(2048, 2048), (256, 2048), (2048, 11008), (130, 1040)])
def test_reloaded_weight_matches_the_oracle(gpu, tmp_path, n, k):
    """Quantized on the GPU, stored, loaded back onto the GPU: the reloaded
    q and scale equal the oracle quantizer's bit for bit, and its linear
    outputs (decode and prefill sizes) match the oracle linear of the
    original weight within the specification's tolerance, and the output
    of the weight before storing bit for bit."""
    from helpers import activations, bf16_gpu, report, to_np, weights

    w = weights(600 + n + k, n, k)
    q_ref, s_ref = O.quantize_per_channel(w)
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    path = str(tmp_path / "w.safetensors")
    Q.save_quantized(path, {"o_w": qw})
    back = Q.load_quantized(path, device=gpu)["o_w"]
    assert back.device == qw.device and back.shape == (n, k) and back.dtype == torch.float32
    np.testing.assert_array_equal(back.q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(back.scale.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    for m in (1, 5, 64, 200):
        x = activations(610 + m, m, k)
        xt = bf16_gpu(x, gpu)
        y = back.linear(xt)
        report(to_np(y), O.linear(x, q_ref, s_ref), k, f"reloaded m={m} n={n} k={k}",
               acc=O.acc_bound(x, q_ref, s_ref))
        assert torch.equal(y, qw.linear(xt))
