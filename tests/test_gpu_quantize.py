"""Quantizer and dequantizer kernels against the oracle: bit-exact.

engine/quantization.py:16-27.  q and scale must equal the oracle bit for bit
(integer and exactly specified fp32 arithmetic); dequantize likewise.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import weights
from oracle import quantization_oracle as O
from pageserve_amd import quantization as Q
from test_oracle_pins import adversarial_rows, kat_rows, random_matrix

pytestmark = pytest.mark.gpu


def _gpu_quant(w_np: np.ndarray, device, dtype=torch.float32):
    w = torch.from_numpy(w_np).to(device)
    if dtype == torch.bfloat16:
        w = torch.from_numpy(O.f32_to_bf16_bits(w_np).view(np.int16).copy()).view(torch.bfloat16).to(device)
    q, s = Q.quantize_per_channel(w)
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy()


def _assert_bit_exact(q, s, q_ref, s_ref, what):
    assert q.dtype == np.int8 and s.dtype == np.float32 and s.shape == s_ref.shape, what
    bad = np.flatnonzero(s.view(np.uint32).ravel() != s_ref.view(np.uint32).ravel())
    assert bad.size == 0, f"{what}: {bad.size} scales differ, first row {bad[:5]}"
    diff = np.argwhere(q != q_ref)
    assert diff.size == 0, f"{what}: {len(diff)} q values differ, first {diff[:5].tolist()}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_known_answer_rows(gpu, dtype):
    w, q_exp, s_exp = kat_rows()
    q, s = _gpu_quant(w, gpu, dtype)
    _assert_bit_exact(q, s, q_exp, s_exp, f"KAT {dtype}")


def test_adversarial_rows(gpu):
    w = adversarial_rows(rows=64, per_row=64)
    q, s = _gpu_quant(w, gpu)
    q_ref, s_ref = O.quantize_per_channel(w)
    _assert_bit_exact(q, s, q_ref, s_ref, "adversarial")


@pytest.mark.parametrize(
    "n,k",
    [(1, 1), (3, 7), (17, 100), (8, 40), (64, 128), (4864, 896), (256, 2048), (2048, 11008), (300, 4100)],
)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_random_shapes_bit_exact(gpu, n, k, dtype):
    w = random_matrix(1000 + n + k, n, k) if n >= 4 else weights(7, n, k)
    if dtype == torch.bfloat16:
        w = O.round_to_bf16(w)
    q, s = _gpu_quant(w, gpu, dtype)
    if dtype == torch.bfloat16:
        q_ref, s_ref = O.quantize_per_channel(O.f32_to_bf16_bits(w), bf16_bits=True)
    else:
        q_ref, s_ref = O.quantize_per_channel(w)
    _assert_bit_exact(q, s, q_ref, s_ref, f"[{n},{k}] {dtype}")


def test_misaligned_view_takes_the_scalar_path(gpu):
    base = weights(5, 33 * 65 + 1, 1).reshape(-1)
    w_np = base[1:].reshape(33, 65)
    wt = torch.from_numpy(base).to(gpu)[1:].view(33, 65)  # data pointer off by 4 bytes
    q, s = Q.quantize_per_channel(wt)
    q_ref, s_ref = O.quantize_per_channel(w_np)
    _assert_bit_exact(q.cpu().numpy(), s.cpu().numpy(), q_ref, s_ref, "misaligned")


def test_cpu_and_gpu_weights_quantize_alike(gpu):
    """A CPU weight is quantized by torch on the CPU, a GPU one by the HIP
    kernel: the same bytes either way, and a weight moved between them keeps
    them."""
    w = weights(8, 96, 256)
    q, s = Q.quantize_per_channel(torch.from_numpy(w))
    assert q.device.type == "cpu" and s.device.type == "cpu"
    q_ref, s_ref = O.quantize_per_channel(w)
    _assert_bit_exact(q.numpy(), s.numpy(), q_ref, s_ref, "cpu-resident weight")
    qg, sg = Q.quantize_per_channel(torch.from_numpy(w).to(gpu))
    assert torch.equal(qg.cpu(), q) and torch.equal(sg.cpu(), s)
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(torch.bfloat16))
    dense_cpu = qw.get()
    assert qw.to(gpu) is qw and torch.equal(qw.dense().cpu(), dense_cpu)
    assert torch.equal(qw.to("cpu").get(), dense_cpu)


def test_lm_head_shape_full_size(gpu):
    """[151936, 2048] (the Qwen2.5 vocabulary): bit-exact on a row sample,
    and exact invariants on every row."""
    n, k = 151936, 2048
    gen = torch.Generator(device=gpu).manual_seed(1234)
    w = torch.randn((n, k), generator=gen, device=gpu, dtype=torch.float32) * 0.02
    q, s = Q.quantize_per_channel(w)
    # every nonzero row's absmax element maps to exactly +-127; |q| <= 127
    qmax = q.abs().amax(dim=1)
    assert int(qmax.min()) == 127 and int(qmax.max()) == 127
    assert int(q.min()) >= -127
    # scale == max(absmax, 1e-8) / 127 with an IEEE fp32 divide (numpy on the
    # host; torch's GPU division by a scalar multiplies by a reciprocal)
    absmax = w.abs().amax(dim=1, keepdim=True).cpu().numpy()
    s_all = (np.maximum(absmax, np.float32(1e-8)) / np.float32(127.0)).astype(np.float32)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_all.view(np.uint32))
    rows = np.concatenate([np.arange(0, 4096), np.random.default_rng(0).choice(n, 4096, replace=False),
                           np.arange(n - 64, n)])
    w_rows = w[torch.from_numpy(rows).to(gpu)].cpu().numpy()
    q_ref, s_ref = O.quantize_per_channel(w_rows)
    _assert_bit_exact(q[torch.from_numpy(rows).to(gpu)].cpu().numpy(),
                      s[torch.from_numpy(rows).to(gpu)].cpu().numpy(), q_ref, s_ref, "lm_head rows")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("n,k", [(64, 128), (5, 7), (2048, 2048)])
def test_dequantize_bit_exact(gpu, dtype, n, k):
    w = random_matrix(77 + k, n, k)
    q_ref, s_ref = O.quantize_per_channel(w)
    qt = torch.from_numpy(q_ref).to(gpu)
    st = torch.from_numpy(s_ref).to(gpu)
    out = Q.dequantize(qt, st, dtype)
    assert out.dtype == dtype and out.shape == (n, k) and out.device == qt.device
    name = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16", torch.float64: "f32"}[dtype]
    ref = O.dequantize(q_ref, s_ref, name)
    got = out.cpu()
    if dtype == torch.bfloat16:
        np.testing.assert_array_equal(got.view(torch.int16).numpy().view(np.uint16), ref)
    elif dtype == torch.float64:
        np.testing.assert_array_equal(got.numpy(), ref.astype(np.float64))
    else:
        np.testing.assert_array_equal(got.numpy().view(np.uint8), ref.view(np.uint8))


def test_quantized_weight_matches_reference_contract(gpu):
    """tests/test_quantization.py:14-46 run on the GPU path."""
    torch.manual_seed(0)
    w = torch.randn(64, 128, dtype=torch.float32)
    qw = Q.QuantizedWeight(w.to(gpu))
    assert qw.q.dtype == torch.int8 and qw.scale.shape == (64, 1) and qw.dtype == torch.float32
    rec = qw.get()
    err = (w - rec.cpu()).abs().max().item()
    step = (w.abs().amax(dim=1, keepdim=True) / 127.0).max().item()
    assert err <= step
    big = Q.QuantizedWeight(torch.randn(2048, 2048).to(gpu))
    assert big.storage_bytes < 2048 * 2048 * 4 / 3
    torch.manual_seed(1)
    x = torch.randn(8, 128)
    wt = torch.randn(64, 128)
    qw = Q.QuantizedWeight(wt.to(gpu))
    exp = x @ wt.T
    act = x @ qw.get().cpu().T
    assert (exp - act).abs().max().item() / exp.abs().max().item() < 0.05
    # .to() moves in place and returns self (engine/quantization.py:43-46)
    assert qw.to("cpu") is qw and qw.q.device.type == "cpu"


@pytest.mark.parametrize("n,k", [(1, 1), (3, 7), (17, 100), (4864, 896), (300, 4100), (2048, 11008), (5, 2048)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_packed_storage_bit_exact(gpu, n, k, dtype):
    """QuantizedWeight stores the packed layout: equal, byte for byte, to the
    oracle's packing of the oracle's q; .q unpacks to the reference layout."""
    w = random_matrix(3000 + n + k, n, k) if n >= 4 else weights(9, n, k)
    if dtype == torch.bfloat16:
        w = O.round_to_bf16(w)
        wt = torch.from_numpy(O.f32_to_bf16_bits(w).view(np.int16).copy()).view(torch.bfloat16).to(gpu)
    else:
        wt = torch.from_numpy(w).to(gpu)
    qw = Q.QuantizedWeight(wt)
    q_ref, s_ref = O.quantize_per_channel(w)
    np.testing.assert_array_equal(qw.qp.cpu().numpy(), O.pack_tiles(q_ref))
    np.testing.assert_array_equal(qw.q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(qw.scale.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert qw.q.shape == (n, k) and qw.scale.shape == (n, 1)
    # pack / unpack of an arbitrary row-major int8 matrix
    r = np.random.default_rng(n).integers(-128, 128, (n, k)).astype(np.int8)
    rp = Q.pack(torch.from_numpy(r).to(gpu))
    np.testing.assert_array_equal(rp.cpu().numpy(), O.pack_tiles(r))
    np.testing.assert_array_equal(Q.unpack(rp, n, k).cpu().numpy(), r)
    # dequantize from the packed storage == the reference's dequantize
    dense = qw.dense()
    assert dense.dtype == dtype and dense.shape == (n, k)
    ref = O.dequantize(q_ref, s_ref, "bf16" if dtype == torch.bfloat16 else "f32")
    got = dense.cpu().view(torch.int16).numpy().view(np.uint16) if dtype == torch.bfloat16 else dense.cpu().numpy()
    np.testing.assert_array_equal(got, ref)


def test_assigning_q_repacks(gpu):
    qw = Q.QuantizedWeight(torch.randn(40, 96, device=gpu))
    new = torch.randint(-127, 128, (40, 96), dtype=torch.int8, device=gpu)
    qw.q = new
    assert torch.equal(qw.q, new)
    np.testing.assert_array_equal(qw.qp.cpu().numpy(), O.pack_tiles(new.cpu().numpy()))


# seeded random soak: any N and K, rows from denormal to 1e30 in magnitude,
# zero rows and the adversarial tie rows, fp32 and bf16 inputs, row-major and
# packed storage -- every q and scale bit-exact
QUANT_CASES = int(__import__("os").environ.get("PGS_RANDOM_QUANT_CASES", "16"))


@pytest.mark.parametrize("i", range(QUANT_CASES))
def test_random_quantize_bit_exact(gpu, i):
    rng = np.random.default_rng(40_000 + i)
    n, k = int(rng.integers(1, 600)), int(rng.integers(1, 3000))
    w = rng.standard_normal((n, k)).astype(np.float32)
    w = (w * (10.0 ** rng.uniform(-38, 30, size=(n, 1)))).astype(np.float32)
    w[rng.random(n) < 0.05] = 0.0
    if i % 3 == 0 and n >= 8 and k >= 8:
        adv = adversarial_rows(rows=min(n, 32), per_row=min(k, 64))
        w[: adv.shape[0], : adv.shape[1]] = adv
    dtype = torch.bfloat16 if i % 2 else torch.float32
    if dtype == torch.bfloat16:
        w = O.round_to_bf16(w)
        q_ref, s_ref = O.quantize_per_channel(O.f32_to_bf16_bits(w), bf16_bits=True)
    else:
        q_ref, s_ref = O.quantize_per_channel(w)
    q, s = _gpu_quant(w, gpu, dtype)
    _assert_bit_exact(q, s, q_ref, s_ref, f"case {i} [{n},{k}] {dtype}")
    wt = torch.from_numpy(w).to(gpu) if dtype == torch.float32 else \
        torch.from_numpy(O.f32_to_bf16_bits(w).view(np.int16).copy()).view(torch.bfloat16).to(gpu)
    qw = Q.QuantizedWeight(wt)
    _assert_bit_exact(qw.q.cpu().numpy(), qw.scale.cpu().numpy(), q_ref, s_ref, f"packed case {i} [{n},{k}] {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_non_finite_rows_follow_the_reference(gpu, dtype):
    """A row holding a NaN gets a NaN scale, a row holding an infinity an
    infinite scale, and every NaN quotient q = 0 (the reference's torch CPU
    arithmetic, pinned in the oracle tests); other rows are unaffected."""
    w = random_matrix(77, 8, 192)
    w[1, 7] = np.nan
    w[2, 3] = np.inf
    w[3, 0] = -np.inf
    w[4, 9], w[4, 100] = np.nan, np.inf
    if dtype == torch.bfloat16:
        w = O.round_to_bf16(w)
    q, s = _gpu_quant(w, gpu, dtype)
    q_ref, s_ref = O.quantize_per_channel(w)
    np.testing.assert_array_equal(q, q_ref)
    np.testing.assert_array_equal(np.isnan(s), np.isnan(s_ref))
    fin = ~np.isnan(s_ref)
    np.testing.assert_array_equal(s[fin].view(np.uint32), s_ref[fin].view(np.uint32))
    assert np.isnan(s[1, 0]) and np.isnan(s[4, 0]) and np.isinf(s[2, 0]) and np.isinf(s[3, 0])
    # the packed store agrees
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu) if dtype == torch.float32 else
                           torch.from_numpy(O.f32_to_bf16_bits(w).view(np.int16).copy()).view(torch.bfloat16).to(gpu))
    np.testing.assert_array_equal(qw.q.cpu().numpy(), q_ref)
