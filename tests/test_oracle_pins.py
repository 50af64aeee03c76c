"""Pins the CPU oracle (oracle/quantization_oracle.py) before it is trusted.

The reference (Rakshit-gen/pageserve) ships no golden vectors for this path,
only the bounds of tests/test_quantization.py:14-46.  The oracle is pinned by:

1. hand-computed known answers (ties, zero rows, tiny rows, exact scales);
2. an independent exact-rational restatement (tests/exact.py) on random and
   adversarial matrices, bit for bit;
3. planted mistakes: plausible wrong versions of the oracle (reciprocal
   multiply, ties away from zero, row/column mix-up, missing clamp, ...) must
   each fail at least one of the checks above;
4. the reference's own bounds.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

import exact
from oracle import quantization_oracle as O

F32 = np.float32


# ---------------------------------------------------------------------------
# inputs
# ---------------------------------------------------------------------------

def kat_rows() -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Rows with hand-derived q and scale.

    Row 0: absmax 127 -> scale exactly 1.0, so q = round-half-even(w).
    Row 1: zero row -> scale = fp32(1e-8) / 127, q = 0.
    Row 2: absmax 254 -> scale 2.0; w = 2 * (k + 0.5) probes ties at odd/even k.
    Row 3: negative absmax wins; scale 0.5.
    """
    w = np.array(
        [
            [127.0, 63.5, -63.5, 0.5, 1.5, 2.5, -2.5, -127.0],
            [0.0, -0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
            [254.0, 1.0, 3.0, 5.0, -1.0, -3.0, 7.0, 9.0],
            [-63.5, 0.25, 0.75, -0.25, 31.75, 1.25, 0.0, 63.0],
        ],
        dtype=np.float32,
    )
    q = np.array(
        [
            [127, 64, -64, 0, 2, 2, -2, -127],
            [0, 0, 0, 0, 0, 0, 0, 0],
            [127, 0, 2, 2, 0, -2, 4, 4],
            [-127, 0, 2, 0, 64, 2, 0, 126],
        ],
        dtype=np.int8,
    )
    scale = np.array([[1.0], [float(F32(F32(1e-8) / F32(127.0)))], [2.0], [0.5]], dtype=np.float32)
    return w, q, scale


def adversarial_rows(seed: int = 7, rows: int = 12, per_row: int = 24) -> np.ndarray:
    """Rows whose elements sit within a few ulps of a half-integer multiple of
    the scale: the cases where a reciprocal multiply, a double-precision
    quotient or a different rounding rule changes q."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(rows):
        a = F32(rng.uniform(0.01, 3.0))
        s = F32(a / F32(127.0))
        row = [a]
        while len(row) < per_row:
            k = int(rng.integers(-126, 126))
            base = F32(s * F32(k + 0.5))
            v = base
            for _ in range(int(rng.integers(-3, 4))):
                v = np.nextafter(v, F32(np.inf))
            if abs(v) < a:
                row.append(F32(v))
        out.append(row)
    return np.array(out, dtype=np.float32)


def random_matrix(seed: int, n: int, k: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[0, :] = 0.0                                     # zero row
    w[1, :] *= F32(1e-7)                              # absmax below the 1e-8 clamp? (mostly not)
    w[2, :] = (rng.standard_normal(k) * 1e-10).astype(np.float32)  # clamped row
    w[3, 5 % k] = -w[3].__abs__().max() * 2            # negative absmax
    return w


# ---------------------------------------------------------------------------
# 1. known answers
# ---------------------------------------------------------------------------

def test_quantizer_known_answers():
    w, q_exp, s_exp = kat_rows()
    q, s = O.quantize_per_channel(w)
    assert q.dtype == np.int8 and s.dtype == np.float32 and s.shape == (4, 1)
    np.testing.assert_array_equal(q, q_exp)
    np.testing.assert_array_equal(s.view(np.uint32), s_exp.view(np.uint32))


def test_quantizer_zero_row_scale_bits():
    q, s = O.quantize_per_channel(np.zeros((3, 5), dtype=np.float32))
    # 1e-8 rounds to fp32 0x322BCC77; / 127 correctly rounded
    assert np.float32(1e-8).view(np.uint32) == 0x322BCC77
    expected = exact.round_f32(Fraction(float(np.float32(1e-8))) / 127)
    assert s[0, 0] == expected and (q == 0).all()


def test_quantizer_bf16_input_widens_exactly():
    w, q_exp, s_exp = kat_rows()  # every KAT value is bf16-representable
    bits = O.f32_to_bf16_bits(w)
    np.testing.assert_array_equal(O.bf16_bits_to_f32(bits), w)
    q, s = O.quantize_per_channel(bits, bf16_bits=True)
    np.testing.assert_array_equal(q, q_exp)
    np.testing.assert_array_equal(s, s_exp)


# ---------------------------------------------------------------------------
# 2. exact-rational restatement
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("maker", ["adversarial", "random", "tiny", "ties"])
def test_quantizer_matches_exact_rationals(maker):
    if maker == "adversarial":
        w = adversarial_rows()
    elif maker == "random":
        w = random_matrix(11, 8, 40)
    elif maker == "tiny":
        rng = np.random.default_rng(3)
        w = (rng.standard_normal((4, 16)) * 1e-9).astype(np.float32)
        w[0, 0] = F32(1.17549435e-38) * F32(0.5)   # subnormal
    else:
        rng = np.random.default_rng(5)
        s = F32(2.0) ** rng.integers(-8, 4, size=6).astype(np.float32)
        ks = rng.integers(-126, 126, size=(6, 20))
        w = ((ks + 0.5) * s[:, None]).astype(np.float32)
        w[:, 0] = F32(127.0) * s
    q, s = O.quantize_per_channel(w)
    q_ref, s_ref = exact.quantize(w)
    np.testing.assert_array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(q, q_ref)


def test_linear_matches_exact_rationals():
    rng = np.random.default_rng(21)
    w = random_matrix(22, 6, 32)
    q, s = O.quantize_per_channel(w)
    x = O.round_to_bf16(rng.standard_normal((3, 32)).astype(np.float32))
    bias = O.round_to_bf16(rng.standard_normal(6).astype(np.float32))
    y = O.linear(x, q, s, bias)
    y_ex = exact.linear(x, q, s, bias)
    for i in range(3):
        for r in range(6):
            assert abs(Fraction(float(y[i, r])) - y_ex[i][r]) <= Fraction(exact.ulp_f32(float(y_ex[i][r])))


def test_swiglu_matches_scalar_math():
    import math

    rng = np.random.default_rng(4)
    w1 = random_matrix(31, 5, 16)
    w2 = random_matrix(32, 5, 16)
    qg, sg = O.quantize_per_channel(w1)
    qu, su = O.quantize_per_channel(w2)
    x = O.round_to_bf16(rng.standard_normal((2, 16)).astype(np.float32))
    act = O.swiglu(x, qg, sg, qu, su)
    g = exact.linear(x, qg, sg)
    u = exact.linear(x, qu, su)
    for i in range(2):
        for r in range(5):
            gv, uv = float(g[i][r]), float(u[i][r])
            expect = gv / (1.0 + math.exp(-gv)) * uv
            assert abs(act[i, r] - expect) <= 2 * exact.ulp_f32(expect) + 1e-30


# ---------------------------------------------------------------------------
# 3. planted mistakes must be caught
# ---------------------------------------------------------------------------

def _q_reciprocal(w):
    absmax = np.maximum(np.abs(w).max(axis=1, keepdims=True), F32(1e-8))
    s = (absmax / F32(127)).astype(np.float32)
    return np.clip(np.rint(w * (F32(1) / s)), -127, 127).astype(np.int8), s


def _q_half_away(w):
    absmax = np.maximum(np.abs(w).max(axis=1, keepdims=True), F32(1e-8))
    s = (absmax / F32(127)).astype(np.float32)
    r = (w / s).astype(np.float32)
    return np.clip(np.sign(r) * np.floor(np.abs(r) + F32(0.5)), -127, 127).astype(np.int8), s


def _q_double_quotient(w):
    absmax = np.maximum(np.abs(w).max(axis=1, keepdims=True), F32(1e-8))
    s = (absmax / F32(127)).astype(np.float32)
    r = w.astype(np.float64) / s.astype(np.float64)
    return np.clip(np.rint(r), -127, 127).astype(np.int8), s


def _q_column_absmax(w):
    absmax = np.maximum(np.abs(w).max(axis=0, keepdims=True), F32(1e-8))
    s = (absmax / F32(127)).astype(np.float32)
    return np.clip(np.rint(w / s), -127, 127).astype(np.int8), s.reshape(-1, 1)[: w.shape[0]]


def _q_no_clamp_min(w):
    absmax = np.abs(w).max(axis=1, keepdims=True)
    s = (absmax / F32(127)).astype(np.float32)
    with np.errstate(all="ignore"):
        q = np.nan_to_num(np.clip(np.rint(w / s), -127, 127)).astype(np.int8)
    return q, s


def _q_div128(w):
    absmax = np.maximum(np.abs(w).max(axis=1, keepdims=True), F32(1e-8))
    s = (absmax / F32(128)).astype(np.float32)
    return np.clip(np.rint(w / s), -127, 127).astype(np.int8), s


def _q_truncate(w):
    absmax = np.maximum(np.abs(w).max(axis=1, keepdims=True), F32(1e-8))
    s = (absmax / F32(127)).astype(np.float32)
    return np.clip(np.trunc(w / s), -127, 127).astype(np.int8), s


MUTANTS = {
    "reciprocal_multiply": _q_reciprocal,
    "ties_away_from_zero": _q_half_away,
    "fp64_quotient": _q_double_quotient,
    "absmax_over_columns": _q_column_absmax,
    "no_1e-8_clamp": _q_no_clamp_min,
    "divide_by_128": _q_div128,
    "truncate": _q_truncate,
}


def _quantizer_pins_pass(fn) -> bool:
    """True when ``fn`` passes every quantizer pin (KATs + exact rationals)."""
    try:
        w, q_exp, s_exp = kat_rows()
        q, s = fn(w)
        if not (np.array_equal(q, q_exp) and np.array_equal(np.asarray(s).reshape(-1, 1), s_exp)):
            return False
        for w in (adversarial_rows(), random_matrix(11, 8, 40)):
            q, s = fn(w)
            q_ref, s_ref = exact.quantize(w)
            if not (np.array_equal(q, q_ref) and np.array_equal(np.asarray(s).reshape(-1, 1), s_ref)):
                return False
        return True
    except Exception:
        return False


def test_oracle_passes_its_own_pins():
    assert _quantizer_pins_pass(O.quantize_per_channel)


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_quantizer_mistake_is_caught(name):
    assert not _quantizer_pins_pass(MUTANTS[name]), f"mutant {name} slipped through the pins"


def _linear_pins_pass(fn) -> bool:
    rng = np.random.default_rng(21)
    w = random_matrix(22, 6, 6)  # square on purpose: a transpose still type-checks
    q, s = O.quantize_per_channel(w)
    x = O.round_to_bf16(rng.standard_normal((3, 6)).astype(np.float32))
    bias = O.round_to_bf16(rng.standard_normal(6).astype(np.float32))
    try:
        y = fn(x, q, s, bias)
    except Exception:
        return False
    y_ex = exact.linear(x, q, s, bias)
    for i in range(3):
        for r in range(6):
            if abs(Fraction(float(y[i, r])) - y_ex[i][r]) > Fraction(exact.ulp_f32(float(y_ex[i][r]))):
                return False
    return True


LINEAR_MUTANTS = {
    "transposed_weight": lambda x, q, s, b: (x.astype(np.float64) @ O.dequantize(q, s).astype(np.float64)
                                             + b).astype(np.float32),
    "scale_per_column": lambda x, q, s, b: (x.astype(np.float64) @ (q.astype(np.float32) * s.reshape(1, -1)).T
                                            + b).astype(np.float32),
    "no_bias": lambda x, q, s, b: O.linear(x, q, s, None),
    "bf16_weights": lambda x, q, s, b: (x.astype(np.float64)
                                        @ O.round_to_bf16(O.dequantize(q, s)).astype(np.float64).T
                                        + b).astype(np.float32),
    "no_scale": lambda x, q, s, b: O.linear(x, q, np.ones_like(s), b),
}


def test_linear_oracle_passes_its_own_pins():
    assert _linear_pins_pass(O.linear)


@pytest.mark.parametrize("name", sorted(LINEAR_MUTANTS))
def test_planted_linear_mistake_is_caught(name):
    assert not _linear_pins_pass(LINEAR_MUTANTS[name]), f"mutant {name} slipped through the pins"


# ---------------------------------------------------------------------------
# 4. the reference's own bounds (tests/test_quantization.py:14-46)
# ---------------------------------------------------------------------------

def test_reference_round_trip_bound():
    torch = pytest.importorskip("torch")
    torch.manual_seed(0)
    w = torch.randn(64, 128, dtype=torch.float32).numpy()
    q, s = O.quantize_per_channel(w)
    assert q.dtype == np.int8 and s.shape == (64, 1)
    rec = O.dequantize(q, s, "f32")
    max_err = np.abs(w - rec).max()
    max_step = (np.abs(w).max(axis=1, keepdims=True) / F32(127.0)).max()
    assert max_err <= max_step
    # the half-step bound the reference's comment states also holds
    assert max_err <= max_step * 0.5 * (1 + 1e-6)


def test_reference_storage_bound():
    q, s = O.quantize_per_channel(np.random.default_rng(0).standard_normal((2048, 2048)).astype(np.float32))
    assert q.nbytes + s.nbytes < 2048 * 2048 * 4 / 3


def test_reference_matmul_bound():
    torch = pytest.importorskip("torch")
    torch.manual_seed(1)
    x = torch.randn(8, 128).numpy()
    w = torch.randn(64, 128).numpy()
    q, s = O.quantize_per_channel(w)
    expected = x.astype(np.float64) @ w.astype(np.float64).T
    actual = O.linear(x, q, s)
    rel = np.abs(expected - actual).max() / np.abs(expected).max()
    assert rel < 0.05


def test_bf16_rounding_helper_is_round_to_nearest_even():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(9)
    v = np.concatenate([
        rng.standard_normal(4096).astype(np.float32) * F32(1000),
        # exact ties between two bf16 values: low 16 bits = 0x8000
        (np.arange(64, dtype=np.uint32) << 16 | 0x3F808000).view(np.float32),
    ])
    ours = O.f32_to_bf16_bits(v)
    theirs = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


# ---------------------------------------------------------------------------
# the packed tile layout (pageserve_amd's weight storage)
# ---------------------------------------------------------------------------

def test_packed_layout_lane_order():
    """Byte 16*l + b of a block is row l%16, column 16*(l//16) + b."""
    q = ((np.arange(16 * 64).reshape(16, 64) % 251) - 125).astype(np.int8)
    p = O.pack_tiles(q)
    assert p.size == 1024
    for lane in range(64):
        np.testing.assert_array_equal(p[16 * lane:16 * lane + 16], q[lane % 16, 16 * (lane // 16):16 * (lane // 16) + 16])


@pytest.mark.parametrize("n,k", [(1, 1), (16, 64), (17, 65), (37, 150), (32, 128), (5, 2048)])
def test_packed_layout_round_trip_and_padding(n, k):
    q = np.random.default_rng(n * k).integers(-127, 128, (n, k)).astype(np.int8)
    p = O.pack_tiles(q)
    assert p.size == -(-n // 16) * -(-k // 64) * 1024
    np.testing.assert_array_equal(O.unpack_tiles(p, n, k), q)
    # block order: block (tr, tc) starts at (tr * ceil(k/64) + tc) KiB
    tk = -(-k // 64)
    for (r, j) in [(0, 0), (n - 1, k - 1), (n // 2, k // 3)]:
        off = ((r // 16) * tk + j // 64) * 1024 + ((r % 16) + 16 * ((j % 64) // 16)) * 16 + j % 16
        assert p[off] == q[r, j]
    # padding bytes are zero: everything not covered by a real element
    covered = np.zeros(p.size, dtype=bool)
    for r in range(n):
        for j in range(k):
            covered[((r // 16) * tk + j // 64) * 1024 + ((r % 16) + 16 * ((j % 64) // 16)) * 16 + j % 16] = True
    assert (p[~covered] == 0).all() and covered.sum() == n * k


# ---------------------------------------------------------------------------
# 5. non-finite weights: the reference's op sequence in torch on the CPU (an
#    independent implementation of engine/quantization.py:20-22) gives a NaN
#    scale to a row holding a NaN, an infinite scale to a row holding an
#    infinity, and q = 0 wherever the quotient is NaN
# ---------------------------------------------------------------------------

def test_quantizer_non_finite_rows_follow_torch_cpu():
    torch = pytest.importorskip("torch")
    w = random_matrix(41, 6, 96)
    w[1, 7] = np.nan
    w[2, 3] = np.inf
    w[3, 0] = -np.inf
    w[4, 9], w[4, 10] = np.nan, np.inf
    t = torch.from_numpy(w)
    absmax = t.float().abs().amax(dim=1, keepdim=True).clamp(min=1e-8)
    scale = absmax / 127.0
    q = torch.clamp((t.float() / scale).round(), -127, 127).to(torch.int8)
    oq, os_ = O.quantize_per_channel(w)
    np.testing.assert_array_equal(oq, q.numpy())
    np.testing.assert_array_equal(np.isnan(os_), np.isnan(scale.numpy()))
    fin = ~np.isnan(os_)
    np.testing.assert_array_equal(os_[fin].view(np.uint32), scale.numpy()[fin].view(np.uint32))
    assert np.isnan(os_[1, 0]) and np.isnan(os_[4, 0]) and np.isinf(os_[2, 0]) and np.isinf(os_[3, 0])
    assert (oq[1:5] == 0).all() and (oq[5] != 0).any()


# ---------------------------------------------------------------------------
# 6. the accumulation bound of the bf16 tolerance (O.acc_bound, O.swiglu_acc)
#    must hold for fp32 evaluations in any summation order -- including an
#    input where sequential fp32 addition absorbs every small term -- and a
#    bound without its factor K must not
# ---------------------------------------------------------------------------

def _fp32_linear(x, q, s, order):
    """fp32 evaluation of x (q s)^T: exact fp32 products summed in fp32 in
    the given order, then one multiply by the scale."""
    p = (x.astype(np.float32)[:, None, :] * q.astype(np.float32)[None, :, :]).astype(np.float32)
    if order == "forward":
        acc = np.add.accumulate(p, axis=-1, dtype=np.float32)[..., -1]
    elif order == "reverse":
        acc = np.add.accumulate(p[..., ::-1], axis=-1, dtype=np.float32)[..., -1]
    else:  # blocks of 32 (an MFMA's k extent) summed in fp32, then the blocks in sequence
        blocks = p.reshape(p.shape[0], p.shape[1], -1, 32).sum(axis=-1, dtype=np.float32)
        acc = np.add.accumulate(blocks, axis=-1, dtype=np.float32)[..., -1]
    return (acc * s.reshape(1, -1)).astype(np.float32)


def _acc_inputs():
    rng = np.random.default_rng(43)
    k = 4096
    q, s = O.quantize_per_channel(random_matrix(44, 12, k))
    x = O.round_to_bf16(rng.standard_normal((3, k)).astype(np.float32))
    # row 0 of q / token 0 of x: one large product, then K-1 products below
    # half an fp32 ulp of it, each absorbed by a sequential fp32 sum
    q[0, :] = 1
    q[0, 0] = 127
    x[0, :] = np.float32(2.0 ** -20)
    x[0, 0] = 1.0
    return x, q, s


@pytest.mark.parametrize("order", ["forward", "reverse", "blocked"])
def test_accumulation_bound_holds_in_any_order(order):
    x, q, s = _acc_inputs()
    exact64 = x.astype(np.float64) @ O.dequantize(q, s, "f32").astype(np.float64).T
    y32 = _fp32_linear(x, q, s, order)
    acc = O.acc_bound(x, q, s)
    assert (np.abs(y32 - exact64) <= acc).all()


def test_accumulation_bound_without_k_is_caught():
    x, q, s = _acc_inputs()
    exact64 = x.astype(np.float64) @ O.dequantize(q, s, "f32").astype(np.float64).T
    y32 = _fp32_linear(x, q, s, "forward")
    k = q.shape[1]
    mutant = O.acc_bound(x, q, s) * (8.0 / (k + 8))
    assert (np.abs(y32 - exact64) > mutant).any()


def test_swiglu_bound_holds_for_an_fp32_evaluation():
    rng = np.random.default_rng(45)
    k = 2048
    qg, sg = O.quantize_per_channel(random_matrix(46, 16, k))
    qu, su = O.quantize_per_channel(random_matrix(47, 16, k))
    x = O.round_to_bf16((rng.standard_normal((4, k)) * 3).astype(np.float32))
    g = _fp32_linear(x, qg, sg, "forward")
    u = _fp32_linear(x, qu, su, "reverse")
    act32 = (g / (np.float32(1) + np.exp(-g, dtype=np.float32)) * u).astype(np.float32)
    ref = O.swiglu(x, qg, sg, qu, su)
    bound = O.swiglu_acc(x, qg, sg, qu, su)
    assert (np.abs(act32.astype(np.float64) - ref) <= bound + np.abs(ref) * 2.0 ** -24).all()
