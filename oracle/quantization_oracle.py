"""numpy restatement of pageserve's INT8 weight-only quantization arithmetic.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the reference results
the HIP kernels are compared against, never part of the product.

Reference: Rakshit-gen/pageserve ``engine/quantization.py`` and the call sites
in ``engine/model.py``.  The reference runs these ops with PyTorch on the CPU;
the semantics restated here are:

* ``Tensor.float()``: exact widening (bf16 -> fp32 is a 16-bit shift).
* ``abs().amax(dim=1)``: exact (a max is order independent).
* ``clamp(min=1e-8)``: the Python scalar becomes ``float32(1e-8)``.
* ``absmax / 127.0`` and ``weight / scale``: IEEE-754 fp32 division, correctly
  rounded (no reciprocal multiply).
* ``round()``: round half to even.
* ``clamp(-127, 127).to(int8)``: saturate to the symmetric range.
* ``.to(bfloat16)``: round to nearest even.

Pinning (tests/test_oracle_pins.py): the quantizer is checked against an
independent exact-rational computation (``fractions.Fraction`` quotients
rounded to fp32 by hand, Python's own ties-to-even ``round``) on hand-built
known-answer rows and random matrices; the matmul against exact rational dot
products; each against a list of planted mistakes that must fail.  The
reference itself holds no golden vectors, only the bounds of
``tests/test_quantization.py:14-46``, which are re-asserted here too.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
EPS_ABSMAX = F32(1e-8)  # engine/quantization.py:20  .clamp(min=1e-8)
QMAX = F32(127.0)       # engine/quantization.py:21  absmax / 127.0


# --------------------------------------------------------------------------
# bf16 helpers (numpy has no bfloat16; bf16 values travel as uint16 bits)
# --------------------------------------------------------------------------

def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns (uint16) to float32."""
    b = np.asarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even; NaN -> canonical quiet NaN.

    Matches torch's ``Tensor.to(torch.bfloat16)`` on finite inputs.
    """
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    out = rounded.astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        out = np.where(nan, np.uint16(0x7FC0), out)
    return out


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16 value (returned as float32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# --------------------------------------------------------------------------
# a1: quantize_per_channel  (engine/quantization.py:16-23)
# --------------------------------------------------------------------------

def quantize_per_channel(weight: np.ndarray, *, bf16_bits: bool = False):
    """Returns ``(q int8 [N,K], scale float32 [N,1])``.

    ``weight``: float32 ``[N,K]``, or uint16 bf16 bit patterns when
    ``bf16_bits`` is true.  Follows engine/quantization.py:20-23 op by op.
    """
    w = bf16_bits_to_f32(weight) if bf16_bits else np.asarray(weight, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("weight must be 2-D (out_features, in_features)")
    # :20  absmax = weight.float().abs().amax(dim=1, keepdim=True).clamp(min=1e-8)
    if w.shape[1] == 0:
        absmax = np.full((w.shape[0], 1), EPS_ABSMAX, dtype=np.float32)
    else:
        absmax = np.abs(w).max(axis=1, keepdims=True)
        absmax = np.maximum(absmax, EPS_ABSMAX)  # NaN propagates, as clamp does
    # :21  scale = absmax / 127.0      (fp32 / fp32, IEEE)
    scale = (absmax / QMAX).astype(np.float32)
    # :22  q = clamp((weight.float() / scale).round(), -127, 127).to(int8)
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = (w / scale).astype(np.float32)
    q = np.clip(np.rint(ratio), F32(-127.0), F32(127.0))
    q = np.nan_to_num(q, nan=0.0).astype(np.int8)  # NaN -> 0: torch's CPU int8 conversion of NaN
    return q, scale


# --------------------------------------------------------------------------
# a2: dequantize  (engine/quantization.py:26-27)
# --------------------------------------------------------------------------

def dequantize(q: np.ndarray, scale: np.ndarray, dtype: str = "f32") -> np.ndarray:
    """``(q.to(float32) * scale).to(dtype)``.

    dtype "f32" -> float32 array; "bf16" -> uint16 bf16 bits; "f16" -> float16.
    """
    prod = (np.asarray(q).astype(np.float32) * np.asarray(scale, dtype=np.float32).reshape(-1, 1)).astype(np.float32)
    if dtype == "f32":
        return prod
    if dtype == "bf16":
        return f32_to_bf16_bits(prod)
    if dtype == "f16":
        return prod.astype(np.float16)
    raise ValueError(f"unknown dtype {dtype!r}")


# --------------------------------------------------------------------------
# packed tile layout of the int8 weight (pageserve_amd's storage format; no
# counterpart in the reference, whose q is row-major)
# --------------------------------------------------------------------------

def pack_tiles(q: np.ndarray) -> np.ndarray:
    """Row-major int8 [N,K] -> flat packed bytes: 16-row x 64-column blocks of
    1 KiB in [ceil(N/16)][ceil(K/64)] order; inside a block byte 16*l + b is
    q[16*tr + l%16, 64*tc + 16*(l//16) + b]; padding zero."""
    q = np.asarray(q, dtype=np.int8)
    n, k = q.shape
    tn, tk = -(-n // 16), -(-k // 64)
    padded = np.zeros((tn * 16, tk * 64), dtype=np.int8)
    padded[:n, :k] = q
    # [tn, 16 rows, tk, 4 groups, 16 bytes] -> [tn, tk, group, row, byte]
    blocks = padded.reshape(tn, 16, tk, 4, 16).transpose(0, 2, 3, 1, 4)
    return np.ascontiguousarray(blocks).reshape(-1)


def unpack_tiles(packed: np.ndarray, n: int, k: int) -> np.ndarray:
    tn, tk = -(-n // 16), -(-k // 64)
    blocks = np.asarray(packed, dtype=np.int8).reshape(tn, tk, 4, 16, 16).transpose(0, 3, 1, 2, 4)
    return np.ascontiguousarray(blocks).reshape(tn * 16, tk * 64)[:n, :k]


# --------------------------------------------------------------------------
# a5-a8: the fp32 dequant-and-matmul (engine/model.py:168-170,184,188-190,193)
# --------------------------------------------------------------------------

def linear(x: np.ndarray, q: np.ndarray, scale: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """fp32 oracle of ``F.linear(x, dequantize(q, scale, float32), bias)``.

    ``x``: float32 ``[M,K]`` (activation values, already bf16-representable in
    the GPU workloads).  ``bias``: float32 ``[N]`` or None.  The dequantized
    weight is formed in fp32 exactly as engine/quantization.py:27 forms it; the
    sum runs in float64 so the oracle is deterministic (BLAS fp32 results vary
    with blocking and thread count) and is then rounded to float32.
    """
    w = dequantize(q, scale, "f32").astype(np.float64)
    y = np.asarray(x, dtype=np.float64) @ w.T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64).reshape(1, -1)
    return y.astype(np.float32)


def silu(x: np.ndarray) -> np.ndarray:
    """``F.silu``: x * sigmoid(x), in float64."""
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def swiglu(x, q_gate, s_gate, q_up, s_up) -> np.ndarray:
    """``F.silu(F.linear(h, Wg)) * F.linear(h, Wu)`` (engine/model.py:188-190), fp32."""
    g = linear(x, q_gate, s_gate).astype(np.float64)
    u = linear(x, q_up, s_up).astype(np.float64)
    return (silu(g) * u).astype(np.float32)


def mlp(x, q_gate, s_gate, q_up, s_up, q_down, s_down) -> np.ndarray:
    """``F.linear(F.silu(gate) * up, Wd)`` (engine/model.py:188-190) in fp32 throughout."""
    act = swiglu(x, q_gate, s_gate, q_up, s_up)
    return linear(act, q_down, s_down)


# --------------------------------------------------------------------------
# the linears' neighbours (engine/model.py:29-34, 166, 184, 187, 190)
# --------------------------------------------------------------------------

def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """``rms_norm(x, weight, eps)`` (engine/model.py:29-34) for bf16 tensors:
    var = mean(x^2) over the last dim in fp32, r = rsqrt(var + eps) in fp32,
    h = bf16(weight * bf16(x * r)).  ``x``, ``weight``: bf16-representable
    float32 arrays.  The mean is formed in float64 and rounded once to fp32 (a
    fp32 reduction in any order agrees with it to a few fp32 ulps); the
    rsqrt is correctly rounded.  Returns bf16-representable float32."""
    x = np.asarray(x, dtype=np.float32)
    var = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    r = (1.0 / np.sqrt((var + np.float32(eps)).astype(np.float64))).astype(np.float32)
    t = round_to_bf16((x * r).astype(np.float32))
    return round_to_bf16((np.asarray(weight, dtype=np.float32) * t).astype(np.float32))


def rmsnorm_bracket(x: np.ndarray, weight: np.ndarray, eps: float, ulps: int = 4) -> tuple[np.ndarray, np.ndarray]:
    """Elementwise [lo, hi] of ``rms_norm`` over every r within ``ulps`` fp32
    ulps of the correctly rounded r = rsqrt(mean(x^2) + eps).  An fp32 sum of
    squares in another order moves r by a few ulps; where that flips the
    inner rounding bf16(x * r), the multiply by the weight and the second
    rounding carry the step into h (up to two bf16 ulps of h).  Every other
    part of the formula is fixed, so a correct implementation lies inside the
    bracket on every element.  h is monotone in r, so the extremes over the
    2 ulps + 1 values of r bound it."""
    x = np.asarray(x, dtype=np.float32)
    w = np.asarray(weight, dtype=np.float32)
    var = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(np.float32)
    r = (1.0 / np.sqrt((var + np.float32(eps)).astype(np.float64))).astype(np.float32)
    lo = hi = None
    for k in range(-ulps, ulps + 1):
        rk = r.copy()
        for _ in range(abs(k)):
            rk = np.nextafter(rk, np.float32(np.inf) if k > 0 else np.float32(0)).astype(np.float32)
        h = round_to_bf16((w * round_to_bf16((x * rk).astype(np.float32))).astype(np.float32))
        lo = h if lo is None else np.minimum(lo, h)
        hi = h if hi is None else np.maximum(hi, h)
    return lo, hi


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """``apply_rope(x, cos, sin)`` (engine/model.py:53-56, ``rotate_half`` at
    :37-39) for bf16 tensors: ``x * cos + rotate_half(x) * sin`` where every
    bf16 op computes in fp32 and rounds once.  x: (tokens, heads, head_dim)
    float32 holding bf16 values; cos / sin: (tokens, head_dim) the same.
    Returns float32 holding the bf16 result."""
    x = np.asarray(x, np.float32)
    h = x.shape[-1] // 2
    rot = np.concatenate([-x[..., h:], x[..., :h]], axis=-1)   # rotate_half: exact negation
    c = np.asarray(cos, np.float32)[:, None, :]
    s = np.asarray(sin, np.float32)[:, None, :]
    t1 = round_to_bf16(x * c)
    t2 = round_to_bf16(rot * s)
    return round_to_bf16(t1 + t2)


def linear_residual_intermediate(x, q, scale, bias=None) -> np.ndarray:
    """The intermediate of :func:`linear_residual` with a bf16 output: the
    linear output rounded to bf16 before the add."""
    return round_to_bf16(linear(x, q, scale, bias))


def linear_residual(x, q, scale, residual, bias=None, bf16_out: bool = True) -> np.ndarray:
    """``residual + F.linear(h, W, b)`` (engine/model.py:184, 190): the linear
    output is rounded to the output dtype first, then added to the bf16
    residual and rounded once more (bf16 output)."""
    lin = linear(x, q, scale, bias)
    if bf16_out:
        return round_to_bf16((round_to_bf16(lin) + np.asarray(residual, dtype=np.float32)).astype(np.float32))
    return (lin + np.asarray(residual, dtype=np.float32)).astype(np.float32)


# --------------------------------------------------------------------------
# Tolerances stated by the path's specification
# --------------------------------------------------------------------------

REL_TOL = 1e-2  # max|y - y_ref| / max|y_ref|   (tests/test_quantization.py:45 definition)


def abs_tol(k: int) -> float:
    """Max elementwise abs error allowed for a reduction of length k."""
    return 2e-2 * float(np.sqrt(k / 1024.0))


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |v| (8 significant bits)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


U32 = 2.0 ** -24  # unit roundoff of fp32


def acc_bound(x: np.ndarray, q: np.ndarray, scale: np.ndarray, bias: np.ndarray | None = None,
              dx: np.ndarray | None = None) -> np.ndarray:
    """Elementwise bound on how far an fp32 evaluation of :func:`linear` can
    be from the exact value, whatever the summation order: the products
    x_i * q_i are exact in fp32 (8 + 8 significant bits), at most K additions
    and the scale multiply and bias add each round once, so the error is at
    most (K + 8) * u * (s * sum_i |x_i q_i| + |b|) with u = 2^-24 (first order;
    the margin of 8 covers the cross-wave and split sums and the second-order
    terms).  ``dx``: an elementwise bound on how far the kernel's input may
    be from ``x`` (an RMSNorm computed in another summation order), which
    moves the output by at most |dx| |W|^T.  float64, shape [M, N]."""
    k = np.asarray(q).shape[1]
    w = np.abs(dequantize(q, scale, "f32").astype(np.float64))
    s = np.abs(np.asarray(x, dtype=np.float64)) @ w.T
    if bias is not None:
        s = s + np.abs(np.asarray(bias, dtype=np.float64)).reshape(1, -1)
    out = (k + 8) * U32 * s
    if dx is not None:
        out = out + np.abs(np.asarray(dx, dtype=np.float64)) @ w.T
    return out


def swiglu_acc(x, q_gate, s_gate, q_up, s_up, dx=None) -> np.ndarray:
    """Elementwise bound on how far an fp32 evaluation of :func:`swiglu` can
    be from the exact value: the gate and up sums carry :func:`acc_bound`
    errors dg, du; act = silu(g) * u moves by at most |silu'| dg |u| +
    |silu(g)| du + dg du (|silu'| <= 1.1 everywhere; its value at g is used),
    and the fp32 evaluation of silu (exp, add, divide) and the product add
    at most (16 + |g| log2 e) u |act|: the exp2 argument -g log2 e is itself
    rounded, an error that grows with |g|.  ``dx`` as for :func:`acc_bound`."""
    g = linear(x, q_gate, s_gate).astype(np.float64)
    u = linear(x, q_up, s_up).astype(np.float64)
    dg = acc_bound(x, q_gate, s_gate, dx=dx)
    du = acc_bound(x, q_up, s_up, dx=dx)
    sig = 1.0 / (1.0 + np.exp(-g))
    dsilu = np.abs(sig * (1.0 + g * (1.0 - sig))) + dg  # the slope anywhere within dg of g (|silu''| <= 0.5)
    return dsilu * dg * np.abs(u) + np.abs(g * sig) * du + dg * du + (16 + np.abs(g) * 1.4426950408889634) * U32 * np.abs(g * sig * u)


def mlp_acc(x, q_gate, s_gate, q_up, s_up, q_down, s_down) -> np.ndarray:
    """Elementwise bound for :func:`mlp` evaluated as the kernels do it: the
    SwiGLU activations rounded once to bf16 (half an ulp plus
    :func:`swiglu_acc` from the exact ones) feed the down projection, whose
    own accumulation adds :func:`acc_bound`."""
    act = swiglu(x, q_gate, s_gate, q_up, s_up)
    dact = 0.5 * bf16_ulp(act) + swiglu_acc(x, q_gate, s_gate, q_up, s_up)
    return acc_bound(act, q_down, s_down, dx=dact)


def rmsnorm_dx(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """Elementwise width of :func:`rmsnorm_bracket`: how far an RMSNorm in
    another fp32 summation order may be from :func:`rmsnorm`."""
    lo, hi = rmsnorm_bracket(x, weight, eps)
    return np.abs(hi.astype(np.float64) - lo.astype(np.float64))


def compare(y: np.ndarray, y_ref: np.ndarray, k: int, bf16_out: bool = False,
            ulp_of: np.ndarray | None = None, acc=None) -> dict:
    """Error report of y against the oracle; ``ok`` when both bounds hold.

    ``rel`` = max|y - y_ref| / max|y_ref| must be <= 1e-2 and every element
    must satisfy |y - y_ref| <= 2e-2 * sqrt(k/1024).

    bf16 outputs (``bf16_out``): a correctly rounded bf16 result of an fp32
    value that is within ``acc`` of the exact one lies within half a bf16 ulp
    + ``acc`` of the oracle's (unrounded) value, so the elementwise bound is
    floored there: half an ulp at the larger of |y| and |y_ref| (two results
    on either side of a power of two are half an ulp of the upper binade from
    the value between them) plus ``acc``, the elementwise accumulation bound
    (:func:`acc_bound`, :func:`swiglu_acc`), which a single-rounding bf16
    comparison must be given.  Below that spacing no bf16 result can resolve
    the stated bound (a value in [8, 16) has a half-ulp of 0.031 > 2e-2 *
    sqrt(2)).  ``ulp_of``: the intermediate bf16 value of a result rounded
    twice (residual + bf16(linear), engine/model.py:184) against an oracle
    that rounds the same twice: the two intermediates may sit on either side
    of a rounding midpoint, one ulp apart, and that step survives the sum
    (also when it cancels to a smaller binade) while the final rounding can
    add one ulp of the result, so the floor is ulp(intermediate) +
    ulp(result) (+ ``acc`` when given).
    """
    y = np.asarray(y, dtype=np.float64)
    r = np.asarray(y_ref, dtype=np.float64)
    if y.shape != r.shape:
        raise ValueError(f"shape mismatch {y.shape} vs {r.shape}")
    tol = abs_tol(k)
    if y.size == 0:
        return {"max_abs": 0.0, "rel": 0.0, "abs_tol": tol, "ok": True}
    if bf16_out and ulp_of is None and acc is None:
        raise ValueError("compare: a single-rounding bf16 comparison needs the accumulation bound `acc`")
    diff = np.abs(y - r)
    max_abs = float(diff.max())
    denom = float(np.abs(r).max())
    rel = max_abs / denom if denom > 0 else max_abs
    big = np.maximum(np.abs(r), np.abs(y))
    extra = np.zeros_like(diff) if acc is None else np.broadcast_to(np.asarray(acc, dtype=np.float64), diff.shape)
    if ulp_of is not None:
        floor = bf16_ulp(big) + bf16_ulp(np.asarray(ulp_of, dtype=np.float64)) + extra
    else:
        floor = 0.5 * bf16_ulp(big) + extra
    bound = np.maximum(tol, floor) if bf16_out else tol
    worst = float((diff / bound).max())
    ok = bool(np.isfinite(y).all()) and rel <= REL_TOL and worst <= 1.0
    return {"max_abs": max_abs, "rel": rel, "abs_tol": tol, "worst_vs_bound": worst, "ok": ok}


def argmax_rows(logits: np.ndarray) -> np.ndarray:
    """First index of the row maximum (torch.argmax tie rule), per row."""
    return np.argmax(np.asarray(logits), axis=-1)


def top2_gap(logits: np.ndarray) -> np.ndarray:
    """Per-row gap between the largest and second-largest logit."""
    part = np.partition(np.asarray(logits, dtype=np.float64), -2, axis=-1)
    return part[..., -1] - part[..., -2]
