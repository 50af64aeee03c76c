"""Exact-arithmetic restatement used to pin the oracle.

Independent of numpy's floating-point kernels: every value is converted to a
``fractions.Fraction`` (exact), quotients and sums are exact rationals, and
rounding to fp32 is done here by comparing exact distances to the neighbouring
fp32 values (ties to the even significand).  Python's ``round`` supplies the
round-half-to-even step.  Slow: for tiny inputs only.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np

F32 = np.float32
_ONE_E_MINUS_8 = Fraction(float(np.float32(1e-8)))


def frac(v) -> Fraction:
    return Fraction(float(v))


def round_f32(fr: Fraction) -> np.float32:
    """Correctly rounded (nearest, ties to even) fp32 value of a rational."""
    if fr == 0:
        return F32(0.0)
    c = F32(float(fr))
    best = None
    for v in (c, np.nextafter(c, F32(np.inf)), np.nextafter(c, F32(-np.inf))):
        if not np.isfinite(v):
            continue
        d = abs(frac(v) - fr)
        key = (d, int(np.array(v, dtype=np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, v)
    return F32(best[1])


def quantize_row(row) -> tuple[list[int], np.float32]:
    """engine/quantization.py:20-22 for one row, in exact arithmetic."""
    vals = [frac(v) for v in row]
    absmax = max([abs(v) for v in vals] + [Fraction(0)])
    absmax = max(absmax, _ONE_E_MINUS_8)
    scale = round_f32(absmax / 127)
    s = frac(scale)
    q = []
    for v in vals:
        r = round_f32(v / s)          # IEEE fp32 quotient
        qi = round(float(r))          # Python's round: ties to even
        q.append(max(-127, min(127, qi)))
    return q, scale


def quantize(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    qs, ss = [], []
    for row in np.asarray(w, dtype=np.float32):
        q, s = quantize_row(row)
        qs.append(q)
        ss.append(s)
    return np.array(qs, dtype=np.int8).reshape(w.shape), np.array(ss, dtype=np.float32).reshape(-1, 1)


def linear(x, q, scale, bias=None) -> list[list[Fraction]]:
    """Exact y[i][r] = sum_j x[i][j] * fp32(q[r][j] * scale[r]) (+ bias[r])."""
    x = np.asarray(x, dtype=np.float32)
    q = np.asarray(q)
    s = np.asarray(scale, dtype=np.float32).reshape(-1)
    w = [[frac(round_f32(Fraction(int(q[r, j])) * frac(s[r]))) for j in range(q.shape[1])] for r in range(q.shape[0])]
    out = []
    for i in range(x.shape[0]):
        xi = [frac(v) for v in x[i]]
        row = []
        for r in range(q.shape[0]):
            acc = sum((a * b for a, b in zip(xi, w[r])), Fraction(0))
            if bias is not None:
                acc += frac(np.float32(bias[r]))
            row.append(acc)
        out.append(row)
    return out


def ulp_f32(v: float) -> float:
    a = abs(F32(v))
    return float(np.nextafter(a, F32(np.inf)) - a)
