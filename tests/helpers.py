"""Shared input builders for the parity tests: seeded numpy inputs, their
oracle results, and the same data placed on the GPU."""

from __future__ import annotations

import numpy as np
import torch

from oracle import quantization_oracle as O


def weights(seed: int, n: int, k: int, std: float = 0.02) -> np.ndarray:
    """fp32 ~ N(0, std) weight [n, k]."""
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, k), dtype=np.float32) * np.float32(std)).astype(np.float32)


def activations(seed: int, m: int, k: int) -> np.ndarray:
    """bf16-representable fp32 activations ~ N(0, 1) [m, k]."""
    rng = np.random.default_rng(seed)
    return O.round_to_bf16(rng.standard_normal((m, k), dtype=np.float32))


def bf16_gpu(a: np.ndarray, device) -> torch.Tensor:
    """float32 numpy values (already bf16-representable) -> bf16 GPU tensor, exact."""
    bits = O.f32_to_bf16_bits(a)
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(device)


def to_np(t: torch.Tensor) -> np.ndarray:
    """GPU tensor -> float32 numpy (bf16 widens exactly)."""
    return t.detach().float().cpu().numpy()


def report(y: np.ndarray, y_ref: np.ndarray, k: int, what: str, bf16_out: bool = True, ulp_of=None,
           acc=None) -> dict:
    """Asserts the specification's tolerance (oracle.compare) and returns the
    report.  ``acc``: the elementwise accumulation bound of a bf16 output
    (O.acc_bound / O.swiglu_acc of the same inputs)."""
    r = O.compare(y, y_ref, k, bf16_out=bf16_out, ulp_of=ulp_of, acc=acc)
    assert r["ok"], f"{what}: {r}"
    return r


def linear_ref(x: np.ndarray, q: np.ndarray, s: np.ndarray, b: np.ndarray | None = None) -> dict:
    """Oracle output and accumulation bound of a linear, as report() keywords:
    ``report(y, **linear_ref(x, q, s, b), k=..., what=...)``."""
    return {"y_ref": O.linear(x, q, s, b), "acc": O.acc_bound(x, q, s, b)}


def swiglu_ref(x: np.ndarray, qg, sg, qu, su) -> dict:
    """Oracle output and accumulation bound of the SwiGLU pair."""
    return {"y_ref": O.swiglu(x, qg, sg, qu, su), "acc": O.swiglu_acc(x, qg, sg, qu, su)}
