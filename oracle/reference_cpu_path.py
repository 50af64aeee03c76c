"""The reference's per-call CPU path, restated with the same torch ops.

TEST/BENCH INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): timed by
``bench.py`` as the CPU baseline, never part of the product.

Per projection the reference runs ``QuantizedWeight.get()`` ->
``dequantize(q, scale, dtype)`` = ``(q.to(float32) * scale).to(dtype)``
(engine/quantization.py:27, 40-41) and then ``F.linear(h, W, b)``
(engine/model.py:168-170, 184, 188-190).  This module issues exactly those
torch calls on CPU tensors.
"""

from __future__ import annotations

import os
import statistics
import time

import torch
import torch.nn.functional as F


def per_call_linear(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor,
                    bias: torch.Tensor | None = None, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``F.linear(x, dequantize(q, scale, dtype), bias)`` as the reference runs it."""
    w = (q.to(torch.float32) * scale).to(dtype)
    return F.linear(x, w, bias)


def cpu_threads() -> int:
    """Threads to use: the host's CPU share for this job (OMP_NUM_THREADS when
    the scheduler sets it), never more than the affinity mask allows."""
    aff = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(aff, int(env))) if env and env.isdigit() else aff


def cpu_model() -> dict:
    info = {"model": "unknown", "amx_bf16": False, "avx512f": False}
    try:
        with open("/proc/cpuinfo") as f:
            text = f.read()
        for line in text.splitlines():
            if line.startswith("model name"):
                info["model"] = line.split(":", 1)[1].strip()
                break
        flags = next((l for l in text.splitlines() if l.startswith("flags")), "")
        info["amx_bf16"] = " amx_bf16" in flags
        info["avx512f"] = " avx512f" in flags
    except OSError:
        pass
    return info


def _layer_runner(x, xi, order=("q", "k", "v", "o", "gate", "up", "down")):
    m = x.shape[0]

    def run_layer(L):
        nbytes = flops = 0
        for name in order:
            q, s = L[name]
            inp = xi if name == "down" else x
            b = L.get(name + "_b")
            per_call_linear(inp, q, s, b)
            n, k = q.shape
            nbytes += n * k + 4 * n + 2 * m * k + 2 * m * n + (2 * n if b is not None else 0)
            flops += 2 * m * n * k
        return nbytes, flops

    return run_layer


def time_layers(get_layer, n_layers: int, m: int, budget_s: float = 12.0, seed: int = 99, warmup: int = 3,
                runs: int = 10) -> dict:
    """Times the reference's 7 per-call linears over a sample of layers:
    ``warmup`` untimed passes, then the median of ``runs`` timed passes over
    the first ``count`` layers, ``count`` chosen so that all passes fit about
    ``budget_s`` seconds.

    ``get_layer(i)`` returns layer i as CPU tensors {name: (q int8 [N,K],
    scale fp32 [N,1])} plus optional "q_b"/"k_b"/"v_b" bf16 biases (all
    sampled layers are fetched before any timing).  Returns the median pass's
    seconds, the layers per pass, the algorithmic bytes / flops of one pass,
    every pass's seconds and the thread count.
    """
    torch.set_num_threads(cpu_threads())
    g = torch.Generator().manual_seed(seed)
    first = get_layer(0)
    hidden = first["q"][0].shape[1]
    inter = first["gate"][0].shape[0]
    x = torch.randn(m, hidden, generator=g).to(torch.bfloat16)
    xi = torch.randn(m, inter, generator=g).to(torch.bfloat16)
    run_layer = _layer_runner(x, xi)
    with torch.inference_mode():
        run_layer(first)  # thread pools, allocator
        t0 = time.perf_counter()
        run_layer(first)
        per_layer = time.perf_counter() - t0
        count = max(1, min(n_layers, int(budget_s / max(per_layer, 1e-6) / (warmup + runs))))
        layers = [first] + [get_layer(i) for i in range(1, count)]
        secs = []
        for rep in range(warmup + runs):
            t0 = time.perf_counter()
            totals = [run_layer(L) for L in layers]
            if rep >= warmup:
                secs.append(time.perf_counter() - t0)
    med = statistics.median(secs)
    return {"seconds": med, "layers": count, "bytes": sum(b for b, _ in totals), "flops": sum(f for _, f in totals),
            "threads": cpu_threads(), "runs": secs, "warmup": warmup}
