"""Benchmark of the INT8 weight-only (W8A16) linear path on one MI355X.

Workload (one "step"): the linear projections of one decode token through
all 36 layers of a Qwen2.5-3B-shaped model, as a dependent chain with the
neighbours a real decode step runs between them (attention output fixed):
layer 0's RMSNorm + q|k|v (with bias) + RoPE, then per layer o + residual,
RMSNorm, gate|up (2x 11008x2048, SwiGLU), down (2048x11008) + residual and the
next layer's RMSNorm + q|k|v + RoPE -- one persistent launch per layer where a
single-launch configuration exists (one or two tokens), the per-projection
kernels otherwise -- on distinct synthetic int8 weights per layer (2.77 GB,
far beyond the 256 MB MALL), activations ~N(0,1) bf16 resident in HBM.  The
launches of a step are captured once in a HIP graph and replayed.  Bytes are
the linears' algorithmic bytes (the norms and RoPE are not counted).

Reported (one JSON line on stdout):
  value          whole-sweep algorithmic GB/s at M=1 (int8 W + fp32 scale +
                 bf16 x + bf16 y + bf16 bias, as the launches read/write them)
  roofline       the dominant kernel (the one launch per layer at M=1):
                 algorithmic bytes per launch / mean launch time from HIP
                 events, vs 8 TB/s
  prefill        the same sweep at M=512 in TFLOP/s vs the 2.5 PFLOP/s bf16
                 dense MFMA peak, with its own dominant-kernel roofline
  per_call_sweep the reference's call structure (7 separate linears/layer)
  decode_detail  eager (no graph) time; the same chain with per-projection
                 kernels (norm inside the projections, as separate kernels,
                 and as the reference's torch op chains); the independent
                 four-launch sweep on fixed inputs; the gate|up and down_proj
                 kernels' rooflines
  other_configs  decode at M=4 and 16, prefill at M=128 and 2048, the fused
                 SwiGLU MLP, the int8 lm_head at M=1/8/256 (fp32 logits) and
                 the single 4864x896 linear beside its CPU reference path
  torch_gpu      the reference's computation with torch on this GPU
  cpu_baseline   the reference's per-call path (dequantize to bf16, then
                 F.linear) with torch on this host's CPU cores, on a sample
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
LAYERS, HIDDEN, INTER, KV = 36, 2048, 11008, 256


def log(*a):
    print(*a, file=sys.stderr, flush=True)


SHAPES = {"q": (HIDDEN, HIDDEN), "k": (KV, HIDDEN), "v": (KV, HIDDEN), "o": (HIDDEN, HIDDEN),
          "gate": (INTER, HIDDEN), "up": (INTER, HIDDEN), "down": (HIDDEN, INTER)}


def layer_weight(dev, l: int, j: int, n: int, k: int):
    """fp32 weight j of layer l, ~N(0, 0.02) from its own seed (regenerated
    bit for bit by the correctness gate)."""
    g = torch.Generator(device=dev).manual_seed(1234 + 100 * l + j)
    return torch.randn((n, k), generator=g, device=dev, dtype=torch.float32) * 0.02


def make_layers(dev, layers: int):
    from pageserve_amd import quantization as Q

    out = []
    for l in range(layers):
        L = {}
        for j, (name, (n, k)) in enumerate(SHAPES.items()):
            w = layer_weight(dev, l, j, n, k)
            L[name] = Q.QuantizedWeight(w)
            del w
        for j, (name, n) in enumerate((("q_b", HIDDEN), ("k_b", KV), ("v_b", KV))):
            g = torch.Generator(device=dev).manual_seed(5000 + 100 * l + j)
            L[name] = (torch.randn(n, generator=g, device=dev) * 0.1).to(torch.bfloat16)
        out.append(L)
    torch.cuda.synchronize()
    return out


def linear_bytes(m, n, k, bias=False, out_bytes=2):
    return n * k + 4 * n + 2 * m * k + out_bytes * m * n + (2 * n if bias else 0)


def fused_sweep(layers, x, xo, m):
    """One step with the fused call structure; returns (callable, bytes, flops, launches)."""
    from pageserve_amd import quantization as Q

    def step():
        outs = None
        for L in layers:
            outs = Q.linear_group(x, [L["q"], L["k"], L["v"]], [L["q_b"], L["k_b"], L["v_b"]])
            L["o"].linear(xo)
            act = Q.swiglu(x, L["gate"], L["up"])
            outs.append(L["down"].linear(act))
        return outs

    per_layer_f = 2 * m * HIDDEN * (HIDDEN + 2 * KV + HIDDEN + 2 * INTER) + 2 * m * INTER * HIDDEN
    return step, layer_bytes(m) * len(layers), per_layer_f * len(layers), 4 * len(layers)


def layer_bytes(m):
    """Algorithmic bytes of one layer's linears: q|k|v with bias (x read
    once), o, gate|up -> act, down (int8 W + fp32 scale + bf16 x and y)."""
    return (linear_bytes(m, HIDDEN + 2 * KV, HIDDEN, bias=True)
            + linear_bytes(m, HIDDEN, HIDDEN)
            + 2 * INTER * HIDDEN + 8 * INTER + 2 * m * HIDDEN + 2 * m * INTER
            + linear_bytes(m, HIDDEN, INTER))


def per_call_sweep(layers, x, xo, xi, m):
    """The reference's structure: 7 separate linears per layer (engine/model.py:168-190)."""

    def step():
        y = None
        for L in layers:
            L["q"].linear(x, L["q_b"])
            L["k"].linear(x, L["k_b"])
            L["v"].linear(x, L["v_b"])
            L["o"].linear(xo)
            L["gate"].linear(x)
            L["up"].linear(x)
            y = L["down"].linear(xi)
        return y

    per_layer_b = (linear_bytes(m, HIDDEN, HIDDEN, True) + 2 * linear_bytes(m, KV, HIDDEN, True)
                   + linear_bytes(m, HIDDEN, HIDDEN) + 2 * linear_bytes(m, INTER, HIDDEN)
                   + linear_bytes(m, HIDDEN, INTER))
    per_layer_f = 2 * m * (2 * HIDDEN * HIDDEN + 2 * KV * HIDDEN + 3 * INTER * HIDDEN)
    return step, per_layer_b * len(layers), per_layer_f * len(layers), 7 * len(layers)


def dropin_sweep(layers, x, xo, xi):
    """The reference's own call structure through the drop-in (engine/model.py
    :25-26, 168-190): ``F.linear(h, _resolve(W), b)`` with ``_resolve(W) =
    W.get()`` on bf16-model QuantizedWeights (the same int8 storage), the
    SwiGLU as ``F.silu(gate) * up`` in torch; 7 linears per layer."""
    import torch.nn.functional as F

    from pageserve_amd import quantization as Q

    def bf16_view(w):
        st = dict(w.state())
        st["meta"] = torch.tensor([w.shape[0], w.shape[1], 1], dtype=torch.int64)
        return Q.QuantizedWeight.from_state(st)

    views = [{name: bf16_view(L[name]) for name in SHAPES} for L in layers]

    def step():
        y = None
        for L, W in zip(layers, views):
            F.linear(x, W["q"].get(), L["q_b"])
            F.linear(x, W["k"].get(), L["k_b"])
            F.linear(x, W["v"].get(), L["v_b"])
            F.linear(xo, W["o"].get())
            act = F.silu(F.linear(x, W["gate"].get())) * F.linear(x, W["up"].get())
            y = F.linear(act, W["down"].get())
        return y

    return step


def torch_gpu_entry(ref_ms, dense_ms, ours_ms, work, unit):
    """Report line for the torch comparison: the same work per sweep (this
    package's algorithmic bytes or flops) over each path's time."""
    scale = 1e9 if unit == "GB/s" else 1e12
    return {
        "what": "same 36-layer sweep with torch on this GPU: the reference's per-call dequantize "
                "(engine/quantization.py:26-27) + F.linear, and F.linear on dense bf16 weights",
        "reference_path_ms_per_step": round(ref_ms, 5),
        "reference_path_rate": round(work / (ref_ms * 1e-3) / scale, 2),
        "dense_bf16_ms_per_step": round(dense_ms, 5),
        "dense_bf16_rate": round(work / (dense_ms * 1e-3) / scale, 2),
        "unit": unit,
        "speedup_vs_reference_path": round(ref_ms / ours_ms, 3),
        "speedup_vs_dense_bf16": round(dense_ms / ours_ms, 3),
    }


def torch_reference_sweeps(layers, x, xo, steps):
    """The reference's own computation with torch on this GPU, no kernel of
    this package inside the timed graphs: per layer the 7 linears of
    engine/model.py:168-190, each weight dequantized per call exactly as
    engine/quantization.py:26-27 ((q.float() * scale).to(bf16)) and then
    F.linear (hipBLASLt); and the same linears on weights dequantized once
    beforehand (dense bf16, twice the weight bytes).  Returns ms per sweep."""
    import torch.nn.functional as F

    names = ("q", "k", "v", "o", "gate", "up", "down")
    q8 = [{n: (L[n].q, L[n].scale.reshape(-1, 1)) for n in names} for L in layers]

    def deq(q, s):
        return (q.float() * s).to(torch.bfloat16)

    def run(get):
        y = None
        for L, W in zip(layers, get):
            F.linear(x, W("q"), L["q_b"])
            F.linear(x, W("k"), L["k_b"])
            F.linear(x, W("v"), L["v_b"])
            F.linear(xo, W("o"))
            act = F.silu(F.linear(x, W("gate"))) * F.linear(x, W("up"))
            y = F.linear(act, W("down"))
        return y

    per_call = [(lambda d: (lambda n: deq(*d[n])))(d) for d in q8]
    g, _ = capture(lambda: run(per_call))
    ms_ref = time_graph(g, steps, 3)
    del g
    dense = [{n: deq(*d[n]) for n in names} for d in q8]
    del q8, per_call
    pre = [(lambda d: (lambda n: d[n]))(d) for d in dense]
    g, _ = capture(lambda: run(pre))
    ms_dense = time_graph(g, steps, 3)
    del g, dense, pre
    torch.cuda.empty_cache()
    return ms_ref, ms_dense


def reference_rms_norm(x, weight, eps):
    """engine/model.py:29-34 as the reference runs it (a chain of torch ops)."""
    dtype = x.dtype
    xf = x.float()
    variance = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(variance + eps)
    return weight * xf.to(dtype)


def reference_apply_rope(x, cos, sin):
    """engine/model.py:37-39,53-56 (rotate_half, apply_rope), the torch op chain."""
    x1, x2 = x.chunk(2, dim=-1)
    return x * cos.unsqueeze(1) + torch.cat((-x2, x1), dim=-1) * sin.unsqueeze(1)


def layer_chain(layers, x0, attn, norms, rope, mode):
    """The decoder layers' linears with their neighbours (engine/model.py:165-190,
    attention replaced by a fixed input): norm -> q|k|v -> RoPE of q and k,
    x += o(attn), norm -> gate|up -> down, x += down.  mode "reference": the
    reference's torch op chains and separate adds around the same linears;
    "kernels": the RMSNorm and RoPE kernels and the residual adds in the
    linear epilogues; "norm_in_linear": as "kernels" with each RMSNorm inside
    the projection launch that consumes it."""
    from pageserve_amd import quantization as Q

    cos, sin = rope
    m = x0.shape[0]
    heads, kv_heads, hd = HIDDEN // 128, KV // 128, 128

    def step():
        x = x0
        for L, (ln1, ln2) in zip(layers, norms):
            if mode == "norm_in_linear":
                q, k, _ = Q.rmsnorm_linear_group(x, ln1, 1e-6, [L["q"], L["k"], L["v"]],
                                                 [L["q_b"], L["k_b"], L["v_b"]])
                Q.rope_qk(q.view(m, heads, hd), k.view(m, kv_heads, hd), cos, sin, inplace=True)
                x = L["o"].linear(attn, residual=x)
                x = Q.rmsnorm_mlp(x, ln2, 1e-6, L["gate"], L["up"], L["down"], residual=x)
            elif mode == "kernels":
                h = Q.rmsnorm(x, ln1, 1e-6)
                q, k, _ = Q.linear_group(h, [L["q"], L["k"], L["v"]], [L["q_b"], L["k_b"], L["v_b"]])
                Q.rope_qk(q.view(m, heads, hd), k.view(m, kv_heads, hd), cos, sin, inplace=True)
                x = L["o"].linear(attn, residual=x)
                h = Q.rmsnorm(x, ln2, 1e-6)
                x = Q.mlp(h, L["gate"], L["up"], L["down"], residual=x)
            else:
                h = reference_rms_norm(x, ln1, 1e-6)
                q, k, _ = Q.linear_group(h, [L["q"], L["k"], L["v"]], [L["q_b"], L["k_b"], L["v_b"]])
                reference_apply_rope(q.view(m, heads, hd), cos, sin)
                reference_apply_rope(k.view(m, kv_heads, hd), cos, sin)
                x = x + L["o"].linear(attn)
                h = reference_rms_norm(x, ln2, 1e-6)
                x = x + Q.mlp(h, L["gate"], L["up"], L["down"])
        return x

    return step


def decode_chain(layers, x0, attn, norms, rope, m, persistent=None):
    """The headline decode sweep: the linear path of one decode step through
    every layer, each stage data-dependent on the one before (attention
    output fixed, engine/model.py:165-190): layer 0's norm -> q|k|v (+ bias)
    -> RoPE, then per layer o + residual -> norm -> gate|up -> down +
    residual -> the next layer's norm -> q|k|v -> RoPE.  Where
    pageserve_amd.span picks it (``persistent`` as in decode_span) each
    layer's part between two attention calls is one persistent launch;
    otherwise the per-projection kernels.  Returns (step, algorithmic bytes,
    launches, single_launch)."""
    from pageserve_amd import quantization as Q
    from pageserve_amd import span as S

    cos, sin = rope
    sizes = (m, HIDDEN, INTER, HIDDEN, KV, 128)
    single = S.span_supported(*sizes) and (persistent is True or (persistent is None and S.span_default(*sizes)))

    def step():
        L0 = layers[0]
        q, k, v = Q.rmsnorm_linear_group(x0, norms[0][0], 1e-6, [L0["q"], L0["k"], L0["v"]],
                                         [L0["q_b"], L0["k_b"], L0["v_b"]])
        Q.rope_qk(q.view(m, -1, 128), k.view(m, -1, 128), cos, sin, inplace=True)
        x = x0
        outs = [q, k, v]
        for i, L in enumerate(layers):
            N = layers[i + 1] if i + 1 < len(layers) else None
            kw = {} if N is None else dict(next_ln=norms[i + 1][0], next_qkv=(N["q"], N["k"], N["v"]),
                                           next_bias=(N["q_b"], N["k_b"], N["v_b"]), cos=cos, sin=sin)
            x, qkv = S.decode_span(attn, x, L["o"], norms[i][1], L["gate"], L["up"], L["down"], 1e-6,
                                   persistent=persistent, **kw)
            if qkv is not None:
                outs = list(qkv)
        return [x] + outs

    nbytes = len(layers) * layer_bytes(m)
    launches = 2 + (len(layers) if single else 5 * len(layers) - 2)
    return step, nbytes, launches, single


def chain_operands(dev, n_layers, m):
    """Per layer (input norm, post-attention norm) weights ~ 1 + N(0, 0.1),
    and the rotary rows of the reference's cache (engine/model.py:42-47) at
    one position per token (positions 4096..)."""
    ng = torch.Generator(device=dev).manual_seed(77)
    norms = [tuple((1 + 0.1 * torch.randn(HIDDEN, generator=ng, device=dev)).to(torch.bfloat16)
                   for _ in range(2)) for _ in range(n_layers)]
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, 128, 2, device=dev).float() / 128))
    emb = torch.cat((torch.outer(torch.arange(4096, 4096 + m, device=dev).float(), inv_freq),) * 2, dim=-1)
    return norms, (emb.cos().to(torch.bfloat16), emb.sin().to(torch.bfloat16))


def span_timeline(dev, layers_n, m, command):
    """Stage timeline of the single-launch decode chain: per-workgroup
    timestamps of every stage boundary (pageserve_amd.span tracing), from a
    graph of the chain captured with tracing on and replayed; returns a
    markdown summary.  Times are relative to the launch's first workgroup
    start, in microseconds (the trace clock runs at 100 MHz)."""
    import statistics

    from pageserve_amd import span as S

    layers = make_layers(dev, layers_n)
    gen = torch.Generator(device=dev).manual_seed(99 + m)
    x = torch.randn((m, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
    xo = torch.randn((m, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
    norms, rope = chain_operands(dev, layers_n, m)
    step, _, _, single = decode_chain(layers, x, xo, norms, rope, m, persistent=True)
    if not single:
        raise SystemExit(f"bench.py: no single-launch decode span at m={m}")
    plain, _ = capture(step)
    plain_ms = time_graph(plain, 50, 10)
    del plain
    slots = 64
    buf = torch.zeros(slots * 256 * 16, dtype=torch.int64, device=dev)
    S.decode_span_trace(buf)
    try:
        traced, _ = capture(step)  # the launches capture the trace pointer
        traced_ms = time_graph(traced, 50, 10)
        buf.zero_()
        traced.replay()
        torch.cuda.synchronize()
        del traced
    finally:
        S.decode_span_trace(None)
    tr = buf.view(slots, 256, 16).cpu()
    # each replay's workspace starts from a cleared epoch: launch i carries tag i + 1
    launches = [tr[(i + 1) % slots] for i in range(layers_n)]
    names = S.TRACE_MARKS
    full = launches[:-1]  # the last layer ends after publishing x2 (no next q|k|v)
    rows = []
    for i in range(1, 13):
        p50s, maxs, durs = [], [], []
        for t in full:
            t0 = int(t[:, 0].min())
            rel = (t[:, i].double() - t0) / 100.0  # us
            prev = (t[:, i - 1].double() - t0) / 100.0
            p50s.append(float(rel.median()))
            maxs.append(float(rel.max()))
            durs.append(float((rel - prev).median()))
        rows.append((names[i], statistics.median(durs), statistics.median(p50s), statistics.median(maxs)))
    spans = [(int(t[:, 12].max()) - int(t[:, 0].min())) / 100.0 for t in full]
    starts = [(int(t[:, 0].max()) - int(t[:, 0].min())) / 100.0 for t in full]
    gaps = [(int(launches[i + 1][:, 0].min()) - int(launches[i][:, 12].max())) / 100.0 for i in range(layers_n - 2)]
    polls = [[int(v) for v in t[:, 13 + g]] for g in range(3) for t in launches]
    poll_med = [statistics.median([statistics.median(p) for p in polls[g * layers_n:(g + 1) * layers_n]])
                for g in range(3)]
    poll_max = [max(max(p) for p in polls[g * layers_n:(g + 1) * layers_n]) for g in range(3)]
    lines = [f"# Decode span stage timeline, M={m}, Qwen2.5-3B ({layers_n} layers, one persistent launch per layer)",
             "", "Command (repository root):", "", "```", command, "```", "",
             "Per-workgroup timestamps (`s_memrealtime`, 100 MHz) written by lane 0 of each workgroup's control wave "
             "at every stage boundary of `span_kernel` (tracing on: `pgs_w8a16_decode_span_trace`), from one replay "
             "of a HIP graph of the whole chain. Times in microseconds from the launch's first workgroup start; "
             "each figure is the median over the launches of layers 0.."
             f"{layers_n - 2} (the last layer's launch has no q|k|v stage).", "",
             f"- graph replay of the chain: {plain_ms * 1e3:.1f} us untraced, {traced_ms * 1e3:.1f} us traced "
             f"({plain_ms * 1e3 / layers_n:.2f} / {traced_ms * 1e3 / layers_n:.2f} us per layer)",
             f"- launch span (first start to last end): median {statistics.median(spans):.2f} us, "
             f"min {min(spans):.2f}, max {max(spans):.2f}",
             f"- spread of the 256 workgroup starts: median {statistics.median(starts):.2f} us",
             f"- gap from a launch's last end to the next one's first start: median {statistics.median(gaps):.2f} us",
             f"- polls of wave 0 of each workgroup before each gather saw every word (median / max): x1 "
             f"{poll_med[0]:.0f} / {poll_max[0]}, act {poll_med[1]:.0f} / {poll_max[1]}, x2 {poll_med[2]:.0f} / "
             f"{poll_max[2]}", "",
             "| stage boundary | phase us (p50 over workgroups) | at us, p50 workgroup | at us, last workgroup |",
             "|---|---:|---:|---:|"]
    for name, d, a, b in rows:
        lines.append(f"| {name} | {d:.2f} | {a:.2f} | {b:.2f} |")
    return "\n".join(lines) + "\n"


def capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up outside capture (one-time attribute setup, allocator)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def time_graph(g, steps, warmup):
    """Mean ms per replay over exactly ``steps`` replays after ``warmup``,
    bracketed by synchronisation; events on the replay stream."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        g.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def time_eager(fn, steps, warmup, reps=5):
    """ms per step of `fn` launched eagerly: the median over `reps` timings of
    `steps` back-to-back steps each (a rare host pause, such as a full Python
    garbage collection, lands in one timing instead of the figure)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    runs = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        runs.append((time.perf_counter() - t0) * 1e3 / steps)
    return statistics.median(runs)


def kernel_roofline(layers, launch, bytes_per_launch, flops_per_launch, bound, reps=20):
    """Mean duration of one kernel, launched once per layer back to back
    (distinct weights each time) inside a graph, from HIP events."""
    g, _ = capture(lambda: [launch(L) for L in layers])
    ms = time_graph(g, reps, 3)
    per_launch_s = ms * 1e-3 / len(layers)
    if bound == "hbm":
        achieved = bytes_per_launch / per_launch_s / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
    else:
        achieved = flops_per_launch / per_launch_s / 1e12
        peak, unit = MFMA_BF16_PEAK_TFLOPS, "TFLOP/s"
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": None,
            "launch_us": round(per_launch_s * 1e6, 3), "algorithmic_bytes_per_launch": bytes_per_launch,
            "algorithmic_flops_per_launch": flops_per_launch}


# ---------------------------------------------------------------------------
# HBM traffic from hardware counters.  Two rocprofv3 --pmc passes (FETCH_SIZE,
# then WRITE_SIZE, KiB per dispatch) over `--pmc-workload`; each counter is
# scaled by bytes / reading of a plain streaming kernel of known size (a
# float32 negation, COPY_BYTES read + COPY_BYTES written), then divided into
# per-launch bytes by `--pmc-summary`, which writes TRAFFIC_FILE.
# ---------------------------------------------------------------------------
COPY_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.txt")
# summary key -> pattern on the demangled kernel name: the number-of-matrices
# template argument is 2 for the gate|up pair (skinny_kernel<NW, U, NB, NMAT,
# ...>, gemm_dma_kernel<BM, BN, NMAT, ...>; the profiler's demangler may drop
# the first template argument, hence the optional group)
PMC_KERNELS = {
    "copy": r"neg_kernel",
    "skinny_gate_up_m1": r"skinny_kernel<(\d+, )?\d+, \d+, 2, false",
    "gemm_gate_up_m512": r"gemm_(dma|k64)_kernel<(\d+, )?\d+, 2, false|gemm_kernel<(\d+, )?\d+, 2, false",
    "span_m1": r"span_kernel",
}


def pmc_workload(dev, layers_n):
    """Known-size copy, then the fused gate|up kernel at M=1 and at M=512 once
    per layer: the dispatches the counter passes read."""
    from pageserve_amd import quantization as Q

    src = torch.randn(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    layers = make_layers(dev, layers_n)
    gen = torch.Generator(device=dev).manual_seed(7)
    for m in (1, 512):
        x = torch.randn((m, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
        for L in layers:
            Q.swiglu(x, L["gate"], L["up"])
        torch.cuda.synchronize()
    # the single launch per layer of the decode chain at one token
    from pageserve_amd import span as S

    x = torch.randn((1, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
    ln = torch.ones(HIDDEN, device=dev, dtype=torch.bfloat16)
    for i, L in enumerate(layers):
        N = layers[(i + 1) % len(layers)]
        S.decode_span(x, x, L["o"], ln, L["gate"], L["up"], L["down"], 1e-6, next_ln=ln,
                      next_qkv=(N["q"], N["k"], N["v"]), next_bias=(N["q_b"], N["k_b"], N["v_b"]))
    torch.cuda.synchronize()
    log(f"[bench] pmc workload done: copy x3, gate|up m=1 and m=512, decode span m=1 x {layers_n} layers")


def _pmc_means(dirs):
    """{counter: {key: (mean KiB per dispatch, dispatches, kernel name)}} from rocprofv3 CSV output."""
    import csv
    import glob

    out = {}
    for d in dirs:
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            vals = {}
            with open(path, newline="") as f:
                for row in csv.DictReader(f):
                    name = row["Kernel_Name"]
                    for key, pattern in PMC_KERNELS.items():
                        if re.search(pattern, name):
                            vals.setdefault((row["Counter_Name"], key), []).append((float(row["Counter_Value"]), name))
            for (counter, key), v in vals.items():
                out.setdefault(counter, {})[key] = (sum(a for a, _ in v) / len(v), len(v), v[0][1])
    return out


def pmc_summary(dirs, commands):
    means = _pmc_means(dirs)
    fetch, write = means.get("FETCH_SIZE", {}), means.get("WRITE_SIZE", {})
    if "copy" not in fetch or "copy" not in write:
        raise SystemExit(f"pmc summary: the copy kernel's FETCH_SIZE and WRITE_SIZE are both required "
                         f"(found {sorted((c, k) for c in means for k in means[c])})")
    f_fac = COPY_BYTES / (fetch["copy"][0] * 1024)
    w_fac = COPY_BYTES / (write["copy"][0] * 1024)
    lines = ["# HBM traffic per launch from rocprofv3 --pmc (KiB per dispatch, mean over dispatches),",
             "# each counter scaled by the factor that maps a plain streaming kernel of known size",
             f"# (float32 negation, {COPY_BYTES} B read + {COPY_BYTES} B written) onto its true bytes.",
             "# commands (from the repository root):"]
    lines += [f"#   {c}" for c in commands]
    lines.append(f"copy fetch_kib={fetch['copy'][0]:.1f} write_kib={write['copy'][0]:.1f} "
                 f"factor_fetch={f_fac:.4f} factor_write={w_fac:.4f}")
    for key in PMC_KERNELS:
        if key == "copy" or key not in fetch or key not in write:
            continue
        fk, n, name = fetch[key]
        wk = write[key][0]
        traffic = fk * 1024 * f_fac + wk * 1024 * w_fac
        lines.append(f"{key} dispatches={n} fetch_kib={fk:.1f} write_kib={wk:.1f} "
                     f"traffic_bytes={traffic:.0f} kernel={name}")
    return "\n".join(lines) + "\n"


def read_traffic(key):
    """Per-launch HBM bytes for `key` from TRAFFIC_FILE, or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if parts and parts[0] == key:
                    kv = dict(p.split("=", 1) for p in parts[1:] if "=" in p)
                    return int(float(kv["traffic_bytes"]))
    except (OSError, KeyError, ValueError):
        return None
    return None


# ---------------------------------------------------------------------------
# MFMA utilisation of the prefill launches from hardware counters: a
# rocprofv3 --pmc pass (MfmaUtil, MfmaFlopsBF16, GRBM_GUI_ACTIVE) over
# `--prefill-workload M`, which runs the four launch kinds of the prefill
# sweep once per layer and records each kind's kernel instance
# (pgs_last_plan) in a JSON file; `--mfma-summary` joins the two.
# ---------------------------------------------------------------------------
PREFILL_KINDS = ("q|k|v", "o", "gate|up", "down")


def prefill_flops(m):
    return {"q|k|v": 2 * m * (HIDDEN + 2 * KV) * HIDDEN, "o": 2 * m * HIDDEN * HIDDEN,
            "gate|up": 4 * m * INTER * HIDDEN, "down": 2 * m * HIDDEN * INTER}


def prefill_workload(dev, layers_n, m, plan_path):
    from pageserve_amd import _native
    from pageserve_amd import quantization as Q

    layers = make_layers(dev, layers_n)
    gen = torch.Generator(device=dev).manual_seed(31 + m)
    x = torch.randn((m, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
    xo = torch.randn((m, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
    plans = {}
    for L in layers:
        Q.linear_group(x, [L["q"], L["k"], L["v"]], [L["q_b"], L["k_b"], L["v_b"]])
        plans["q|k|v"] = _native.last_plan()
        L["o"].linear(xo)
        plans["o"] = _native.last_plan()
        act = Q.swiglu(x, L["gate"], L["up"])
        plans["gate|up"] = _native.last_plan()
        L["down"].linear(act)
        plans["down"] = _native.last_plan()
    torch.cuda.synchronize()
    with open(plan_path, "w") as f:
        json.dump({"m": m, "layers": layers_n, "plans": plans, "flops": prefill_flops(m)}, f, indent=1)
    log(f"[bench] prefill workload done: m={m}, {layers_n} layers x {len(PREFILL_KINDS)} launch kinds -> {plan_path}")


def kernel_pattern(plan: str) -> tuple[str, str | None]:
    """The demangled kernel name (template argument list) of a launch plan
    string, and of its follow-up reduce kernel, if any."""
    m = re.search(r"(launch_k64|launch_dma|launch_once|launch_cfg|launch_instance|launch_pair_tiles)\(.*?\) "
                  r"\[(.*?)\]", plan)
    if not m:
        raise ValueError(f"unrecognised launch plan {plan!r}")
    vals = [kv.split(" = ")[1] for kv in m.group(2).split(", ")]
    name = {"launch_k64": "gemm_k64_kernel", "launch_dma": "gemm_dma_kernel", "launch_once": "gemm_once_kernel",
            "launch_cfg": "gemm_kernel", "launch_instance": "skinny_kernel",
            "launch_pair_tiles": "pair_tiles_kernel"}[m.group(1)]
    reduce = None
    if "then gemm_reduce_kernel" in plan:
        reduce = "gemm_reduce_kernel<" + ", ".join(vals[:4])  # then the split count
    return f"{name}<{', '.join(vals)}>", reduce


def _prefill_dispatches(pmc_dir, plan_path):
    """(plan, [(kind, kernel pattern)], {kind: [dispatch rows]}) of a
    --prefill-workload counter pass: every counter of each dispatch, keyed by
    counter name, and its duration ("ns")."""
    import csv
    import glob

    with open(plan_path) as f:
        plan = json.load(f)
    rows = {}
    for path in glob.glob(os.path.join(pmc_dir, "**", "*counter_collection.csv"), recursive=True):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                d = rows.setdefault((r["Kernel_Name"], r["Dispatch_Id"]), {"name": r["Kernel_Name"],
                                                                          "id": r["Dispatch_Id"]})
                d[r["Counter_Name"]] = float(r["Counter_Value"])
                d["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    # the workload issues, per layer, the launch kinds in PREFILL_KINDS order
    # (each followed by its reduce kernel when it has one): walk this
    # package's dispatches in dispatch order and hand each to the next
    # expected launch (q|k|v and o can be the same kernel instance)
    seq = []
    for kind in PREFILL_KINDS:
        kname, reduce = kernel_pattern(plan["plans"][kind])
        seq.append((kind, kname))
        if reduce:
            seq.append((kind + " (reduce)", reduce))
    ours = sorted((d for d in rows.values() if any(pat in d["name"] for _, pat in seq)),
                  key=lambda d: int(d["id"]))
    by_kind = {kind: [] for kind, _ in seq}
    i = 0
    for d in ours:
        for step in range(len(seq)):
            kind, pat = seq[(i + step) % len(seq)]
            if pat in d["name"]:
                by_kind[kind].append(d)
                i = (i + step + 1) % len(seq)
                break
    return plan, seq, by_kind


def mfma_summary(pmc_dir, plan_path, command):
    """Per launch kind: mean dispatch duration (the counter pass's own
    timestamps), MfmaUtil, MFMA flops counted by the hardware, and the
    algorithmic TFLOP/s against the 2.5 PFLOP/s bf16 dense peak."""
    import statistics

    plan, seq, by_kind = _prefill_dispatches(pmc_dir, plan_path)
    m = plan["m"]
    lines = [f"# MFMA utilisation of the prefill launches, M={m}, Qwen2.5-3B linears ({plan['layers']} layers)", "",
             "Command (repository root):", "", "```", command, "```", "",
             "Counters per dispatch from `rocprofv3 --pmc` (one pass: `MfmaUtil` = SQ_VALU_MFMA_BUSY_CYCLES summed "
             "over SIMDs / (GRBM_GUI_ACTIVE x SIMDs), `MfmaFlopsBF16` = SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512), "
             "mean over the dispatches of each launch kind (assigned in dispatch order: the workload issues "
             "q|k|v, o, gate|up, down per layer); durations from the same pass's dispatch timestamps "
             "(kernels serialised by counter collection). Algorithmic flops = 2 M N K per linear (4 M N K for the "
             "gate|up pair); the hardware count also includes the zero padding of partial tiles.", "",
             "| launch | kernel | dispatches | mean us | MfmaUtil % | hw MFMA GFLOP | algorithmic GFLOP | "
             "algorithmic TFLOP/s | % of 2.5 PFLOP/s |",
             "|---|---|---:|---:|---:|---:|---:|---:|---:|"]
    for kind, pat in seq:
        ds = by_kind[kind]
        if not ds:
            lines.append(f"| {kind} | `{pat}` | 0 | | | | | | |")
            continue
        us = statistics.mean(d["ns"] for d in ds) / 1e3
        util = statistics.mean(d.get("MfmaUtil", float("nan")) for d in ds)
        hw = statistics.mean(d.get("MfmaFlopsBF16", float("nan")) for d in ds) / 1e9
        alg = plan["flops"][kind] / 1e9 if kind in plan["flops"] else 0.0
        tf = alg * 1e9 / (us * 1e-6) / 1e12 if alg else 0.0
        lines.append(f"| {kind} | `{pat}` | {len(ds)} | {us:.2f} | {util:.1f} | {hw:.2f} | {alg:.2f} | "
                     f"{tf:.1f} | {100 * tf / MFMA_BF16_PEAK_TFLOPS:.1f} |")
    return "\n".join(lines) + "\n"


# what the counter table says about each counter it may find
COUNTER_NOTES = {
    "VALUBusy": "% of GPU time the CUs issue vector ALU instructions (100 SQ_ACTIVE_INST_VALU / CUs / GRBM_GUI_ACTIVE)",
    "LdsUtil": "% of GPU time the LDS is active (100 SQ_LDS_IDX_ACTIVE / (GRBM_GUI_ACTIVE x CUs))",
    "MfmaUtil": "% of SIMD cycles the MFMA unit is busy",
    "SQ_LDS_BANK_CONFLICT": "cycles LDS is stalled by bank conflicts (sum over CUs)",
    "SQ_INSTS_LDS": "LDS instructions issued (all waves)",
    "SQ_INSTS_VALU": "vector ALU instructions issued, MFMAs included",
    "SQ_INSTS_MFMA": "MFMA instructions issued",
}


def counter_summary(pmc_dir, plan_path, command):
    """Per launch kind of a --prefill-workload counter pass: mean dispatch
    duration and the mean of every counter the pass collected."""
    import statistics

    plan, seq, by_kind = _prefill_dispatches(pmc_dir, plan_path)
    names = sorted({k for ds in by_kind.values() for d in ds for k in d if k not in ("name", "id", "ns")})
    lines = [f"# Counters of the prefill launches, M={plan['m']}, Qwen2.5-3B linears ({plan['layers']} layers)", "",
             "Command (repository root):", "", "```", command, "```", "",
             "Counters per dispatch from one `rocprofv3 --pmc` pass, mean over the dispatches of each launch kind "
             "(assigned in dispatch order: the workload issues q|k|v, o, gate|up, down per layer); durations from "
             "the same pass's dispatch timestamps (kernels serialised by counter collection).", ""]
    for n in names:
        lines.append(f"- `{n}`: {COUNTER_NOTES.get(n, 'raw counter, summed over instances')}")
    lines += ["", "| launch | kernel | dispatches | mean us | " + " | ".join(names) + " |",
              "|---|---|---:|---:|" + "---:|" * len(names)]
    for kind, pat in seq:
        ds = by_kind[kind]
        if not ds:
            continue
        us = statistics.mean(d["ns"] for d in ds) / 1e3
        vals = []
        for n in names:
            v = statistics.mean(d.get(n, float("nan")) for d in ds)
            vals.append(f"{v:.1f}" if abs(v) < 1e4 else f"{v:.4g}")
        lines.append(f"| {kind} | `{pat}` | {len(ds)} | {us:.2f} | " + " | ".join(vals) + " |")
    return "\n".join(lines) + "\n"


def other_configs(layers, dev, steps, gate_inputs=None):
    """The remaining workload sizes, one compact figure each: decode sweeps at
    M=4 and 16, the dependent decode chain at M=2 and 4, prefill sweeps at M=128 and 2048, the fused SwiGLU MLP at M=1
    and 512, the int8 lm_head [151936, 2048] at M=1, 8 and 256 (two copies
    alternated so the 256 MB MALL cannot hold the weight), and the single
    [4864, 896] linear at M=1 with the reference's CPU path beside it.  The
    sweeps' and the MLP's inputs are added to ``gate_inputs`` for the
    correctness gate."""
    from pageserve_amd import quantization as Q

    gen = torch.Generator(device=dev).manual_seed(4242)

    def act(m, k):
        return torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)

    out = {}
    gate_inputs = {} if gate_inputs is None else gate_inputs
    for m in (4, 16):
        x, xo = act(m, HIDDEN), act(m, HIDDEN)
        gate_inputs[m] = (x, xo)
        step, nbytes, _, _ = fused_sweep(layers, x, xo, m)
        g, _ = capture(step)
        ms = time_graph(g, steps, 3)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[f"decode_sweep_m{m}"] = {"us_per_sweep": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                     "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        del g
    from pageserve_amd import span as S

    # the dependent decode chain at 2 and 4 tokens, as the headline's at one:
    # the single launch and the per-projection kernels, and which of the two
    # decode_span picks by default at that size
    for m in (2, 4):
        x0, attn = act(m, HIDDEN), act(m, HIDDEN)
        norms, rope = chain_operands(dev, len(layers), m)
        chain = {"default": "single_launch" if S.span_default(m, HIDDEN, INTER, HIDDEN, KV, 128)
                 else "per_projection"}
        for name, pers in (("single_launch", True), ("per_projection", False)):
            step, nbytes, _, single = decode_chain(layers, x0, attn, norms, rope, m, persistent=pers)
            g, _ = capture(step)
            ms = time_graph(g, steps, 3)
            gbs = nbytes / (ms * 1e-3) / 1e9
            chain[name] = {"us_per_sweep": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                           "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "single_launch_per_layer": single}
            del g
        out[f"decode_chain_m{m}"] = chain
    for m in (128, 2048):
        x, xo = act(m, HIDDEN), act(m, HIDDEN)
        gate_inputs[m] = (x, xo)
        step, _, nflops, _ = fused_sweep(layers, x, xo, m)
        g, _ = capture(step)
        ms = time_graph(g, max(5, steps // 4), 2)
        tf = nflops / (ms * 1e-3) / 1e12
        out[f"prefill_sweep_m{m}"] = {"ms_per_sweep": round(ms, 4), "TFLOP/s": round(tf, 1),
                                      "frac_of_mfma_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}
        del g
    for m in (1, 512):
        x = act(m, HIDDEN)
        gate_inputs[("mlp", m)] = x
        g, _ = capture(lambda: [Q.mlp(x, L["gate"], L["up"], L["down"]) for L in layers])
        ms = time_graph(g, max(5, steps // 4), 2)
        per = ms * 1e3 / len(layers)
        nbytes = 3 * INTER * HIDDEN + 8 * INTER + 4 * HIDDEN + 2 * m * HIDDEN + 4 * m * INTER + 2 * m * HIDDEN
        nflops = 6 * m * INTER * HIDDEN
        out[f"swiglu_mlp_m{m}"] = {"us_per_layer": round(per, 2), "GB/s": round(nbytes / (per * 1e-6) / 1e9, 1),
                                   "TFLOP/s": round(nflops / (per * 1e-6) / 1e12, 1)}
        del g
    vocab = 151936
    heads = []
    for c in range(2):
        hg = torch.Generator(device=dev).manual_seed(9000 + c)
        w = torch.randn((vocab, HIDDEN), generator=hg, device=dev) * 0.02
        heads.append(Q.QuantizedWeight(w))
        del w
    torch.cuda.empty_cache()
    gate_x, gate_logits = {}, {}
    for m in (1, 8, 256):
        x = act(m, HIDDEN)
        gate_x[m] = x.float().cpu().numpy()
        gate_logits[m] = heads[0].linear(x, out_dtype=torch.float32).cpu().numpy()
        g, _ = capture(lambda: [hw.linear(x, out_dtype=torch.float32) for hw in heads * 4])
        ms = time_graph(g, max(5, steps // 10), 2)
        per = ms * 1e3 / 8
        nbytes = vocab * HIDDEN + 4 * vocab + 2 * m * HIDDEN + 4 * m * vocab
        out[f"lm_head_m{m}"] = {"us_per_launch": round(per, 2), "GB/s": round(nbytes / (per * 1e-6) / 1e9, 1),
                                "TFLOP/s": round(2 * m * vocab * HIDDEN / (per * 1e-6) / 1e12, 1)}
        del g
    # the greedy next token (server.py:51): logits + torch.argmax against the
    # argmax reduced inside the projection (no logits written)
    for m in (1, 8):
        x = act(m, HIDDEN)
        g, _ = capture(lambda: [hw.linear(x, out_dtype=torch.float32).argmax(dim=-1) for hw in heads * 4])
        sep = time_graph(g, max(5, steps // 10), 2) * 1e3 / 8
        del g
        g, _ = capture(lambda: [Q.linear_argmax(x, hw) for hw in heads * 4])
        fused = time_graph(g, max(5, steps // 10), 2) * 1e3 / 8
        del g
        same = bool(torch.equal(Q.linear_argmax(x, heads[0]), heads[0].linear(x, out_dtype=torch.float32).argmax(-1)))
        out[f"lm_head_argmax_m{m}"] = {"fused_us": round(fused, 2), "logits_then_torch_argmax_us": round(sep, 2),
                                       "same_indices": same}
    log("[bench] lm_head correctness gate (every row's argmax against the oracle)")
    out["lm_head_correctness"] = lm_head_gate((heads[0].q.cpu().numpy(), heads[0].scale.cpu().numpy()), gate_x,
                                              gate_logits)
    del heads, gate_logits
    torch.cuda.empty_cache()
    # the single [4864, 896] linear at M=1 (Qwen2.5-0.5B gate_proj)
    w = torch.randn((4864, 896), generator=gen, device=dev) * 0.02
    qw = Q.QuantizedWeight(w)
    x = act(1, 896)
    g, _ = capture(lambda: [qw.linear(x) for _ in range(20)])
    us = time_graph(g, 20, 3) * 1e3 / 20
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import reference_cpu_path as R

    q_cpu, s_cpu, x_cpu = qw.q.cpu(), qw.scale.cpu(), x.cpu()
    torch.set_num_threads(R.cpu_threads())
    R.per_call_linear(x_cpu, q_cpu, s_cpu)
    t0 = time.perf_counter()
    for _ in range(20):
        R.per_call_linear(x_cpu, q_cpu, s_cpu)
    cpu_us = (time.perf_counter() - t0) / 20 * 1e6
    nbytes = linear_bytes(1, 4864, 896)
    out["single_linear_4864x896_m1"] = {"gpu_us": round(us, 2), "gpu_GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                                        "cpu_reference_path_us": round(cpu_us, 1), "cpu_threads": R.cpu_threads()}
    return out


def cpu_baseline(layers, m, budget_s):
    """The reference's per-call path on this host's CPU cores over a sample
    of layers: 3 warm-ups, the median of 10 timed passes."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import reference_cpu_path as R

    def get_layer(i):
        L = layers[i]
        h = {name: (L[name].q.cpu(), L[name].scale.cpu()) for name in SHAPES}
        for b in ("q_b", "k_b", "v_b"):
            h[b] = L[b].cpu()
        return h

    r = R.time_layers(get_layer, len(layers), m, budget_s=budget_s)
    info = R.cpu_model()
    return r, info


def _sha(a) -> str:
    import hashlib

    return hashlib.sha256(a.tobytes()).hexdigest()[:16]


def span_gate(dev, layers, l, ref_q, norms, rope, x, attn, O, np32):
    """Layer l's single-launch decode span (o + residual, norm, gate|up,
    down + residual, the next layer's norm + q|k|v + bias, RoPE) against the
    oracle, each stage on its own GPU input (the launch's exchanged
    intermediates); the fused RoPE bit for bit against the oracle's RoPE of
    the same launch's un-rotated q and k."""
    import numpy as np

    from pageserve_amd import span as S

    L = layers[l]
    m = x.shape[0]
    N = layers[l + 1] if l + 1 < len(layers) else None
    kw = {}
    nq = {}
    if N is not None:
        for j, name in enumerate(("q", "k", "v")):
            n, k = SHAPES[name]
            nq[name] = O.quantize_per_channel(layer_weight(dev, l + 1, j, n, k).cpu().numpy())
        kw = dict(next_ln=norms[l + 1][0], next_qkv=(N["q"], N["k"], N["v"]), next_bias=(N["q_b"], N["k_b"], N["v_b"]))
    x_out, qkv = S.decode_span(attn, x, L["o"], norms[l][1], L["gate"], L["up"], L["down"], 1e-6, **kw)
    torch.cuda.synchronize()
    x1, act, tags = S.exchange_values(m, HIDDEN, INTER)
    x1, act = x1.numpy(), act.numpy()
    xn, an, xo_ = np32(x), np32(attn), np32(x_out)
    ln2, ln1 = np32(norms[l][1]), np32(norms[l + 1][0]) if N is not None else None
    res = []

    def check(name, y, ref, k, **bound):
        r = O.compare(y, ref, k, bf16_out=True, **bound)
        res.append({"layer": l, "m": m, "launch": f"span {name}", "ok": r["ok"], "rel": round(r["rel"], 6),
                    "worst_vs_bound": round(r["worst_vs_bound"], 4), "rows": m})

    check("o + residual", x1, O.linear_residual(an, *ref_q["o"], xn), HIDDEN,
          ulp_of=O.linear_residual_intermediate(an, *ref_q["o"]))
    h2, dh2 = O.rmsnorm(x1, ln2, 1e-6), O.rmsnorm_dx(x1, ln2, 1e-6)
    check("gate|up", act, O.swiglu(h2, *ref_q["gate"], *ref_q["up"]), HIDDEN,
          acc=O.swiglu_acc(h2, *ref_q["gate"], *ref_q["up"], dx=dh2))
    check("down + residual", xo_, O.linear_residual(act, *ref_q["down"], x1), INTER,
          ulp_of=O.linear_residual_intermediate(act, *ref_q["down"]))
    ok_tags = len(tags) == 1 and 0 not in tags
    if N is not None:
        h1, dh1 = O.rmsnorm(xo_, ln1, 1e-6), O.rmsnorm_dx(xo_, ln1, 1e-6)
        for y, name in zip(qkv, ("q", "k", "v")):
            b = np32(N[name + "_b"])
            check(name, np32(y), O.linear(h1, *nq[name], b), HIDDEN, acc=O.acc_bound(h1, *nq[name], b, dx=dh1))
        _, rot = S.decode_span(attn, x, L["o"], norms[l][1], L["gate"], L["up"], L["down"], 1e-6, cos=rope[0],
                               sin=rope[1], **kw)
        cs, sn = np32(rope[0]), np32(rope[1])
        rope_ok = all(np.array_equal(np32(r_).reshape(m, -1), O.rope(np32(u_).reshape(m, -1, 128), cs, sn).reshape(m, -1))
                      for r_, u_ in zip(rot[:2], qkv[:2])) and bool(torch.equal(rot[2], qkv[2]))
        res.append({"layer": l, "m": m, "launch": "span RoPE (bit-exact)", "ok": bool(rope_ok), "rows": m})
    res.append({"layer": l, "m": m, "launch": "span exchange tags", "ok": ok_tags, "rows": m})
    return res


def correctness_gate(dev, layers, inputs, check_layers):
    """After the timed runs: the same launches as the timed sweeps, on the
    same weights and inputs, against the oracle (oracle/quantization_oracle.py
    on this host's CPU).  Per checked layer: every q and scale bit for bit
    against the oracle quantizer run on the regenerated fp32 weights (their
    sha256 prefixes recorded), and at each token count every launch kind of
    the sweep -- q|k|v with bias, o, the fused gate|up, down on the kernel's
    own gate|up output -- within the specification's tolerance (all rows at
    up to 16 tokens, 16 sampled rows above); for ``("mlp", m)`` keys the
    fused MLP (gate|up then down) against the oracle's fp32 MLP."""
    import numpy as np

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import quantization_oracle as O
    from pageserve_amd import quantization as Q

    def np32(t):
        return t.detach().float().cpu().numpy()

    out = {"ok": True, "quantizer": [], "linears": []}
    inputs = dict(inputs)
    span = inputs.pop("span", None)
    for l in check_layers:
        L = layers[l]
        ref_q = {}
        for j, (name, (n, k)) in enumerate(SHAPES.items()):
            qr, sr = O.quantize_per_channel(layer_weight(dev, l, j, n, k).cpu().numpy())
            qg, sg = L[name].q.cpu().numpy(), L[name].scale.cpu().numpy()
            ok = bool(np.array_equal(qg, qr) and np.array_equal(sg.view(np.uint32), sr.view(np.uint32)))
            out["quantizer"].append({"layer": l, "weight": name, "bit_exact": ok, "q_sha256": _sha(qg),
                                     "scale_sha256": _sha(sg)})
            out["ok"] &= ok
            ref_q[name] = (qr, sr)
        for m, xs in inputs.items():
            if isinstance(m, tuple):  # ("mlp", tokens): Q.mlp as other_configs times it
                x = xs
                rows = np.arange(m[1]) if m[1] <= 16 else np.linspace(0, m[1] - 1, 16).astype(int)
                xn = np32(x)[rows]
                w3 = (*ref_q["gate"], *ref_q["up"], *ref_q["down"])
                y = Q.mlp(x, L["gate"], L["up"], L["down"])
                r = O.compare(np32(y)[rows], O.mlp(xn, *w3), INTER, bf16_out=True, acc=O.mlp_acc(xn, *w3))
                out["linears"].append({"layer": l, "m": m[1], "launch": "mlp", "ok": r["ok"], "rel": round(r["rel"], 6),
                                       "worst_vs_bound": round(r["worst_vs_bound"], 4), "rows": len(rows)})
                out["ok"] &= r["ok"]
                continue
            x, xo = xs
            rows = np.arange(m) if m <= 16 else np.linspace(0, m - 1, 16).astype(int)
            xn, xon = np32(x)[rows], np32(xo)[rows]
            outs = Q.linear_group(x, [L["q"], L["k"], L["v"]], [L["q_b"], L["k_b"], L["v_b"]])
            act = Q.swiglu(x, L["gate"], L["up"])
            got = {"q": outs[0], "k": outs[1], "v": outs[2], "o": L["o"].linear(xo), "gate|up": act,
                   "down": L["down"].linear(act)}
            actn = np32(act)[rows]
            for name, y in got.items():
                if name in ("q", "k", "v"):
                    b = np32(L[name + "_b"])
                    ref, acc, k = O.linear(xn, *ref_q[name], b), O.acc_bound(xn, *ref_q[name], b), HIDDEN
                elif name == "o":
                    ref, acc, k = O.linear(xon, *ref_q["o"]), O.acc_bound(xon, *ref_q["o"]), HIDDEN
                elif name == "gate|up":
                    qg_, qu_ = ref_q["gate"], ref_q["up"]
                    ref, acc, k = O.swiglu(xn, *qg_, *qu_), O.swiglu_acc(xn, *qg_, *qu_), HIDDEN
                else:
                    ref, acc, k = O.linear(actn, *ref_q["down"]), O.acc_bound(actn, *ref_q["down"]), INTER
                r = O.compare(np32(y)[rows], ref, k, bf16_out=True, acc=acc)
                out["linears"].append({"layer": l, "m": m, "launch": name, "ok": r["ok"], "rel": round(r["rel"], 6),
                                       "worst_vs_bound": round(r["worst_vs_bound"], 4), "rows": len(rows)})
                out["ok"] &= r["ok"]
        if span is not None:
            from pageserve_amd import span as S

            norms, rope, sx, sattn = span
            if S.span_supported(sx.shape[0], HIDDEN, INTER, HIDDEN, KV, 128):
                for r in span_gate(dev, layers, l, ref_q, norms, rope, sx, sattn, O, np32):
                    out["linears"].append(r)
                    out["ok"] &= r["ok"]
    return out


def lm_head_gate(heads_q, x_by_m, logits_by_m):
    """int8 lm_head: fp32 logits of every row within the tolerance and the
    argmax of every row equal to the oracle's (blocked float64 oracle)."""
    import numpy as np

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import quantization_oracle as O

    q, s = heads_q
    res = {"ok": True}
    for m, x in x_by_m.items():
        ref = np.concatenate([O.linear(x, q[i:i + 16384], s[i:i + 16384]) for i in range(0, q.shape[0], 16384)], axis=1)
        got = logits_by_m[m]
        r = O.compare(got, ref, HIDDEN)
        am = bool(np.array_equal(O.argmax_rows(got), O.argmax_rows(ref)))
        res[f"m{m}"] = {"rows": m, "argmax_equal_every_row": am, "rel": r["rel"], "ok": r["ok"] and am,
                        "min_top2_gap": float(O.top2_gap(ref).min())}
        res["ok"] &= r["ok"] and am
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--m", type=int, default=1, help="tokens per decode step")
    ap.add_argument("--prefill-m", type=int, default=512)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU work for the baseline")
    ap.add_argument("--cpu-prefill-budget", type=float, default=8.0,
                    help="seconds of CPU work for the prefill baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-gate", action="store_true", help="skip the correctness gate (profiling runs)")
    ap.add_argument("--only", choices=["all", "decode", "prefill", "configs"], default="all")
    ap.add_argument("--no-configs", action="store_true", help="skip the other workload sizes")
    ap.add_argument("--no-torch-ref", action="store_true",
                    help="skip the torch comparison sweeps (reference dequantize + F.linear, dense bf16)")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="run only the dispatches the rocprofv3 --pmc traffic passes read")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="reduce rocprofv3 --pmc output directories to the traffic summary (no GPU)")
    ap.add_argument("--span-timeline", metavar="OUT",
                    help="write the single-launch decode chain's stage timeline (markdown) to OUT and exit")
    ap.add_argument("--prefill-workload", type=int, metavar="M",
                    help="run only the prefill sweep's launches once per layer at M tokens (counter passes)")
    ap.add_argument("--plan-file", default="prefill_plans.json",
                    help="where --prefill-workload records each launch kind's kernel instance")
    ap.add_argument("--mfma-summary", nargs=2, metavar=("PMC_DIR", "PLAN_FILE"),
                    help="reduce a rocprofv3 --pmc pass over --prefill-workload to an MFMA table (no GPU)")
    ap.add_argument("--counter-summary", nargs=2, metavar=("PMC_DIR", "PLAN_FILE"),
                    help="tabulate every counter of a --prefill-workload counter pass per launch kind (no GPU)")
    ap.add_argument("--summary-out", help="file --mfma-summary / --counter-summary writes (stdout too)")
    ap.add_argument("--pmc-command", action="append", default=[],
                    help="command line recorded in the traffic summary (repeatable)")
    args = ap.parse_args()

    if args.counter_summary:
        text = counter_summary(args.counter_summary[0], args.counter_summary[1], " ".join(args.pmc_command))
        if args.summary_out:
            with open(args.summary_out, "w") as f:
                f.write(text)
        print(text, end="")
        return
    if args.mfma_summary:
        text = mfma_summary(args.mfma_summary[0], args.mfma_summary[1], " ".join(args.pmc_command))
        if args.summary_out:
            with open(args.summary_out, "w") as f:
                f.write(text)
        print(text, end="")
        return

    if args.pmc_summary:
        text = pmc_summary(args.pmc_summary, args.pmc_command)
        os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
        with open(TRAFFIC_FILE, "w") as f:
            f.write(text)
        print(text, end="")
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this path is measured on one GPU only; --gpus must be 1 "
              "(multi-GPU sharding is described, not run)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)

    from pageserve_amd import _native
    from pageserve_amd import quantization as Q

    _native.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.pmc_workload:
        with torch.inference_mode():
            pmc_workload(dev, args.layers)
        return
    if args.span_timeline:
        os.makedirs(os.path.dirname(os.path.abspath(args.span_timeline)), exist_ok=True)
        with torch.inference_mode():
            md = span_timeline(dev, args.layers, args.m, "python3 bench.py " + " ".join(sys.argv[1:]))
        with open(args.span_timeline, "w") as f:
            f.write(md)
        log(f"[bench] span timeline written to {args.span_timeline}")
        return
    if args.prefill_workload:
        os.makedirs(os.path.dirname(os.path.abspath(args.plan_file)), exist_ok=True)
        with torch.inference_mode():
            prefill_workload(dev, args.layers, args.prefill_workload, args.plan_file)
        return
    log(f"[bench] device {torch.cuda.get_device_name(dev)}; building {args.layers} layers of int8 weights")
    layers = make_layers(dev, args.layers)
    gen = torch.Generator(device=dev).manual_seed(99 + args.m)

    result = {}
    gate_inputs = {}
    with torch.inference_mode():
        # ---------------- decode, M = m ----------------
        m = args.m
        x = torch.randn((m, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
        xo = torch.randn((m, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
        xi = torch.randn((m, INTER), generator=gen, device=dev).to(torch.bfloat16)
        if args.only in ("all", "decode"):
            gate_inputs[m] = (x, xo)
            norms, rope = chain_operands(dev, len(layers), m)
            gate_inputs["span"] = (norms, rope, x, xo)
            # the headline: the dependent decode chain
            step, nbytes, launches, single = decode_chain(layers, x, xo, norms, rope, m)
            eager_out = step()
            g, graph_out = capture(step)
            g.replay()
            torch.cuda.synchronize()
            for a_, b_ in zip(eager_out, graph_out):
                assert torch.equal(a_, b_), "graph replay differs from eager"
            log("[bench] decode chain captured; timing")
            ms = time_graph(g, args.steps, args.warmup)
            ms_eager = time_eager(step, max(5, args.steps // 10), 3)
            value = nbytes / (ms * 1e-3) / 1e9
            log(f"[bench] decode m={m} (dependent chain, {'one launch per layer' if single else 'per-projection kernels'}): "
                f"{ms * 1e3:.1f} us/sweep, {value:.1f} GB/s ({100 * value / HBM_PEAK_GBS:.1f}% of HBM peak); "
                f"eager {ms_eager * 1e3:.1f} us")
            del g
            # the same chain with the per-projection kernels, and with the
            # reference's torch op chains for the neighbours
            chain = {}
            for mode in ("reference", "kernels", "norm_in_linear"):
                cg, _ = capture(layer_chain(layers, x, xo, norms, rope, mode))
                chain[mode] = time_graph(cg, max(20, args.steps // 4), 5) * 1e3 / len(layers)
                del cg
            chain_eager = time_eager(layer_chain(layers, x, xo, norms, rope, "norm_in_linear"),
                                     max(5, args.steps // 10), 3) * 1e3 / len(layers)
            log(f"[bench] decode chain per-projection kernels (us/layer): norm in the linear {chain['norm_in_linear']:.2f}"
                f" (eager {chain_eager:.2f}), separate kernels {chain['kernels']:.2f}, reference structure "
                f"{chain['reference']:.2f}")
            # the independent four-launch sweep (every launch on fixed inputs)
            istep, ibytes, _, ilaunches = fused_sweep(layers, x, xo, m)
            ig, _ = capture(istep)
            ims = time_graph(ig, args.steps, args.warmup)
            ims_eager = time_eager(istep, max(5, args.steps // 10), 3)
            ival = ibytes / (ims * 1e-3) / 1e9
            log(f"[bench] independent sweep (4 launches/layer, fixed inputs): {ims * 1e3:.1f} us, {ival:.1f} GB/s; "
                f"eager {ims_eager * 1e3:.1f} us")
            del ig
            pstep, pbytes, _, plaunch = per_call_sweep(layers, x, xo, xi, m)
            pg, _ = capture(pstep)
            pms = time_graph(pg, args.steps, args.warmup)
            pval = pbytes / (pms * 1e-3) / 1e9
            pms_eager = time_eager(pstep, max(5, args.steps // 10), 3)
            dstep = dropin_sweep(layers, x, xo, xi)
            dms_eager = time_eager(dstep, max(5, args.steps // 10), 3)
            log(f"[bench] per-call sweep (7 launches/layer): {pms * 1e3:.1f} us graph, {pms_eager * 1e3:.1f} us eager; "
                f"through F.linear(x, W.get(), b) eagerly: {dms_eager * 1e3:.1f} us")
            del pg
            ref_ms = dense_ms = None
            if not args.no_torch_ref:
                ref_ms, dense_ms = torch_reference_sweeps(layers, x, xo, max(10, args.steps // 10))
                log(f"[bench] reference computation with torch on this GPU: dequantize + F.linear "
                    f"{ref_ms * 1e3:.1f} us, dense bf16 F.linear {dense_ms * 1e3:.1f} us per sweep")
            # dominant kernel of the headline: the single launch per layer
            if single:
                from pageserve_amd import span as S

                nxt = {id(L): layers[(i + 1) % len(layers)] for i, L in enumerate(layers)}

                def span_launch(L):
                    N = nxt[id(L)]
                    return S.decode_span(xo, x, L["o"], norms[0][1], L["gate"], L["up"], L["down"], 1e-6,
                                         next_ln=norms[0][0], next_qkv=(N["q"], N["k"], N["v"]),
                                         next_bias=(N["q_b"], N["k_b"], N["v_b"]), cos=rope[0], sin=rope[1])

                roof = kernel_roofline(layers, span_launch, layer_bytes(m),
                                       2 * m * HIDDEN * (2 * HIDDEN + 3 * INTER + 2 * KV), "hbm")
                roof["kernel"] = ("span_kernel (o + residual, RMSNorm, gate|up SwiGLU, down + residual, RMSNorm, "
                                  "next layer's q|k|v + bias + RoPE: one launch per layer)")
                roof["traffic"] = read_traffic("span_m1") if m == 1 else None
            swiglu_b = 2 * INTER * HIDDEN + 8 * INTER + 2 * m * HIDDEN + 2 * m * INTER
            gu_roof = kernel_roofline(layers, lambda L: Q.swiglu(x, L["gate"], L["up"]), swiglu_b,
                                      4 * m * INTER * HIDDEN, "hbm")
            gu_roof["kernel"] = "skinny_kernel<NMAT=2> (fused gate|up, 2x[11008,2048] int8)"
            gu_roof["traffic"] = read_traffic("skinny_gate_up_m1") if m == 1 else None
            if not single:
                roof = gu_roof
            log(f"[bench] dominant kernel: {roof['launch_us']} us/launch, {roof['achieved']} GB/s")
            down_roof = kernel_roofline(layers, lambda L: L["down"].linear(xi), linear_bytes(m, HIDDEN, INTER),
                                        2 * m * HIDDEN * INTER, "hbm")
            result.update({
                "value": round(value, 2), "ms_per_step": round(ms, 5), "roofline": roof,
                "decode_detail": {"what": ("dependent decode chain: layer 0's norm + q|k|v + RoPE, then per layer "
                                           "o + residual, norm, gate|up, down + residual, the next layer's norm + "
                                           "q|k|v + bias + RoPE (attention output fixed); HIP-graph replay"),
                                  "single_launch_per_layer": single,
                                  "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
                                  "bytes_per_step": nbytes, "launches_per_step": launches,
                                  "eager_ms_per_step": round(ms_eager, 5),
                                  "eager_gbs": round(nbytes / (ms_eager * 1e-3) / 1e9, 2),
                                  "per_projection_chain": {
                                      "what": "the same chain with per-projection kernels (norm inside q|k|v and "
                                              "gate|up, RoPE kernel, residual epilogues), 5 launches per layer",
                                      "us_per_layer": round(chain["norm_in_linear"], 3),
                                      "eager_us_per_layer": round(chain_eager, 3),
                                      "separate_norm_kernel_us_per_layer": round(chain["kernels"], 3),
                                      "reference_structure_us_per_layer": round(chain["reference"], 3)},
                                  "independent_sweep": {
                                      "what": "q|k|v, o, gate|up, down per layer on fixed inputs (no norms, no "
                                              "RoPE), 4 launches per layer",
                                      "ms_per_step": round(ims, 5), "gbs": round(ival, 2),
                                      "frac_of_hbm_peak": round(ival / HBM_PEAK_GBS, 4),
                                      "bytes_per_step": ibytes, "launches_per_step": ilaunches,
                                      "eager_ms_per_step": round(ims_eager, 5)},
                                  "gate_up_roofline": gu_roof,
                                  "down_proj_roofline": down_roof},
                "per_call_sweep": {"ms_per_step": round(pms, 5), "gbs": round(pval, 2),
                                   "frac_of_hbm_peak": round(pval / HBM_PEAK_GBS, 4),
                                   "bytes_per_step": pbytes, "launches_per_step": plaunch,
                                   "eager_ms_per_step": round(pms_eager, 5),
                                   "dropin_f_linear_eager_ms_per_step": round(dms_eager, 5),
                                   "dropin_what": "engine/model.py's own calls, F.linear(h, W.get(), b) on bf16-model "
                                                  "QuantizedWeights and F.silu(gate) * up in torch, launched eagerly"},
            })
            if ref_ms is not None:
                result["torch_gpu"] = torch_gpu_entry(ref_ms, dense_ms, ms, nbytes, "GB/s")

        # ---------------- prefill, M = prefill_m ----------------
        if args.only in ("all", "prefill") and args.prefill_m > 0:
            pm = args.prefill_m
            px = torch.randn((pm, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
            pxo = torch.randn((pm, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
            gate_inputs[pm] = (px, pxo)
            step, nbytes, nflops, launches = fused_sweep(layers, px, pxo, pm)
            g, _ = capture(step)
            psteps = max(10, args.steps // 4)
            ms = time_graph(g, psteps, max(3, args.warmup // 4))
            tflops = nflops / (ms * 1e-3) / 1e12
            log(f"[bench] prefill m={pm}: {ms:.3f} ms/sweep, {tflops:.1f} TFLOP/s "
                f"({100 * tflops / MFMA_BF16_PEAK_TFLOPS:.1f}% of bf16 MFMA peak)")
            del g
            pref_ms = pdense_ms = None
            if not args.no_torch_ref:
                pref_ms, pdense_ms = torch_reference_sweeps(layers, px, pxo, 10)
                log(f"[bench] prefill, reference computation with torch on this GPU: dequantize + F.linear "
                    f"{pref_ms:.3f} ms, dense bf16 F.linear {pdense_ms:.3f} ms per sweep")
            proof = kernel_roofline(layers, lambda L: Q.swiglu(px, L["gate"], L["up"]),
                                    2 * INTER * HIDDEN + 8 * INTER + 2 * pm * HIDDEN + 2 * pm * INTER,
                                    4 * pm * INTER * HIDDEN, "mfma", reps=5)
            proof["kernel"] = "gemm_dma_kernel<BM=128,BN=64,NMAT=2> (fused gate|up, 2x[11008,2048] int8, 512 tokens)"
            proof["traffic"] = read_traffic("gemm_gate_up_m512") if pm == 512 else None
            result["prefill"] = {"m": pm, "value": round(tflops, 2), "unit": "TFLOP/s",
                                 "frac_of_mfma_peak": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                                 "ms_per_step": round(ms, 5), "flops_per_step": nflops, "steps": psteps,
                                 "roofline": proof}
            if pref_ms is not None:
                result["prefill"]["torch_gpu"] = torch_gpu_entry(pref_ms, pdense_ms, ms, nflops, "TFLOP/s")

        # ---------------- the other workload sizes ----------------
        if args.only in ("all", "configs") and not args.no_configs:
            oc = other_configs(layers, dev, args.steps, gate_inputs)
            for key, v in oc.items():
                log(f"[bench] {key}: {v}")
            result["other_configs"] = oc

        # ---------------- correctness gate (after all timing) ----------------
        if gate_inputs and not args.no_gate:
            log("[bench] correctness gate: quantizer bits and every launch kind of the sweeps against the oracle")
            t0 = time.perf_counter()
            gate = correctness_gate(dev, layers, gate_inputs, sorted({0, len(layers) - 1}))
            gate["seconds"] = round(time.perf_counter() - t0, 1)
            result["correctness"] = gate
            log(f"[bench] correctness gate: ok={gate['ok']} ({gate['seconds']} s)")

        # ---------------- CPU baseline ----------------
        if not args.no_cpu_baseline and args.only in ("all", "decode"):
            r, info = cpu_baseline(layers, args.m, args.cpu_budget)
            gbs = r["bytes"] / r["seconds"] / 1e9
            log(f"[bench] CPU baseline: {r['layers']} layers per pass, median {r['seconds']:.3f} s on "
                f"{r['threads']} threads ({info['model']}): {gbs:.3f} GB/s")
            result["cpu_baseline"] = {
                "value": round(gbs, 4), "unit": "GB/s", "cores": r["threads"], "kind": "port",
                "sample": (f"layers 0..{r['layers'] - 1} of the {args.layers}-layer M={args.m} sweep, 7 per-call "
                           f"linears each: (q.float()*scale).to(bf16) then F.linear, torch CPU; {r['warmup']} "
                           f"warm-up passes, median of {len(r['runs'])} timed passes ({r['seconds']:.3f} s each)"),
                "cpu": info["model"], "amx_bf16": info["amx_bf16"], "avx512f": info["avx512f"],
                "runs_s": [round(v, 4) for v in r["runs"]],
            }
            if args.prefill_m > 0 and args.only == "all":
                pr, _ = cpu_baseline(layers, args.prefill_m, args.cpu_prefill_budget)
                tf = pr["flops"] / pr["seconds"] / 1e12
                log(f"[bench] CPU baseline, prefill M={args.prefill_m}: {pr['layers']} layer per pass, median "
                    f"{pr['seconds']:.3f} s: {tf:.3f} TFLOP/s")
                result["cpu_baseline"]["prefill"] = {
                    "value": round(tf, 4), "unit": "TFLOP/s", "cores": pr["threads"], "kind": "port",
                    "ms_per_step_scaled": round(pr["seconds"] * 1e3 * args.layers / pr["layers"], 1),
                    "sample": (f"layers 0..{pr['layers'] - 1} at M={args.prefill_m}, the same 7 per-call linears; "
                               f"{pr['warmup']} warm-ups, median of {len(pr['runs'])} passes "
                               f"({pr['seconds']:.3f} s each); ms_per_step_scaled = that median x "
                               f"{args.layers}/{pr['layers']} layers"),
                    "runs_s": [round(v, 4) for v in pr["runs"]],
                }

    line = {
        "metric": "W8A16 linear GB/s (% HBM peak) at M=1; TFLOPS (% MFMA peak) at M=512",
        "value": result.get("value"), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": result.get("ms_per_step"), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"Qwen2.5-3B decode linears as a dependent chain: {args.layers} layers x (o + "
                               f"residual, RMSNorm, gate|up SwiGLU, down + residual, the next layer's RMSNorm + "
                               f"q|k|v with bias + RoPE; attention output fixed), M={args.m}, int8 per-row weights "
                               f"from N(0,0.02), HIP-graph replay; bytes = the linears' int8 W + fp32 scale + bf16 "
                               f"x/y",
                   "m": args.m, "layers": args.layers, "hidden": HIDDEN, "intermediate": INTER, "kv_dim": KV,
                   "weight_dtype": "int8", "activation_dtype": "bf16", "accumulate": "fp32",
                   "parallelism": "none (1 GPU)"},
    }
    for key in ("roofline", "cpu_baseline", "correctness", "prefill", "per_call_sweep", "torch_gpu", "decode_detail",
                "other_configs"):
        if key in result:
            line[key] = result[key]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
