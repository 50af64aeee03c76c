"""The decode step between two attention calls as one persistent launch
(pgs_w8a16_decode_span) against the oracle, stage by stage.

engine/model.py:184-190 of layer l, then :165-173 of layer l + 1, at the
Qwen2.5-3B shapes (hidden 2048, intermediate 11008, 16 q heads and 2 kv heads
of 128).  Every stage is checked on the GPU's own input to it (the
intermediates are read back from the launch's exchange buffers), so errors do
not compound: o_proj + residual, the SwiGLU pair on rms_norm of that, down +
residual, then q|k|v (+ bias) of rms_norm of the new residual stream, within
the specification's tolerance; the fused RoPE bit for bit against the RoPE
of the same launch's un-rotated q and k.  Also: graph replays and repeated
calls equal the first eager call bit for bit (the epoch tag changes every
launch), the bounded wait's give-up path (forced from the host) reports
PGS_ERR_TIMEOUT and leaves the workspace reusable, and sizes without a
compiled configuration run the per-projection kernels.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quantization_oracle as O
from pageserve_amd import _native
from pageserve_amd import quantization as Q
from pageserve_amd import span as S

from helpers import activations, bf16_gpu, report, to_np, weights

pytestmark = pytest.mark.gpu

H, I, KV, HD = 2048, 11008, 256, 128
EPS = 1e-6


@pytest.fixture(scope="module")
def layer(gpu):
    """One layer's post-attention weights and the next layer's q/k/v, with
    their oracle quantizations."""
    def qw(seed, n, k):
        w = weights(seed, n, k)
        return Q.QuantizedWeight(torch.from_numpy(w).to(gpu)), O.quantize_per_channel(w)

    L = {"o": qw(301, H, H), "gate": qw(302, I, H), "up": qw(303, I, H), "down": qw(304, H, I),
         "q": qw(305, H, H), "k": qw(306, KV, H), "v": qw(307, KV, H)}
    rng = np.random.default_rng(308)
    ln2 = O.round_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    ln1 = O.round_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    bias = [O.round_to_bf16(rng.standard_normal(n).astype(np.float32)) for n in (H, KV, KV)]
    L["ln2"], L["ln1"], L["bias"] = ln2, ln1, bias
    L["ln2_t"], L["ln1_t"] = bf16_gpu(ln2, gpu), bf16_gpu(ln1, gpu)
    L["bias_t"] = tuple(bf16_gpu(b, gpu) for b in bias)
    return L


def rope_tables(m, start=7):
    pos = np.arange(start, start + m, dtype=np.float64)
    inv = 1.0 / (1e6 ** (np.arange(0, HD, 2) / HD))
    emb = np.concatenate([np.outer(pos, inv)] * 2, axis=-1)
    return O.round_to_bf16(np.cos(emb).astype(np.float32)), O.round_to_bf16(np.sin(emb).astype(np.float32))


def run_span(L, attn_t, x_t, cos_t=None, sin_t=None, last=False, persistent=None):
    nxt = {} if last else dict(next_ln=L["ln1_t"], next_qkv=(L["q"][0], L["k"][0], L["v"][0]),
                               next_bias=L["bias_t"], cos=cos_t, sin=sin_t)
    return S.decode_span(attn_t, x_t, L["o"][0], L["ln2_t"], L["gate"][0], L["up"][0], L["down"][0], EPS,
                         persistent=persistent, **nxt)


def exchange(gpu, m):
    """(x1, act) as the launch left them in its exchange buffers (bf16 values
    in the low half of each tagged word; 8 rows x m tokens per 128-byte
    slot), and the set of tags seen."""
    ws = S._eager[(gpu.index, Q._raw_stream(gpu))]
    words = ws.view(torch.int32).cpu().numpy().view(np.uint32)
    hdr = 256 // 4

    def unpack(base, units):
        w = words[base: base + units * 32].reshape(units, 32)[:, : 8 * m].reshape(units, m, 8)
        vals = O.bf16_bits_to_f32((w & 0xFFFF).astype(np.uint16))
        return vals.transpose(1, 0, 2).reshape(m, units * 8), set(np.unique(w >> 16).tolist())

    x1, t1 = unpack(hdr, H // 8)
    act, t2 = unpack(hdr + (H // 8) * 32, I // 8)
    return x1, act, t1 | t2


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_span_stages_match_oracle(gpu, layer, m):
    L = layer
    assert S.span_supported(m, H, I, H, KV, HD)
    assert S.span_default(m, H, I, H, KV, HD) == (m <= 2)
    x, attn = activations(310 + m, m, H), activations(320 + m, m, H)
    xt, at = bf16_gpu(x, gpu), bf16_gpu(attn, gpu)
    x_out, (q, k, v) = run_span(L, at, xt, persistent=True)
    torch.cuda.synchronize()
    S.decode_span_status(gpu)
    assert "launch_span" in _native.last_plan()
    x1, act, tags = exchange(gpu, m)
    assert len(tags) == 1 and 0 not in tags, f"exchange words from more than one launch: {tags}"
    oo, og, ou, od = L["o"][1], L["gate"][1], L["up"][1], L["down"][1]
    report(x1, O.linear_residual(attn, *oo, x), H, f"m={m} o + residual",
           ulp_of=O.linear_residual_intermediate(attn, *oo))
    h2, dh2 = O.rmsnorm(x1, L["ln2"], EPS), O.rmsnorm_dx(x1, L["ln2"], EPS)
    report(act, O.swiglu(h2, *og, *ou), H, f"m={m} gate|up", acc=O.swiglu_acc(h2, *og, *ou, dx=dh2))
    xo = to_np(x_out)
    report(xo, O.linear_residual(act, *od, x1), I, f"m={m} down + residual",
           ulp_of=O.linear_residual_intermediate(act, *od))
    h1, dh1 = O.rmsnorm(xo, L["ln1"], EPS), O.rmsnorm_dx(xo, L["ln1"], EPS)
    for y, nm, b in ((q, "q", L["bias"][0]), (k, "k", L["bias"][1]), (v, "v", L["bias"][2])):
        qq, ss = L[nm][1]
        report(to_np(y), O.linear(h1, qq, ss, b), H, f"m={m} {nm}", acc=O.acc_bound(h1, qq, ss, b, dx=dh1))


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_span_rope_equals_rope_of_its_projection(gpu, layer, m):
    """The RoPE in the q|k|v epilogue equals the RoPE kernel (and the oracle's
    RoPE) of the same launch's un-rotated q and k, bit for bit; v is not
    rotated."""
    x, attn = activations(330 + m, m, H), activations(340 + m, m, H)
    xt, at = bf16_gpu(x, gpu), bf16_gpu(attn, gpu)
    cos, sin = rope_tables(m)
    x0, (q0, k0, v0) = run_span(layer, at, xt, persistent=True)
    x1, (q1, k1, v1) = run_span(layer, at, xt, bf16_gpu(cos, gpu), bf16_gpu(sin, gpu), persistent=True)
    torch.cuda.synchronize()
    assert torch.equal(x0, x1) and torch.equal(v0, v1)
    for un, rot in ((q0, q1), (k0, k1)):
        ref = O.rope(to_np(un).reshape(m, -1, HD), cos, sin).reshape(m, -1)
        np.testing.assert_array_equal(to_np(rot), ref)
    qk, kk = Q.rope_qk(q0.view(m, H // HD, HD), k0.view(m, KV // HD, HD), bf16_gpu(cos, gpu), bf16_gpu(sin, gpu))
    assert torch.equal(qk.reshape(m, H), q1) and torch.equal(kk.reshape(m, KV), k1)


def test_span_last_layer_and_chain_agree(gpu, layer):
    """next = None (the last layer): the residual stream only.  The single
    launch and the per-projection kernels agree within the tolerance (their
    fp32 sums run in different orders)."""
    x, attn = activations(350, 1, H), activations(351, 1, H)
    xt, at = bf16_gpu(x, gpu), bf16_gpu(attn, gpu)
    xs, none = run_span(layer, at, xt, last=True)
    assert none is None
    xc, _ = run_span(layer, at, xt, last=True, persistent=False)
    x_full, _ = run_span(layer, at, xt)
    torch.cuda.synchronize()
    assert torch.equal(xs, x_full), "the last-layer launch computes the same residual stream"
    ref = to_np(xc)
    d = np.abs(to_np(xs) - ref)
    assert d.max() <= 4 * O.bf16_ulp(ref).max() + O.abs_tol(I), d.max()


def test_span_repeats_and_graph_replays_are_bit_equal(gpu, layer):
    """Two layers' spans chained (the second's residual is the first's
    output) in a captured graph: every replay, with eager calls and other
    work between replays, equals the eager result bit for bit; so do
    repeated eager calls (a new tag each launch)."""
    m = 1
    x, attn = activations(360, m, H), activations(361, m, H)
    xt, at = bf16_gpu(x, gpu), bf16_gpu(attn, gpu)
    cos, sin = (bf16_gpu(t, gpu) for t in rope_tables(m))

    def step():
        xa, (qa, ka, va) = run_span(layer, at, xt, cos, sin)
        xb, (qb, kb, vb) = run_span(layer, at, xa, cos, sin)
        return xa, qa, ka, va, xb, qb, kb, vb

    ref = [t.clone() for t in step()]
    torch.cuda.synchronize()
    for _ in range(4):
        again = step()
        torch.cuda.synchronize()
        for a, b in zip(ref, again):
            assert torch.equal(a, b)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        cap = step()
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(4):
        junk = torch.randn(1 << 20, device=gpu).sum()
        step()
        g.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(ref, cap)):
            assert torch.equal(a, b), f"replay {rep}, output {i}"
        del junk
    S.decode_span_status(gpu)


def test_span_trace_records_every_stage_and_changes_nothing(gpu, layer):
    """Tracing on: the outputs equal an untraced launch's bit for bit; each
    of the 256 workgroups of each launch writes its 13 marks into the slot
    of the launch's tag, non-decreasing, and the poll counts; a launch with
    the next layer's q|k|v reaches the last mark, one without stops after
    the x2 mark.  Bad buffers are refused; off again, nothing is written."""
    m = 1
    x, attn = activations(380, m, H), activations(381, m, H)
    xt, at = bf16_gpu(x, gpu), bf16_gpu(attn, gpu)
    cos, sin = (bf16_gpu(t, gpu) for t in rope_tables(m))
    ref = [t.clone() for t in (lambda r: [r[0], *r[1]])(run_span(layer, at, xt, cos, sin))]
    torch.cuda.synchronize()
    slots = 4
    buf = torch.zeros(slots * 256 * 16, dtype=torch.int64, device=gpu)
    with pytest.raises(ValueError):
        S.decode_span_trace(buf[:100])
    with pytest.raises(ValueError):
        S.decode_span_trace(buf.view(torch.float64))
    S.decode_span_trace(buf)
    try:
        got, (q, k, v) = run_span(layer, at, xt, cos, sin)
        last, _ = run_span(layer, at, xt, last=True)
        torch.cuda.synchronize()
    finally:
        S.decode_span_trace(None)
    for a, b in zip(ref, [got, q, k, v]):
        assert torch.equal(a, b)
    tr = buf.view(slots, 256, 16).cpu()
    used = [i for i in range(slots) if tr[i, :, 0].ne(0).any()]
    assert len(used) == 2 and (used[1] - used[0]) % slots in (1, slots - 1)
    first, second = (used[0], used[1]) if (used[0] + 1) % slots == used[1] else (used[1], used[0])
    full, tail = tr[first], tr[second]
    assert bool((full[:, :13] > 0).all())
    assert bool((full[:, 1:13] >= full[:, 0:12]).all())
    assert bool((full[:, 13:16] >= 1).all())  # every gather polled at least once
    assert bool((tail[:, :10] > 0).all()) and bool((tail[:, 10:13] == 0).all())
    assert bool((tail[:, 1:10] >= tail[:, 0:9]).all())
    buf.zero_()
    run_span(layer, at, xt, cos, sin)
    torch.cuda.synchronize()
    assert not bool(buf.ne(0).any())
    S.decode_span_status(gpu)


def test_span_giveup_reports_timeout_and_recovers(gpu, layer, native_lib):
    """The bounded wait's give-up path, forced from the host (every gather
    waits for a tag no workgroup writes, two polls): the launch ends, the
    status call raises DeviceWaitTimeout, a launch on the flagged workspace
    does nothing, and after the reset the next launch is correct."""
    x, attn = activations(370, 1, H), activations(371, 1, H)
    xt, at = bf16_gpu(x, gpu), bf16_gpu(attn, gpu)
    good, (gq, gk, gv) = run_span(layer, at, xt)
    torch.cuda.synchronize()
    try:
        assert native_lib.pgs_w8a16_decode_span_test_hooks(2, 1) == 0
        run_span(layer, at, xt)
        torch.cuda.synchronize()
        with pytest.raises(_native.DeviceWaitTimeout):
            S.decode_span_status(gpu, reset=False)
        assert native_lib.pgs_w8a16_decode_span_test_hooks(0, 0) == 0
        blocked, _ = run_span(layer, at, xt)  # the error word is still set: nothing runs
        torch.cuda.synchronize()
        with pytest.raises(_native.DeviceWaitTimeout):
            S.decode_span_status(gpu, reset=True)
    finally:
        native_lib.pgs_w8a16_decode_span_test_hooks(0, 0)
    S.decode_span_status(gpu)  # cleared
    again, (q, k, v) = run_span(layer, at, xt)
    torch.cuda.synchronize()
    S.decode_span_status(gpu)
    assert torch.equal(again, good) and torch.equal(q, gq) and torch.equal(k, gk) and torch.equal(v, gv)


def test_span_without_configuration_runs_the_projection_kernels(gpu, layer):
    """Five tokens have no single-launch configuration: decode_span runs the
    per-projection kernels, exactly the explicit chain."""
    m = 5
    assert not S.span_supported(m, H, I, H, KV, HD)
    x, attn = activations(380, m, H), activations(381, m, H)
    xt, at = bf16_gpu(x, gpu), bf16_gpu(attn, gpu)
    cos, sin = (bf16_gpu(t, gpu) for t in rope_tables(m))
    xs, (q, k, v) = run_span(layer, at, xt, cos, sin)
    with pytest.raises(ValueError):
        run_span(layer, at, xt, cos, sin, persistent=True)
    L = layer
    x1 = L["o"][0].linear(at, residual=xt)
    xr = Q.rmsnorm_mlp(x1, L["ln2_t"], EPS, L["gate"][0], L["up"][0], L["down"][0], residual=x1)
    qr, kr, vr = Q.rmsnorm_linear_group(xr, L["ln1_t"], EPS, [L["q"][0], L["k"][0], L["v"][0]], list(L["bias_t"]))
    Q.rope_qk(qr.view(m, -1, HD), kr.view(m, -1, HD), cos, sin, inplace=True)
    torch.cuda.synchronize()
    for a, b in ((xs, xr), (q, qr), (k, kr), (v, vr)):
        assert torch.equal(a, b)


def test_span_default_is_the_single_launch_at_one_and_two_tokens_only(gpu, layer):
    """The single launch is compiled for 1..4 tokens and picked by default at
    one and two tokens only (from three tokens on the per-projection kernels
    are faster); persistent=None then runs exactly the per-projection chain,
    and persistent=True the single launch."""
    m = 3
    assert S.span_supported(m, H, I, H, KV, HD) and not S.span_default(m, H, I, H, KV, HD)
    assert S.span_default(1, H, I, H, KV, HD) and S.span_default(2, H, I, H, KV, HD)
    x, attn = activations(390, m, H), activations(391, m, H)
    xt, at = bf16_gpu(x, gpu), bf16_gpu(attn, gpu)
    xd, (qd, kd, vd) = run_span(layer, at, xt)
    assert "launch_span" not in _native.last_plan()
    xc, (qc, kc, vc) = run_span(layer, at, xt, persistent=False)
    xs, _ = run_span(layer, at, xt, persistent=True)
    assert "launch_span" in _native.last_plan()
    torch.cuda.synchronize()
    S.decode_span_status(gpu)
    for a, b in ((xd, xc), (qd, qc), (kd, kc), (vd, vc)):
        assert torch.equal(a, b)
    ref = to_np(xc)
    d = np.abs(to_np(xs) - ref)
    assert d.max() <= 4 * O.bf16_ulp(ref).max() + O.abs_tol(I), d.max()
