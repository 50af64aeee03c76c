"""The decode step between two attention calls as one launch.

:func:`decode_span` runs what ``PagedCausalLM.forward_step`` does from one
layer's attention output to the next layer's q/k/v (engine/model.py:184-190,
then :165-173 of the next layer):

    x1 = residual + o_proj(attn)
    x  = x1 + down_proj(silu(gate_proj(h)) * up_proj(h)),  h = rms_norm(x1)
    q, k, v = q|k|v_proj(rms_norm(x)) (+ bias), RoPE of q and k

The compiled configurations (``pgs_w8a16_decode_span_supported``: the
Qwen2.5-3B shapes at one to four tokens) can run as one persistent launch
(``pgs_w8a16_decode_span``); by default the launch is used where it is the
faster way (:func:`span_default`: one and two tokens), and otherwise the same steps
run as the fused per-projection kernels (``linear`` with its residual
epilogue, ``rmsnorm_mlp``, ``rmsnorm_linear_group``, ``rope_qk``).  Either way
every operation is a gfx950 kernel of this package.
"""

from __future__ import annotations

import ctypes
import threading

import torch

from . import _native
from . import quantization as Q
from ._native import LinearOut, SpanNext, SpanWeights, check

__all__ = ["decode_span", "decode_span_status", "decode_span_trace", "span_default", "span_supported", "TRACE_MARKS"]

# Workspaces of the persistent launch (epoch, error word and exchange
# buffers; zero before first use): one per (device, stream) for eager calls,
# one per capture for calls under HIP graph capture (allocated and zeroed
# inside the capture, so each replay starts from a clean workspace).
_lock = threading.Lock()
_eager: dict[tuple[int, int], torch.Tensor] = {}
_capture: dict[tuple[int, int], tuple[int, torch.Tensor]] = {}


def _span_ws(dev: torch.device, stream: int, need: int) -> torch.Tensor:
    key = (dev.index, stream)
    capturing, cid = _native.capture_state(stream)
    with _lock:
        if capturing:
            cur = _capture.get(key)
            if cur is None or cur[0] != cid or cur[1].numel() < need:
                _capture[key] = (cid, torch.zeros(need, dtype=torch.uint8, device=dev))
            return _capture[key][1]
        _capture.pop(key, None)
        ws = _eager.get(key)
        if ws is None or ws.numel() < need:
            ws = torch.zeros(need, dtype=torch.uint8, device=dev)
            _eager[key] = ws
        return ws


def span_supported(m: int, hidden: int, inter: int, nq: int, nkv: int, head_dim: int) -> bool:
    """Whether :func:`decode_span` can run as one persistent launch for these
    sizes (``persistent=True``)."""
    return bool(_native.load().pgs_w8a16_decode_span_supported(m, hidden, inter, nq, nkv, head_dim))


def span_default(m: int, hidden: int, inter: int, nq: int, nkv: int, head_dim: int) -> bool:
    """Whether :func:`decode_span` picks the persistent launch by default: where
    it is compiled and faster than the per-projection kernels, i.e. at one and
    two tokens.  The dependent 36-layer Qwen2.5-3B decode chain on MI355X,
    single launch against per-projection kernels: 1 / 2 / 3 / 4 tokens 788 /
    918 / 1031 / 1111 against 963 / 973 / 1005 / 1016 us (from two tokens on
    every wave holds pieces of the normed-input gathers, so no wave issues the
    next stage's loads before those gathers)."""
    return m <= 2 and span_supported(m, hidden, inter, nq, nkv, head_dim)


def decode_span_status(device: torch.device | None = None, reset: bool = True) -> None:
    """Synchronises the current stream and raises
    :class:`_native.DeviceWaitTimeout` if a persistent launch on it gave up
    waiting (the outputs of that launch and of later ones on the same
    workspace are then invalid); with ``reset`` the workspace is cleared so
    that the next launch runs."""
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    stream = Q._raw_stream(dev)
    ws = _eager.get((dev.index, stream))
    if ws is None:
        return
    lib = _native.load()
    with Q._on_device(dev):
        rc = lib.pgs_w8a16_decode_span_status(ctypes.c_void_p(ws.data_ptr()), int(reset), ctypes.c_void_p(stream))
    check(rc, "decode_span")


# stage names of the 13 timestamps a traced launch writes per workgroup
TRACE_MARKS = ("start", "prologue", "o streamed", "x1 published", "x1 gathered + norm", "gate|up streamed",
               "act published", "act gathered", "down streamed", "x2 published", "x2 gathered + norm",
               "q|k|v streamed", "end")
_trace_buf: torch.Tensor | None = None


def decode_span_trace(buffer: torch.Tensor | None) -> None:
    """Turns stage tracing of the single-launch span on (``buffer``: a
    contiguous int64 CUDA tensor of ``slots * 256 * 16`` entries) or off
    (None).  While on, each launch writes per-workgroup timestamps (100 MHz
    ticks) into ``buffer.view(slots, 256, 16)[tag % slots]``: entries 0..12
    the :data:`TRACE_MARKS`, 13..15 the poll counts of the three gathers
    (those of each workgroup's first wave).
    The buffer is kept referenced until tracing is turned off.  A HIP graph
    captured while tracing is on holds the buffer's address and writes to it
    on every replay: keep the buffer for as long as such a graph exists."""
    global _trace_buf
    lib = _native.load()
    if buffer is None:
        check(lib.pgs_w8a16_decode_span_trace(None, 0), "decode_span_trace")
        _trace_buf = None
        return
    if (not isinstance(buffer, torch.Tensor) or not buffer.is_cuda or buffer.dtype != torch.int64
            or not buffer.is_contiguous() or buffer.numel() % (256 * 16) or buffer.numel() == 0):
        raise ValueError("decode_span_trace: buffer must be a contiguous int64 CUDA tensor of slots * 4096 entries")
    check(lib.pgs_w8a16_decode_span_trace(ctypes.c_void_p(buffer.data_ptr()), buffer.numel() * 8),
          "decode_span_trace")
    _trace_buf = buffer


def _bf16_vec(t: torch.Tensor, n: int, dev, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16 or t.numel() != n or t.device != dev:
        raise ValueError(f"decode_span: {name} must be a bf16 [{n}] tensor on {dev}")
    t = t.reshape(n).contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def decode_span(attn: torch.Tensor, residual: torch.Tensor, o: "Q.QuantizedWeight", ln_post: torch.Tensor,
                gate: "Q.QuantizedWeight", up: "Q.QuantizedWeight", down: "Q.QuantizedWeight", eps: float,
                next_ln: torch.Tensor | None = None, next_qkv: tuple | None = None,
                next_bias: tuple | None = None, cos: torch.Tensor | None = None, sin: torch.Tensor | None = None,
                head_dim: int = 128, persistent: bool | None = None):
    """engine/model.py:184-190 of one layer and :165-173 of the next.

    attn: the attention output ``[m, hidden]`` bf16 (the o_proj input);
    residual: the residual stream before the layer.  ``next_qkv`` = the next
    layer's (q, k, v) QuantizedWeights with ``next_ln`` its input norm weight
    and ``next_bias`` its (q_b, k_b, v_b) (entries may be None); cos / sin:
    the ``[m, head_dim]`` RoPE rows for q and k (None: no RoPE).  Returns
    ``x`` (the residual stream after the layer) and, with ``next_qkv``,
    ``(q, k, v)`` as ``[m, n]`` tensors; else ``(x, None)``.

    ``persistent``: None picks the single launch where :func:`span_default`
    says so; False forces the per-projection kernels; True requires the
    single launch (any compiled configuration)."""
    if attn.dtype != torch.bfloat16 or residual.dtype != torch.bfloat16:
        raise TypeError("decode_span: attn and residual must be bf16")
    if (next_qkv is None) != (next_ln is None):
        raise ValueError("decode_span: next_qkv and next_ln go together")
    if (cos is None) != (sin is None):
        raise ValueError("decode_span: cos and sin go together")
    qo, so, hidden, k_o, dev = o._launch_operands()
    qg, sg, inter, k_g, _ = gate._launch_operands()
    qu, su, inter_u, k_u, _ = up._launch_operands()
    qd, sd, hidden_d, k_d, _ = down._launch_operands()
    if not (k_o == hidden == k_g == k_u == hidden_d and inter == inter_u == k_d):
        raise ValueError("decode_span: o [h, h], gate/up [i, h] and down [h, i] shapes expected")
    x2 = attn.reshape(-1, hidden)
    m = x2.shape[0]
    if residual.shape != attn.shape or attn.device != dev:
        raise ValueError(f"decode_span: attn and residual must be [m, {hidden}] on {dev}")
    nq = nkv = 0
    if next_qkv is not None:
        wq, wk, wv = next_qkv
        nq, nkv = wq.shape[0], wk.shape[0]
        if wv.shape[0] != nkv or any(w.shape[1] != hidden for w in (wq, wk, wv)):
            raise ValueError("decode_span: q [nq, h], k and v [nkv, h] expected")
    sizes = (m, hidden, inter, nq if next_qkv is not None else 2048, nkv if next_qkv is not None else 256, head_dim)
    fits = span_supported(*sizes)
    if persistent is True and not fits:
        raise ValueError(f"decode_span: no single-launch configuration for m={m}, hidden={hidden}, inter={inter}")
    if persistent is False or not fits or (persistent is None and not span_default(*sizes)):
        return _chain(attn, residual, o, ln_post, gate, up, down, eps, next_ln, next_qkv, next_bias, cos, sin,
                      head_dim)

    xa = Q._aligned(x2)
    res = Q._aligned(residual.reshape(m, hidden))
    x_out = torch.empty((m, hidden), dtype=torch.bfloat16, device=dev)
    # (every tensor whose address goes into the argument structures stays
    # referenced until the launch is enqueued)
    ln_p = _bf16_vec(ln_post, hidden, dev, "ln_post")
    w = SpanWeights(qo.data_ptr(), so.data_ptr(), ln_p.data_ptr(), qg.data_ptr(), sg.data_ptr(), qu.data_ptr(),
                    su.data_ptr(), qd.data_ptr(), sd.data_ptr())
    keep = [ln_p]
    nxt = None
    outs = None
    if next_qkv is not None:
        biases = list(next_bias) if next_bias is not None else [None, None, None]
        ln_n = _bf16_vec(next_ln, hidden, dev, "next_ln")
        outs = []
        lo = []
        for wgt, b in zip(next_qkv, biases):
            q_, s_, n_, _, d_ = wgt._launch_operands()
            if d_ != dev:
                raise ValueError("decode_span: every weight must be on one device")
            bb = _bf16_vec(b, n_, dev, "bias") if b is not None else None
            y = torch.empty((m, n_), dtype=torch.bfloat16, device=dev)
            outs.append(y)
            keep.append(bb)
            lo.append(LinearOut(q_.data_ptr(), s_.data_ptr(), bb.data_ptr() if bb is not None else None,
                                y.data_ptr(), n_))
        cs = sn = None
        if cos is not None:
            if cos.dtype != torch.bfloat16 or tuple(cos.shape) != (m, head_dim) or tuple(sin.shape) != (m, head_dim):
                raise ValueError(f"decode_span: cos and sin must be bf16 [{m}, {head_dim}]")
            cs, sn = cos.contiguous(), sin.contiguous()
            keep += [cs, sn]
        nxt = SpanNext(ln_n.data_ptr(), lo[0], lo[1], lo[2], cs.data_ptr() if cs is not None else None,
                       sn.data_ptr() if sn is not None else None, head_dim)
        keep.append(ln_n)
    lib = _native.load()
    need = int(lib.pgs_w8a16_decode_span_workspace_bytes(m, hidden, inter))
    with Q._on_device(dev):
        stream = Q._raw_stream(dev)
        ws = _span_ws(dev, stream, need)
        rc = lib.pgs_w8a16_decode_span(ctypes.c_void_p(xa.data_ptr()), ctypes.c_void_p(res.data_ptr()),
                                       ctypes.c_void_p(x_out.data_ptr()), ctypes.byref(w),
                                       ctypes.byref(nxt) if nxt is not None else None, ctypes.c_float(eps), m,
                                       hidden, inter, ctypes.c_void_p(ws.data_ptr()), ws.numel(),
                                       ctypes.c_void_p(stream))
    check(rc, "decode_span")
    shape = attn.shape
    if outs is None:
        return x_out.reshape(shape), None
    return x_out.reshape(shape), tuple(outs)


def _chain(attn, residual, o, ln_post, gate, up, down, eps, next_ln, next_qkv, next_bias, cos, sin, head_dim):
    """The same steps as per-projection kernels (any size)."""
    x1 = o.linear(attn, residual=residual)
    x = Q.rmsnorm_mlp(x1, ln_post, eps, gate, up, down, residual=x1)
    if next_qkv is None:
        return x, None
    q, k, v = Q.rmsnorm_linear_group(x, next_ln, eps, list(next_qkv), list(next_bias) if next_bias else None)
    if cos is not None:
        m = q.shape[0] if q.dim() == 2 else q.numel() // q.shape[-1]
        q3 = q.reshape(m, -1, head_dim)
        k3 = k.reshape(m, -1, head_dim)
        Q.rope_qk(q3, k3, cos, sin, inplace=True)
    return x, (q, k, v)


def exchange_values(m: int, hidden: int, inter: int, device: torch.device | None = None):
    """(x1, act): the residual stream after o_proj and the SwiGLU activations
    of the last single-launch :func:`decode_span` call on the current stream
    (the values its workgroups exchanged), as float32 ``[m, hidden]`` and
    ``[m, inter]`` CPU tensors, and the set of launch tags seen in them (one
    tag when every word comes from that launch).  For checks of each stage
    on its own GPU input; synchronises the stream."""
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    ws = _eager.get((dev.index, Q._raw_stream(dev)))
    if ws is None:
        raise RuntimeError("decode_span: no single-launch call on this stream yet")
    w = ws.view(torch.int32).cpu().to(torch.int64) & 0xFFFFFFFF
    hdr = 256 // 4

    def unpack(base, units):
        blk = w[base: base + units * 32].reshape(units, 32)[:, : 8 * m].reshape(units, m, 8)
        vals = (blk & 0xFFFF).to(torch.int32).to(torch.int16).view(torch.bfloat16).float()
        return vals.permute(1, 0, 2).reshape(m, units * 8), set((blk >> 16).unique().tolist())

    x1, t1 = unpack(hdr, hidden // 8)
    act, t2 = unpack(hdr + (hidden // 8) * 32, inter // 8)
    return x1, act, t1 | t2
