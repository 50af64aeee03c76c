"""INT8 weight-only quantization with the interface of pageserve's
``engine/quantization.py``, computed by gfx950 HIP kernels.

Same names, argument meaning and return types as the reference:

* ``quantize_per_channel(weight) -> (q int8 [N,K], scale fp32 [N,1])``
  (engine/quantization.py:16-23), bit-identical to the reference's CPU result;
* ``dequantize(q, scale, dtype)`` (engine/quantization.py:26-27), bit-identical;
* ``QuantizedWeight(weight)`` with ``.dtype .q .scale .get() .to(device)
  .storage_bytes`` (engine/quantization.py:30-50).

What changes is the per-call path.  The reference's ``get()`` dequantizes the
whole weight on every access and ``engine/model.py`` then runs a dense GEMM.
Here ``get()`` on a GPU weight returns a :class:`W8A16Weight`, a tensor
subclass of the same shape and dtype whose ``F.linear`` runs the fused W8A16
kernel (int8 read once, scale and bias in the epilogue), so
``F.linear(h, _resolve(w), b)`` in an unchanged ``engine/model.py`` takes the
fused path.  Any other operation on it materialises the dense weight through
the dequantize kernel, which is exactly what the reference's ``get()`` returns.

Explicit entry points that the reference's call sites can use directly:
``QuantizedWeight.linear``, :func:`linear_group` (q/k/v in one launch) and
:func:`swiglu` (gate/up/silu*up in one launch, engine/model.py:188-190).

Device placement follows the reference: results live where the input lives.
GPU tensors always run the gfx950 HIP kernels; without the built library those
calls raise.  CPU tensors keep the reference's own math, evaluated by torch on
the CPU (the reference quantizes on the CPU, engine/model.py:101-112, and its
one ``quantize=True`` caller runs a CPU fp32 model,
scripts/verify_quantization.py:32): a CPU weight is quantized, stored,
unpacked and dequantized there without any copy to a GPU, and ``get()``
returns the dense dequantized weight as the reference's does.  The fused
entry points (``linear``, ``linear_group``, ``swiglu`` ...) take GPU tensors
only.
"""

from __future__ import annotations

import ctypes
import functools
import threading
from collections import OrderedDict

import torch
import torch.nn.functional as F

from . import _native
from ._native import DTYPE_BF16, DTYPE_F16, DTYPE_F32, check

__all__ = [
    "quantize_per_channel",
    "dequantize",
    "QuantizedWeight",
    "W8A16Weight",
    "linear",
    "linear_group",
    "swiglu",
    "mlp",
    "rmsnorm",
    "save_quantized",
    "load_quantized",
    "packed_numel",
    "pack",
    "unpack",
]

_DTYPE_CODE = {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16}


# ---------------------------------------------------------------------------
# plumbing
# ---------------------------------------------------------------------------

# torch's current stream as a raw hipStream_t, without building a Stream
# object per call (the public route costs a few microseconds of host time)
_get_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _raw_stream(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if _get_raw_stream is not None:
        return _get_raw_stream(idx)
    return torch.cuda.current_stream(idx).cuda_stream


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(_raw_stream(device))


class _on_device:
    """Makes ``device`` current for the launch (cheap when it already is)."""

    __slots__ = ("dev", "prev")

    def __init__(self, device: torch.device):
        self.dev = device.index if device.index is not None else torch.cuda.current_device()
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.dev:
            self.prev = cur
            torch.cuda.set_device(self.dev)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def _aligned(t: torch.Tensor, n: int = 16) -> torch.Tensor:
    """Contiguous, with data pointer aligned to ``n`` bytes (copies only if needed)."""
    t = t.contiguous()
    if t.numel() and t.data_ptr() % n:
        t = t.clone()
    return t


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None and t.numel() else 0)


# Workspaces of the K-split plans (pair slots that must start empty, then
# partial tiles):
#  * eager calls use one buffer per (device, stream), zero-filled when it is
#    allocated; every call leaves its pair slots empty, so the stream's later
#    calls reuse it; a larger need replaces it (the old buffer is freed in
#    stream order, which torch's caching allocator makes safe);
#  * calls under HIP graph capture use one buffer per capture (device, stream,
#    capture id), allocated and zero-filled inside the capture: the fill is a
#    node of that graph, so every replay starts from empty slots whatever used
#    the memory between replays (graphs sharing a memory pool), and no eager
#    call shares it.  It is a temporary of the graph's memory pool and leaves
#    this table once its capture is over.
_MAX_EAGER_WS = 16  # (device, stream) pairs kept; the least recently used is dropped
# The tables are shared by every thread: each lookup-and-update holds this
# lock (calls from several threads on one stream then share that stream's
# buffer, which the stream's order makes safe).
_ws_lock = threading.Lock()
_eager_ws: "OrderedDict[tuple[int, int], torch.Tensor]" = OrderedDict()
_capture_ws: dict[tuple[int, int], tuple[int, torch.Tensor]] = {}
_MIN_WS = 4 << 20


@functools.lru_cache(maxsize=4096)
def _ws_need(m: int, ns: tuple, k: int, swiglu: bool, norm: bool) -> int:
    lib = _native.load()
    arr = (ctypes.c_int64 * len(ns))(*ns)
    query = lib.pgs_w8a16_rmsnorm_workspace_bytes if norm else lib.pgs_w8a16_workspace_bytes
    return int(query(m, arr, len(ns), k, int(swiglu)))


def _zeroed(size: int, dev: torch.device) -> torch.Tensor:
    ws = torch.zeros(size, dtype=torch.uint8, device=dev)  # a fill kernel, capturable
    if ws.data_ptr() % 256:
        raise RuntimeError("pageserve_amd: workspace allocation is not 256-byte aligned")
    return ws


def _workspace(lib, dev: torch.device, stream: int, m: int, ns: tuple, k: int, swiglu: bool, norm: bool = False):
    need = _ws_need(m, ns, k, bool(swiglu), bool(norm))
    if need == 0:
        return ctypes.c_void_p(0), 0, None
    key = (dev.index, stream)
    capturing, cid = _native.capture_state(stream)
    with _ws_lock:
        if capturing:
            cur = _capture_ws.get(key)
            if cur is None or cur[0] != cid or cur[1].numel() < need:
                grow = 2 * cur[1].numel() if cur is not None and cur[0] == cid else 0
                _capture_ws[key] = (cid, _zeroed(max(need, grow, _MIN_WS), dev))
            ws = _capture_ws[key][1]
        else:
            _capture_ws.pop(key, None)  # that capture is over
            ws = _eager_ws.get(key)
            if ws is None or ws.numel() < need:
                ws = _zeroed(max(need, 2 * ws.numel() if ws is not None else 0, _MIN_WS), dev)
                _eager_ws[key] = ws
                while len(_eager_ws) > _MAX_EAGER_WS:
                    _eager_ws.popitem(last=False)
            _eager_ws.move_to_end(key)
    # the caller keeps the tensor until its launch is enqueued: a thread that
    # replaces the buffer meanwhile cannot free it under that launch
    return ctypes.c_void_p(ws.data_ptr()), ws.numel(), ws


# ---------------------------------------------------------------------------
# CPU-resident tensors: the reference formula in torch, on the CPU
# ---------------------------------------------------------------------------
# Used only for tensors that live on the CPU; GPU tensors never reach these.

def _cpu_quantize(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """engine/quantization.py:20-22 in torch on the CPU: per-row absmax of the
    fp32 weight floored at 1e-8, divided by 127 (IEEE fp32 divide), then
    w / scale rounded half to even and clamped to +-127."""
    w = weight.float()
    scale = w.abs().amax(dim=1, keepdim=True).clamp(min=1e-8) / 127.0
    return (w / scale).round().clamp(-127, 127).to(torch.int8), scale


def _cpu_dequantize(q: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """engine/quantization.py:27: the fp32 product q * scale, then the cast."""
    return (q.to(torch.float32) * scale.to(torch.float32).reshape(-1, 1)).to(dtype)


def _tiles(n: int, k: int) -> tuple[int, int]:
    return -(-n // 16), -(-k // 64)


def _cpu_pack(q: torch.Tensor) -> torch.Tensor:
    """Row-major int8 [n, k] -> packed bytes (layout of :func:`packed_numel`)."""
    n, k = q.shape
    if n == 0 or k == 0:
        return torch.empty(0, dtype=torch.int8)
    tn, tk = _tiles(n, k)
    padded = torch.zeros((tn * 16, tk * 64), dtype=torch.int8)
    padded[:n, :k] = q
    # [tile row, row, tile col, 16-column group, byte] -> [tile row, tile col, group, row, byte]
    return padded.view(tn, 16, tk, 4, 16).permute(0, 2, 3, 1, 4).reshape(-1)


def _cpu_tiles_to(qp: torch.Tensor, n: int, k: int, dtype: torch.dtype) -> torch.Tensor:
    """Packed bytes -> the row-major [n, k] matrix in ``dtype``, converted in
    the same pass as the reordering."""
    if n == 0 or k == 0:
        return torch.empty((n, k), dtype=dtype)
    tn, tk = _tiles(n, k)
    out = torch.empty((tn, 16, tk, 4, 16), dtype=dtype)
    out.copy_(qp.view(tn, tk, 4, 16, 16).permute(0, 3, 1, 2, 4))
    return out.view(tn * 16, tk * 64)[:n, :k]


def _cpu_unpack(qp: torch.Tensor, n: int, k: int) -> torch.Tensor:
    return _cpu_tiles_to(qp, n, k, torch.int8).contiguous()


def _cpu_dequantize_packed(qp: torch.Tensor, scale: torch.Tensor, n: int, k: int,
                           dtype: torch.dtype) -> torch.Tensor:
    # the same fp32 products as _cpu_dequantize of the unpacked q
    return (_cpu_tiles_to(qp, n, k, torch.float32) * scale.to(torch.float32).reshape(-1, 1)).to(dtype)


# ---------------------------------------------------------------------------
# quantize_per_channel / dequantize
# ---------------------------------------------------------------------------

def quantize_per_channel(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """weight: (out_features, in_features).  Returns (int8_weight, scale),
    scale shape (out_features, 1), such that dequantize(int8_weight, scale)
    ~= weight.  engine/quantization.py:16-23, bit-identical.
    """
    if not isinstance(weight, torch.Tensor):
        raise TypeError("weight must be a torch.Tensor")
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D (out_features, in_features), got shape {tuple(weight.shape)}")
    n, k = weight.shape
    if k == 0 and n > 0:
        # torch's amax refuses an empty reduction dimension; so does the reference
        raise RuntimeError("amax(): Expected reduction dim 1 to have non-zero size.")
    if weight.device.type != "cuda":
        return _cpu_quantize(weight)
    dev = weight.device
    lib = _native.load()
    w = weight
    if w.dtype not in (torch.float32, torch.bfloat16):
        w = w.float()  # the reference's own first step, weight.float()
    w = _aligned(w)
    q = torch.empty((n, k), dtype=torch.int8, device=dev)
    scale = torch.empty((n, 1), dtype=torch.float32, device=dev)
    with _on_device(dev):
        rc = lib.pgs_quantize_per_channel(
            _ptr(w), _DTYPE_CODE[w.dtype], n, k, _ptr(q), _ptr(scale), _stream(dev)
        )
    check(rc, "quantize_per_channel")
    return q, scale


def dequantize(q: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``(q.to(float32) * scale).to(dtype)`` -- engine/quantization.py:26-27,
    bit-identical.  ``scale``: per-row, shape (N, 1) or (N,).
    """
    if q.dim() != 2 or q.dtype != torch.int8:
        raise ValueError("q must be a 2-D int8 tensor")
    n, k = q.shape
    if scale.numel() != n:
        raise ValueError(f"scale must hold one value per row ({n}), got shape {tuple(scale.shape)}")
    if q.device.type != "cuda":
        return _cpu_dequantize(q, scale.to(q.device), dtype)
    dev = q.device
    lib = _native.load()
    kdt = dtype if dtype in _DTYPE_CODE else torch.float32
    qd = _aligned(q)
    sd = _aligned(scale.to(dev, dtype=torch.float32).reshape(n))
    out = torch.empty((n, k), dtype=kdt, device=dev)
    with _on_device(dev):
        rc = lib.pgs_dequantize(_ptr(qd), _ptr(sd), n, k, _ptr(out), _DTYPE_CODE[kdt], _stream(dev))
    check(rc, "dequantize")
    if kdt != dtype:
        out = out.to(dtype)  # fp32 product, then the reference's .to(dtype)
    return out


# ---------------------------------------------------------------------------
# packed storage (the layout the linear kernels stream)
# ---------------------------------------------------------------------------

def _packed_numel(lib, n: int, k: int) -> int:
    return int(lib.pgs_packed_bytes(n, k))


def _quantize_packed(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """quantize_per_channel with q written in the packed layout (on the
    weight's device)."""
    n, k = weight.shape
    if weight.device.type != "cuda":
        q, scale = _cpu_quantize(weight)
        return _cpu_pack(q), scale
    dev = weight.device
    lib = _native.load()
    w = weight if weight.dtype in (torch.float32, torch.bfloat16) else weight.float()
    w = _aligned(w)
    qp = torch.empty(_packed_numel(lib, n, k), dtype=torch.int8, device=dev)
    scale = torch.empty((n, 1), dtype=torch.float32, device=dev)
    with _on_device(dev):
        rc = lib.pgs_quantize_per_channel_packed(_ptr(w), _DTYPE_CODE[w.dtype], n, k, _ptr(qp), _ptr(scale),
                                                 _stream(dev))
    check(rc, "quantize_per_channel")
    return qp, scale


def pack(q: torch.Tensor) -> torch.Tensor:
    """Row-major int8 [N, K] -> the packed layout (same device as ``q``)."""
    if q.dim() != 2 or q.dtype != torch.int8:
        raise ValueError("q must be a 2-D int8 tensor")
    n, k = q.shape
    if q.device.type != "cuda":
        return _cpu_pack(q)
    dev = q.device
    lib = _native.load()
    qd = _aligned(q)
    qp = torch.empty(_packed_numel(lib, n, k), dtype=torch.int8, device=dev)
    with _on_device(dev):
        rc = lib.pgs_pack_weight(_ptr(qd), n, k, _ptr(qp), _stream(dev))
    check(rc, "pack")
    return qp


def unpack(qp: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """The packed layout -> row-major int8 [N, K] (same device as ``qp``)."""
    if qp.numel() != packed_numel(n, k):
        raise ValueError(f"packed buffer holds {qp.numel()} bytes, [{n}, {k}] needs {packed_numel(n, k)}")
    if qp.device.type != "cuda":
        return _cpu_unpack(qp, n, k)
    dev = qp.device
    lib = _native.load()
    qd = _aligned(qp)
    q = torch.empty((n, k), dtype=torch.int8, device=dev)
    with _on_device(dev):
        rc = lib.pgs_unpack_weight(_ptr(qd), n, k, _ptr(q), _stream(dev))
    check(rc, "unpack")
    return q


def _dequantize_packed(qp: torch.Tensor, scale: torch.Tensor, n: int, k: int, dtype: torch.dtype) -> torch.Tensor:
    if qp.device.type != "cuda":
        return _cpu_dequantize_packed(qp, scale.to(qp.device), n, k, dtype)
    dev = qp.device
    lib = _native.load()
    kdt = dtype if dtype in _DTYPE_CODE else torch.float32
    qd = _aligned(qp)
    sd = _aligned(scale.to(dev, dtype=torch.float32).reshape(n))
    out = torch.empty((n, k), dtype=kdt, device=dev)
    with _on_device(dev):
        rc = lib.pgs_dequantize_packed(_ptr(qd), _ptr(sd), n, k, _ptr(out), _DTYPE_CODE[kdt], _stream(dev))
    check(rc, "dequantize")
    if kdt != dtype:
        out = out.to(dtype)
    return out


# ---------------------------------------------------------------------------
# fused linears
# ---------------------------------------------------------------------------

def _ws_args(dev: torch.device, x, k: int, ns: tuple, swiglu: bool, norm: bool) -> tuple:
    """(pointer, bytes, buffer) of the K-split workspace a call needs, (0, 0,
    None) when its plan splits nothing (every decode projection of a
    2048-hidden model).  Hold ``buffer`` until the launch is enqueued."""
    m = x.numel() // k if isinstance(x, torch.Tensor) and k else 0
    if m <= 0 or _ws_need(m, ns, k, swiglu, norm) == 0:
        return 0, 0, None
    lib = _native.load()
    with _on_device(dev):
        ws, nbytes, buf = _workspace(lib, dev, _raw_stream(dev), m, ns, k, swiglu, norm)
    return ws.value or 0, nbytes, buf


def linear(x: torch.Tensor, weight: "QuantizedWeight", bias: torch.Tensor | None = None,
           out_dtype: torch.dtype = torch.bfloat16, residual: torch.Tensor | None = None,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x, dequantize(q, scale, bf16), bias)`` fused: y = x (q s)^T + b.

    x: bf16 [..., K] on the weight's GPU.  out_dtype: bf16 (projections) or
    fp32 (the lm_head logits).  Returns [..., N].

    residual (bf16 [..., N]): returns ``residual + F.linear(x, W, b)`` with the
    reference's roundings (engine/model.py:184, 190) from the same launch.
    out: optional contiguous result buffer of the right shape and dtype; it
    may be the residual itself (in place).
    """
    if out_dtype is not torch.bfloat16 and out_dtype is not torch.float32:
        raise TypeError("out_dtype must be torch.bfloat16 or torch.float32")
    # (is_cuda rather than .device.type: no torch.device built per call)
    if not weight.qp.is_cuda:
        raise RuntimeError("W8A16 linear: the weight must be on a ROCm GPU (call .to('cuda') first)")
    q, s, n, k, dev = weight._launch_operands()
    ws, ws_bytes, _buf = _ws_args(dev, x, k, (n,), False, False)
    return _native.load_host().linear1(x, q, s, bias, n, k, out_dtype is torch.float32, residual, out, ws, ws_bytes)


def linear_argmax(x: torch.Tensor, weight: "QuantizedWeight", bias: torch.Tensor | None = None,
                  return_values: bool = False):
    """``F.linear(x, W, bias).float().argmax(-1)`` -- the greedy next token
    of server.py:51 after the lm_head of engine/model.py:193 -- without
    writing the logits: the fp32 logits (as :func:`linear` with
    ``out_dtype=torch.float32`` computes them) are reduced to their row
    argmax inside the projection (torch.argmax's choice: the first index of
    the maximum, NaN counting as the maximum).  x: bf16 [..., K] with at most
    32 rows (pass only the rows whose argmax is needed, e.g. ``h[-1:]``).
    Returns int64 indices of shape x.shape[:-1], and with ``return_values``
    also the fp32 maxima."""
    if weight.device.type != "cuda":
        raise RuntimeError("linear_argmax: the weight must be on a ROCm GPU")
    q, s, n, k, dev = weight._launch_operands()
    if not isinstance(x, torch.Tensor) or x.device != dev:
        raise ValueError(f"linear_argmax: input must be on {dev}")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"linear_argmax: the W8A16 kernels take bf16 activations, got {x.dtype}")
    if x.dim() < 1 or x.shape[-1] != k:
        raise ValueError(f"linear_argmax: input has {x.shape[-1] if x.dim() else 0} features, weight expects {k}")
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous().clone()
    m = x2.shape[0]
    if bias is not None:
        if bias.device != dev or bias.dtype != torch.bfloat16 or bias.numel() != n:
            raise ValueError(f"linear_argmax: bias must be a bf16 [{n}] tensor on {dev}")
        bias = bias.reshape(n).contiguous()
    idx = torch.empty(m, dtype=torch.int64, device=dev)
    vmax = torch.empty(m, dtype=torch.float32, device=dev) if return_values else None
    lib = _native.load()
    need = lib.pgs_w8a16_argmax_workspace_bytes(m, n, k)
    if need == 0:
        raise ValueError(f"linear_argmax: {m} rows; 1..32 are supported (pass the rows whose argmax is needed)")
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    with _on_device(dev):
        rc = lib.pgs_w8a16_linear_argmax(_ptr(x2), _ptr(q), _ptr(s), _ptr(bias) if bias is not None else None,
                                         _ptr(idx), _ptr(vmax) if vmax is not None else None, m, n, k, _ptr(ws),
                                         need, ctypes.c_void_p(_raw_stream(dev)))
    check(rc, "linear_argmax")
    shape = x.shape[:-1]
    if return_values:
        return idx.reshape(shape), vmax.reshape(shape)
    return idx.reshape(shape)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``rms_norm(x, weight, eps)`` of engine/model.py:29-34 as one kernel:
    h = bf16(weight * bf16(x * rsqrt(mean(x^2) + eps))), the mean in fp32.
    x: bf16 [..., K] on a ROCm GPU; weight: bf16 [K] on the same GPU."""
    if not isinstance(x, torch.Tensor) or x.device.type != "cuda":
        raise RuntimeError("rmsnorm: x must be on a ROCm GPU")
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("rmsnorm: x and weight must be bf16")
    k = x.shape[-1]
    if weight.device != x.device or weight.numel() != k:
        raise ValueError(f"rmsnorm: weight must be a bf16 [{k}] tensor on {x.device}")
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    w = weight.reshape(k).contiguous()
    h = torch.empty_like(x2)
    lib = _native.load()
    with _on_device(x.device):
        stream = _raw_stream(x.device)
        rc = lib.pgs_rmsnorm(_ptr(x2), _ptr(w), ctypes.c_float(eps), _ptr(h), x2.shape[0], k, ctypes.c_void_p(stream))
    check(rc, "rmsnorm")
    return h.reshape(x.shape)


def _rope_tables(cos: torch.Tensor, sin: torch.Tensor, m: int, head_dim: int, device) -> tuple:
    if cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16:
        raise TypeError("rope: cos and sin must be bf16")
    if tuple(cos.shape) != (m, head_dim) or tuple(sin.shape) != (m, head_dim):
        raise ValueError(f"rope: cos and sin must be [{m}, {head_dim}]")
    if cos.device != device or sin.device != device:
        raise ValueError("rope: cos and sin must be on the tensors' device")
    return cos.contiguous(), sin.contiguous()


def _rope_input(x: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(x, torch.Tensor) or x.device.type != "cuda":
        raise RuntimeError(f"rope: {name} must be on a ROCm GPU")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"rope: {name} must be bf16")
    if x.dim() != 3:
        raise ValueError(f"rope: {name} must be (tokens, heads, head_dim)")
    return x.contiguous()


def rope_qk(q: torch.Tensor, k: torch.Tensor | None, cos: torch.Tensor, sin: torch.Tensor,
            inplace: bool = False) -> tuple:
    """``q = apply_rope(q, cos, sin); k = apply_rope(k, cos, sin)``
    (engine/model.py:53-56, applied at :172-173) in one launch, with the
    reference's bf16 roundings.  q: (tokens, heads, head_dim) bf16, k:
    (tokens, kv_heads, head_dim) bf16 or None; cos / sin: (tokens, head_dim)
    bf16 (the reference's cache rows).  Returns (q_out, k_out); in place when
    ``inplace`` (the inputs must then be contiguous)."""
    qc = _rope_input(q, "q")
    m, qh, hd = qc.shape
    if k is not None:
        kc = _rope_input(k, "k")
        if kc.shape[0] != m or kc.shape[2] != hd or kc.device != qc.device:
            raise ValueError("rope: k must match q in tokens, head_dim and device")
        kh = kc.shape[1]
    else:
        kc, kh = None, 0
    if hd % 2:
        raise ValueError("rope: head_dim must be even")
    if inplace and (qc is not q or (k is not None and kc is not k)):
        raise ValueError("rope: in place needs contiguous q and k")
    c, s = _rope_tables(cos, sin, m, hd, qc.device)
    qo = qc if inplace else torch.empty_like(qc)
    ko = (kc if inplace else torch.empty_like(kc)) if kc is not None else None
    lib = _native.load()
    with _on_device(qc.device):
        stream = _raw_stream(qc.device)
        rc = lib.pgs_rope(_ptr(qc), _ptr(qo), qh, _ptr(kc) if kc is not None else None,
                          _ptr(ko) if ko is not None else None, kh, _ptr(c), _ptr(s), m, hd,
                          ctypes.c_void_p(stream))
    check(rc, "rope")
    return qo, ko


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``apply_rope(x, cos, sin)`` of engine/model.py:53-56 as one kernel
    (same arguments, same bf16 result)."""
    return rope_qk(x, None, cos, sin)[0]


def linear_group(x: torch.Tensor, weights: list["QuantizedWeight"], biases: list | None = None,
                 out_dtype: torch.dtype = torch.bfloat16) -> list[torch.Tensor]:
    """Several projections of the same input in one launch (q/k/v,
    engine/model.py:168-170).  Returns one output per weight."""
    return _linear_group(x, weights, biases, out_dtype, None, 0.0)


def rmsnorm_linear_group(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, weights: list["QuantizedWeight"],
                         biases: list | None = None, out_dtype: torch.dtype = torch.bfloat16) -> list[torch.Tensor]:
    """``h = rms_norm(x, norm_weight, eps)`` then the projections of ``h``
    (engine/model.py:166-170), in one launch for up to 4 tokens (the kernel
    normalises the activations it stages; its fixed-order sum of squares may
    make ``h`` differ from :func:`rmsnorm` in the last bf16 bit), otherwise
    :func:`rmsnorm` then :func:`linear_group`."""
    return _linear_group(x, weights, biases, out_dtype, norm_weight, eps)


def _linear_group(x, weights, biases, out_dtype, norm_weight, eps) -> list[torch.Tensor]:
    if not weights or len(weights) > _native.MAX_GROUP:
        raise ValueError(f"linear_group takes 1..{_native.MAX_GROUP} weights")
    biases = list(biases) if biases is not None else [None] * len(weights)
    if len(biases) != len(weights):
        raise ValueError("one bias (or None) per weight")
    if out_dtype is not torch.bfloat16 and out_dtype is not torch.float32:
        raise TypeError("out_dtype must be torch.bfloat16 or torch.float32")
    if not weights[0].qp.is_cuda:
        raise RuntimeError("W8A16 linear: the weight must be on a ROCm GPU (call .to('cuda') first)")
    ops = [w._launch_operands() for w in weights]
    _, _, _, k, dev = ops[0]
    for o in ops:
        if o[3] != k or o[4] != dev:
            raise ValueError("linear_group: weights must share device and in_features")
    qs, ss, ns = [o[0] for o in ops], [o[1] for o in ops], tuple(o[2] for o in ops)
    ws, ws_bytes, _buf = _ws_args(dev, x, k, ns, False, norm_weight is not None)
    return _native.load_host().linear(x, qs, ss, biases, ns, k, out_dtype is torch.float32, None, None, norm_weight,
                                      eps, ws, ws_bytes)


def swiglu(x: torch.Tensor, gate: "QuantizedWeight", up: "QuantizedWeight") -> torch.Tensor:
    """``F.silu(F.linear(x, gate)) * F.linear(x, up)`` in one launch
    (engine/model.py:188-190); fp32 inside, one rounding to bf16."""
    return _swiglu(x, gate, up, None, 0.0)


def rmsnorm_swiglu(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, gate: "QuantizedWeight",
                   up: "QuantizedWeight") -> torch.Tensor:
    """``h = rms_norm(x, norm_weight, eps)`` then :func:`swiglu` of ``h``
    (engine/model.py:187-189), in one launch for up to 4 tokens (as
    :func:`rmsnorm_linear_group`)."""
    return _swiglu(x, gate, up, norm_weight, eps)


def _swiglu(x, gate, up, norm_weight, eps) -> torch.Tensor:
    if not gate.qp.is_cuda or not up.qp.is_cuda:
        raise RuntimeError("swiglu: gate and up weights must be on the same ROCm GPU")
    qg, sg, n, k, dev = gate._launch_operands()
    qu, su, nu, ku, dev_u = up._launch_operands()
    if dev_u != dev:
        raise RuntimeError("swiglu: gate and up weights must be on the same ROCm GPU")
    if (n, k) != (nu, ku):
        raise ValueError("swiglu: gate and up weights must have the same shape")
    ws, ws_bytes, _buf = _ws_args(dev, x, k, (n,), True, norm_weight is not None)
    return _native.load_host().swiglu(x, qg, sg, qu, su, n, k, norm_weight, eps, ws, ws_bytes)


def mlp(x: torch.Tensor, gate: "QuantizedWeight", up: "QuantizedWeight", down: "QuantizedWeight",
        residual: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(F.silu(gate(x)) * up(x), down)`` (engine/model.py:188-190): the
    fused gate/up kernel, then the down projection; with ``residual`` the
    add of engine/model.py:190 runs in the down projection's epilogue."""
    return linear(swiglu(x, gate, up), down, residual=residual)


def rmsnorm_mlp(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, gate: "QuantizedWeight",
                up: "QuantizedWeight", down: "QuantizedWeight", residual: torch.Tensor | None = None) -> torch.Tensor:
    """engine/model.py:187-190: ``rms_norm`` and the fused gate/up kernel in
    one launch (:func:`rmsnorm_swiglu`), then the down projection with the
    optional residual add in its epilogue."""
    return linear(rmsnorm_swiglu(x, norm_weight, eps, gate, up), down, residual=residual)


# ---------------------------------------------------------------------------
# QuantizedWeight and the drop-in tensor view
# ---------------------------------------------------------------------------

class QuantizedWeight:
    """Drop-in replacement for a plain weight tensor: stores int8 + scale,
    dequantizes on access (engine/quantization.py:30-50).

    Storage is the packed tile layout the kernels stream (``qp``, one byte per
    weight plus zero padding to 16 rows x 64 columns).  ``q`` gives the
    reference's row-major int8 view, rebuilt on access by the unpack kernel
    (bit-identical to ``quantize_per_channel(weight)[0]``); assigning ``q``
    repacks it.  ``get()`` gives a tensor that behaves as the dequantized
    weight; ``F.linear`` on it runs the fused W8A16 kernel.
    """

    def __init__(self, weight: torch.Tensor):
        if not isinstance(weight, torch.Tensor) or weight.dim() != 2:
            raise ValueError("weight must be a 2-D tensor (out_features, in_features)")
        if weight.shape[1] == 0 and weight.shape[0] > 0:
            raise RuntimeError("amax(): Expected reduction dim 1 to have non-zero size.")
        self.dtype = weight.dtype
        self.shape = torch.Size(weight.shape)
        self.qp, self.scale = _quantize_packed(weight)

    @property
    def q(self) -> torch.Tensor:
        return unpack(self.qp, *self.shape)

    @q.setter
    def q(self, value: torch.Tensor) -> None:
        self.qp = pack(value)
        self.shape = torch.Size(value.shape)

    @property
    def device(self) -> torch.device:
        return self.qp.device

    def get(self) -> torch.Tensor:
        if self.qp.device.type == "cuda":
            # one view per (qp, scale) storage: engine/model.py's _resolve calls
            # get() before every projection, and building the tensor subclass
            # costs about a microsecond of host time
            v = getattr(self, "_view", None)
            if v is None or v[0] is not self.qp or v[1] is not self.scale:
                v = (self.qp, self.scale, W8A16Weight(self))
                self._view = v
            return v[2]
        return self.dense()  # a CPU weight: the reference's dequantized tensor, computed on the CPU

    def to(self, device) -> "QuantizedWeight":
        self.qp = self.qp.to(device)
        self.scale = self.scale.to(device)
        return self

    @property
    def storage_bytes(self) -> int:
        return self.qp.numel() * self.qp.element_size() + self.scale.numel() * self.scale.element_size()

    def dense(self) -> torch.Tensor:
        """The reference's ``get()``: the dequantized weight in ``self.dtype``."""
        return _dequantize_packed(self.qp, self.scale, *self.shape, self.dtype)

    def linear(self, x: torch.Tensor, bias: torch.Tensor | None = None,
               out_dtype: torch.dtype = torch.bfloat16, residual: torch.Tensor | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
        return linear(x, self, bias, out_dtype=out_dtype, residual=residual, out=out)

    # -- persistent form (the reference re-quantizes at every load,
    # engine/model.py:101-112; the stored packed form loads as a copy) --

    def state(self) -> dict[str, torch.Tensor]:
        """The stored form: packed int8 ``qp``, fp32 ``scale`` [N, 1] and
        ``meta`` = int64 [N, K, dtype code] (0 fp32, 1 bf16, 2 fp16)."""
        code = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}.get(self.dtype)
        if code is None:
            raise TypeError(f"cannot store a QuantizedWeight of dtype {self.dtype}")
        return {"qp": self.qp, "scale": self.scale,
                "meta": torch.tensor([self.shape[0], self.shape[1], code], dtype=torch.int64)}

    @classmethod
    def from_state(cls, state: dict[str, torch.Tensor]) -> "QuantizedWeight":
        """Rebuilds a QuantizedWeight from :meth:`state` (no quantization, no
        kernel launch); the tensors stay on their device."""
        try:
            qp, scale, meta = state["qp"], state["scale"], state["meta"]
        except KeyError as e:
            raise ValueError(f"QuantizedWeight state lacks {e}") from None
        n, k, code = (int(v) for v in meta.reshape(-1).tolist())
        dtype = {0: torch.float32, 1: torch.bfloat16, 2: torch.float16}.get(code)
        if dtype is None or n < 0 or k < 0:
            raise ValueError(f"bad QuantizedWeight meta {meta.tolist()}")
        if qp.dtype != torch.int8 or qp.numel() != packed_numel(n, k):
            raise ValueError(f"packed weight must be int8 with {packed_numel(n, k)} elements for [{n}, {k}]")
        if scale.dtype != torch.float32 or scale.numel() != n or scale.device != qp.device:
            raise ValueError(f"scale must be fp32 [{n}, 1] on {qp.device}")
        obj = cls.__new__(cls)
        obj.dtype, obj.shape = dtype, torch.Size((n, k))
        obj.qp, obj.scale = qp.reshape(-1), scale.reshape(n, 1)
        return obj

    def _kernel_operands(self) -> tuple[torch.Tensor, torch.Tensor]:
        # cached for the current (qp, scale) objects when both are used as
        # they are (no copy that an in-place update could leave stale);
        # rebuilt when either is replaced (to(), assigning q)
        qp0, sc0 = self.qp, self.scale
        cached = getattr(self, "_ops", None)
        if cached is not None and cached[0] is qp0 and cached[1] is sc0:
            return cached[2], cached[3]
        qp = qp0
        if not qp.is_contiguous() or (qp.numel() and qp.data_ptr() % 16):
            qp = _aligned(qp)
        s = sc0.reshape(-1)
        if s.dtype != torch.float32 or not s.is_contiguous():
            s = s.to(torch.float32).contiguous()
        if qp is qp0 and (not s.numel() or s.data_ptr() == sc0.data_ptr()):
            self._ops = (qp0, sc0, qp, s)
        return qp, s

    def _launch_operands(self) -> tuple:
        """(packed q, fp32 scale [N], N, K, device) for a launch, cached for
        the current (qp, scale) objects (the per-call host path)."""
        c = getattr(self, "_launch", None)
        if c is not None and c[0] is self.qp and c[1] is self.scale:
            return c[2]
        q, s = self._kernel_operands()
        ops = (q, s, self.shape[0], self.shape[1], q.device)
        cached = getattr(self, "_ops", None)  # set when q and s are the stored tensors themselves
        if cached is not None and cached[0] is self.qp and cached[1] is self.scale:
            self._launch = (self.qp, self.scale, ops)
        return ops


def packed_numel(n: int, k: int) -> int:
    """Bytes of the packed tile layout of an [n, k] int8 matrix (16-row x
    64-column blocks of 1 KiB, zero padded)."""
    return ((n + 15) // 16) * ((k + 63) // 64) * 1024 if n > 0 and k > 0 else 0


_FORMAT = "pageserve_amd.w8a16.packed.v1"


def save_quantized(path: str, weights: dict[str, "QuantizedWeight"]) -> None:
    """Writes quantized weights to a safetensors file (tensors ``<name>.qp``,
    ``<name>.scale``, ``<name>.meta``); executes nothing when loaded."""
    from safetensors.torch import save_file

    tensors = {}
    for name, w in weights.items():
        for key, t in w.state().items():
            tensors[f"{name}.{key}"] = t.detach().to("cpu").contiguous()
    save_file(tensors, path, metadata={"format": _FORMAT})


def load_quantized(path: str, device: str | torch.device = "cpu") -> dict[str, "QuantizedWeight"]:
    """Reads :func:`save_quantized` output onto ``device`` (a copy: no
    quantization at load)."""
    from safetensors import safe_open

    out: dict[str, dict[str, torch.Tensor]] = {}
    with safe_open(path, framework="pt", device=str(device)) as f:
        if (f.metadata() or {}).get("format") != _FORMAT:
            raise ValueError(f"{path}: not a pageserve_amd quantized-weight file")
        for key in f.keys():
            name, _, field = key.rpartition(".")
            out.setdefault(name, {})[field] = f.get_tensor(key)
    return {name: QuantizedWeight.from_state(st) for name, st in out.items()}


class W8A16Weight(torch.Tensor):
    """The value of ``QuantizedWeight.get()`` on a GPU.

    Shape, dtype and device of the dense weight, but no dense storage.
    ``F.linear(x, w, b)`` with bf16 ``x`` runs the fused W8A16 kernel; every
    other operation (and ``F.linear`` on other activation dtypes) receives the
    dense weight produced by the dequantize kernel, i.e. the reference's
    ``get()`` result.
    """

    _qw: QuantizedWeight

    @staticmethod
    def __new__(cls, qw: QuantizedWeight):
        t = torch.Tensor._make_wrapper_subclass(
            cls, tuple(qw.shape), dtype=qw.dtype, device=qw.qp.device, requires_grad=False
        )
        t._qw = qw
        return t

    def __repr__(self, *, tensor_contents=None):
        return f"W8A16Weight(shape={tuple(self.shape)}, dtype={self.dtype}, device={self.device})"

    def dense(self) -> torch.Tensor:
        return self._qw.dense()

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func is F.linear:
            x = args[0] if args else kwargs.get("input")
            w = args[1] if len(args) > 1 else kwargs.get("weight")
            b = args[2] if len(args) > 2 else kwargs.get("bias")
            # metadata is read from the plain QuantizedWeight: a property of the
            # subclass itself would re-enter this handler
            # (dtypes are singletons, and device indices compare without
            # building torch.device objects: this runs once per projection)
            if (type(w) is W8A16Weight and type(x) is torch.Tensor
                    and (b is None or type(b) is torch.Tensor)
                    and w._qw.dtype is torch.bfloat16 and x.dtype is torch.bfloat16
                    and x.get_device() == w._qw.qp.get_device()):
                return w._qw.linear(x, b)
        # everything else keeps torch's own behaviour: metadata reads use the
        # wrapper's shape/dtype/device, and compute reaches __torch_dispatch__,
        # which hands the op the dense weight
        with torch._C.DisableTorchFunctionSubclass():
            return func(*args, **kwargs)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        args, kwargs = _densify((args, kwargs or {}))
        return func(*args, **kwargs)


def _densify(obj):
    if isinstance(obj, W8A16Weight):
        return obj._qw.dense()
    if isinstance(obj, tuple):
        return tuple(_densify(o) for o in obj)
    if isinstance(obj, list):
        return [_densify(o) for o in obj]
    if isinstance(obj, dict):
        return {k: _densify(v) for k, v in obj.items()}
    return obj
