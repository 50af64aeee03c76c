"""ctypes binding of the gfx950 C-ABI library (``include/pageserve_amd.h``).

The library is built in-tree by ``pageserve_amd.build`` into
``pageserve_amd/_lib/libpageserve_amd.so``.  Nothing here falls back to
another implementation: if the library is missing or cannot be loaded, every
entry point raises :class:`NativeLibraryError`.
"""

from __future__ import annotations

import ctypes
import os
import re
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("PAGESERVE_AMD_LIB", Path(__file__).resolve().parent / "_lib" / "libpageserve_amd.so"))
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "pageserve_amd.h"

# element type codes and return codes (include/pageserve_amd.h)
DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
OK = 0
MAX_GROUP = 4
ABI_VERSION = 10
ERR_TIMEOUT = 5


class NativeLibraryError(RuntimeError):
    """The gfx950 library is missing, stale or failed a call."""


class DeviceWaitTimeout(NativeLibraryError):
    """A bounded wait inside a persistent launch gave up (PGS_ERR_TIMEOUT)."""


class LinearOut(ctypes.Structure):
    """``pgs_linear_out`` of include/pageserve_amd.h."""

    _fields_ = [
        ("qp", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("n", ctypes.c_int64),
    ]


class SpanWeights(ctypes.Structure):
    """``pgs_span_weights`` of include/pageserve_amd.h."""

    _fields_ = [
        ("qp_o", ctypes.c_void_p), ("s_o", ctypes.c_void_p),
        ("ln_post", ctypes.c_void_p),
        ("qp_gate", ctypes.c_void_p), ("s_gate", ctypes.c_void_p),
        ("qp_up", ctypes.c_void_p), ("s_up", ctypes.c_void_p),
        ("qp_down", ctypes.c_void_p), ("s_down", ctypes.c_void_p),
    ]


class SpanNext(ctypes.Structure):
    """``pgs_span_next`` of include/pageserve_amd.h."""

    _fields_ = [
        ("ln_in", ctypes.c_void_p),
        ("q", LinearOut), ("k", LinearOut), ("v", LinearOut),
        ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
        ("head_dim", ctypes.c_int64),
    ]


_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); every symbol the header declares
SIGNATURES = {
    "pgs_abi_version": (_INT, []),
    "pgs_error_string": (ctypes.c_char_p, [_INT]),
    "pgs_last_error": (ctypes.c_char_p, []),
    "pgs_last_plan": (ctypes.c_char_p, []),
    "pgs_stream_capture_state": (_INT, [_VP, ctypes.POINTER(_INT), ctypes.POINTER(ctypes.c_ulonglong)]),
    "pgs_quantize_per_channel": (_INT, [_VP, _INT, _I64, _I64, _VP, _VP, _VP]),
    "pgs_dequantize": (_INT, [_VP, _VP, _I64, _I64, _VP, _INT, _VP]),
    "pgs_quantize_per_channel_packed": (_INT, [_VP, _INT, _I64, _I64, _VP, _VP, _VP]),
    "pgs_packed_bytes": (_I64, [_I64, _I64]),
    "pgs_pack_weight": (_INT, [_VP, _I64, _I64, _VP, _VP]),
    "pgs_unpack_weight": (_INT, [_VP, _I64, _I64, _VP, _VP]),
    "pgs_dequantize_packed": (_INT, [_VP, _VP, _I64, _I64, _VP, _INT, _VP]),
    "pgs_w8a16_linear": (_INT, [_VP, _VP, _VP, _VP, _VP, _INT, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "pgs_w8a16_linear_noalloc": (_INT, [_VP, _VP, _VP, _VP, _VP, _INT, _I64, _I64, _I64, _VP]),
    "pgs_w8a16_linear_group": (_INT, [_VP, ctypes.POINTER(LinearOut), _INT, _INT, _I64, _I64, _VP, _SZ, _VP]),
    "pgs_w8a16_linear_residual": (_INT, [_VP, _VP, _VP, _VP, _VP, _VP, _INT, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "pgs_rmsnorm": (_INT, [_VP, _VP, ctypes.c_float, _VP, _I64, _I64, _VP]),
    "pgs_rope": (_INT, [_VP, _VP, _I64, _VP, _VP, _I64, _VP, _VP, _I64, _I64, _VP]),
    "pgs_w8a16_swiglu": (_INT, [_VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "pgs_w8a16_workspace_bytes": (_SZ, [_I64, ctypes.POINTER(_I64), _INT, _I64, _INT]),
    "pgs_w8a16_rmsnorm_linear_group": (_INT, [_VP, _VP, ctypes.c_float, ctypes.POINTER(LinearOut), _INT, _INT,
                                              _I64, _I64, _VP, _SZ, _VP]),
    "pgs_w8a16_rmsnorm_swiglu": (_INT, [_VP, _VP, ctypes.c_float, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _VP,
                                        _SZ, _VP]),
    "pgs_w8a16_rmsnorm_workspace_bytes": (_SZ, [_I64, ctypes.POINTER(_I64), _INT, _I64, _INT]),
    "pgs_w8a16_linear_argmax": (_INT, [_VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "pgs_w8a16_argmax_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "pgs_w8a16_decode_span": (_INT, [_VP, _VP, _VP, ctypes.POINTER(SpanWeights), ctypes.POINTER(SpanNext),
                                     ctypes.c_float, _I64, _I64, _I64, _VP, _SZ, _VP]),
    "pgs_w8a16_decode_span_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "pgs_w8a16_decode_span_supported": (_INT, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "pgs_w8a16_decode_span_status": (_INT, [_VP, _INT, _VP]),
    "pgs_w8a16_decode_span_test_hooks": (_INT, [_INT, _INT]),
    "pgs_w8a16_decode_span_trace": (_INT, [_VP, _SZ]),
}

_lock = threading.Lock()
_lib = None


def header_symbols(path: Path = HEADER_PATH) -> list[str]:
    """Function names declared in the public header."""
    text = path.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pgs_[a-z0-9_]+)\s*\(", text)))


def load(path: Path | None = None) -> ctypes.CDLL:
    """Loads (once) and returns the library with typed entry points."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        # torch first: its HIP runtime (soname libamdhip64.so.7) is then the
        # one the library binds to, so streams and pointers from torch are
        # valid handles for the library's launches
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not p.exists():
            raise NativeLibraryError(
                f"pageserve_amd: gfx950 library not found at {p}; build it with "
                "`python -m pageserve_amd.build` (there is no fallback implementation)"
            )
        try:
            # global: the C++ host module (_pgs_host) links against this
            # library and binds to the copy loaded here
            lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_GLOBAL)
        except OSError as e:
            raise NativeLibraryError(f"pageserve_amd: cannot load {p}: {e}") from e
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.pgs_abi_version()
        if ver != ABI_VERSION:
            raise NativeLibraryError(f"pageserve_amd: library ABI {ver} != expected {ABI_VERSION}; rebuild it")
        if path is None:
            _lib = lib
        return lib


_host = None


def load_host():
    """The C++ host module (``_lib/_pgs_host*.so``, built by
    ``pageserve_amd.build``): the argument checks, output allocation and
    C-ABI call of the linear entry points without Python per-call overhead.
    Loaded once, after the library it calls."""
    global _host
    if _host is not None:
        return _host
    load()
    import importlib.machinery
    import importlib.util

    cands = sorted(LIB_PATH.parent.glob("_pgs_host*.so"))
    if not cands:
        raise NativeLibraryError(f"pageserve_amd: C++ host module not found in {LIB_PATH.parent}; build it with "
                                 "`python -m pageserve_amd.build`")
    loader = importlib.machinery.ExtensionFileLoader("_pgs_host", str(cands[0]))
    spec = importlib.util.spec_from_file_location("_pgs_host", str(cands[0]), loader=loader)
    try:
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
    except ImportError as e:
        raise NativeLibraryError(f"pageserve_amd: cannot load the C++ host module {cands[0]}: {e}") from e
    if mod.abi_version() != ABI_VERSION:
        raise NativeLibraryError(f"pageserve_amd: host module bound to ABI {mod.abi_version()} != {ABI_VERSION}")
    _host = mod
    return mod


def last_plan() -> str:
    """Kernel instance, grid and K split of this thread's last linear launch."""
    return load().pgs_last_plan().decode(errors="replace")


def capture_state(stream: int) -> tuple[int, int]:
    """(capturing, capture id) of a raw hipStream_t (0, 0 when not capturing)."""
    lib = load()
    cap, cid = _INT(0), ctypes.c_ulonglong(0)
    rc = lib.pgs_stream_capture_state(ctypes.c_void_p(stream), ctypes.byref(cap), ctypes.byref(cid))
    check(rc, "stream capture state")
    return cap.value, cid.value


def check(rc: int, what: str) -> None:
    """Raises on a non-zero return code, with the library's own message."""
    if rc == OK:
        return
    lib = load()
    detail = lib.pgs_last_error().decode(errors="replace")
    kind = lib.pgs_error_string(rc).decode(errors="replace")
    exc = ValueError if rc in (1, 2) else DeviceWaitTimeout if rc == ERR_TIMEOUT else NativeLibraryError
    raise exc(f"{what}: {kind}: {detail}")
