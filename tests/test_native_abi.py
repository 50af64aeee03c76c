"""The C-ABI library: loads, exports exactly what include/pageserve_amd.h
declares, and rejects bad arguments before touching a GPU (CPU-only)."""

from __future__ import annotations

import ctypes
import subprocess

import pytest

from pageserve_amd import _native


def test_header_declares_the_bound_symbols():
    assert sorted(_native.SIGNATURES) == _native.header_symbols()


def test_library_exports_every_header_symbol(native_lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    exported = {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}
    for name in _native.header_symbols():
        assert name in exported, f"{name} declared in the header but not exported"
        assert hasattr(native_lib, name)


def test_abi_version_and_error_strings(native_lib):
    assert native_lib.pgs_abi_version() == _native.ABI_VERSION
    assert native_lib.pgs_error_string(0) == b"ok"
    for code in (1, 2, 3, 4):
        assert native_lib.pgs_error_string(code) not in (b"ok", b"unknown error")
    assert native_lib.pgs_error_string(99) == b"unknown error"


@pytest.mark.parametrize(
    "call, needle",
    [
        (lambda L: L.pgs_quantize_per_channel(None, 0, -1, 4, None, None, None), b"negative size"),
        (lambda L: L.pgs_quantize_per_channel(None, 7, 4, 4, None, None, None), b"dtype"),
        (lambda L: L.pgs_quantize_per_channel(None, 0, 4, 4, None, None, None), b"null pointer"),
        (lambda L: L.pgs_dequantize(None, None, 2, -3, None, 0, None), b"negative size"),
        (lambda L: L.pgs_dequantize(ctypes.c_void_p(16), ctypes.c_void_p(16), 2, 16, ctypes.c_void_p(16), 9, None),
         b"dtype"),
        (lambda L: L.pgs_w8a16_linear(None, None, None, None, None, 1, 1, 4, 8, None, 0, None), b"multiple of 16"),
        (lambda L: L.pgs_w8a16_linear(ctypes.c_void_p(8), None, None, None, None, 1, 1, 4, 16, None, 0, None),
         b"aligned"),
        (lambda L: L.pgs_w8a16_linear(ctypes.c_void_p(16), None, None, None, None, 5, 1, 4, 16, None, 0, None),
         b"dtype"),
        (lambda L: L.pgs_w8a16_linear_group(ctypes.c_void_p(16), None, 0, 1, 1, 16, None, 0, None), b"n_outs"),
        (lambda L: L.pgs_w8a16_swiglu(None, None, None, None, None, None, -1, 4, 16, None, 0, None),
         b"negative size"),
        (lambda L: L.pgs_pack_weight(None, 4, 64, None, None), b"null pointer"),
        (lambda L: L.pgs_unpack_weight(ctypes.c_void_p(8), 4, 64, ctypes.c_void_p(16), None), b"aligned"),
        (lambda L: L.pgs_dequantize_packed(None, None, -1, 64, None, 0, None), b"negative size"),
        (lambda L: L.pgs_quantize_per_channel_packed(None, 3, 4, 64, None, None, None), b"dtype"),
        (lambda L: L.pgs_w8a16_rmsnorm_linear_group(None, None, 1e-6, None, 1, 1, 1, 64, None, 0, None),
         b"null norm weight"),
        (lambda L: L.pgs_w8a16_rmsnorm_linear_group(None, ctypes.c_void_p(17), 1e-6, None, 1, 1, 1, 64, None, 0,
                                                    None), b"norm weight misaligned"),
        (lambda L: L.pgs_w8a16_rmsnorm_swiglu(None, ctypes.c_void_p(16), -1.0, None, None, None, None, None, 1, 16,
                                              64, None, 0, None), b"eps"),
        (lambda L: L.pgs_w8a16_rmsnorm_swiglu(None, ctypes.c_void_p(16), float("nan"), None, None, None, None, None,
                                              1, 16, 64, None, 0, None), b"eps"),
        (lambda L: L.pgs_w8a16_rmsnorm_linear_group(ctypes.c_void_p(16), ctypes.c_void_p(16), 1e-6, None, 0, 1, 1,
                                                    64, None, 0, None), b"n_outs"),
    ],
)
def test_bad_arguments_are_rejected_without_launching(native_lib, call, needle):
    rc = call(native_lib)
    assert rc in (1, 2)
    assert needle in native_lib.pgs_last_error()


def test_empty_problems_are_no_ops(native_lib):
    # m == 0 or n == 0: nothing to compute, success, nothing launched
    assert native_lib.pgs_w8a16_linear(ctypes.c_void_p(256), None, None, None, None, 1, 0, 8, 64, None, 0,
                                       None) == 0
    assert native_lib.pgs_quantize_per_channel(None, 0, 0, 64, None, None, None) == 0
    assert native_lib.pgs_dequantize(None, None, 0, 64, None, 0, None) == 0


def test_check_raises_with_library_message(native_lib):
    rc = native_lib.pgs_w8a16_linear(None, None, None, None, None, 1, 1, 4, 8, None, 0, None)
    with pytest.raises(ValueError, match="multiple of 16"):
        _native.check(rc, "w8a16 linear")


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_native.NativeLibraryError, match="not found"):
        _native.load(tmp_path / "nope.so")


def test_workspace_query(native_lib):
    """Short-N shapes at 9..16 tokens split K and need a workspace; at up
    to 8 tokens they fold (no workspace), and wide ones do not split."""
    def need(m, ns, k, swiglu=0):
        arr = (ctypes.c_int64 * len(ns))(*ns)
        return native_lib.pgs_w8a16_workspace_bytes(m, arr, len(ns), k, swiglu)

    assert need(16, [2048], 11008) > 0                          # down_proj at 16 tokens: K split
    assert need(1, [2048], 11008) == 0                          # down_proj at 1 token: folded
    assert need(1, [151936], 2048) == 0                         # lm_head: plenty of tiles
    assert need(0, [2048], 2048) == 0 and need(1, [2048], -5) == 0
    assert need(1, [0], 2048) == 0
    assert need(12, [1024, 256, 256], 2048) >= need(12, [2048], 2048) > 0   # o / a small q|k|v group
    assert need(8, [1024, 256, 256], 2048) == 0                 # folded
    # 17..32 tokens: two 16-token blocks per tile (pair slots for 128 tiles;
    # partials of 16 x 32 outputs per tile and matrix for the SwiGLU pair)
    assert need(32, [2048], 11008) == 256 * 256 * 8
    assert need(24, [1000], 8192, 1) == 256 * 256 * 8 + 63 * 2 * 2 * 512 * 4
    assert need(16, [1000], 8192, 1) == 256 * 256 * 8 + 63 * 2 * 2 * 256 * 4


def test_tiled_plan_splits(native_lib):
    """The tiled GEMM planner's K splits, read through the workspace query:
    512 KiB of pair slots plus tiles x splits x matrices x tile bytes (fp32),
    or 0 when nothing is split."""
    def need(m, ns, k, swiglu=0):
        arr = (ctypes.c_int64 * len(ns))(*ns)
        return native_lib.pgs_w8a16_workspace_bytes(m, arr, len(ns), k, swiglu)

    slots = 256 * 256 * 8

    def split(tiles, splits, bm, bn, nmat=1):
        return slots + tiles * splits * nmat * bm * bn * 4

    # 33..128 tokens, long K: 64 x 64 tiles split until one workgroup per CU (at most 8)
    assert need(64, [2048], 11008) == split(32, 8, 64, 64)
    assert need(40, [300], 8192) == split(5, 8, 64, 64)
    assert need(128, [2048], 11008) == split(64, 4, 64, 64)
    # above 256 tokens, long K: 128 x 128 tiles split until 512 workgroups (at most 8)
    assert need(384, [2048], 11008) == split(48, 8, 128, 128)
    assert need(512, [2048], 11008) == split(64, 8, 128, 128)
    assert need(1024, [2048], 11008) == split(128, 4, 128, 128)
    assert need(1920, [2048], 11008) == split(240, 4, 128, 128)   # 60.5 MiB, the model's largest
    assert need(2048, [2048], 11008) == split(256, 2, 128, 128)
    # 129..256 tokens, long K: 64 x 128 tiles, split while under 1024 units
    assert need(256, [2048], 11008) == split(64, 8, 64, 128)
    # short K above 128 tokens: 32 x 64 tiles, split only when very few
    assert need(512, [2048], 2048) == 0 and need(160, [2048, 256, 256], 2048) == 0
    assert need(200, [100], 2048) == split(14, 4, 32, 64)
    # the SwiGLU pair at these sizes never splits
    assert need(128, [11008], 2048, 1) == 0 and need(512, [11008], 2048, 1) == 0


def test_rmsnorm_workspace_query(native_lib):
    """The fused-norm calls need room for h = rms_norm(x) (m x k bf16) past
    the linear's own workspace, for the cases that cannot normalise inside
    the projection kernel."""
    def need(fn, m, ns, k, swiglu=0):
        arr = (ctypes.c_int64 * len(ns))(*ns)
        return fn(m, arr, len(ns), k, swiglu)

    for m, ns, k, sw in [(1, [2048, 256, 256], 2048, 0), (16, [2048], 11008, 0), (512, [11008], 2048, 1),
                         (3, [1104], 640, 0)]:
        base = need(native_lib.pgs_w8a16_workspace_bytes, m, ns, k, sw)
        fused = need(native_lib.pgs_w8a16_rmsnorm_workspace_bytes, m, ns, k, sw)
        # h lies past the linear's workspace and past the pair slots (256 x 256 x 8 bytes at its start)
        assert fused - m * k * 2 >= max(base, 256 * 256 * 8) and fused - m * k * 2 < max(base, 256 * 256 * 8) + 256
    assert need(native_lib.pgs_w8a16_rmsnorm_workspace_bytes, 0, [2048], 2048) == 0


@pytest.mark.parametrize("n,k,expect", [(16, 64, 1024), (17, 64, 2048), (16, 65, 2048), (0, 64, 0), (2048, 11008,
                                                                                                    2048 * 11008),
                                        (-1, 4, -1)])
def test_packed_bytes(native_lib, n, k, expect):
    assert native_lib.pgs_packed_bytes(n, k) == expect


def _has_gpu() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.mark.parametrize(
    "call",
    [
        lambda L: L.pgs_rmsnorm(ctypes.c_void_p(256), ctypes.c_void_p(256), 1e-6, ctypes.c_void_p(512), 1, 16, None),
        lambda L: L.pgs_w8a16_linear(ctypes.c_void_p(256), ctypes.c_void_p(256), ctypes.c_void_p(256), None,
                                     ctypes.c_void_p(256), 1, 1, 16, 64, None, 0, None),
        lambda L: L.pgs_quantize_per_channel(ctypes.c_void_p(256), 0, 4, 64, ctypes.c_void_p(256),
                                             ctypes.c_void_p(256), None),
        lambda L: L.pgs_pack_weight(ctypes.c_void_p(256), 4, 64, ctypes.c_void_p(256), None),
    ],
)
def test_no_device_is_an_error_not_a_launch(native_lib, call):
    """Well-formed calls on a machine without a (gfx950) device return
    PGS_ERR_NO_DEVICE before launching anything."""
    if _has_gpu():
        pytest.skip("a GPU is visible: the device check passes there")
    assert call(native_lib) == 4
    assert b"device" in native_lib.pgs_last_error()


def test_last_plan_is_empty_before_any_launch(native_lib):
    import threading

    seen = []
    t = threading.Thread(target=lambda: seen.append(native_lib.pgs_last_plan()))
    t.start()
    t.join()
    assert seen == [b""]


def test_capture_state_arguments(native_lib):
    assert native_lib.pgs_stream_capture_state(None, None, None) == 1
    cap, cid = ctypes.c_int(7), ctypes.c_ulonglong(7)
    rc = native_lib.pgs_stream_capture_state(None, ctypes.byref(cap), ctypes.byref(cid))
    if rc == 0:
        assert (cap.value, cid.value) == (0, 0)  # the null stream is not capturing
    else:
        assert rc == 4 and not _has_gpu()


def test_host_module_loads_and_matches_the_abi(native_lib):
    """The C++ host module (the eager fast path of linear / linear_group /
    swiglu) loads on a machine without a GPU and is bound to this ABI."""
    host = _native.load_host()
    assert host.abi_version() == _native.ABI_VERSION
    assert callable(host.linear) and callable(host.swiglu)


def test_span_configurations_and_default(native_lib):
    """The persistent decode span is compiled for the Qwen2.5-3B shapes at 1..4
    tokens (its workspace is sized for them) and is the default path of
    decode_span at one and two tokens only; other sizes run the
    per-projection kernels."""
    from pageserve_amd import span as S

    qwen = (2048, 11008, 2048, 256, 128)
    for m in range(0, 7):
        assert S.span_supported(m, *qwen) == (1 <= m <= 4), m
        assert S.span_default(m, *qwen) == (1 <= m <= 2), m
    assert not S.span_supported(1, 2048, 11008, 2048, 256, 64)
    assert not S.span_supported(1, 4096, 11008, 2048, 256, 128)
    ws = native_lib.pgs_w8a16_decode_span_workspace_bytes
    assert ws(1, 2048, 11008) == ws(4, 2048, 11008) > 0
    assert ws(5, 2048, 11008) == 0 and ws(0, 2048, 11008) == 0
