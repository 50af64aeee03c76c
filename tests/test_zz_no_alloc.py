"""pgs_w8a16_linear_noalloc, the entry point that allocates nothing: called
through the C ABI, its outputs equal pgs_w8a16_linear's (same launch plan,
the workspace taken from the library's fixed device array instead of the
caller) bit for bit, on two calls in a row, the second with a smaller input,
for plans that use the scratch (split-K partials, pair slots) and one that
does not; a call whose plan needs more than the array holds is rejected."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import activations, bf16_gpu, report, to_np, weights
from oracle import quantization_oracle as O
from pageserve_amd import _native
from pageserve_amd import quantization as Q

pytestmark = pytest.mark.gpu

VP = ctypes.c_void_p


def _noalloc(lib):
    return lib.pgs_w8a16_linear_noalloc  # typed by the binding (pageserve_amd._native)


def _ptr(t):
    return VP(t.data_ptr()) if t is not None else None


def _reference_call(lib, x, qp, sc, b, y, m, n, k, stream):
    """pgs_w8a16_linear with a freshly zeroed workspace of the exact size."""
    need = lib.pgs_w8a16_workspace_bytes(m, (ctypes.c_int64 * 1)(n), 1, k, 0)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=x.device) if need else None
    rc = lib.pgs_w8a16_linear(_ptr(x), _ptr(qp), _ptr(sc), _ptr(b), _ptr(y), 1, m, n, k,
                              _ptr(ws) if ws is not None else None, need, VP(stream))
    assert rc == 0, lib.pgs_last_error()
    return need


# (m, n, k): down_proj at 200 tokens (split-K partials, 16.5 MiB) then o_proj
# at 9 tokens (pair slots); down_proj at 5 tokens (pair slots) then 1 token
# (folded, no scratch); a ragged tiled split then a smaller one; down_proj at
# 1920 tokens (128 x 128 tiles split four ways, 60.5 MiB, the largest of the
# model's shapes) then 1280 tokens (the same plan, 40.5 MiB); a narrow short-K
# matrix (32 x 64 tiles, K split 4) then o_proj at 160 tokens (32 x 64, unsplit)
PAIRS = [((200, 2048, 11008), (9, 2048, 2048)), ((5, 2048, 11008), (1, 2048, 11008)),
         ((150, 300, 4160), (40, 200, 4160)), ((1920, 2048, 11008), (1280, 2048, 11008)),
         ((200, 100, 2048), (160, 2048, 2048)),
         # down_proj at 4096 tokens: 128 x 128 tiles, no split, no scratch needed
         ((4096, 2048, 11008), (2304, 2048, 11008))]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_equals_the_workspace_entry_point(gpu, first, second):
    lib = _native.load()
    stream = torch.cuda.current_stream().cuda_stream
    for rep, (m, n, k) in enumerate((first, second)):
        w = weights(900 + n + k, n, k)
        qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
        qp, sc = qw._kernel_operands()
        x = activations(910 + m, m, k)
        b = O.round_to_bf16(np.random.default_rng(920 + n).standard_normal(n).astype(np.float32))
        xt, bt = bf16_gpu(x, gpu), bf16_gpu(b, gpu)
        y_ref = torch.empty((m, n), dtype=torch.bfloat16, device=gpu)
        need = _reference_call(lib, xt, qp, sc, bt, y_ref, m, n, k, stream)
        plan_ref = _native.last_plan()
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=gpu)
        rc = _noalloc(lib)(_ptr(xt), _ptr(qp), _ptr(sc), _ptr(bt), _ptr(y), 1, m, n, k, VP(stream))
        assert rc == 0, lib.pgs_last_error()
        assert _native.last_plan() == plan_ref, (plan_ref, _native.last_plan())
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), f"call {rep} (m={m} n={n} k={k}, scratch {need} B) differs"
        rows = np.arange(m) if m <= 16 else np.linspace(0, m - 1, 16).astype(int)
        q, s = O.quantize_per_channel(w)
        report(to_np(y)[rows], O.linear(x[rows], q, s, b), k, f"noalloc m={m}", acc=O.acc_bound(x[rows], q, s, b))


def test_noalloc_rejects_plans_beyond_its_scratch(gpu):
    lib = _native.load()
    # a shape whose split plan needs more than the fixed 64 MiB
    m, n, k = 192, 10880, 32768  # 255 tiles of 64 x 128, K split 8: 64.25 MiB
    need = lib.pgs_w8a16_workspace_bytes(m, (ctypes.c_int64 * 1)(n), 1, k, 0)
    assert need > (64 << 20), need
    rc = _noalloc(lib)(VP(256), VP(256), VP(256), None, VP(256), 1, m, n, k,
                                      VP(torch.cuda.current_stream().cuda_stream))
    assert rc == 1 and b"maximum" in lib.pgs_last_error()


_CAPTURE_SCRIPT = r"""
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
from helpers import activations, bf16_gpu, weights
from pageserve_amd import _native
from pageserve_amd import quantization as Q
lib = _native.load()
VP = ctypes.c_void_p
dev = torch.device("cuda", 0)
m, n, k = 200, 2048, 11008
qw = Q.QuantizedWeight(torch.from_numpy(weights(931, n, k)).to(dev))
qp, sc = qw._kernel_operands()
x = bf16_gpu(activations(932, m, k), dev)
y_ref = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
need = lib.pgs_w8a16_workspace_bytes(m, (ctypes.c_int64 * 1)(n), 1, k, 0)
assert need > 0
ws = torch.zeros(need, dtype=torch.uint8, device=dev)
st = torch.cuda.current_stream().cuda_stream
assert lib.pgs_w8a16_linear(VP(x.data_ptr()), VP(qp.data_ptr()), VP(sc.data_ptr()), None, VP(y_ref.data_ptr()), 1,
                            m, n, k, VP(ws.data_ptr()), need, VP(st)) == 0
y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=dev)
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    # the first call on this device in this process: takes the scratch
    # address and clears its pair slots inside the capture
    rc = lib.pgs_w8a16_linear_noalloc(VP(x.data_ptr()), VP(qp.data_ptr()), VP(sc.data_ptr()), None,
                                      VP(y.data_ptr()), 1, m, n, k, VP(s.cuda_stream))
assert rc == 0, lib.pgs_last_error()
torch.cuda.current_stream().wait_stream(s)
y_eager = torch.empty_like(y)
for rep in range(4):
    y.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref), f"replay {rep} differs from pgs_w8a16_linear"
    # an eager call in between on the same stream, sharing the scratch
    assert lib.pgs_w8a16_linear_noalloc(VP(x.data_ptr()), VP(qp.data_ptr()), VP(sc.data_ptr()), None,
                                        VP(y_eager.data_ptr()), 1, m, n, k, VP(st)) == 0
    torch.cuda.synchronize()
    assert torch.equal(y_eager, y_ref), f"eager call {rep} differs"
print("capture ok")
"""


def test_noalloc_first_call_inside_a_graph_capture(gpu):
    """In a fresh process, the first call of the entry point is made inside
    a HIP graph capture (split-K plan): the scratch address is taken and the
    pair slots cleared during the capture; every replay, with eager calls on
    the same stream between replays, equals pgs_w8a16_linear bit for bit."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parent.parent)
    res = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, root], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and "capture ok" in res.stdout, res.stdout[-2000:] + res.stderr[-2000:]
