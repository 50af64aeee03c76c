"""W8A16 linear kernels against the fp32 dequant+matmul oracle.

engine/model.py:168-170 (q/k/v, with bias), :184 (o), :188-190 (gate/up/down)
and :193 (lm_head, fp32 logits).  Tolerance from the path's specification:
max|y - y_ref| / max|y_ref| <= 1e-2 and max|y - y_ref| <= 2e-2 * sqrt(K/1024),
with y_ref = x . fp32(q * scale)^T (+ b) summed in float64 (oracle.linear).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import activations, bf16_gpu, report, to_np, weights
from oracle import quantization_oracle as O
from pageserve_amd import quantization as Q

pytestmark = pytest.mark.gpu


def _problem(gpu, seed, m, n, k, bias=False):
    w = weights(seed, n, k)
    x = activations(seed + 1, m, k)
    b = O.round_to_bf16(np.random.default_rng(seed + 2).standard_normal(n).astype(np.float32)) if bias else None
    qw = Q.QuantizedWeight(torch.from_numpy(w).to(gpu))
    q, s = O.quantize_per_channel(w)
    return qw, q, s, x, b


# decode (skinny kernel, m <= 32) and prefill (tile kernel) shapes, including
# ragged n (not a multiple of 16 / 128) and k not a multiple of 64
SHAPES = [
    (1, 2048, 2048), (1, 256, 2048), (1, 11008, 2048), (1, 2048, 11008),
    (4, 2048, 2048), (4, 11008, 2048), (16, 2048, 11008), (16, 256, 2048),
    (2, 100, 80), (3, 1, 16), (5, 17, 48), (7, 4864, 896), (15, 130, 1040), (1, 33, 112),
    (17, 64, 64), (31, 300, 208), (64, 2048, 2048), (100, 1000, 336), (127, 129, 2048),
    (128, 2048, 2048), (129, 256, 2048), (256, 11008, 2048), (512, 2048, 2048), (512, 2048, 11008),
    (300, 2560, 2048),
    # K below one 64-column block and K tails on the tiled path; a split-K
    # plan (few tiles, long K) whose last block is partial
    (20, 48, 16), (33, 130, 32), (40, 96, 48), (40, 256, 4112), (70, 2048, 11024),
    # 33..128 tokens, K % 64 == 0: 64-row tiles in four K groups (long K also
    # split: 4 ways over 64 tiles, 8 ways over 32 or fewer)
    (70, 2048, 11008), (128, 2048, 11008), (96, 2560, 2048), (17, 300, 128), (64, 2048, 11008),
    (40, 300, 8192),
    # 33..128 tokens, K <= 2048: one-shot 16-token tiles of 64 / 32 / 16 rows,
    # ragged M and N, a one-chunk K, a K shorter than the tile holds
    (48, 2560, 2048), (40, 1000, 1024), (100, 300, 2048), (128, 64, 64), (33, 4000, 512),
    # folded decode (8-row halves of a tile, two K chunks per MFMA, m <= 8):
    # 2m = 16 columns, an odd chunk count with a K tail, 6 tokens
    (3, 2048, 11008), (8, 130, 1040), (6, 48, 1104), (2, 2560, 2048),
    # past the fold (paired K split): 8 tokens with a long K
    (8, 2048, 11008),
    # one to four tokens, folded, activations staged through LDS: odd chunk counts
    (1, 2048, 1088), (1, 300, 4160), (2, 2048, 1088), (4, 300, 4160), (3, 130, 2112),
    # 17..32 tokens, two token blocks: paired o and down_proj (looping), wide
    # unsplit, K tails, a long K over few tiles
    (17, 2048, 2048), (24, 2048, 11008), (32, 11008, 2048), (32, 2048, 2048), (25, 1000, 1040),
    (30, 130, 4160), (19, 4864, 896),
    # folded wide matrices (>= 256 row tiles, up to 2 tokens, short K)
    (2, 5000, 2048), (1, 8192, 1024),
    # unfolded single matrices at 3..8 tokens, activations staged (4 / 8 tokens):
    # wide, 129..255 tiles, paired K halves, a long K over few tiles, 16-wave shapes
    (3, 4096, 1024), (5, 4096, 2048), (8, 2560, 1024), (6, 2048, 11008), (7, 300, 8192),
    # unfolded single matrices at 9..16 tokens, activations staged one batch at a
    # time: unsplit (q|k|v-, gate-like, wide), paired halves (o, down_proj), an odd
    # chunk count over paired halves
    (16, 2560, 2048), (16, 11008, 2048), (10, 4096, 1024), (12, 2048, 2048), (9, 2048, 11008),
    (13, 300, 4160),
    (4, 5000, 4096), (8, 9000, 3072),
]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_linear_matches_oracle(gpu, m, n, k):
    qw, q, s, x, _ = _problem(gpu, 100 + m + n + k, m, n, k)
    y = qw.linear(bf16_gpu(x, gpu))
    assert y.dtype == torch.bfloat16 and y.shape == (m, n)
    report(to_np(y), O.linear(x, q, s), k, f"linear m={m} n={n} k={k}", acc=O.acc_bound(x, q, s))


@pytest.mark.parametrize("m", [1, 3, 16, 24, 40, 256])
def test_linear_with_bias(gpu, m):
    qw, q, s, x, b = _problem(gpu, 7 + m, m, 2048, 2048, bias=True)
    y = qw.linear(bf16_gpu(x, gpu), bf16_gpu(b, gpu))
    report(to_np(y), O.linear(x, q, s, b), 2048, f"linear+bias m={m}", acc=O.acc_bound(x, q, s, b))


@pytest.mark.parametrize("m", [1, 8, 20, 32, 256])
def test_fp32_output(gpu, m):
    qw, q, s, x, _ = _problem(gpu, 50 + m, m, 1536, 2048)
    y = qw.linear(bf16_gpu(x, gpu), out_dtype=torch.float32)
    assert y.dtype == torch.float32
    r = report(to_np(y), O.linear(x, q, s), 2048, f"fp32 out m={m}", bf16_out=False)
    # fp32 output carries no bf16 rounding: far inside the bound
    assert r["rel"] < 1e-4


@pytest.mark.parametrize("m", [1, 5, 16, 24, 32, 48, 64, 96, 128, 160, 512, 800])
def test_grouped_qkv_matches_separate_calls(gpu, m):
    """q/k/v (engine/model.py:168-170) in one launch: each output matches the
    oracle and its single-weight launch within tolerance.  (Not bit for bit:
    the K-split plan depends on the launch's total tile count, so a member
    can be summed in a different order in the group than on its own.)"""
    k = 2048
    x = activations(7000 + m, m, k)  # seeds distinct from the weights
    xs = bf16_gpu(x, gpu)
    ws, qs, ss, bs = [], [], [], []
    for j, n in enumerate((2048, 256, 256)):
        w = weights(901 + j, n, k)
        ws.append(Q.QuantizedWeight(torch.from_numpy(w).to(gpu)))
        q, s = O.quantize_per_channel(w)
        qs.append(q)
        ss.append(s)
        bs.append(O.round_to_bf16(np.random.default_rng(950 + j).standard_normal(n).astype(np.float32)))
    bt = [bf16_gpu(b, gpu) for b in bs]
    outs = Q.linear_group(xs, ws, bt)
    for j in range(3):
        single = ws[j].linear(xs, bt[j])
        report(to_np(outs[j]), O.linear(x, qs[j], ss[j], bs[j]), k, f"qkv[{j}] m={m}", acc=O.acc_bound(x, qs[j], ss[j], bs[j]))
        # two correctly rounded results of the same value in different
        # summation orders: within one ulp plus both accumulation bounds
        report(to_np(outs[j]), to_np(single), k, f"qkv[{j}] m={m} group vs single",
               acc=0.5 * O.bf16_ulp(to_np(single)) + 2 * O.acc_bound(x, qs[j], ss[j], bs[j]))


def test_leading_dims_and_noncontiguous_input(gpu):
    qw, q, s, x, _ = _problem(gpu, 3, 6, 512, 256)
    xt = bf16_gpu(x, gpu).reshape(2, 3, 256)
    y = qw.linear(xt)
    assert y.shape == (2, 3, 512)
    report(to_np(y.reshape(6, 512)), O.linear(x, q, s), 256, "3-D input", acc=O.acc_bound(x, q, s))
    # a transposed view: the wrapper copies it to a contiguous buffer
    xT = bf16_gpu(np.ascontiguousarray(x.T), gpu).t()
    report(to_np(qw.linear(xT)), O.linear(x, q, s), 256, "non-contiguous input", acc=O.acc_bound(x, q, s))


def test_leading_dims_through_group_and_swiglu(gpu):
    """A 3-D input, a 1-D input and a [1, n] bias through the group and
    SwiGLU calls: outputs keep the input's leading dims and equal the 2-D
    calls bit for bit (same launch plan), and a group's members are separate
    tensors with their own storage offsets in one allocation."""
    k = 256
    x = activations(7801, 6, k)
    x2 = bf16_gpu(x, gpu)
    ws = [Q.QuantizedWeight(torch.from_numpy(weights(7802 + j, n, k)).to(gpu)) for j, n in enumerate((96, 40, 40))]
    bs = [bf16_gpu(O.round_to_bf16(np.random.default_rng(7810 + j).standard_normal(n).astype(np.float32)), gpu)
          for j, n in enumerate((96, 40, 40))]
    flat = Q.linear_group(x2, ws, bs)
    three = Q.linear_group(x2.reshape(2, 3, k), ws, [bs[0].reshape(1, 96), bs[1], bs[2]])
    for j, (a, b) in enumerate(zip(flat, three)):
        assert b.shape == (2, 3, a.shape[1]) and torch.equal(a, b.reshape(a.shape)), j
        assert a.is_contiguous() and a.data_ptr() % 128 == 0, j
    assert flat[0].data_ptr() != flat[1].data_ptr() != flat[2].data_ptr()
    one = Q.linear_group(x2[0], ws, bs)
    for a, b in zip(flat, one):
        assert b.shape == (a.shape[1],) and torch.equal(a[0], b)
    g, u = (Q.QuantizedWeight(torch.from_numpy(weights(7820 + j, 200, k)).to(gpu)) for j in range(2))
    act = Q.swiglu(x2, g, u)
    assert torch.equal(Q.swiglu(x2.reshape(2, 3, k), g, u), act.reshape(2, 3, 200))
    assert torch.equal(Q.swiglu(x2[0], g, u), act[0])


def test_full_size_prefill_sampled(gpu):
    """m = 2048 (the largest prefill chunk) on gate_proj's shape: every output
    row and column block checked on a random sample against the oracle."""
    m, n, k = 2048, 11008, 2048
    qw, q, s, x, _ = _problem(gpu, 4242, m, n, k)
    y = to_np(qw.linear(bf16_gpu(x, gpu)))
    rng = np.random.default_rng(1)
    rows = rng.choice(m, 96, replace=False)
    cols = rng.choice(n, 512, replace=False)
    ref = O.linear(x[rows], q[cols], s[cols])
    report(y[np.ix_(rows, cols)], ref, k, "m=2048 sample", acc=O.acc_bound(x[rows], q[cols], s[cols]))
    assert np.isfinite(y).all()


def test_wide_matrix_128_token_tiles_sampled(gpu):
    """A single matrix with very many 128-token tiles (as lm_head at 256
    tokens) runs 128 x 128 tiles: ragged last token and row tiles, bias, bf16
    output; a random sample of rows and columns against the oracle."""
    m, n, k = 300, 87500, 512
    qw, q, s, x, b = _problem(gpu, 5151, m, n, k, bias=True)
    y = to_np(qw.linear(bf16_gpu(x, gpu), bf16_gpu(b, gpu)))
    rng = np.random.default_rng(2)
    rows = np.concatenate([rng.choice(m, 60, replace=False), [0, 255, 256, m - 1]])
    cols = np.concatenate([rng.choice(n, 400, replace=False), [0, 127, 128, n - 1]])
    ref = O.linear(x[rows], q[cols], s[cols], b[cols])
    report(y[np.ix_(rows, cols)], ref, k, "128-token tiles sample", acc=O.acc_bound(x[rows], q[cols], s[cols], b[cols]))
    assert np.isfinite(y).all()


def test_paired_split_leaves_the_workspace_clean(gpu):
    """Decode shapes with few row tiles at 9..16 tokens split K in two and
    combine the halves through slots at the front of the shared workspace;
    each call must leave them empty.  Interleave differently shaped paired
    calls (o, down, a ragged one) with folded ones (up to 8 tokens, no
    slots) and repeat: every result must match the oracle."""
    cases = [_problem(gpu, 300 + j, m, n, k) for j, (m, n, k) in
             enumerate([(1, 2048, 2048), (12, 2048, 11008), (9, 1000, 1040), (16, 256, 2048), (1, 33, 1024),
                        (16, 2048, 2048), (3, 1000, 1040), (24, 2048, 11008), (32, 2048, 2048),
                        (17, 1000, 1040)])]
    xs = [bf16_gpu(c[3], gpu) for c in cases]
    refs = [O.linear(c[3], c[1], c[2]) for c in cases]
    accs = [O.acc_bound(c[3], c[1], c[2]) for c in cases]
    for rep in range(3):
        outs = [c[0].linear(x) for c, x in zip(cases, xs)]
        for (qw, q, s, x, _), y, ref, acc in zip(cases, outs, refs, accs):
            report(to_np(y), ref, x.shape[1], f"paired m={x.shape[0]} n={q.shape[0]} k={x.shape[1]} rep={rep}",
                   acc=acc)


@pytest.mark.parametrize("m,n,k", [(3, 1000, 1040), (8, 256, 2048), (16, 256, 2048), (2, 2048, 11008), (5, 17, 48),
                                   (20, 2048, 2048), (32, 256, 2048), (27, 300, 1040), (7, 4864, 896),
                                   (6, 2048, 11008), (4, 4096, 1024), (12, 2048, 2048), (16, 2048, 11008),
                                   (11, 2560, 2048)])
def test_nonfinite_token_stays_in_its_row(gpu, m, n, k):
    """A token whose activations hold inf and nan poisons only its own
    outputs (as in x @ W^T): padding columns and the K range of another
    workgroup or MFMA column must not carry it into the other tokens."""
    qw, q, s, x, _ = _problem(gpu, 90, m, n, k)
    bad = m // 2
    x = x.copy()
    x[bad, :16] = np.inf
    x[bad, -16:] = np.nan
    y = to_np(qw.linear(bf16_gpu(x, gpu)))
    ok = [t for t in range(m) if t != bad]
    assert not np.isfinite(y[bad]).any()
    ref = O.linear(x[ok], q, s)
    report(y[ok], ref, k, f"non-finite token m={m} n={n} k={k}", acc=O.acc_bound(x[ok], q, s))


def test_deterministic(gpu):
    qw, q, s, x, _ = _problem(gpu, 77, 512, 2048, 11008)
    xs = bf16_gpu(x, gpu)
    a = qw.linear(xs)
    b = qw.linear(xs)
    assert torch.equal(a, b)
    qw1, *_ = _problem(gpu, 78, 1, 2048, 11008)
    xs1 = bf16_gpu(activations(5, 1, 11008), gpu)
    assert torch.equal(qw1.linear(xs1), qw1.linear(xs1))


def test_empty_inputs(gpu):
    qw, *_ = _problem(gpu, 1, 4, 64, 64)
    y = qw.linear(torch.zeros((0, 64), dtype=torch.bfloat16, device=gpu))
    assert y.shape == (0, 64)


def test_bad_inputs_raise(gpu):
    qw, *_ = _problem(gpu, 1, 4, 64, 64)
    with pytest.raises(TypeError, match="bf16"):
        qw.linear(torch.zeros((2, 64), dtype=torch.float32, device=gpu))
    with pytest.raises(ValueError, match="features"):
        qw.linear(torch.zeros((2, 32), dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError, match="bias"):
        qw.linear(torch.zeros((2, 64), dtype=torch.bfloat16, device=gpu), torch.zeros(3, dtype=torch.bfloat16,
                                                                                      device=gpu))
    odd = Q.QuantizedWeight(torch.randn(8, 40, device=gpu))
    with pytest.raises(ValueError, match="multiple of 16"):
        odd.linear(torch.zeros((2, 40), dtype=torch.bfloat16, device=gpu))


def test_launch_stream_and_cached_operands(gpu):
    """Launches go to torch's current stream (also a side stream), and the
    cached kernel operands follow a weight whose storage is replaced."""
    from pageserve_amd.quantization import _raw_stream
    assert _raw_stream(gpu) == torch.cuda.current_stream(gpu).cuda_stream
    side = torch.cuda.Stream(device=gpu)
    with torch.cuda.stream(side):
        assert _raw_stream(gpu) == side.cuda_stream
    qw, q, s, x, _ = _problem(gpu, 5, 3, 256, 512)
    xt = bf16_gpu(x, gpu)
    report(to_np(qw.linear(xt)), O.linear(x, q, s), 512, "before", acc=O.acc_bound(x, q, s))
    q2 = np.ascontiguousarray(q[::-1])
    qw.q = torch.from_numpy(q2).to(gpu)
    report(to_np(qw.linear(xt)), O.linear(x, q2, s), 512, "after assigning q", acc=O.acc_bound(x, q2, s))


def test_calls_from_a_worker_thread(gpu):
    """The reference's runner calls forward_step from a daemon thread
    (engine/runner.py:52-84): launches from another thread use that thread's
    current stream, give the same results, and errors stay per thread."""
    import threading

    qw, q, s, x, _ = _problem(gpu, 61, 4, 2048, 2048)
    xt = bf16_gpu(x, gpu)
    main = qw.linear(xt)
    out, errs = {}, []

    def work():
        try:
            side = torch.cuda.Stream(device=gpu)
            with torch.cuda.stream(side):
                y = qw.linear(xt)
                g = Q.swiglu(xt, qw, qw)
            side.synchronize()
            out["y"], out["g"] = y, g
            with pytest.raises(ValueError):
                qw.linear(xt[:, :100])
        except BaseException as e:  # reported in the main thread
            errs.append(e)

    t = threading.Thread(target=work, daemon=True)
    t.start()
    t.join(60)
    assert not t.is_alive() and not errs, errs
    assert torch.equal(out["y"], main)
    assert torch.equal(out["g"], Q.swiglu(xt, qw, qw))


def test_split_plans_from_concurrent_threads(gpu):
    """Four threads, each on its own stream, run K-split plans (each needs a
    workspace: one per stream, made on first use, some grown later) at the
    same time as the main thread: every result equals the single-threaded
    one bit for bit."""
    import threading

    cases = [_problem(gpu, 70 + j, m, n, k) for j, (m, n, k) in
             enumerate([(200, 2048, 11008), (64, 2048, 11008), (12, 2048, 11008), (600, 2048, 11008)])]
    xs = [bf16_gpu(c[3], gpu) for c in cases]
    want = [c[0].linear(x) for c, x in zip(cases, xs)]
    torch.cuda.synchronize()
    got, errs = {}, []
    start = threading.Barrier(5)

    def work(t):
        try:
            side = torch.cuda.Stream(device=gpu)
            start.wait(30)
            with torch.cuda.stream(side):
                for rep in range(6):
                    j = (t + rep) % len(cases)
                    got[(t, rep)] = (j, cases[j][0].linear(xs[j]))
            side.synchronize()
        except BaseException as e:  # reported in the main thread
            errs.append(e)

    threads = [threading.Thread(target=work, args=(t,), daemon=True) for t in range(4)]
    for t in threads:
        t.start()
    start.wait(30)
    main = [c[0].linear(x) for c, x in zip(cases, xs)]
    for t in threads:
        t.join(120)
    torch.cuda.synchronize()
    assert not any(t.is_alive() for t in threads) and not errs, errs
    assert all(torch.equal(a, b) for a, b in zip(main, want))
    assert len(got) == 24
    for (t, rep), (j, y) in got.items():
        assert torch.equal(y, want[j]), (t, rep, j)


def _plan_kernel() -> str:
    from pageserve_amd import _native

    return _native.last_plan()


def test_four_k_group_plan(gpu):
    """The 256-tile, long-K plan (four K groups of four waves per
    workgroup, launch_k64<64, 128, 1, *, 2, 2, 1, 4>): a wide long-K shape at
    256 tokens (256 tiles, no split), and a few-tile long-K shape with a
    workspace (K split 8 plus the reduce kernel) and without one (the C ABI
    with a NULL workspace: no split)."""
    import ctypes

    from pageserve_amd import _native

    kg4 = "BM = 64, BN = 128, NMAT = 1, OUT_F32 = false, WLEAD = 2, XLEAD = 2, OCC = 1, KG = 4"
    m, n, k = 256, 8192, 4160
    qw, q, s, x, _ = _problem(gpu, 7711, m, n, k)
    y = to_np(qw.linear(bf16_gpu(x, gpu)))
    assert kg4 in _plan_kernel() and "splits=1" in _plan_kernel(), _plan_kernel()
    rows = np.concatenate([np.random.default_rng(3).choice(m, 40, replace=False), [0, 63, 64, m - 1]])
    report(y[rows], O.linear(x[rows], q, s), k, "kg4 m=256", acc=O.acc_bound(x[rows], q, s))

    m, n, k = 200, 200, 4160
    qw, q, s, x, b = _problem(gpu, 7712, m, n, k, bias=True)
    xt, bt = bf16_gpu(x, gpu), bf16_gpu(b, gpu)
    y = to_np(qw.linear(xt, bt))
    plan = _plan_kernel()
    assert kg4 in plan and "splits=8" in plan and "gemm_reduce_kernel" in plan, plan
    report(y, O.linear(x, q, s, b), k, "kg4 split", acc=O.acc_bound(x, q, s, b))
    lib = _native.load()
    qp, sc = qw._kernel_operands()
    out = torch.empty((m, n), dtype=torch.bfloat16, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.pgs_w8a16_linear(ctypes.c_void_p(xt.data_ptr()), ctypes.c_void_p(qp.data_ptr()),
                              ctypes.c_void_p(sc.data_ptr()), ctypes.c_void_p(bt.data_ptr()),
                              ctypes.c_void_p(out.data_ptr()), 1, m, n, k, None, 0, ctypes.c_void_p(stream))
    assert rc == 0, lib.pgs_last_error()
    plan = _plan_kernel()
    assert kg4 in plan and "splits=1" in plan, plan
    report(to_np(out), O.linear(x, q, s, b), k, "kg4 no workspace", acc=O.acc_bound(x, q, s, b))


def test_long_k_128_tile_plan(gpu):
    """Above 256 tokens a long K (more than 64 steps of 64) runs 128 x 128
    LDS-DMA tiles with the K split (up to 8 ways) until 512 workgroups
    (launch_dma<128, 128, 1, *, 2, 3, 2> plus the reduce kernel): a ragged
    few-tile shape (eight splits) against the full oracle, down_proj's shape
    at 2048 tokens (two splits) and at 384 (eight) on sampled rows, and the C
    ABI without a workspace, which keeps the unsplit plan."""
    import ctypes

    from pageserve_amd import _native

    t128 = "BM = 128, BN = 128, NMAT = 1, OUT_F32 = false, WLEAD = 2, S = 3, OCC = 2"
    m, n, k = 1536, 300, 4160
    qw, q, s, x, b = _problem(gpu, 7721, m, n, k, bias=True)
    xt, bt = bf16_gpu(x, gpu), bf16_gpu(b, gpu)
    y = to_np(qw.linear(xt, bt))
    plan = _plan_kernel()
    assert t128 in plan and "splits=8" in plan and "gemm_reduce_kernel" in plan, plan
    report(y, O.linear(x, q, s, b), k, "128 tile m=1536", acc=O.acc_bound(x, q, s, b))

    lib = _native.load()
    qp, sc = qw._kernel_operands()
    out = torch.empty((m, n), dtype=torch.bfloat16, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.pgs_w8a16_linear(ctypes.c_void_p(xt.data_ptr()), ctypes.c_void_p(qp.data_ptr()),
                              ctypes.c_void_p(sc.data_ptr()), ctypes.c_void_p(bt.data_ptr()),
                              ctypes.c_void_p(out.data_ptr()), 1, m, n, k, None, 0, ctypes.c_void_p(stream))
    assert rc == 0, lib.pgs_last_error()
    plan = _plan_kernel()
    assert t128 not in plan and "splits=1" in plan, plan
    report(to_np(out), O.linear(x, q, s, b), k, "no workspace m=1536", acc=O.acc_bound(x, q, s, b))

    for m, splits, seed in ((2048, 2, 7731), (384, 8, 7732)):
        n, k = 2048, 11008
        qw, q, s, x, _ = _problem(gpu, seed, m, n, k)
        y = to_np(qw.linear(bf16_gpu(x, gpu)))
        plan = _plan_kernel()
        assert t128 in plan and f"splits={splits}" in plan, plan
        rows = np.concatenate([np.random.default_rng(5).choice(m, 40, replace=False), [0, 127, 128, m - 1]])
        report(y[rows], O.linear(x[rows], q, s), k, f"128 tile m={m}", acc=O.acc_bound(x[rows], q, s))


def test_narrow_tile_plan(gpu):
    """Short-K single matrices above 128 tokens whose 32 x 128 tiles would
    number at most 384 run 32 x 64 tiles in two K groups
    (launch_k64<32, 64, 1, *, 2, 2, 2, 2>): o_proj's shape at 160 tokens (no
    split) against the full oracle, q|k|v's at 512 on sampled rows, a
    ragged narrow matrix whose few tiles split K (reduce kernel of 32 x 64
    tiles) and a ragged K; at 1024 tokens (512 tiles) o_proj keeps the
    32 x 128 plan."""
    narrow = "BM = 32, BN = 64, NMAT = 1, OUT_F32 = false, WLEAD = 2, XLEAD = 2, OCC = 2, KG = 2"
    for m, n, k, seed, split in ((160, 2048, 2048, 7761, False), (200, 100, 2048, 7762, True),
                                 (300, 1000, 1088, 7763, False)):
        qw, q, s, x, b = _problem(gpu, seed, m, n, k, bias=n != 2048)
        y = to_np(qw.linear(bf16_gpu(x, gpu), bf16_gpu(b, gpu) if b is not None else None))
        plan = _plan_kernel()
        assert narrow in plan and ("gemm_reduce_kernel" in plan) == split, plan
        report(y, O.linear(x, q, s, b), k, f"narrow m={m} n={n} k={k}", acc=O.acc_bound(x, q, s, b))
    m, k = 512, 2048
    x = activations(7764, m, k)
    xs = bf16_gpu(x, gpu)
    ws, qs, ss = [], [], []
    for j, n in enumerate((2048, 256, 256)):
        w = weights(7765 + j, n, k)
        ws.append(Q.QuantizedWeight(torch.from_numpy(w).to(gpu)))
        q, s = O.quantize_per_channel(w)
        qs.append(q)
        ss.append(s)
    outs = Q.linear_group(xs, ws)
    assert narrow in _plan_kernel(), _plan_kernel()
    rows = np.concatenate([np.random.default_rng(9).choice(m, 40, replace=False), [0, 31, 32, m - 1]])
    for j in range(3):
        report(to_np(outs[j])[rows], O.linear(x[rows], qs[j], ss[j]), k, f"narrow qkv[{j}]",
               acc=O.acc_bound(x[rows], qs[j], ss[j]))
    qw, q, s, x, _ = _problem(gpu, 7768, 1024, 2048, 2048)
    qw.linear(bf16_gpu(x, gpu))
    assert narrow not in _plan_kernel() and "BN = 128" in _plan_kernel(), _plan_kernel()


def test_one_shot_32_token_plan(gpu):
    """65..128 tokens, one matrix, K <= 2048: one-shot tiles of 32 tokens
    (launch_once<*, *, *, 2>, each widened weight fragment feeding two MFMAs)
    where they give at least as many workgroups as 16-token tiles: o_proj's
    shape at 96 and 128 tokens, a ragged M (97: one token in the last tile)
    and N with a bias, and q|k|v at 128 tokens (64-row tiles) against the
    full oracle; at 64 tokens and where 16-token tiles are more (100 x 300)
    the 16-token tile stays."""
    tm2 = "TM = 2"
    for m, n, k, seed, want in ((96, 2048, 2048, 7781, "NT = 2"), (128, 2048, 2048, 7782, "NT = 2"),
                                (97, 2048, 2048, 7783, "NT = 2"), (70, 1000, 1024, 7784, "NT = 1"),
                                (64, 2048, 2048, 7785, None), (100, 300, 2048, 7786, None)):
        qw, q, s, x, b = _problem(gpu, seed, m, n, k, bias=n != 2048)
        y = to_np(qw.linear(bf16_gpu(x, gpu), bf16_gpu(b, gpu) if b is not None else None))
        plan = _plan_kernel()
        assert "launch_once" in plan, plan
        assert (tm2 in plan) == (want is not None) and (want is None or want in plan), plan
        report(y, O.linear(x, q, s, b), k, f"once m={m} n={n} k={k}", acc=O.acc_bound(x, q, s, b))
    m, k = 128, 2048
    x = activations(7787, m, k)
    ws, qs, ss = [], [], []
    for j, n in enumerate((2048, 256, 256)):
        w = weights(7788 + j, n, k)
        ws.append(Q.QuantizedWeight(torch.from_numpy(w).to(gpu)))
        q, s = O.quantize_per_channel(w)
        qs.append(q)
        ss.append(s)
    outs = Q.linear_group(bf16_gpu(x, gpu), ws)
    plan = _plan_kernel()
    assert "launch_once" in plan and tm2 in plan and "NT = 4" in plan, plan
    for j in range(3):
        report(to_np(outs[j]), O.linear(x, qs[j], ss[j]), k, f"once qkv[{j}]", acc=O.acc_bound(x, qs[j], ss[j]))
