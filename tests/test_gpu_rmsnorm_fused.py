"""rms_norm fused into the projections that consume it (engine/model.py:166-170
and :187-189): ``rmsnorm_linear_group`` and ``rmsnorm_swiglu``.

Up to four tokens, K % 64 == 0 and a bf16 output run one launch whose
skinny kernel normalises the activations it stages; every other case runs
the RMSNorm kernel into the workspace and then the plain projection.  Both
are checked:

- against the oracle chain ``linear(rmsnorm(x))`` within the linear
  tolerance (random inputs);
- bit for bit against the unfused calls ``linear_group(rmsnorm(x))`` on
  inputs whose sum of squares is exact in fp32 in any order (entries in
  {0, +-0.5, +-1, +-2}): the mean, r and both bf16 roundings then agree, so
  any difference is a wrong column, token or chunk in the fused prologue
  (a chunk past K counted into the sum, another token's row, a dropped
  piece) and fails the test.
"""

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

# (token counts, group widths, K): Qwen2.5 q|k|v at 2048 and 896 hidden
# (the 896 case has 14 chunks: unfolded, two staged slots past K), a
# single wide matrix, and short groups that fold
GROUPS = [([2048, 256, 256], 2048), ([896, 128, 128], 896), ([11008], 2048), ([2048], 11008), ([512, 64], 1024),
          ([1104], 640), ([300, 48], 1040)]  # (K % 64 != 0: always the unfused route)


def exact_sum_inputs(seed: int, m: int, k: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.choice(np.array([0.0, 0.5, -0.5, 1.0, -1.0, 2.0, -2.0], np.float32), size=(m, k))


def norm_weight(seed: int, k: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return O.round_to_bf16((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32))


def group(gpu, seed: int, ns: list[int], k: int):
    ws = [weights(seed + j, n, k) for j, n in enumerate(ns)]
    return ws, [Q.QuantizedWeight(torch.from_numpy(w).to(gpu)) for w in ws], [O.quantize_per_channel(w) for w in ws]


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 16, 24])
@pytest.mark.parametrize("ns,k", GROUPS)
def test_rmsnorm_linear_group_equals_unfused(gpu, m, ns, k):
    _, qws, _ = group(gpu, 3 * k + len(ns), ns, k)
    x = bf16_gpu(exact_sum_inputs(m * 7 + k, m, k), gpu)
    w = bf16_gpu(norm_weight(k + 1, k), gpu)
    fused = Q.rmsnorm_linear_group(x, w, 1e-6, qws)
    plain = Q.linear_group(Q.rmsnorm(x, w, 1e-6), qws)
    for j, (a, b) in enumerate(zip(fused, plain)):
        assert a.shape == (m, ns[j]) and a.dtype == torch.bfloat16
        assert torch.equal(a, b), f"output {j}: max diff {(a.float() - b.float()).abs().max().item()}"


@pytest.mark.parametrize("m", [1, 2, 3, 4, 6])
@pytest.mark.parametrize("ns,k", [([2048, 256, 256], 2048), ([896, 128, 128], 896), ([1104], 640)])
def test_rmsnorm_linear_group_matches_oracle(gpu, m, ns, k):
    ws, qws, qs = group(gpu, 5 * k + m, ns, k)
    rng = np.random.default_rng(m + k)
    x = O.round_to_bf16(rng.standard_normal((m, k), dtype=np.float32) * np.float32(3.0))
    w = norm_weight(k, k)
    biases = [O.round_to_bf16(rng.standard_normal(n).astype(np.float32)) for n in ns]
    outs = Q.rmsnorm_linear_group(bf16_gpu(x, gpu), bf16_gpu(w, gpu), 1e-6, qws, [bf16_gpu(b, gpu) for b in biases])
    h, dh = O.rmsnorm(x, w, 1e-6), O.rmsnorm_dx(x, w, 1e-6)
    for j, (q, s) in enumerate(qs):
        report(to_np(outs[j]), O.linear(h, q, s, biases[j]), k, f"rmsnorm+linear m={m} n={ns[j]} k={k}",
               acc=O.acc_bound(h, q, s, biases[j], dx=dh))


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("n,k", [(11008, 2048), (4864, 896), (1408, 512)])
def test_rmsnorm_swiglu_equals_unfused_and_oracle(gpu, m, n, k):
    wg, wu = weights(40 + n, n, k), weights(41 + n, n, k)
    g, u = Q.QuantizedWeight(torch.from_numpy(wg).to(gpu)), Q.QuantizedWeight(torch.from_numpy(wu).to(gpu))
    w = bf16_gpu(norm_weight(n, k), gpu)
    xe = bf16_gpu(exact_sum_inputs(m + n, m, k), gpu)
    assert torch.equal(Q.rmsnorm_swiglu(xe, w, 1e-6, g, u), Q.swiglu(Q.rmsnorm(xe, w, 1e-6), g, u))
    x = activations(m * 3 + n, m, k)
    act = Q.rmsnorm_swiglu(bf16_gpu(x, gpu), w, 1e-6, g, u)
    h, dh = O.rmsnorm(x, norm_weight(n, k), 1e-6), O.rmsnorm_dx(x, norm_weight(n, k), 1e-6)
    qg, qu = O.quantize_per_channel(wg), O.quantize_per_channel(wu)
    report(to_np(act), O.swiglu(h, *qg, *qu), k, f"rmsnorm+swiglu m={m} n={n} k={k}",
           acc=O.swiglu_acc(h, *qg, *qu, dx=dh))


@pytest.mark.parametrize("m", [1, 3])
def test_rmsnorm_mlp_with_residual(gpu, m):
    H, I = 896, 4864
    ws = {nm: weights(90 + j, n, kk) for j, (nm, n, kk) in enumerate([("g", I, H), ("u", I, H), ("d", H, I)])}
    qw = {nm: Q.QuantizedWeight(torch.from_numpy(w).to(gpu)) for nm, w in ws.items()}
    x = bf16_gpu(exact_sum_inputs(m, m, H), gpu)
    res = bf16_gpu(activations(m + 1, m, H), gpu)
    w = bf16_gpu(norm_weight(7, H), gpu)
    fused = Q.rmsnorm_mlp(x, w, 1e-5, qw["g"], qw["u"], qw["d"], residual=res)
    plain = Q.mlp(Q.rmsnorm(x, w, 1e-5), qw["g"], qw["u"], qw["d"], residual=res)
    assert torch.equal(fused, plain)


def test_fallbacks_fp32_output_and_leading_dims(gpu):
    """A fp32 output and 3-D inputs take the unfused route or reshape; the
    results equal the unfused calls."""
    k = 2048
    _, qws, _ = group(gpu, 1, [1024, 256], k)
    x = bf16_gpu(exact_sum_inputs(2, 2, k), gpu)
    w = bf16_gpu(norm_weight(3, k), gpu)
    f32 = Q.rmsnorm_linear_group(x, w, 1e-6, qws, out_dtype=torch.float32)
    p32 = Q.linear_group(Q.rmsnorm(x, w, 1e-6), qws, out_dtype=torch.float32)
    assert all(a.dtype == torch.float32 and torch.equal(a, b) for a, b in zip(f32, p32))
    x3 = x.view(1, 2, k)
    out3 = Q.rmsnorm_linear_group(x3, w, 1e-6, qws)
    assert out3[0].shape == (1, 2, 1024)
    assert torch.equal(out3[1].view(2, 256), Q.linear_group(Q.rmsnorm(x, w, 1e-6), qws)[1])


def test_misaligned_norm_weight_through_the_c_abi(gpu):
    """A norm weight that is 2-byte but not 16-byte aligned cannot feed the
    staged 16-byte loads: the library runs the RMSNorm kernel first.  The
    output equals the aligned call's."""
    m, n, k = 2, 2048, 2048
    qw = Q.QuantizedWeight(torch.from_numpy(weights(5, n, k)).to(gpu))
    x = bf16_gpu(exact_sum_inputs(9, m, k), gpu)
    wv = norm_weight(10, k)
    holder = torch.zeros(k + 8, dtype=torch.bfloat16, device=gpu)
    holder[1:k + 1] = bf16_gpu(wv, gpu)
    wmis = holder[1:k + 1]
    assert wmis.data_ptr() % 16 == 2
    lib = _native.load()
    qp, sc = qw._kernel_operands()
    y = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    outs = (_native.LinearOut * 1)()
    outs[0].qp, outs[0].scale, outs[0].bias, outs[0].y, outs[0].n = qp.data_ptr(), sc.data_ptr(), None, y.data_ptr(), n
    ns = (ctypes.c_int64 * 1)(n)
    nbytes = lib.pgs_w8a16_rmsnorm_workspace_bytes(m, ns, 1, k, 0)
    assert nbytes >= m * k * 2
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    rc = lib.pgs_w8a16_rmsnorm_linear_group(x.data_ptr(), wmis.data_ptr(), ctypes.c_float(1e-6), outs, 1, 1, m, k,
                                             ws.data_ptr(), nbytes, ctypes.c_void_p(stream))
    _native.check(rc, "rmsnorm linear")
    ref = qw.linear(Q.rmsnorm(x, bf16_gpu(wv, gpu), 1e-6))
    assert torch.equal(y, ref)
    # without a workspace the misaligned weight has nowhere to put h: an error, nothing launched
    rc = lib.pgs_w8a16_rmsnorm_linear_group(x.data_ptr(), wmis.data_ptr(), ctypes.c_float(1e-6), outs, 1, 1, m, k,
                                             None, 0, ctypes.c_void_p(stream))
    assert rc != 0 and b"workspace" in lib.pgs_last_error()


def test_zero_rows_eps_and_repeat_calls(gpu):
    """A zero row normalises to zeros (eps > 0), so its outputs are the bias;
    eps = 0 on non-zero rows matches the oracle; repeated calls are
    identical."""
    m, k = 3, 2048
    ns = [1024, 256]
    _, qws, qs = group(gpu, 21, ns, k)
    x = activations(22, m, k)
    x[1] = 0.0
    w = norm_weight(23, k)
    b = [O.round_to_bf16(np.random.default_rng(24 + j).standard_normal(n).astype(np.float32)) for j, n in
         enumerate(ns)]
    xt, wt, bt = bf16_gpu(x, gpu), bf16_gpu(w, gpu), [bf16_gpu(v, gpu) for v in b]
    outs = Q.rmsnorm_linear_group(xt, wt, 1e-6, qws, bt)
    for j in range(2):
        np.testing.assert_array_equal(to_np(outs[j])[1], b[j])
        assert torch.equal(outs[j], Q.rmsnorm_linear_group(xt, wt, 1e-6, qws, bt)[j])
    x0 = np.delete(x, 1, axis=0)
    outs0 = Q.rmsnorm_linear_group(bf16_gpu(x0, gpu), wt, 0.0, qws)
    h, dh = O.rmsnorm(x0, w, 0.0), O.rmsnorm_dx(x0, w, 0.0)
    for j, (q, s) in enumerate(qs):
        report(to_np(outs0[j]), O.linear(h, q, s), k, f"eps=0 output {j}", acc=O.acc_bound(h, q, s, dx=dh))


def test_empty_and_bad_norm_weight(gpu):
    _, qws, _ = group(gpu, 31, [256], 512)
    w = bf16_gpu(norm_weight(32, 512), gpu)
    out = Q.rmsnorm_linear_group(torch.empty(0, 512, dtype=torch.bfloat16, device=gpu), w, 1e-6, qws)
    assert out[0].shape == (0, 256)
    x = bf16_gpu(activations(33, 2, 512), gpu)
    with pytest.raises(ValueError, match="norm weight"):
        Q.rmsnorm_linear_group(x, w[:256], 1e-6, qws)
    with pytest.raises(ValueError, match="norm weight"):
        Q.rmsnorm_linear_group(x, w.float(), 1e-6, qws)
    with pytest.raises(ValueError, match="eps"):
        Q.rmsnorm_linear_group(x, w, -1.0, qws)


def test_fallback_leaves_the_pair_slots_empty(gpu):
    """The unfused route writes h into the shared workspace; a later paired
    K split on the same workspace (down_proj at 5 tokens) must still find
    its pair slots empty, also after a call whose own plan used none."""
    wide = Q.QuantizedWeight(torch.from_numpy(weights(51, 11008, 2048)).to(gpu))
    down = Q.QuantizedWeight(torch.from_numpy(weights(52, 2048, 11008)).to(gpu))
    x5 = bf16_gpu(activations(53, 5, 11008), gpu)
    before = down.linear(x5)
    x16 = bf16_gpu(activations(54, 16, 2048) * np.float32(4.0), gpu)
    Q.rmsnorm_linear_group(x16, bf16_gpu(norm_weight(55, 2048), gpu), 1e-6, [wide])
    torch.cuda.synchronize()
    assert torch.equal(down.linear(x5), before)
