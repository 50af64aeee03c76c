"""Fused SwiGLU (engine/model.py:188-190) against the oracle.

act = silu(x Wg^T) * (x Wu^T) computed in fp32 and rounded once to bf16;
out = act Wd^T.  The oracle keeps everything in fp32/float64.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import activations, bf16_gpu, report, to_np, weights
from oracle import quantization_oracle as O
from pageserve_amd import quantization as Q

pytestmark = pytest.mark.gpu


def _mlp_weights(gpu, seed, inter, hidden):
    ws = {}
    for j, (name, shape) in enumerate((("gate", (inter, hidden)), ("up", (inter, hidden)),
                                       ("down", (hidden, inter)))):
        w = weights(seed + j, *shape)
        ws[name] = (Q.QuantizedWeight(torch.from_numpy(w).to(gpu)), *O.quantize_per_channel(w))
    return ws


@pytest.mark.parametrize("m,inter,hidden", [(1, 11008, 2048), (4, 11008, 2048), (16, 11008, 2048),
                                            (17, 11008, 2048), (128, 11008, 2048), (512, 11008, 2048),
                                            (3, 100, 48), (40, 300, 208), (20, 64, 16),
                                            (50, 130, 48), (24, 256, 4112),
                                            # 128-token x 64-row tiles: split K, ragged M and N
                                            (100, 256, 4096), (300, 1000, 2048), (65, 64, 64),
                                            (33, 1000, 2048),
                                            # 65..128 tokens: 64-token tiles, LDS-DMA activations
                                            (80, 11008, 2048), (96, 1000, 2112),
                                            # above 128 tokens with a last 128-token tile at most
                                            # half full: 64-token tiles
                                            (160, 11008, 2048), (320, 1000, 2112),
                                            # two token blocks: unsplit, and a long K split into partials
                                            (32, 11008, 2048), (24, 1000, 8192), (21, 300, 1040),
                                            # 14..16 tokens, K <= 2048: three row tiles per workgroup
                                            # (ragged N, tile counts not a multiple of three, a K of
                                            # 17 chunks, a single chunk)
                                            (14, 11008, 2048), (15, 1000, 2048), (16, 130, 1088),
                                            (14, 48, 64), (16, 100, 2048)])
def test_swiglu_matches_oracle(gpu, m, inter, hidden):
    ws = _mlp_weights(gpu, 10 + m + inter, inter, hidden)
    x = activations(m, m, hidden)
    act = Q.swiglu(bf16_gpu(x, gpu), ws["gate"][0], ws["up"][0])
    assert act.dtype == torch.bfloat16 and act.shape == (m, inter)
    ref = O.swiglu(x, ws["gate"][1], ws["gate"][2], ws["up"][1], ws["up"][2])
    acc = O.swiglu_acc(x, ws["gate"][1], ws["gate"][2], ws["up"][1], ws["up"][2])
    report(to_np(act), ref, hidden, f"swiglu m={m}", acc=acc)


@pytest.mark.parametrize("m", [1, 512])
def test_mlp_config(gpu, m):
    """The fused SwiGLU MLP workload: x [m, 2048], gate/up [11008, 2048],
    down [2048, 11008]; out = down(silu(gate(x)) * up(x))."""
    ws = _mlp_weights(gpu, 4000, 11008, 2048)
    x = activations(4100 + m, m, 2048)
    out = Q.mlp(bf16_gpu(x, gpu), ws["gate"][0], ws["up"][0], ws["down"][0])
    ref = O.mlp(x, ws["gate"][1], ws["gate"][2], ws["up"][1], ws["up"][2], ws["down"][1], ws["down"][2])
    report(to_np(out), ref, 11008, f"mlp m={m}", acc=O.mlp_acc(x, ws["gate"][1], ws["gate"][2], ws["up"][1],
                                                              ws["up"][2], ws["down"][1], ws["down"][2]))


def test_swiglu_equals_unfused_composition(gpu):
    """Same as gate and up as separate fp32-output linears, combined in fp32."""
    ws = _mlp_weights(gpu, 77, 1024, 512)
    x = bf16_gpu(activations(3, 8, 512), gpu)
    g = ws["gate"][0].linear(x, out_dtype=torch.float32)
    u = ws["up"][0].linear(x, out_dtype=torch.float32)
    expect = (torch.nn.functional.silu(g) * u).to(torch.bfloat16).float()
    got = Q.swiglu(x, ws["gate"][0], ws["up"][0]).float()
    # same fp32 accumulations; silu rounding may differ by one bf16 ulp
    assert ((got - expect).abs() <= expect.abs() * 2 ** -7 + 1e-6).all()


def test_pair_tiles_plan(gpu):
    """14..16 tokens with K % 64 == 0 and at most 32 chunks run the pair as three
    16-row tiles per workgroup (pair_tiles_kernel); 13 tokens and a 33-chunk K keep
    the one-tile skinny plan.  Every case against the oracle."""
    from pageserve_amd import _native

    for m, inter, hidden, want in ((16, 11008, 2048, True), (14, 1000, 2048, True), (15, 35, 128, True),
                                   (13, 11008, 2048, False), (16, 1000, 2112, False)):
        ws = _mlp_weights(gpu, 900 + m + inter, inter, hidden)
        x = activations(950 + m, m, hidden)
        act = Q.swiglu(bf16_gpu(x, gpu), ws["gate"][0], ws["up"][0])
        plan = _native.last_plan()
        assert ("launch_pair_tiles" in plan) == want, plan
        ref = O.swiglu(x, ws["gate"][1], ws["gate"][2], ws["up"][1], ws["up"][2])
        acc = O.swiglu_acc(x, ws["gate"][1], ws["gate"][2], ws["up"][1], ws["up"][2])
        report(to_np(act), ref, hidden, f"pair tiles m={m} n={inter} k={hidden}", acc=acc)
