"""CPU checks of the bench's plan-string parsing: the counter summaries map
each launch kind's recorded plan (pgs_last_plan) onto the kernel instance
rocprofv3 names, for every launcher the GEMM and skinny paths use."""
from __future__ import annotations

import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402

_SIG = "(const uint16_t *, const GemmArgs &, hipStream_t)"


@pytest.mark.parametrize("plan, kernel, reduce", [
    (f"int pgs::(anonymous namespace)::launch_k64{_SIG} [BM = 64, BN = 128, NMAT = 1, OUT_F32 = false, WLEAD = 2, "
     "XLEAD = 2, OCC = 2, KG = 2] | grid=512 splits=4 | then gemm_reduce_kernel",
     "gemm_k64_kernel<64, 128, 1, false, 2, 2, 2, 2>", "gemm_reduce_kernel<64, 128, 1, false"),
    (f"int pgs::(anonymous namespace)::launch_dma{_SIG} [BM = 128, BN = 64, NMAT = 2, OUT_F32 = false, WLEAD = 2, "
     "S = 3, OCC = 3] | grid=688 splits=1",
     "gemm_dma_kernel<128, 64, 2, false, 2, 3, 3>", None),
    (f"int pgs::(anonymous namespace)::launch_once{_SIG} [CPG = 8, NT = 4, OUT_F32 = false] | grid=256 splits=1",
     "gemm_once_kernel<8, 4, false>", None),
    (f"int pgs::(anonymous namespace)::launch_cfg{_SIG} [BM = 32, BN = 128, NMAT = 1, OUT_F32 = false, OCC = 2, "
     "LEAD = 1] | grid=64 splits=1",
     "gemm_kernel<32, 128, 1, false, 2, 1>", None),
    ("int pgs::(anonymous namespace)::launch_instance(Problem &, const SkinnyPlan &, hipStream_t) [NW = 8, U = 2, "
     "NB = 2, NMAT = 2, OUT_F32 = false, K64 = true, FOLD = false, XM = 0, NORM = false, TM = 1] | grid=688 splits=1",
     "skinny_kernel<8, 2, 2, 2, false, true, false, 0, false, 1>", None),
    ("int pgs::(anonymous namespace)::launch_pair_tiles(Problem &, const SkinnyPlan &, hipStream_t) [RT = 3, "
     "NW = 16, CPW = 2] | grid=230 splits=1",
     "pair_tiles_kernel<3, 16, 2>", None),
])
def test_kernel_pattern_names_the_launched_instance(plan, kernel, reduce):
    assert bench.kernel_pattern(plan) == (kernel, reduce)


def test_kernel_pattern_rejects_an_unknown_launcher():
    with pytest.raises(ValueError):
        bench.kernel_pattern("int pgs::launch_unknown(void) [A = 1] | grid=1 splits=1")


@pytest.mark.parametrize("argv, env", [(["--gpus", "2"], {}), (["--gpus", "8", "--steps", "1"], {}),
                                       ([], {"WORLD_SIZE": "4"})])
def test_more_than_one_gpu_exits_with_a_message(argv, env):
    """`bench.py --gpus N` with N > 1 (or a multi-rank launch) exits before
    touching a GPU, saying that this path is measured on one GPU."""
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), *argv], capture_output=True, text=True,
                       env={**os.environ, **env}, timeout=300)
    assert r.returncode == 2 and "one GPU only" in r.stderr and r.stdout == ""
