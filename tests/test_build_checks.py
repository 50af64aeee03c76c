"""The library compile's resource-usage check: the compiler's per-kernel remarks are
parsed, and a kernel that spills registers to scratch fails the build."""

from __future__ import annotations

from pageserve_amd import build

SAMPLE = """\
x.hip:27:1: remark: Function Name: k_good [-Rpass-analysis=kernel-resource-usage]
x.hip:27:1: remark:     VGPRs: 24 [-Rpass-analysis=kernel-resource-usage]
x.hip:27:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
x.hip:27:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]
   27 | __global__ void k_good() {}
x.hip:40:1: remark: Function Name: k_spill [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark:     ScratchSize [bytes/lane]: 144 [-Rpass-analysis=kernel-resource-usage]
x.hip:40:1: remark:     VGPRs Spill: 36 [-Rpass-analysis=kernel-resource-usage]
"""


def test_kernel_usage_parses_remarks():
    u = build.kernel_usage(SAMPLE)
    assert set(u) == {"k_good", "k_spill"}
    assert u["k_good"]["VGPRs"] == "24" and u["k_good"]["ScratchSize [bytes/lane]"] == "0"
    assert u["k_spill"]["ScratchSize [bytes/lane]"] == "144" and u["k_spill"]["VGPRs Spill"] == "36"


def test_build_passes_the_usage_flag():
    assert build.USAGE_FLAG == "-Rpass-analysis=kernel-resource-usage"
