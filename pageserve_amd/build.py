"""Builds the gfx950 shared library ``pageserve_amd/_lib/libpageserve_amd.so``.

``python -m pageserve_amd.build`` (or ``build()``) compiles every ``csrc/*.hip``
with hipcc for gfx950 and links them into one C-ABI shared library that the
Python host code loads with ctypes.  hipcc cross-compiles, so this runs on a
machine without a GPU.

Flags that matter for results:
* no fast-math, and ``-fhip-fp32-correctly-rounded-divide-sqrt``: the
  quantizer's ``w / scale`` must be a correctly rounded IEEE division;
* ``-packed-fp32-ops`` off: packed fp32 VALU forms are not emitted.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIBDIR = PKG / "_lib"
LIBNAME = "libpageserve_amd.so"
OBJDIR = ROOT / "_build" / "obj"
HOST_SRC = CSRC / "host_ops.cpp"
HOST_NAME = "_pgs_host"
HOST_BUILD = ROOT / "_build" / "host"

ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


# the compiler's per-kernel resource report (registers, scratch, occupancy)
USAGE_FLAG = "-Rpass-analysis=kernel-resource-usage"


def kernel_usage(stderr: str) -> dict:
    """Kernel name -> {field: value} from the resource-usage remarks."""
    usage, name = {}, None
    for line in stderr.splitlines():
        if "remark:" not in line or USAGE_FLAG not in line:
            continue
        body = line.split("remark:", 1)[1].rsplit("[", 1)[0].strip()
        key, _, val = body.partition(":")
        if key == "Function Name":
            name = val.strip()
            usage[name] = {}
        elif name is not None:
            usage[name][key.strip()] = val.strip()
    return usage


def _compile(hipcc: str, src: Path) -> Path:
    OBJDIR.mkdir(parents=True, exist_ok=True)
    obj = OBJDIR / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, USAGE_FLAG, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    # Every kernel is tuned to live in registers: a spill to scratch memory
    # (after a change, or with another compiler) is a build error, not a
    # silent slowdown.
    spills = [f"{k}: scratch {u.get('ScratchSize [bytes/lane]')} B/lane, VGPR spill {u.get('VGPRs Spill')}"
              for k, u in kernel_usage(res.stderr).items()
              if u.get("ScratchSize [bytes/lane]", "0") != "0" or u.get("VGPRs Spill", "0") != "0"]
    if spills:
        raise RuntimeError(f"{src.name}: kernels spill registers to scratch:\n  " + "\n  ".join(spills))
    noise = "is not a recognized feature for this target"
    lines = [l for l in res.stderr.splitlines()
             if l.strip() and noise not in l and USAGE_FLAG not in l and not re.match(r"^\s*\d*\s*\|", l)]
    warn = "\n".join(lines)
    if warn:
        print(f"[pageserve_amd.build] {src.name}:\n{warn}", file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles and links the library; returns its path.  Always rebuilds."""
    hipcc = _hipcc()
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s), srcs))
    LIBDIR.mkdir(parents=True, exist_ok=True)
    out = LIBDIR / LIBNAME
    tmp = LIBDIR / (LIBNAME + ".tmp")
    # the soname lets the host module's dependency on this library resolve
    # to the copy already loaded from the package directory
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,-soname,{LIBNAME}", *map(str, objs), "-o",
           str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"[pageserve_amd.build] built {out} from {len(srcs)} sources for {ARCH}")
    build_host(verbose)
    return out


def build_host(verbose: bool = True) -> Path:
    """Compiles the C++ host module (host_ops.cpp, a PyTorch extension that
    calls the C ABI) into ``_lib/_pgs_host*.so``.  Always rebuilds."""
    import ctypes

    import torch.utils.cpp_extension as ext

    # the module's dependency on the library resolves by soname to a copy
    # already loaded (load() imports the module right after linking it)
    ctypes.CDLL(str(LIBDIR / LIBNAME), mode=ctypes.RTLD_GLOBAL)
    shutil.rmtree(HOST_BUILD, ignore_errors=True)
    HOST_BUILD.mkdir(parents=True, exist_ok=True)
    ext.load(
        name=HOST_NAME,
        sources=[str(HOST_SRC)],
        build_directory=str(HOST_BUILD),
        extra_include_paths=[str(INCLUDE), "/opt/rocm/include"],
        # torch's HIP headers need the platform macro outside hipcc
        extra_cflags=["-O2", "-D__HIP_PLATFORM_AMD__"],
        extra_ldflags=[f"-L{LIBDIR}", "-lpageserve_amd"],
        with_cuda=False,
        verbose=False,
    )
    built = next(HOST_BUILD.glob(f"{HOST_NAME}*.so"))
    dst = LIBDIR / built.name
    tmp = LIBDIR / (built.name + ".tmp")
    shutil.copyfile(built, tmp)
    os.replace(tmp, dst)
    if verbose:
        print(f"[pageserve_amd.build] built {dst} (C++ host module)")
    return dst


if __name__ == "__main__":
    build()
