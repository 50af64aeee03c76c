"""Shared test configuration.

Markers: ``gpu`` tests need a ROCm GPU and call the HIP kernels through the C
ABI; everything else runs on the CPU.  The gfx950 library is built in-tree if
it is missing (hipcc cross-compiles without a GPU).
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (gfx950) and runs the HIP kernels")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def native_lib():
    """The loaded C-ABI library (built first if absent)."""
    from pageserve_amd import _native

    if not _native.LIB_PATH.exists():
        from pageserve_amd import build

        build.build()
    return _native.load()


@pytest.fixture(scope="session")
def gpu(native_lib):
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda", 0)
