"""Host-side API of pageserve_amd.quantization on the CPU: the reference's
names and argument checks, and no silent CPU implementation."""

from __future__ import annotations

import inspect

import pytest
import torch

import pageserve_amd
from pageserve_amd import quantization as Q


def test_reference_api_surface():
    # engine/quantization.py:16,26,30-50
    assert list(inspect.signature(Q.quantize_per_channel).parameters) == ["weight"]
    assert list(inspect.signature(Q.dequantize).parameters) == ["q", "scale", "dtype"]
    assert list(inspect.signature(Q.QuantizedWeight.__init__).parameters) == ["self", "weight"]
    for attr in ("get", "to", "storage_bytes", "q"):
        assert hasattr(Q.QuantizedWeight, attr)
    assert pageserve_amd.QuantizedWeight is Q.QuantizedWeight


def test_product_never_imports_the_oracle():
    import pathlib

    pkg = pathlib.Path(Q.__file__).parent
    for src in pkg.rglob("*.py"):
        text = src.read_text()
        assert "import oracle" not in text and "from oracle" not in text, src


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_no_gpu_fused_path_is_an_error_not_a_fallback():
    """Without a GPU the fused linears raise; only CPU tensors' own reference
    math (quantize, dequantize, get) runs on the CPU."""
    qw = Q.QuantizedWeight(torch.randn(8, 16))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        Q.linear(torch.zeros(1, 16, dtype=torch.bfloat16), qw)
    with pytest.raises(RuntimeError):
        qw.to("cuda")


def test_shape_errors_match_reference_behaviour():
    with pytest.raises(ValueError, match="2-D"):
        Q.quantize_per_channel(torch.randn(16))
    with pytest.raises(RuntimeError, match="non-zero size"):
        Q.quantize_per_channel(torch.randn(4, 0))
    with pytest.raises(ValueError, match="int8"):
        Q.dequantize(torch.zeros(2, 16), torch.ones(2, 1), torch.float32)
    with pytest.raises(ValueError, match="one value per row"):
        Q.dequantize(torch.zeros(2, 16, dtype=torch.int8), torch.ones(3, 1), torch.float32)


def test_linear_requires_a_gpu_resident_weight():
    class Fake:
        qp = torch.zeros(1024, dtype=torch.int8)
        shape = torch.Size((4, 16))
        device = torch.device("cpu")
        scale = torch.ones(4, 1)

    with pytest.raises(RuntimeError, match="ROCm GPU"):
        Q.linear(torch.zeros(1, 16, dtype=torch.bfloat16), Fake())
    with pytest.raises(ValueError, match="1..4"):
        Q.linear_group(torch.zeros(1, 16, dtype=torch.bfloat16), [])
