"""pageserve_amd: MI355X (gfx950) INT8 weight-only linear path.

A drop-in for pageserve's ``engine/quantization.py``: the same Python API,
computed by hand-written HIP kernels behind a C ABI
(``include/pageserve_amd.h``).
"""

from .quantization import (  # noqa: F401
    QuantizedWeight,
    W8A16Weight,
    apply_rope,
    dequantize,
    linear,
    linear_argmax,
    linear_group,
    load_quantized,
    mlp,
    quantize_per_channel,
    rmsnorm,
    rmsnorm_linear_group,
    rmsnorm_mlp,
    rmsnorm_swiglu,
    rope_qk,
    save_quantized,
    swiglu,
)

__version__ = "0.1.0"
