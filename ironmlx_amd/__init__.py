"""ironmlx_amd — MI355X (gfx950) quantized-matmul path for ironmlx.

The product is ``libiqmm.so`` (C ABI in ``include/iqmm.h``); this package is
its host-side mirror of ironmlx's Rust surface: ``ops`` (quantized_matmul,
dequantize, gather_qmm, quantize) and ``nn`` (QuantizedLinear,
QuantizedEmbedding, MLP/Expert, MoE, the fused-expert split).
"""
from ._lib import IqmmError  # noqa: F401

__version__ = "0.1.0"
