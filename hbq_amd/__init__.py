"""HBQ hot path on MI355X (gfx950): fused quantize-dequantize kernels and
block-quant GEMMs behind a C ABI (include/hbq_amd.h), with Python front ends
that mirror the reference's quantizer classes and blockquant_ext ops."""
from . import quantizer  # noqa: F401

__all__ = ["quantizer"]
