"""Offline (CPU) quantization primitives that produce the packed int4 tensors."""

from .hqq import hqq_pack, hqq_quantize_weight, hqq_search
from .primitives import (dequantize_asym, dequantize_sym, fake_quantize, pack_int4,
                         quantize_asym, quantize_sym, unpack_int4)

__all__ = ["hqq_quantize_weight", "hqq_search", "hqq_pack", "quantize_sym", "dequantize_sym", "quantize_asym", "dequantize_asym",
           "fake_quantize", "pack_int4", "unpack_int4"]
