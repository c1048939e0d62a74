"""Model-side call surface: Q4Linear and the int8 KV cache."""

from .kv_cache import QuantizedKVCache, dequantize_kv, make_quantized_cache, quantize_kv
from .q4_linear import Q4Linear

__all__ = ["Q4Linear", "QuantizedKVCache", "quantize_kv", "dequantize_kv", "make_quantized_cache"]
