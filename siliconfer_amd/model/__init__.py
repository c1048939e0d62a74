"""Model-side call surface: Q4Linear, the int8 KV cache and the transformer
layer modules."""

from .kv_cache import QuantizedKVCache, dequantize_kv, make_quantized_cache, quantize_kv
from .layers import MLP, Attention, RMSNorm, TransformerBlock, apply_rope, compute_rope_freqs
from .q4_linear import Q4Linear

__all__ = ["Q4Linear", "QuantizedKVCache", "quantize_kv", "dequantize_kv", "make_quantized_cache",
           "RMSNorm", "Attention", "MLP", "TransformerBlock", "apply_rope", "compute_rope_freqs"]
