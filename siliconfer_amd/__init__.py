"""siliconfer_amd — MI355X (gfx950) HIP implementation of siliconfer's quantized
inference hot path: int4 Q4Linear GEMV/GEMM and fused decode attention over an
int8 KV cache, behind the reference's own call surface.

Subpackages:
  kernels  — pack_weights_*, gemv_*, gemm_*, Q4Weight, fused attention
  model    — Q4Linear, QuantizedKVCache, quantize_kv / dequantize_kv
  quant    — offline CPU quantizers producing the packed tensors
"""

__version__ = "0.1.0"
