"""int4 kernel interface — same names and argument meaning as the reference's
`siliconfer.kernels.neon` (/root/reference/siliconfer/kernels/neon/__init__.py:42-239).

Differences a caller can see:
  * `HIP_AVAILABLE` replaces `NEON_AVAILABLE`; there is no fallback backend —
    without the built library and a gfx950 GPU every compute call raises.
  * Inputs may be numpy arrays (the reference's types) or torch tensors. numpy
    in -> numpy float32 out (computed on the GPU, synchronously); torch in ->
    torch float32 out on the device, enqueued on the current stream.
  * Scales are stored as fp16 on the device; zero-points must be integral
    (the reference's asymmetric quantizer always produces integral zeros,
    siliconfer/quant/primitives.py:111).
  * gemv_asym works without a compiled NEON extension (the reference raises,
    :168-169) and computes the asymmetric formula on every host (the
    reference's non-ARM build silently computes the symmetric one,
    q4_gemv.cpp:249-255).
"""

from __future__ import annotations

import numpy as np
import torch

from .. import _lib
from ..quant.primitives import quantize_asym, quantize_sym
from .q4 import GEMV_MAX_ROWS, Q4Weight

HIP_AVAILABLE = _lib.hip_available()
_BACKEND = "hip-gfx950" if HIP_AVAILABLE else "unavailable"


def pack_weights_sym(W: np.ndarray, group_size: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """Quantize (symmetric RTN) and pack: -> (packed uint8 [N, K/2], scales float32 [N, K/g]).
    Low nibble = even column, high nibble = odd column, two's-complement codes."""
    q, scales = quantize_sym(np.asarray(W, dtype=np.float32), group_size)
    lo = q[:, 0::2].astype(np.uint8) & 0x0F
    hi = q[:, 1::2].astype(np.uint8) & 0x0F
    return (lo | (hi << 4)).astype(np.uint8), scales


def pack_weights_asym(W: np.ndarray, group_size: int = 128):
    """Quantize (asymmetric RTN) and pack: -> (packed, scales float32, zeros float32)."""
    q, scales, zeros = quantize_asym(np.asarray(W, dtype=np.float32), group_size)
    lo = q[:, 0::2] & 0x0F
    hi = q[:, 1::2] & 0x0F
    return (lo | (hi << 4)).astype(np.uint8), scales, zeros


def _run(packed, scales, zeros, X, group_size: int, want_2d: bool):
    """Shared body of the functional API: build the device weight, run, convert back."""
    numpy_io = not isinstance(X, torch.Tensor)
    if numpy_io:
        if not _lib.hip_available():
            raise _lib.SFError("no gfx950 HIP device: siliconfer_amd has no CPU fallback")
        dev = torch.device("cuda", torch.cuda.current_device())
        Xt = torch.from_numpy(np.ascontiguousarray(np.asarray(X, dtype=np.float32))).to(dev)
    else:
        dev = X.device
        Xt = X.contiguous()
        if Xt.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            Xt = Xt.float()
    if want_2d:
        if Xt.dim() != 2:
            raise _lib.SFError("X must be 2-D [T, in_f]")
        X2 = Xt
    else:
        if Xt.dim() != 1:
            raise _lib.SFError("x must be 1-D [in_f]")
        if Xt.shape[0] != 2 * packed.shape[1]:
            raise _lib.SFError("x length mismatch")
        X2 = Xt.reshape(1, -1)
    w = Q4Weight(packed, scales, zeros, group_size, device=dev)
    y = w.matmul(X2, out_dtype=torch.float32)
    if not want_2d:
        y = y.reshape(-1)
    if numpy_io:
        return y.cpu().numpy()
    return y


def gemv_sym(packed, scales, x, group_size: int = 128):
    """y = dequant(W) @ x, symmetric int4 (reference q4_gemv_sym)."""
    return _run(packed, scales, None, x, group_size, want_2d=False)


def gemv_scalar(packed, scales, x, group_size: int = 128):
    """Same result as gemv_sym; the reference keeps a scalar C twin for testing,
    here both names run the one GPU kernel."""
    return _run(packed, scales, None, x, group_size, want_2d=False)


def gemv_asym(packed, scales, zeros, x, group_size: int = 128):
    """y = dequant_asym(W) @ x with per-group zero-points (reference q4_gemv_asym)."""
    return _run(packed, scales, zeros, x, group_size, want_2d=False)


def gemm_sym(packed, scales, X, group_size: int = 128):
    """Y[T, out] = X[T, in] @ dequant(W).T, symmetric (reference q4_gemm_sym)."""
    return _run(packed, scales, None, X, group_size, want_2d=True)


def gemm_asym(packed, scales, zeros, X, group_size: int = 128):
    """Y[T, out] = X[T, in] @ dequant_asym(W).T (reference q4_gemm_asym)."""
    return _run(packed, scales, zeros, X, group_size, want_2d=True)


__all__ = [
    "HIP_AVAILABLE",
    "Q4Weight",
    "GEMV_MAX_ROWS",
    "pack_weights_sym",
    "pack_weights_asym",
    "gemv_sym",
    "gemv_scalar",
    "gemv_asym",
    "gemm_sym",
    "gemm_asym",
]
