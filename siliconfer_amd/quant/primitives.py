"""Offline int4 quantization primitives (CPU, numpy) — the producer of packed tensors.

Same API as the reference's `siliconfer/quant/primitives.py` (quantize_sym
:24-51, dequantize_sym :54-75, quantize_asym :82-114, dequantize_asym
:117-140, pack_int4 :332-349, unpack_int4 :352-376, fake_quantize :442-472).
These run once per model load, on the host, as in the reference: the GPU path
consumes their packed output. Codes are computed with float32 arithmetic and
numpy's round-half-to-even, which is what fixes the reference's bits.
"""

from __future__ import annotations

import numpy as np

INT4_SYM_MIN, INT4_SYM_MAX, INT4_UINT_MAX = -8, 7, 15


def _split_groups(w: np.ndarray, group_size: int) -> np.ndarray:
    *lead, cols = w.shape
    if cols % group_size:
        raise ValueError(f"cols={cols} not divisible by group_size={group_size}")
    return w.reshape(*lead, cols // group_size, group_size)


def quantize_sym(w: np.ndarray, group_size: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """Group-wise symmetric int4 along the last axis -> (q int8 in [-8,7], scales f32)."""
    w = np.asarray(w, dtype=np.float32)
    groups = _split_groups(w, group_size)
    scale = np.abs(groups).max(axis=-1, keepdims=True) / np.float32(INT4_SYM_MAX)
    scale = scale.astype(np.float32)
    safe = np.where(scale == 0, np.float32(1.0), scale)
    q = np.clip(np.round(groups / safe), INT4_SYM_MIN, INT4_SYM_MAX).astype(np.int8)
    return q.reshape(w.shape), scale[..., 0]


def dequantize_sym(q: np.ndarray, scales: np.ndarray, group_size: int = 128) -> np.ndarray:
    groups = _split_groups(np.asarray(q), group_size).astype(np.float32)
    return (groups * np.asarray(scales, np.float32)[..., None]).reshape(q.shape)


def quantize_asym(w: np.ndarray, group_size: int = 128):
    """Group-wise asymmetric int4 -> (q uint8 in [0,15], scales f32, zeros f32 integral)."""
    w = np.asarray(w, dtype=np.float32)
    groups = _split_groups(w, group_size)
    lo = groups.min(axis=-1, keepdims=True)
    hi = groups.max(axis=-1, keepdims=True)
    scale = ((hi - lo) / np.float32(INT4_UINT_MAX)).astype(np.float32)
    safe = np.where(scale == 0, np.float32(1.0), scale)
    zero = np.clip(np.round(-lo / safe), 0, INT4_UINT_MAX).astype(np.float32)
    q = np.clip(np.round(groups / safe) + zero, 0, INT4_UINT_MAX).astype(np.uint8)
    return q.reshape(w.shape), scale[..., 0], zero[..., 0]


def dequantize_asym(q: np.ndarray, scales: np.ndarray, zeros: np.ndarray,
                    group_size: int = 128) -> np.ndarray:
    groups = _split_groups(np.asarray(q), group_size).astype(np.float32)
    s = np.asarray(scales, np.float32)[..., None]
    z = np.asarray(zeros, np.float32)[..., None]
    return ((groups - z) * s).reshape(q.shape)


def fake_quantize(w: np.ndarray, group_size: int = 128, sym: bool = True) -> np.ndarray:
    """RTN quantize then dequantize (4-bit)."""
    if sym:
        return dequantize_sym(*quantize_sym(w, group_size), group_size)
    return dequantize_asym(*quantize_asym(w, group_size), group_size)


def pack_int4(q: np.ndarray) -> np.ndarray:
    """Two int4 per byte: low nibble = even element, high nibble = odd element."""
    flat = np.asarray(q).reshape(-1).astype(np.int32)
    if flat.size % 2 != 0:
        raise ValueError("Total elements must be even for int4 packing")
    pairs = (flat & 0xF).astype(np.uint8).reshape(-1, 2)
    return pairs[:, 0] | (pairs[:, 1] << 4)


def unpack_int4(packed: np.ndarray, n: int, signed: bool = True) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8).reshape(-1)
    out = np.empty(p.size * 2, dtype=np.int16)
    out[0::2] = p & 0x0F
    out[1::2] = p >> 4
    out = out[:n]
    if signed:
        return np.where(out > 7, out - 16, out).astype(np.int8)
    return out.astype(np.uint8)
