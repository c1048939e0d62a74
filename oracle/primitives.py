"""Oracle restatement of the reference's int4 quantize / pack / unpack / dequant.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).

Every computation that produces integer codes is done in float32, exactly as the
reference does it with numpy float32 arrays, because the codes must be
bit-identical: `round(w / s)` on float32 operands, with numpy's round-half-even.

Reference anchors (all under /root/reference):
  quantize_sym          siliconfer/quant/primitives.py:24-51
  dequantize_sym        siliconfer/quant/primitives.py:54-75
  quantize_asym         siliconfer/quant/primitives.py:82-114
  dequantize_asym       siliconfer/quant/primitives.py:117-140
  pack_int4             siliconfer/quant/primitives.py:332-349
  unpack_int4           siliconfer/quant/primitives.py:352-376
  fake_quantize (4-bit) siliconfer/quant/primitives.py:442-472
  pack_weights_sym      siliconfer/kernels/neon/__init__.py:42-63
  pack_weights_asym     siliconfer/kernels/neon/__init__.py:66-81

Pinning (tests/test_oracle_primitives.py):
  * unpack: exhaustive over all 256 byte values, signed and unsigned, plus the
    reference's literal boundary vector `[-8,-1,0,1,7,-8,7,-1]`
    (tests/test_primitives.py:148).
  * quantize_sym/asym: closed-form invariants (|q|<=7, -8 never produced, z
    integral in [0,15], zero groups give s=0 / q=0), brute-force argmin of the
    reconstruction error on tiny groups, and round-half-even ties.
  * pack/unpack round trips and the lo=even / hi=odd layout.
"""

from __future__ import annotations

import numpy as np

SYM_QMIN, SYM_QMAX = -8, 7
ASYM_QMAX = 15


def _grouped(w: np.ndarray, group_size: int) -> np.ndarray:
    cols = w.shape[-1]
    if cols % group_size != 0:
        raise ValueError(f"cols={cols} not divisible by group_size={group_size}")
    return w.reshape(*w.shape[:-1], cols // group_size, group_size)


def quantize_sym(w: np.ndarray, group_size: int = 128):
    """Symmetric RTN per group: s = max|w|/7 (fp32), q = clip(rint(w/s'), -8, 7).

    s' = 1 where s == 0 (the stored scale stays 0). Returns (q int8 [...,K],
    s float32 [...,K/g]).
    """
    wg = _grouped(np.asarray(w, dtype=np.float32), group_size)
    amax = np.max(np.abs(wg), axis=-1)                        # float32
    s = (amax / np.float32(SYM_QMAX)).astype(np.float32)
    s_div = np.where(s == np.float32(0), np.float32(1), s).astype(np.float32)
    ratio = (wg / s_div[..., None]).astype(np.float32)
    q = np.clip(np.rint(ratio), SYM_QMIN, SYM_QMAX).astype(np.int8)
    return q.reshape(w.shape), s


def quantize_asym(w: np.ndarray, group_size: int = 128):
    """Asymmetric (min-max) RTN per group.

    s = (max - min)/15 (fp32); z = clip(rint(-min/s'), 0, 15);
    q = clip(rint(w/s') + z, 0, 15). Returns (q uint8, s float32, z float32).
    """
    wg = _grouped(np.asarray(w, dtype=np.float32), group_size)
    lo = np.min(wg, axis=-1)
    hi = np.max(wg, axis=-1)
    s = ((hi - lo) / np.float32(ASYM_QMAX)).astype(np.float32)
    s_div = np.where(s == np.float32(0), np.float32(1), s).astype(np.float32)
    z = np.clip(np.rint((-lo / s_div).astype(np.float32)), 0, ASYM_QMAX).astype(np.float32)
    ratio = (wg / s_div[..., None]).astype(np.float32)
    q = np.clip(np.rint(ratio) + z[..., None], 0, ASYM_QMAX).astype(np.uint8)
    return q.reshape(w.shape), s, z


def dequantize_sym(q: np.ndarray, s: np.ndarray, group_size: int = 128) -> np.ndarray:
    """w ≈ q * s, evaluated in float32 (one rounding per element)."""
    qg = _grouped(q.astype(np.float32), group_size)
    return (qg * s.astype(np.float32)[..., None]).reshape(q.shape)


def dequantize_asym(q: np.ndarray, s: np.ndarray, z: np.ndarray, group_size: int = 128) -> np.ndarray:
    """w ≈ (q - z) * s, evaluated in float32."""
    qg = _grouped(q.astype(np.float32), group_size)
    return ((qg - z.astype(np.float32)[..., None]) * s.astype(np.float32)[..., None]).reshape(q.shape)


def fake_quantize(w: np.ndarray, group_size: int = 128, sym: bool = True) -> np.ndarray:
    """4-bit RTN quantize-then-dequantize."""
    if sym:
        q, s = quantize_sym(w, group_size)
        return dequantize_sym(q, s, group_size)
    q, s, z = quantize_asym(w, group_size)
    return dequantize_asym(q, s, z, group_size)


def pack_int4(q: np.ndarray) -> np.ndarray:
    """Flat packing: byte i = (q[2i] & 0xF) | (q[2i+1] & 0xF) << 4."""
    flat = np.asarray(q).reshape(-1).astype(np.int64)
    if flat.size % 2:
        raise ValueError("Total elements must be even for int4 packing")
    return ((flat[0::2] & 0xF) | ((flat[1::2] & 0xF) << 4)).astype(np.uint8)


def unpack_int4(packed: np.ndarray, n: int, signed: bool = True) -> np.ndarray:
    """Inverse of pack_int4; signed nibbles are two's complement (8..15 -> -8..-1)."""
    b = np.asarray(packed, dtype=np.uint8).reshape(-1).astype(np.int64)
    out = np.stack([b & 0xF, b >> 4], axis=-1).reshape(-1)[:n]
    if signed:
        return (out - 16 * (out >= 8)).astype(np.int8)
    return out.astype(np.uint8)


def pack_rows(q: np.ndarray) -> np.ndarray:
    """Row-wise nibble packing used by the kernels: [N, K] -> uint8 [N, K/2],
    lo nibble = even column, hi nibble = odd column."""
    q = np.asarray(q)
    n, k = q.shape
    return pack_int4(q).reshape(n, k // 2)


def unpack_rows(packed: np.ndarray, signed: bool) -> np.ndarray:
    n, kh = packed.shape
    return unpack_int4(packed, n * kh * 2, signed=signed).reshape(n, kh * 2)


def pack_weights_sym(w: np.ndarray, group_size: int = 128):
    """(packed uint8 [N,K/2], scales float32 [N,K/g]) — symmetric."""
    q, s = quantize_sym(np.asarray(w, dtype=np.float32), group_size)
    return pack_rows(q), s


def pack_weights_asym(w: np.ndarray, group_size: int = 128):
    """(packed uint8 [N,K/2], scales float32 [N,K/g], zeros float32 [N,K/g])."""
    q, s, z = quantize_asym(np.asarray(w, dtype=np.float32), group_size)
    return pack_rows(q), s, z


def dequant_packed(packed: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None,
                   group_size: int, dtype=np.float64) -> np.ndarray:
    """Dequantized weight matrix [N, K] from the packed form, in `dtype`.

    In float64 the products q*s and (q-z)*s are exact for fp16 or fp32 scales,
    so this is the exact real-valued weight the kernels are meant to apply.
    """
    signed = zeros is None
    q = unpack_rows(packed, signed=signed).astype(dtype)
    g = group_size
    n, k = q.shape
    qg = q.reshape(n, k // g, g)
    s = np.asarray(scales, dtype=dtype)[..., None]
    if zeros is not None:
        qg = qg - np.asarray(zeros, dtype=dtype)[..., None]
    return (qg * s).reshape(n, k)
