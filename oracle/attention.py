"""Oracle for the int8 KV cache and the fused decode attention over it.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).

What the reference computes (/root/reference):
  quantize_kv       siliconfer/model/kv_cache.py:49-63 — per (b, head, t) vector
                    over head_dim: s = max|x|/127 (1 if max|x| == 0), fp32;
                    q = clip(round(x/s), -128, 127) int8.
  dequantize_kv     siliconfer/model/kv_cache.py:66-68 — q * s.
  decode attention  siliconfer/kernels/metal/q4_attention.py:200-261 — for one
                    query token per (b, h): softmax(q . K^T / sqrt(D)) . V with
                    K = k_codes * k_scale per token (likewise V), GQA mapping
                    kv_head = h // (H / KVH) (:103), all T positions visible.
  split-T combine   q4_attention.py:63-70, 256-261 — per tile (m, l, acc),
                    M = max m; L = sum l e^(m-M); out = sum acc e^(m-M) / max(L, 1e-20).
  _choose_n_tiles   q4_attention.py:183-197.

The reference tests pin the fused kernel against "dequantize the int8 cache,
then scaled-dot-product attention" (tests/test_metal_attention.py:21-32); the
oracle is exactly that, in float64.

Pinning (tests/test_oracle_attention.py): T=1 returns V[0] exactly; uniform
keys give the mean of V; the split-T combine equals the unsplit softmax for
every split count in the reference's own list (1,2,3,7,16,64,200); GQA equals
MHA with repeated K/V heads; the quantize_kv closed form (zero vector -> s=1,
q=0; |q| <= 127 and -128 never produced; incremental == batch quantization,
tests/test_kv_cache.py:62-81).
"""

from __future__ import annotations

import math

import numpy as np


def quantize_kv(x: np.ndarray):
    """(codes int8, scales float32 [..., 1]) with the reference's fp32 arithmetic."""
    x32 = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x32), axis=-1, keepdims=True)
    s = np.where(amax == np.float32(0), np.float32(1), (amax / np.float32(127))).astype(np.float32)
    q = np.clip(np.rint((x32 / s).astype(np.float32)), -128, 127).astype(np.int8)
    return q, s


def dequantize_kv(q: np.ndarray, s: np.ndarray, dtype=np.float64) -> np.ndarray:
    s = np.asarray(s, dtype=np.float64)
    if s.ndim == q.ndim - 1:
        s = s[..., None]
    return (q.astype(np.float64) * s).astype(dtype)


def attention_decode(q: np.ndarray, k_codes: np.ndarray, k_scales: np.ndarray,
                     v_codes: np.ndarray, v_scales: np.ndarray,
                     scale: float | None = None, T: int | None = None) -> np.ndarray:
    """Textbook single-query attention over the dequantized int8 cache, float64.

    q [B, H, D]; codes [B, KVH, Tcap, D]; scales [B, KVH, Tcap] or [..., 1].
    Only the first T positions (default: all) are visible.
    Returns [B, H, D] float64.
    """
    q = np.asarray(q, dtype=np.float64)
    B, H, D = q.shape
    KVH = k_codes.shape[1]
    if T is None:
        T = k_codes.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    K = dequantize_kv(k_codes[:, :, :T], np.asarray(k_scales).reshape(B, KVH, -1)[:, :, :T])
    V = dequantize_kv(v_codes[:, :, :T], np.asarray(v_scales).reshape(B, KVH, -1)[:, :, :T])
    grp = H // KVH
    out = np.zeros((B, H, D), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            kh = h // grp
            s = (K[b, kh] @ q[b, h]) * scale          # [T]
            s = s - s.max()
            p = np.exp(s)
            out[b, h] = (p @ V[b, kh]) / p.sum()
    return out


def split_partials(q, k_codes, k_scales, v_codes, v_scales, n_tiles: int, scale=None):
    """Per-tile un-normalised partials (m, l, acc) with the reference's tiling:
    tile_size = ceil(T / n_tiles) (q4_attention.py:231-234). Empty tiles give
    m = -inf, l = 0, acc = 0."""
    q = np.asarray(q, dtype=np.float64)
    B, H, D = q.shape
    KVH = k_codes.shape[1]
    T = k_codes.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    n_tiles = max(1, min(n_tiles, T))
    ts = -(-T // n_tiles)
    K = dequantize_kv(k_codes, np.asarray(k_scales).reshape(B, KVH, T))
    V = dequantize_kv(v_codes, np.asarray(v_scales).reshape(B, KVH, T))
    grp = H // KVH
    m = np.full((B, H, n_tiles), -np.inf)
    l = np.zeros((B, H, n_tiles))
    acc = np.zeros((B, H, n_tiles, D))
    for b in range(B):
        for h in range(H):
            kh = h // grp
            for i in range(n_tiles):
                t0, t1 = i * ts, min((i + 1) * ts, T)
                if t0 >= t1:
                    continue
                s = (K[b, kh, t0:t1] @ q[b, h]) * scale
                m[b, h, i] = s.max()
                p = np.exp(s - m[b, h, i])
                l[b, h, i] = p.sum()
                acc[b, h, i] = p @ V[b, kh, t0:t1]
    return m, l, acc


def combine(m: np.ndarray, l: np.ndarray, acc: np.ndarray) -> np.ndarray:
    """Flash combine across the tile axis (q4_attention.py:256-261)."""
    M = np.max(m, axis=2, keepdims=True)
    c = np.exp(m - M)
    L = np.sum(l * c, axis=2)
    ACC = np.sum(acc * c[..., None], axis=2)
    return ACC / np.maximum(L, 1e-20)[..., None]


def choose_n_tiles(T_cache: int, min_tile_size: int = 16, max_tiles: int = 256) -> int:
    """Reference default split heuristic (q4_attention.py:183-197)."""
    if T_cache <= min_tile_size:
        return 1
    return min(max_tiles, -(-T_cache // min_tile_size))
