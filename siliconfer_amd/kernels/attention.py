"""Fused decode attention over the int8 KV cache — the HIP counterpart of the
reference's `siliconfer.kernels.metal.q4_attention`
(/root/reference/siliconfer/kernels/metal/q4_attention.py:183-261).

`fused_quantized_attention_decode(q, k_codes, k_scales, v_codes, v_scales,
n_tiles=None)` keeps the reference's signature, shapes and result:
q [B, H, D]; codes int8 [B, KVH, T, D]; scales [B, KVH, T] or [B, KVH, T, 1]
(fp32 as the reference stores them, or fp16 as this build's cache does);
returns float32 [B, H, D]. `n_tiles` is the split-T count with the reference's
tiling (tile = ceil(T / n_tiles)); by default this build picks its own split
count for MI355X (`default_splits`, which depends on the head dim) rather than
`_choose_n_tiles`, which is kept for callers and tests that use it.
"""

from __future__ import annotations

import math

import torch

from .. import _lib
from .._lib import SFError

_MAX_HEAD_DIM = 256


def _choose_n_tiles(T_cache: int, min_tile_size: int = 16, max_tiles: int = 256) -> int:
    """The reference's split heuristic (q4_attention.py:183-197)."""
    if T_cache <= min_tile_size:
        return 1
    return min(max_tiles, -(-T_cache // min_tile_size))


def default_splits(B: int, n_kv_heads: int, T: int, head_dim: int = 64) -> int:
    """The split count `attention_decode` picks when none is given
    (sf_attn_default_splits_d: one split up to a head_dim-dependent cache
    length, then about 128 tokens per split)."""
    return int(_lib.load().sf_attn_default_splits_d(B, n_kv_heads, T, head_dim))


_workspaces: dict = {}


def workspace(device: torch.device, stream_handle: int, nbytes: int) -> torch.Tensor:
    """Attention workspace (the split partials), one per (device, stream), grown
    on demand; nothing in it needs clearing between calls."""
    key = (device, stream_handle)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def attention_decode(q: torch.Tensor, k_codes: torch.Tensor, k_scales: torch.Tensor,
                     v_codes: torch.Tensor, v_scales: torch.Tensor, T: int | None = None,
                     n_splits: int | None = None, scale: float | None = None,
                     out: torch.Tensor | None = None,
                     out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Decode attention of q [B, H, D] over the first T positions of a cache
    whose codes are [B, KVH, T_cap, D] and scales [B, KVH, T_cap] (contiguous)."""
    if q.dim() != 3:
        raise SFError("q must be [B, n_heads, head_dim]")
    B, H, D = q.shape
    if k_codes.dim() != 4 or k_codes.shape != v_codes.shape:
        raise SFError("k_codes / v_codes must both be [B, n_kv_heads, T, head_dim]")
    KVH, T_cap = k_codes.shape[1], k_codes.shape[2]
    if k_codes.shape[0] != B or k_codes.shape[3] != D:
        raise SFError("cache shape does not match q")
    if D > _MAX_HEAD_DIM:
        raise ValueError(f"head_dim={D} exceeds kernel's compile-time max {_MAX_HEAD_DIM}")
    if T is None:
        T = T_cap
    ks = k_scales.reshape(B, KVH, T_cap)
    vs = v_scales.reshape(B, KVH, T_cap)
    if ks.dtype != vs.dtype or ks.dtype not in (torch.float16, torch.float32):
        raise SFError("k/v scales must both be float16 or both float32")
    if k_codes.dtype != torch.int8 or v_codes.dtype != torch.int8:
        raise SFError("KV codes must be int8")
    for t, n in ((q, "q"), (k_codes, "k_codes"), (v_codes, "v_codes"), (ks, "k_scales"),
                 (vs, "v_scales")):
        _lib.require_device(t, n)
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        q = q.float()
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    lib = _lib.load()
    if n_splits is None or n_splits <= 0:
        n_splits = default_splits(B, KVH, T, D)
    n_splits = max(1, min(int(n_splits), max(T, 1), 512))
    ws_bytes = lib.sf_attn_workspace_bytes(B, H, D, n_splits)
    st = _lib.stream(q)
    ws = workspace(q.device, st, ws_bytes)
    if out is None:
        out = torch.empty((B, H, D), dtype=out_dtype, device=q.device)
    rc = lib.sf_attn_decode_i8kv(q.data_ptr(), _lib.dt(q), k_codes.data_ptr(), ks.data_ptr(),
                                 v_codes.data_ptr(), vs.data_ptr(), _lib.dt(ks), out.data_ptr(),
                                 _lib.dt(out), ws.data_ptr(), ws.numel(), B, H, KVH, T, T_cap, D,
                                 float(scale), n_splits, st)
    _lib.check(rc, "sf_attn_decode_i8kv")
    return out


def fused_quantized_attention_decode(q, k_codes, k_scales, v_codes, v_scales,
                                     n_tiles: int | None = None) -> torch.Tensor:
    """Fused decode-phase attention over an int8-quantized KV cache (reference
    q4_attention.py:200-261): softmax(q K^T / sqrt(D)) V, float32 [B, H, D]."""
    q = q.contiguous()
    return attention_decode(q, k_codes.contiguous(), k_scales.contiguous(), v_codes.contiguous(),
                            v_scales.contiguous(), n_splits=n_tiles)
