"""Group-wise int8 KV cache on the device — the counterpart of the reference's
`siliconfer.model.kv_cache` (/root/reference/siliconfer/model/kv_cache.py:49-126).

Per (b, head, t) vector over head_dim: s = max|x| / 127 (1 if the vector is
zero), code = clip(rint(x / s), -128, 127), all in fp32 (kv_cache.py:59-63).
The reference grows its cache by concatenation every step and returns the
whole cache dequantized (kv_cache.py:99-105); here the codes go into a
preallocated buffer at the current length by one HIP kernel
(`sf_kv_quant_append`), and the fused decode attention reads them in place.
`update()` still returns the dequantized cache for callers that want the
reference's behaviour; `append()` skips that.

Scales are stored as fp16 by default (scale_dtype=torch.float32 keeps the
reference's fp32 scales).
"""

from __future__ import annotations

import torch

from .. import _lib
from .._lib import SFError


def _append(k: torch.Tensor, v: torch.Tensor, qk, sk, qv, sv, t_off: int) -> None:
    for t, n in ((k, "k"), (v, "v")):
        _lib.require_device(t, n)
    B, KVH, Tn, D = k.shape
    if v.shape != k.shape:
        raise SFError("k and v must have the same shape")
    if k.dtype not in (torch.float16, torch.bfloat16, torch.float32) or v.dtype != k.dtype:
        raise SFError(f"unsupported KV dtype {k.dtype}")
    T_cap = qk.shape[2]
    rc = _lib.load().sf_kv_quant_append(k.data_ptr(), v.data_ptr(), _lib.dt(k), qk.data_ptr(),
                                        sk.data_ptr(), qv.data_ptr(), sv.data_ptr(), _lib.dt(sk),
                                        B, KVH, Tn, t_off, T_cap, D, _lib.stream(k))
    _lib.check(rc, "sf_kv_quant_append")


def quantize_kv(x: torch.Tensor, scale_dtype: torch.dtype = torch.float32):
    """Symmetric int8 quantization, one scale per (b, head, token) vector.
    x [B, KVH, T, D] -> (codes int8 [B, KVH, T, D], scales [B, KVH, T, 1])."""
    x = x.contiguous()
    B, KVH, T, D = x.shape
    qk = torch.empty((B, KVH, T, D), dtype=torch.int8, device=x.device)
    sk = torch.empty((B, KVH, T), dtype=scale_dtype, device=x.device)
    # the append kernel quantizes K and V in one launch; quantize x as both
    qv = torch.empty_like(qk)
    sv = torch.empty_like(sk)
    _append(x, x, qk, sk, qv, sv, 0)
    return qk, sk.unsqueeze(-1)


def dequantize_kv(q: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype = torch.float16):
    """Inverse of quantize_kv: q * scale, in `dtype`."""
    s = scale if scale.dim() == q.dim() else scale.unsqueeze(-1)
    return (q.float() * s.float()).to(dtype)


class QuantizedKVCache:
    """Per-layer int8 KV cache in preallocated device buffers.

    `capacity` is the maximum number of positions (grown by doubling if an
    update would overflow and `growable` is set). Buffers are allocated on the
    first update, when batch, heads, head_dim and device are known.
    """

    def __init__(self, capacity: int = 4096, scale_dtype: torch.dtype = torch.float16,
                 growable: bool = True) -> None:
        self.capacity = int(capacity)
        self.scale_dtype = scale_dtype
        self.growable = growable
        self._len = 0
        self._qk = self._sk = self._qv = self._sv = None

    # -- reference API ------------------------------------------------------
    def length(self) -> int:
        return self._len

    @property
    def q_k(self):
        return None if self._qk is None else self._qk[:, :, :self._len]

    @property
    def s_k(self):
        return None if self._sk is None else self._sk[:, :, :self._len].unsqueeze(-1)

    @property
    def q_v(self):
        return None if self._qv is None else self._qv[:, :, :self._len]

    @property
    def s_v(self):
        return None if self._sv is None else self._sv[:, :, :self._len].unsqueeze(-1)

    def update(self, k: torch.Tensor, v: torch.Tensor):
        """Quantize and append new (k, v) [B, KVH, T_new, D]; return the full
        dequantized cache in k's dtype (the reference's contract)."""
        self.append(k, v)
        return (dequantize_kv(self.q_k, self.s_k, k.dtype),
                dequantize_kv(self.q_v, self.s_v, k.dtype))

    def trim(self, n: int) -> None:
        """Keep the first n positions."""
        self._len = max(0, min(int(n), self._len))

    def nbytes(self) -> int:
        """Footprint of the valid prefix (codes + scales), as the reference reports it."""
        if self._qk is None:
            return 0
        B, KVH, _, D = self._qk.shape
        es = torch.empty((), dtype=self.scale_dtype).element_size()
        return 2 * B * KVH * self._len * (D + es)

    # -- device-resident fast path -------------------------------------------
    def reserve(self, B: int, KVH: int, D: int, need: int, device) -> None:
        """Make the buffers hold at least `need` positions of [B, KVH, *, D]
        (allocating them on first use) without appending anything."""
        self._ensure(torch.empty((B, KVH, 0, D), device=device), need)

    def set_length(self, n: int) -> None:
        """Mark the first n positions valid (a kernel wrote them in place)."""
        if self._qk is None or not 0 <= n <= self._qk.shape[2]:
            raise SFError(f"length {n} outside the cache's buffers")
        self._len = int(n)

    def _ensure(self, k: torch.Tensor, need: int) -> None:
        B, KVH, _, D = k.shape
        if self._qk is not None:
            if self._qk.shape[0] != B or self._qk.shape[1] != KVH or self._qk.shape[3] != D:
                raise SFError("KV cache shape changed between updates")
            if need <= self._qk.shape[2]:
                return
            if not self.growable:
                raise SFError(f"KV cache overflow: {need} > capacity {self._qk.shape[2]}")
        cap = max(self.capacity, 1)
        while cap < need:
            cap *= 2
        qk = torch.empty((B, KVH, cap, D), dtype=torch.int8, device=k.device)
        sk = torch.empty((B, KVH, cap), dtype=self.scale_dtype, device=k.device)
        qv, sv = torch.empty_like(qk), torch.empty_like(sk)
        if self._qk is not None and self._len:
            qk[:, :, :self._len].copy_(self._qk[:, :, :self._len])
            sk[:, :, :self._len].copy_(self._sk[:, :, :self._len])
            qv[:, :, :self._len].copy_(self._qv[:, :, :self._len])
            sv[:, :, :self._len].copy_(self._sv[:, :, :self._len])
        self._qk, self._sk, self._qv, self._sv = qk, sk, qv, sv
        self.capacity = cap

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Quantize new (k, v) straight into the buffers at the current length."""
        k = k.contiguous()
        v = v.contiguous()
        self._ensure(k, self._len + k.shape[2])
        _append(k, v, self._qk, self._sk, self._qv, self._sv, self._len)
        self._len += k.shape[2]

    def buffers(self):
        """(k_codes, k_scales, v_codes, v_scales) full-capacity buffers."""
        return self._qk, self._sk, self._qv, self._sv


def make_quantized_cache(n_layers: int, capacity: int = 4096,
                         scale_dtype: torch.dtype = torch.float16) -> list[QuantizedKVCache]:
    """One fresh QuantizedKVCache per transformer layer."""
    return [QuantizedKVCache(capacity, scale_dtype) for _ in range(n_layers)]
