"""Oracle for the end-to-end decoder.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).

A numpy fp32 restatement of the reference's forward pass over int4 weights
and an int8 KV cache:

  RMSNorm           siliconfer/model/layers.py:14-21 (mx.fast.rms_norm):
                    x * 1/sqrt(mean(x^2) + eps) * w
  RoPE              layers.py:24-66: freqs 1/theta^(2i/D) (fp32), angles
                    position * freq, x * [cos, cos] + [-x2, x1] * [sin, sin]
  Attention         layers.py:72-133: q/k/v projections (+bias), RoPE on q and
                    k at offset = cache length, k and v through the int8 cache
                    (kv_cache.py:49-68, 90-105: per (head, token) s = max|x|/127,
                    codes rint(x/s); the cache here stores s in fp16, as the
                    build's cache does), SDPA over the dequantized cache with a
                    causal mask for T > 1 and scale 1/sqrt(D), o projection
  MLP               layers.py:136-144: down(silu(gate(x)) * up(x))
  block             layers.py:157-163: x + attn(norm(x)); x + mlp(norm(x))
  model             llama.py:55-79: embedding, blocks, final norm, logits
                    through the tied embedding (as_linear) or lm_head
  greedy            generate.py:45-46: argmax of the last row

Weights come dequantized (fp32 codes * fp16 scale) from
`LlamaModel.export_weights`, so projections are plain fp32 matmuls, as the
reference's Q4Linear computes them (fp32 activations, q4_linear.py:49-68).

Pinning (tests/test_model_oracle.py): RMSNorm closed form; RoPE at position 0
is the identity and preserves each pair's norm; attention over one cached
token returns its V and equals a per-row loop; a causal block equals the same
tokens fed one by one; and the whole forward pass equals a scalar, per-element
restatement of the reference's layers on a tiny model, which planted mistakes
(gate and up swapped, sigmoid for SiLU, a dropped residual, RoPE on
interleaved pairs or with the sine's sign flipped, the wrong GQA head) fail.
"""

from __future__ import annotations

import numpy as np

from . import attention as A


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, np.float32)
    ms = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    return (x * (np.float32(1.0) / np.sqrt(ms + np.float32(eps)))).astype(np.float32) * w.astype(np.float32)


def rope(x: np.ndarray, positions: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray) -> np.ndarray:
    """x [T, heads, D] rotated at the given absolute positions (tables fp32 [P, D/2])."""
    D = x.shape[-1]
    half = D // 2
    c = cos_t[positions][:, None, :]
    s = sin_t[positions][:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1).astype(np.float32)


class KVCache:
    """Per-layer int8 codes with fp16-stored scales, batch 1: [KVH, T, D]."""

    def __init__(self, n_layers: int):
        self.k = [None] * n_layers
        self.v = [None] * n_layers

    def append(self, layer: int, k: np.ndarray, v: np.ndarray):
        """k, v [T, KVH, D] fp32 -> appended; returns dequantized full K, V [KVH, T_all, D]."""
        out = []
        for which, x in (("k", k), ("v", v)):
            codes, s = A.quantize_kv(np.transpose(x, (1, 0, 2)))  # [KVH, T, D], [KVH, T, 1]
            s16 = s.astype(np.float16).astype(np.float32)
            store = getattr(self, which)
            prev = store[layer]
            if prev is None:
                store[layer] = (codes, s16)
            else:
                store[layer] = (np.concatenate([prev[0], codes], axis=1),
                                np.concatenate([prev[1], s16], axis=1))
            c, sc = store[layer]
            out.append(c.astype(np.float32) * sc)
        return out[0], out[1]

    def length(self) -> int:
        return 0 if self.k[0] is None else self.k[0][0].shape[1]


def attend(q: np.ndarray, K: np.ndarray, V: np.ndarray, pos0: int, scale: float) -> np.ndarray:
    """q [T, H, D] at positions pos0..pos0+T-1 over K, V [KVH, T_all, D]
    (causal: row t sees keys 0..pos0+t; GQA head h reads kv head h // (H/KVH)).
    float64 scores and softmax, one head at a time over all rows."""
    T, H, D = q.shape
    KVH, n_all = K.shape[0], pos0 + T
    G = H // KVH
    visible = np.arange(n_all)[None, :] <= (pos0 + np.arange(T))[:, None]  # [T, n_all]
    out = np.empty((T, H, D), np.float32)
    for h in range(H):
        kh = K[h // G, :n_all].astype(np.float64)
        vh = V[h // G, :n_all].astype(np.float64)
        s = (q[:, h].astype(np.float64) @ kh.T) * scale
        s = np.where(visible, s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p @ vh) / p.sum(axis=1, keepdims=True)
    return out


def swiglu(gu: np.ndarray, inter: int) -> np.ndarray:
    """silu(gate) * up for gate|up rows [T, 2 * inter] (layers.py:143-144)."""
    g, u = gu[:, :inter], gu[:, inter:]
    return (g / (np.float32(1.0) + np.exp(-g))) * u


def residual(x: np.ndarray, delta: np.ndarray) -> np.ndarray:
    """The block's residual add (layers.py:157-163)."""
    return x + delta


def dense(L: dict, name: str, x: np.ndarray) -> np.ndarray:
    """Projection `name` of layer dict L over rows x: x @ W.T with the
    dequantized fp32 weight (Q4Linear's math, q4_linear.py:49-68)."""
    return x @ L[name].T


def forward(weights: dict, cfg, ids, cache: KVCache, cos_t: np.ndarray, sin_t: np.ndarray,
            last_rows: int | None = None, linear=dense) -> np.ndarray:
    """Run tokens `ids` (appending to `cache`) and return the logits of every
    row [T, V], or of the last `last_rows` rows only. `linear(L, name, x)`
    computes each projection (default: `dense`; the CPU baseline passes the
    reference's own int4 kernel over the packed weights)."""
    ids = np.asarray(ids, dtype=np.int64).reshape(-1)
    T = ids.size
    H, Hq, KVH, D = cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    pos0 = cache.length()
    pos = np.arange(pos0, pos0 + T)
    eps = cfg.rms_norm_eps
    x = weights["embed"][ids].astype(np.float32)
    for l, L in enumerate(weights["layers"]):
        xn = rmsnorm(x, L["w_in"], eps)
        qkv = linear(L, "qkv", xn)
        if L["qkv_bias"] is not None:
            qkv = qkv + L["qkv_bias"]
        q = qkv[:, :Hq * D].reshape(T, Hq, D)
        k = qkv[:, Hq * D:(Hq + KVH) * D].reshape(T, KVH, D)
        v = qkv[:, (Hq + KVH) * D:].reshape(T, KVH, D)
        q = rope(q, pos, cos_t, sin_t)
        k = rope(k, pos, cos_t, sin_t)
        K, V = cache.append(l, k, v.astype(np.float32))
        a = attend(q, K, V, pos0, D ** -0.5).reshape(T, Hq * D)
        x = residual(x, linear(L, "o", a))
        xn = rmsnorm(x, L["w_post"], eps)
        act = swiglu(linear(L, "gate_up", xn), cfg.intermediate_size)
        x = residual(x, linear(L, "down", act))
    if last_rows is not None:
        x = x[-last_rows:]
    xn = rmsnorm(x, weights["norm"], eps)
    return (xn @ weights.get("lm_head", weights["embed"]).T).astype(np.float32)


def greedy(logits_row: np.ndarray) -> int:
    return int(np.argmax(logits_row))
