"""Transformer layers as modules over the device kernels — the counterpart of
the reference's `siliconfer.model.layers` (/root/reference/siliconfer/model/
layers.py): RMSNorm (:14-21), the RoPE frequencies and rotation (:24-66),
grouped-query Attention (:69-129), the SwiGLU MLP (:132-144) and
TransformerBlock (:147-163), with the same constructor arguments and call
contracts, for callers that compose their own layers instead of running the
fixed decoder (`LlamaModel`).

Projections are `Q4Linear` (after `from_weights` on a packed checkpoint, or
assigned by the caller) or dense `torch.nn.Linear` modules, as the
reference's are before `_pack_and_replace_linears`. With a
`QuantizedKVCache` at batch 1, an attention call runs the decoder's kernels:
RoPE and the int8 append of k and v in one launch (`sf_rope_kv_append`),
then the split-T decode attention for one new token or the causal prefill
attention for several, both reading the codes in place. The reference's
other cache forms — none, or a (k, v) tuple of full-precision tensors — and
batches above one with an int8 cache take the reference's own route on the
device: RoPE, concatenation (or the int8 append and the dequantized cache)
and softmax attention with the causal mask, in fp32 torch operations.

Activations: projections return fp32 (Q4Linear's contract); RMSNorm returns
its input's dtype; the block's residual stream is kept in the input's dtype.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from .. import _lib
from .._lib import SFError
from .config import ModelConfig, rope_freqs as _rope_freqs_np
from .kv_cache import QuantizedKVCache, dequantize_kv
from .q4_linear import Q4Linear


def _on_device(x: torch.Tensor) -> None:
    if not x.is_cuda:
        raise SFError(f"layer input must be a device tensor (got {x.device}); these layers run "
                      "only on the GPU kernels")


class RMSNorm(torch.nn.Module):
    """x * rsqrt(mean(x^2) + eps) * weight over the last dimension
    (layers.py:14-21), by `sf_rmsnorm` in fp32; the output has x's dtype."""

    def __init__(self, dim: int, eps: float = 1e-5, device=None) -> None:
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(dim, dtype=torch.float32, device=device),
                                         requires_grad=False)
        self.eps = float(eps)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _on_device(x)
        dim = self.weight.numel()
        if x.shape[-1] != dim:
            raise SFError(f"RMSNorm over {dim} features got {x.shape[-1]}")
        x32 = x.reshape(-1, dim).to(torch.float32).contiguous()  # read only (no delta)
        dt = x.dtype if x.dtype in (torch.float16, torch.bfloat16, torch.float32) else torch.float32
        out = torch.empty(x32.shape, dtype=dt, device=x.device)
        w = self.weight.detach().contiguous()
        _lib.check(_lib.load().sf_rmsnorm(x32.data_ptr(), None, w.data_ptr(), _lib.SF_F32, out.data_ptr(),
                                          _lib.dt(out), x32.shape[0], dim, self.eps, _lib.stream(x)),
                   "sf_rmsnorm")
        return out.reshape(x.shape)


def compute_rope_freqs(config: ModelConfig, device=None) -> torch.Tensor:
    """RoPE frequencies 1 / theta^(2i / D), with Llama-3 scaling when the
    config asks for it (layers.py:24-55), fp32 [D / 2]."""
    return torch.as_tensor(_rope_freqs_np(config), dtype=torch.float32, device=device)


def apply_rope(x: torch.Tensor, offset: int, freqs: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of x [B, heads, T, D] at positions offset .. offset + T - 1
    (layers.py:58-66), in fp32 on x's device; returns x's dtype."""
    T, D = x.shape[2], x.shape[3]
    f = freqs.to(device=x.device, dtype=torch.float32)
    pos = torch.arange(offset, offset + T, dtype=torch.float32, device=x.device)
    ang = torch.outer(pos, f)
    c = torch.cat([torch.cos(ang), torch.cos(ang)], dim=-1)[None, None]
    s = torch.cat([torch.sin(ang), torch.sin(ang)], dim=-1)[None, None]
    xf = x.float()
    rot = torch.cat([-xf[..., D // 2:], xf[..., :D // 2]], dim=-1)
    return (xf * c + rot * s).to(x.dtype)


def _host(a) -> np.ndarray:
    """A checkpoint array (numpy, or a torch tensor on any device) as numpy."""
    return a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else np.asarray(a)


def _f32(a) -> torch.Tensor:
    """A checkpoint array as an fp32 torch tensor (on its own device)."""
    return a.detach().float() if isinstance(a, torch.Tensor) else torch.from_numpy(np.asarray(a, np.float32))


def _dense(in_f: int, out_f: int, bias: bool, device) -> torch.nn.Linear:
    return torch.nn.Linear(in_f, out_f, bias=bias, device=device, dtype=torch.float32)


def _project(lin, x: torch.Tensor) -> torch.Tensor:
    """A projection's output in fp32 (Q4Linear returns fp32; a dense layer
    runs on fp32 input)."""
    if isinstance(lin, Q4Linear):
        return lin(x)
    return lin(x.float())


def _sdpa_causal(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, offset: int,
                 scale: float) -> torch.Tensor:
    """softmax(q k^T * scale + causal mask) v in fp32 for q [B, H, T, D] over
    k, v [B, KVH, offset + T, D] (GQA by repeating kv heads; layers.py:114-126)."""
    B, H, T, D = q.shape
    KVH = k.shape[1]
    k = k.float().repeat_interleave(H // KVH, dim=1)
    v = v.float().repeat_interleave(H // KVH, dim=1)
    s = torch.matmul(q.float(), k.transpose(-1, -2).contiguous()) * scale
    if T > 1:
        n = k.shape[2]
        rows = torch.arange(T, device=q.device)[:, None] + offset
        cols = torch.arange(n, device=q.device)[None, :]
        s = s.masked_fill(cols > rows, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v)


class Attention(torch.nn.Module):
    """Grouped-query attention (layers.py:69-129). `__call__(x, cache)` with x
    [B, T, hidden] returns (o_proj(attention) [B, T, hidden] fp32, cache)."""

    def __init__(self, config: ModelConfig, rope_freqs: torch.Tensor, device=None) -> None:
        super().__init__()
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.scale = self.head_dim ** -0.5
        self.rope_freqs = rope_freqs
        H, D, bias = config.hidden_size, self.head_dim, config.attention_bias
        self.q_proj = _dense(H, self.num_heads * D, bias, device)
        self.k_proj = _dense(H, self.num_kv_heads * D, bias, device)
        self.v_proj = _dense(H, self.num_kv_heads * D, bias, device)
        self.o_proj = _dense(self.num_heads * D, H, False, device)
        self._cos = self._sin = None

    def _tables(self, need: int, device) -> tuple[torch.Tensor, torch.Tensor]:
        """fp32 [P, D/2] tables of cos / sin(position * freq), P >= need, built
        as `config.rope_tables` builds them (fp32 angles, host cos / sin)."""
        if self._cos is None or self._cos.shape[0] < need or self._cos.device != device:
            P = 1 << max(6, math.ceil(math.log2(max(need, 1))))
            f = self.rope_freqs.detach().float().cpu().numpy()
            ang = np.outer(np.arange(P, dtype=np.float32), f).astype(np.float32)
            self._cos = torch.from_numpy(np.cos(ang).astype(np.float32)).to(device)
            self._sin = torch.from_numpy(np.sin(ang).astype(np.float32)).to(device)
        return self._cos, self._sin

    def forward(self, x: torch.Tensor, cache=None):
        _on_device(x)  # every route runs on the GPU; none on the host
        B, T, _ = x.shape
        H, KVH, D = self.num_heads, self.num_kv_heads, self.head_dim
        q = _project(self.q_proj, x)
        k = _project(self.k_proj, x)
        v = _project(self.v_proj, x)
        if isinstance(cache, QuantizedKVCache) and B == 1:
            out = self._int8_batch1(q, k, v, cache, T, x.device)
            return _project(self.o_proj, out.reshape(1, T, H * D)), cache
        q = q.reshape(B, T, H, D).transpose(1, 2)
        k = k.reshape(B, T, KVH, D).transpose(1, 2)
        v = v.reshape(B, T, KVH, D).transpose(1, 2)
        if isinstance(cache, QuantizedKVCache):
            offset = cache.length()
        elif cache is not None:
            offset = cache[0].shape[2]
        else:
            offset = 0
        q = apply_rope(q, offset, self.rope_freqs)
        k = apply_rope(k, offset, self.rope_freqs)
        if isinstance(cache, QuantizedKVCache):
            cache.append(k, v)
            kc, vc = dequantize_kv(cache.q_k, cache.s_k, torch.float32), dequantize_kv(cache.q_v, cache.s_v,
                                                                                    torch.float32)
            new_cache = cache
        elif cache is not None:
            kc = torch.cat([cache[0], k.to(cache[0].dtype)], dim=2)
            vc = torch.cat([cache[1], v.to(cache[1].dtype)], dim=2)
            new_cache = (kc, vc)
        else:
            kc, vc = k, v
            new_cache = (k, v)
        a = _sdpa_causal(q, kc, vc, offset, self.scale)
        return _project(self.o_proj, a.transpose(1, 2).reshape(B, T, H * D)), new_cache

    def _int8_batch1(self, q, k, v, cache: QuantizedKVCache, T: int, device) -> torch.Tensor:
        """RoPE + int8 append in one launch, then decode or causal prefill
        attention over the cache in place; returns [T, H, D] fp32."""
        H, KVH, D = self.num_heads, self.num_kv_heads, self.head_dim
        lib = _lib.load()
        offset = cache.length()
        cache.reserve(1, KVH, D, offset + T, device)
        kq, ks, vq, vs = cache.buffers()
        T_cap = kq.shape[2]
        cos_t, sin_t = self._tables(offset + T, device)
        qkv = torch.cat([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], dim=1).contiguous()
        q_rot = torch.empty((T, H, D), dtype=torch.float32, device=device)
        st = _lib.stream(qkv)
        _lib.check(lib.sf_rope_kv_append(qkv.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(), cos_t.shape[0],
                                         q_rot.data_ptr(), _lib.SF_F32, kq.data_ptr(), ks.data_ptr(),
                                         vq.data_ptr(), vs.data_ptr(), _lib.dt(ks), T, H, KVH, D, T_cap,
                                         None, offset, st), "sf_rope_kv_append")
        cache.set_length(offset + T)
        if T == 1:
            from ..kernels.attention import attention_decode
            return attention_decode(q_rot, kq, ks, vq, vs, T=offset + 1, scale=self.scale)
        out = torch.empty((T, H, D), dtype=torch.float32, device=device)
        _lib.check(lib.sf_attn_prefill_i8kv(q_rot.data_ptr(), _lib.SF_F32, kq.data_ptr(), ks.data_ptr(),
                                            vq.data_ptr(), vs.data_ptr(), _lib.dt(ks), out.data_ptr(),
                                            _lib.SF_F32, T, H, KVH, offset, T_cap, D, float(self.scale), st),
                   "sf_attn_prefill_i8kv")
        return out


class MLP(torch.nn.Module):
    """down_proj(silu(gate_proj(x)) * up_proj(x)) (layers.py:132-144); the
    SwiGLU activation by `sf_silu_mul`. Returns fp32."""

    def __init__(self, config: ModelConfig, device=None) -> None:
        super().__init__()
        H, I = config.hidden_size, config.intermediate_size
        self.gate_proj = _dense(H, I, False, device)
        self.up_proj = _dense(H, I, False, device)
        self.down_proj = _dense(I, H, False, device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _on_device(x)
        g = _project(self.gate_proj, x)
        u = _project(self.up_proj, x)
        I = g.shape[-1]
        gu = torch.cat([g.reshape(-1, I), u.reshape(-1, I)], dim=1).contiguous()
        act = torch.empty((gu.shape[0], I), dtype=torch.float32, device=x.device)
        _lib.check(_lib.load().sf_silu_mul(gu.data_ptr(), act.data_ptr(), _lib.SF_F32, gu.shape[0], I,
                                           _lib.stream(gu)), "sf_silu_mul")
        return _project(self.down_proj, act.reshape(*g.shape))


class TransformerBlock(torch.nn.Module):
    """x + attn(norm(x)), then + mlp(norm(x)) (layers.py:147-163)."""

    def __init__(self, config: ModelConfig, rope_freqs: torch.Tensor, device=None) -> None:
        super().__init__()
        self.self_attn = Attention(config, rope_freqs, device)
        self.mlp = MLP(config, device)
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps, device)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps, device)

    def forward(self, x: torch.Tensor, cache=None):
        h, new_cache = self.self_attn(self.input_layernorm(x), cache)
        x = x + h.to(x.dtype)
        x = x + self.mlp(self.post_attention_layernorm(x)).to(x.dtype)
        return x, new_cache

    @classmethod
    def from_weights(cls, config: ModelConfig, weights: dict, layer: int, rope_freqs: torch.Tensor,
                     group_size: int = 128, device=None) -> "TransformerBlock":
        """Layer `layer` of a checkpoint dict in the HuggingFace naming: packed
        projections (`<p>.q4_packed`, `.q4_scales`, `.q4_zeros`, as
        `pack_and_replace_linears` leaves them) become Q4Linear, dense ones
        (`<p>.weight`) torch Linear, biases and norm weights fp32."""
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        blk = cls(config, rope_freqs, dev)
        pre = f"model.layers.{layer}"
        for parent, mod in (("self_attn", blk.self_attn), ("mlp", blk.mlp)):
            for name in (("q_proj", "k_proj", "v_proj", "o_proj") if parent == "self_attn"
                         else ("gate_proj", "up_proj", "down_proj")):
                p = f"{pre}.{parent}.{name}"
                b = weights.get(p + ".bias")
                if p + ".q4_packed" in weights:
                    z = weights.get(p + ".q4_zeros")
                    lin = Q4Linear(_host(weights[p + ".q4_packed"]),
                                   _host(weights[p + ".q4_scales"]).astype(np.float32),
                                   None if z is None else _host(z),
                                   None if b is None else _f32(b), group_size, device=dev)
                else:
                    W = _f32(weights[p + ".weight"])
                    lin = _dense(W.shape[1], W.shape[0], b is not None, dev)
                    with torch.no_grad():
                        lin.weight.copy_(W)
                        if b is not None:
                            lin.bias.copy_(_f32(b))
                setattr(mod, name, lin)
        with torch.no_grad():
            blk.input_layernorm.weight.copy_(_f32(weights[f"{pre}.input_layernorm.weight"]))
            blk.post_attention_layernorm.weight.copy_(_f32(weights[f"{pre}.post_attention_layernorm.weight"]))
        return blk
