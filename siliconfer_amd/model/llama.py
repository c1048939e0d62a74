"""Decoder runner on MI355X — the reference's `LlamaModel` / `TransformerBlock`
(/root/reference/siliconfer/model/llama.py:20-93,
/root/reference/siliconfer/model/layers.py:72-163) with every projection an
int4 `Q4Linear` weight and an int8 `QuantizedKVCache`, batch 1.

The forward pass is the reference's, restated over this build's kernels:

  embed -> per layer: RMSNorm -> q|k|v projection (+bias) -> RoPE + int8 KV
  append -> attention over the int8 cache -> o projection + residual ->
  RMSNorm -> gate|up projection -> silu(gate) * up -> down projection +
  residual -> final RMSNorm -> tied-embedding logits -> greedy token.

Differences of form, not of result:
  * q/k/v and gate/up are each one fused int4 weight (rows concatenated; the
    per-row groups quantize identically);
  * the residual add after o / down rides in the GEMV as its bias (decode) or
    in the next RMSNorm (prefill);
  * the residual stream is fp32; projections run on `act_dtype` activations
    (fp32 by default, like the reference's `Q4Linear`, which casts to fp32);
  * decode positions and the greedy token stay on the device, so a decode
    step is one HIP-graph replay with no host round trip (`capture`).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from .. import _lib
from .._lib import SFError
from ..kernels.q4 import Q4Weight
from .config import ModelConfig, rope_tables

_DT = {torch.float32: _lib.SF_F32, torch.float16: _lib.SF_F16, torch.bfloat16: _lib.SF_BF16}
# sf_q4_gemm runs up to this many rows as 8-row batch GEMVs (no K split)
GEMM_GEMV_ROWS = 16


def pack_sym_device(W: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric RTN int4 of a device fp32 matrix, packed like
    `siliconfer_amd.kernels.pack_weights_sym` (scale = max|w| / 7 per group,
    q = clip(round(w / scale), -8, 7), low nibble = even column): returns
    (packed uint8 [N, K/2], scales fp32 [N, K/g]) on the same device. Same
    IEEE fp32 division and round-half-even as the numpy packer, so the codes
    agree bit for bit."""
    N, K = W.shape
    if K % group_size:
        raise SFError("in_features must be divisible by group_size")
    g = W.float().reshape(N, K // group_size, group_size)
    amax = g.abs().amax(dim=-1, keepdim=True)
    # a tensor divisor: torch divides by a Python scalar through its reciprocal
    scale = amax / torch.full_like(amax, 7.0)
    safe = torch.where(scale == 0, torch.ones_like(scale), scale)
    q = torch.round(g / safe).clamp_(-8, 7).to(torch.int8).reshape(N, K)
    lo = q[:, 0::2].to(torch.uint8) & 0x0F
    hi = q[:, 1::2].to(torch.uint8) & 0x0F
    return (lo | (hi << 4)).contiguous(), scale[..., 0].contiguous()


@dataclass
class LayerWeights:
    qkv: Q4Weight
    qkv_bias: torch.Tensor | None  # fp32 [(H + 2 KVH) * D]
    o: Q4Weight
    gate_up: Q4Weight
    down: Q4Weight
    w_in: torch.Tensor    # fp32 [hidden]
    w_post: torch.Tensor  # fp32 [hidden]


@dataclass
class GenerationResult:
    token_ids: list[int]
    prefill_time: float
    decode_time: float
    num_prefill_tokens: int
    num_decode_tokens: int

    @property
    def prefill_tok_s(self) -> float:
        return self.num_prefill_tokens / self.prefill_time if self.prefill_time else 0.0

    @property
    def decode_tok_s(self) -> float:
        return self.num_decode_tokens / self.decode_time if self.decode_time else 0.0


class LlamaModel:
    """Batch-1 int4 decoder on one GPU. `max_seq` bounds prompt + generated
    tokens (the KV cache capacity and the RoPE table)."""

    VERIFY_ROWS = 8  # rows of one lm_head pass in verify()

    def __init__(self, config: ModelConfig, layers: list[LayerWeights], embed: torch.Tensor,
                 norm_w: torch.Tensor, group_size: int, max_seq: int,
                 act_dtype: torch.dtype = torch.float32, max_prefill: int = 512,
                 fuse: bool = True, lm_head: torch.Tensor | None = None):
        if embed.dtype != torch.bfloat16 or (lm_head is not None and lm_head.dtype != torch.bfloat16):
            raise SFError("the embedding and the lm_head must be bf16")
        if lm_head is not None and tuple(lm_head.shape) != tuple(embed.shape):
            raise SFError("lm_head shape mismatch")
        if act_dtype not in _DT:
            raise SFError("act_dtype must be float32, float16 or bfloat16")
        self.config, self.layers, self.embed, self.norm_w = config, layers, embed, norm_w
        # logits table: the tied embedding (llama.py:77-79 `as_linear`) or lm_head.weight
        self.head = embed if lm_head is None else lm_head
        self.group_size, self.max_seq, self.act_dtype = group_size, max_seq, act_dtype
        self.max_prefill = max_prefill
        # decode folds each RMSNorm and the SwiGLU into the next projection
        # (bit-identical to running them as separate kernels; fuse=False does)
        self.fuse = fuse
        self.device = embed.device
        self.lib = _lib.load()
        c = config
        self.H, self.Hq, self.KVH, self.D = c.hidden_size, c.num_attention_heads, c.num_key_value_heads, c.head_dim
        self.I, self.V = c.intermediate_size, c.vocab_size
        self.qkv_n = (self.Hq + 2 * self.KVH) * self.D
        self.scale = float(self.D ** -0.5)
        dev = self.device
        f32 = torch.float32
        # KV cache: per layer codes [KVH, T_cap, D] int8 and fp16 scales [KVH, T_cap]
        self.k_codes = [torch.zeros((self.KVH, max_seq, self.D), dtype=torch.int8, device=dev) for _ in layers]
        self.v_codes = [torch.zeros_like(t) for t in self.k_codes]
        self.k_scales = [torch.zeros((self.KVH, max_seq), dtype=torch.float16, device=dev) for _ in layers]
        self.v_scales = [torch.zeros_like(t) for t in self.k_scales]
        cos, sin = rope_tables(config, max_seq)
        self.cos = torch.from_numpy(cos).to(dev)
        self.sin = torch.from_numpy(sin).to(dev)
        # decode buffers
        a = act_dtype
        self.h = torch.zeros((1, self.H), dtype=f32, device=dev)
        self.xn = torch.zeros((1, self.H), dtype=a, device=dev)
        self.qkv = torch.zeros((1, self.qkv_n), dtype=f32, device=dev)
        self.q = torch.zeros((1, self.Hq, self.D), dtype=a, device=dev)
        self.attn = torch.zeros((1, self.Hq * self.D), dtype=a, device=dev)
        self.gu = torch.zeros((1, 2 * self.I), dtype=f32, device=dev)
        self.act = torch.zeros((1, self.I), dtype=a, device=dev)
        self.logits = torch.zeros((self.V,), dtype=f32, device=dev)
        self.token = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.pos_dev = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.hist = torch.zeros((max_seq + 1,), dtype=torch.int32, device=dev)
        self.attn_splits = int(self.lib.sf_attn_default_splits_d(1, self.KVH, max_seq, self.D))
        # decode attention: about 128 cached tokens per split (2..8 splits), the
        # split merge folded into the o projection's activation load
        # (sf_q4_gemv_attn_merge); fuse=False runs the same splits through the
        # merge launch and a plain GEMV, which gives the same bits
        L0 = layers[0]
        fold_s = min(8, max(2, -(-max_seq // 128)))
        self._attn_fold = bool(self.lib.sf_q4_gemv_attn_merge_supported(
            1, L0.o.out_features, self.Hq, self.D, fold_s, L0.o.group_size, _DT[act_dtype]))
        self.decode_splits = fold_s if self._attn_fold else self.attn_splits
        ws = max(self.lib.sf_attn_workspace_bytes(1, self.Hq, self.D, self.attn_splits),
                 self.lib.sf_attn_workspace_bytes(1, self.Hq, self.D, self.decode_splits), 1 << 16)
        self.attn_ws = torch.zeros(ws, dtype=torch.uint8, device=dev)
        hw = self.lib.sf_lm_head_workspace_bytes(self.V)
        self.head_ws = torch.zeros(hw, dtype=torch.uint8, device=dev)
        # verify rows (speculative decoding): greedy token and logits per row
        self.vtok = torch.zeros((self.VERIFY_ROWS,), dtype=torch.int32, device=dev)
        self.vlogits = torch.zeros((self.VERIFY_ROWS, self.V), dtype=f32, device=dev)
        rw = self.lib.sf_lm_head_rows_workspace_bytes(self.V, self.VERIFY_ROWS)
        self.rows_ws = torch.zeros(rw, dtype=torch.uint8, device=dev)
        # decode: RoPE + KV append folded into the qkv projection's epilogue
        # where its batch-1 plan gives one head per workgroup (hidden <= 1024)
        self._qkv_rope = bool(fuse and self.lib.sf_q4_gemv_fused_rope_supported(
            L0.qkv.out_features, L0.qkv.in_features, L0.qkv.group_size, self.Hq, self.KVH, self.D,
            _DT[act_dtype]))
        self.pos = 0
        self.graph = None
        self._verify_graphs = {}
        self._rows_plans = {}
        self._vbufs = None
        self._prefill_bufs = None
        # the prefill GEMM's split-K workspace, sized once for every projection
        # at every chunk length up to max_prefill rows: a recorded verify graph
        # keeps its address, so it is never replaced
        ws = 0
        for w in (L0.qkv, L0.o, L0.gate_up, L0.down):
            for M in range(1, max(max_prefill, self.VERIFY_ROWS) + 1):
                ws = max(ws, self.lib.sf_q4_gemm_workspace_bytes(M, w.out_features, w.in_features,
                                                                 w.group_size))
        self._gemm_ws = torch.empty(ws, dtype=torch.uint8, device=dev) if ws else None

    def sibling(self) -> "LlamaModel":
        """A decoder over the same device weights with a KV cache, buffers and
        graphs of its own: the second cache that the reference's models get by
        taking the cache as an argument (speculative decoding with draft ==
        target, engine/speculative.py:224-225)."""
        return LlamaModel(self.config, self.layers, self.embed, self.norm_w, self.group_size,
                          self.max_seq, act_dtype=self.act_dtype, max_prefill=self.max_prefill,
                          fuse=self.fuse, lm_head=None if self.head is self.embed else self.head)

    # ------------------------------------------------------------------ init
    @classmethod
    def random_init(cls, config: ModelConfig, seed: int = 4, group_size: int = 64,
                    device=None, max_seq: int = 1024, act_dtype: torch.dtype = torch.float32,
                    std: float = 0.02, max_prefill: int = 512, fuse: bool = True) -> "LlamaModel":
        """Random weights N(0, std) drawn on the device from `seed` (RMSNorm
        weights 1, q/k/v biases N(0, std) when the config has attention bias),
        every projection RTN int4 symmetric with `group_size`, the embedding
        in bf16, and a bf16 lm_head of its own drawn after the layers when the
        config does not tie it to the embedding."""
        if not _lib.hip_available():
            raise SFError("no gfx950 HIP device: siliconfer_amd has no CPU fallback")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        c = config
        H, I, D = c.hidden_size, c.intermediate_size, c.head_dim
        Hq, KVH = c.num_attention_heads, c.num_key_value_heads

        def randn(*shape):
            return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32) * std

        def q4(*mats):
            W = torch.cat(mats, dim=0) if len(mats) > 1 else mats[0]
            pk, sc = pack_sym_device(W, group_size)
            return Q4Weight(pk, sc, None, group_size, device=dev)

        embed = randn(c.vocab_size, H).to(torch.bfloat16).contiguous()
        layers = []
        for _ in range(c.num_hidden_layers):
            qkv = q4(randn(Hq * D, H), randn(KVH * D, H), randn(KVH * D, H))
            bias = randn((Hq + 2 * KVH) * D) if c.attention_bias else None
            o = q4(randn(H, Hq * D))
            gate_up = q4(randn(I, H), randn(I, H))
            down = q4(randn(H, I))
            ones = torch.ones(H, dtype=torch.float32, device=dev)
            layers.append(LayerWeights(qkv, bias, o, gate_up, down, ones, ones.clone()))
        norm_w = torch.ones(H, dtype=torch.float32, device=dev)
        head = None if c.tie_word_embeddings else randn(c.vocab_size, H).to(torch.bfloat16).contiguous()
        return cls(config, layers, embed, norm_w, group_size, max_seq, act_dtype, max_prefill, fuse,
                   lm_head=head)

    def export_weights(self, packed: bool = False) -> dict:
        """Host copies for a reference restatement: dequantized fp32 weights
        (fp16 scales as stored), biases, norms, the embedding as fp32. With
        `packed`, each projection also as `name + "_q4"`: (codes u8 [N, K/2] in
        the reference's nibble order, scales fp32 [N, G], group size), the
        operands of the reference's q4_gemv_sym (symmetric weights only)."""
        out = {"embed": self.embed.float().cpu().numpy(), "norm": self.norm_w.cpu().numpy(),
               "layers": []}
        if self.head is not self.embed:
            out["lm_head"] = self.head.float().cpu().numpy()
        for L in self.layers:
            d = {}
            for name in ("qkv", "o", "gate_up", "down"):
                w: Q4Weight = getattr(L, name)
                pk, s, z = w.canonical()
                pk = pk.cpu().numpy()
                s = s.float().cpu().numpy()
                lo = (pk & 0x0F).astype(np.int16)
                hi = (pk >> 4).astype(np.int16)
                q = np.empty((pk.shape[0], pk.shape[1] * 2), np.int16)
                q[:, 0::2], q[:, 1::2] = lo, hi
                g = self.group_size
                if z is None:  # two's-complement codes
                    q = np.where(q > 7, q - 16, q).astype(np.float32).reshape(q.shape[0], -1, g)
                else:          # unsigned codes minus the group's zero-point
                    q = q.astype(np.float32).reshape(q.shape[0], -1, g) - z.cpu().numpy()[..., None]
                d[name] = (q * s[..., None]).reshape(pk.shape[0], -1)
                if packed:
                    if z is not None:
                        raise ValueError("packed export takes symmetric weights")
                    d[name + "_q4"] = (np.ascontiguousarray(pk), np.ascontiguousarray(s, np.float32), g)
            d["qkv_bias"] = None if L.qkv_bias is None else L.qkv_bias.cpu().numpy()
            d["w_in"], d["w_post"] = L.w_in.cpu().numpy(), L.w_post.cpu().numpy()
            out["layers"].append(d)
        return out

    # ------------------------------------------------------------- launches
    def _st(self) -> int:
        return torch.cuda.current_stream(self.device).cuda_stream

    def _chk(self, rc, what):
        _lib.check(rc, what)

    def _gemv(self, w: Q4Weight, x: torch.Tensor, y32: torch.Tensor, bias: torch.Tensor | None):
        self._chk(self.lib.sf_q4_gemv(w.blob.data_ptr(), x.data_ptr(), _DT[x.dtype], None, _lib.SF_F32,
                                      y32.data_ptr(), None if bias is None else bias.data_ptr(),
                                      _lib.SF_F32, 1, w.out_features, w.in_features, w.group_size,
                                      int(w.has_zeros), self._st()), "sf_q4_gemv")

    def _gemv_ok(self, M: int, w: Q4Weight) -> bool:
        """The batch GEMV runs these rows on MFMA in one pass (sf_q4_gemv_supported)."""
        return M <= 8 and bool(self.lib.sf_q4_gemv_supported(M, w.out_features, w.in_features,
                                                             w.group_size, _DT[self.act_dtype]))

    def _gemm(self, w: Q4Weight, X: torch.Tensor, Y32: torch.Tensor, bias: torch.Tensor | None):
        M = X.shape[0]
        if self._gemv_ok(M, w):
            # up to 8 rows (a short chunk, a speculative verify): the batch GEMV
            # streams the weights once for all rows
            self._chk(self.lib.sf_q4_gemv(w.blob.data_ptr(), X.data_ptr(), _DT[X.dtype], None,
                                          _lib.SF_F32, Y32.data_ptr(),
                                          None if bias is None else bias.data_ptr(), _lib.SF_F32, M,
                                          w.out_features, w.in_features, w.group_size,
                                          int(w.has_zeros), self._st()), "sf_q4_gemv")
            return
        need = self.lib.sf_q4_gemm_workspace_bytes(M, w.out_features, w.in_features, w.group_size)
        if need and (self._gemm_ws is None or self._gemm_ws.numel() < need):
            raise SFError(f"GEMM workspace: {need} bytes for {M} rows exceeds the preallocated "
                          f"{0 if self._gemm_ws is None else self._gemm_ws.numel()} (max_prefill)")
        ws = self._gemm_ws if need else None
        self._chk(self.lib.sf_q4_gemm(w.blob.data_ptr(), X.data_ptr(), _DT[X.dtype], None, _lib.SF_F32,
                                      Y32.data_ptr(), None if bias is None else bias.data_ptr(),
                                      _lib.SF_F32, M, w.out_features, w.in_features, w.group_size,
                                      int(w.has_zeros), None if ws is None else ws.data_ptr(),
                                      0 if ws is None else ws.numel(), self._st()), "sf_q4_gemm")

    def _gemm_parts(self, w: Q4Weight, X: torch.Tensor) -> int:
        """Where the GEMM splits K for these rows, run it leaving its partials
        in the GEMM workspace (no reduce launch) and return their count; else
        launch nothing and return 0."""
        M = X.shape[0]
        if M <= GEMM_GEMV_ROWS and self._gemv_ok(min(M, 8), w):
            return 0  # sf_q4_gemm runs these rows as 8-row batch GEMVs: no partials
        S = int(self.lib.sf_q4_gemm_splits(M, w.out_features, w.in_features, w.group_size))
        if S <= 1:
            return 0
        need = self.lib.sf_q4_gemm_workspace_bytes(M, w.out_features, w.in_features, w.group_size)
        if self._gemm_ws is None or self._gemm_ws.numel() < need:
            raise SFError(f"GEMM workspace: {need} bytes for {M} rows exceeds the preallocated "
                          f"{0 if self._gemm_ws is None else self._gemm_ws.numel()} (max_prefill)")
        self._chk(self.lib.sf_q4_gemm_partials(
            w.blob.data_ptr(), X.data_ptr(), _DT[X.dtype], M, w.out_features, w.in_features,
            w.group_size, int(w.has_zeros), self._gemm_ws.data_ptr(), self._gemm_ws.numel(),
            self._st()), "sf_q4_gemm_partials")
        return S

    def _gemm_delta(self, w: Q4Weight, X: torch.Tensor, Dl: torch.Tensor) -> int:
        """The projection's output as the residual's delta: its K-split
        partials left for the next RMSNorm to sum (returns their count), else
        written to Dl (returns 0). Either way the norm gets the same bits."""
        S = self._gemm_parts(w, X)
        if not S:
            self._gemm(w, X, Dl, None)
        return S

    def _rmsnorm_delta(self, x, delta, parts: int, w, out, rows):
        """RMSNorm after adding the residual delta: `parts` K-split partials in
        the GEMM workspace (from _gemm_delta), else the `delta` rows (or none)."""
        if not parts:
            self._rmsnorm(x, delta, w, out, rows)
            return
        self._chk(self.lib.sf_rmsnorm_partials(
            x.data_ptr(), self._gemm_ws.data_ptr(), parts, w.data_ptr(), _lib.SF_F32, out.data_ptr(),
            _DT[out.dtype], rows, self.H, float(self.config.rms_norm_eps), self._st()),
            "sf_rmsnorm_partials")

    def _gemv_fused(self, w: Q4Weight, src: torch.Tensor, op: int, norm_w, y32: torch.Tensor,
                    bias: torch.Tensor | None):
        self._chk(self.lib.sf_q4_gemv_fused(
            w.blob.data_ptr(), src.data_ptr(), op, None if norm_w is None else norm_w.data_ptr(),
            float(self.config.rms_norm_eps), _DT[self.act_dtype], None, _lib.SF_F32, y32.data_ptr(),
            None if bias is None else bias.data_ptr(), _lib.SF_F32, w.out_features, w.in_features,
            w.group_size, int(w.has_zeros), self._st()), "sf_q4_gemv_fused")

    def _rmsnorm(self, x, delta, w, out, rows):
        self._chk(self.lib.sf_rmsnorm(x.data_ptr(), None if delta is None else delta.data_ptr(),
                                      w.data_ptr(), _lib.SF_F32, out.data_ptr(), _DT[out.dtype], rows,
                                      self.H, float(self.config.rms_norm_eps), self._st()), "sf_rmsnorm")

    def _rope_append(self, l, qkv, q_out, rows, pos_dev, pos_host):
        self._chk(self.lib.sf_rope_kv_append(
            qkv.data_ptr(), self.cos.data_ptr(), self.sin.data_ptr(), self.max_seq, q_out.data_ptr(),
            _DT[q_out.dtype], self.k_codes[l].data_ptr(), self.k_scales[l].data_ptr(),
            self.v_codes[l].data_ptr(), self.v_scales[l].data_ptr(), _lib.SF_F16, rows, self.Hq,
            self.KVH, self.D, self.max_seq, pos_dev, pos_host, self._st()), "sf_rope_kv_append")

    def _rope_append_parts(self, l, parts, bias, q_out, rows, pos_dev, pos_host):
        self._chk(self.lib.sf_rope_kv_append_partials(
            self._gemm_ws.data_ptr(), parts, None if bias is None else bias.data_ptr(), _lib.SF_F32,
            self.cos.data_ptr(), self.sin.data_ptr(), self.max_seq, q_out.data_ptr(),
            _DT[q_out.dtype], self.k_codes[l].data_ptr(), self.k_scales[l].data_ptr(),
            self.v_codes[l].data_ptr(), self.v_scales[l].data_ptr(), _lib.SF_F16, rows, self.Hq,
            self.KVH, self.D, self.max_seq, pos_dev, pos_host, self._st()), "sf_rope_kv_append_partials")

    def _lm_head_norm(self, h_row, token, pos_inc, logits=True):
        self._chk(self.lib.sf_lm_head_argmax_rmsnorm(
            self.head.data_ptr(), h_row.data_ptr(), self.norm_w.data_ptr(),
            float(self.config.rms_norm_eps), _DT[self.act_dtype],
            self.logits.data_ptr() if logits else None, self.V, self.H, token.data_ptr(), pos_inc,
            self.hist.data_ptr() if pos_inc else None, self.head_ws.data_ptr(), self.head_ws.numel(),
            self._st()), "sf_lm_head_argmax_rmsnorm")

    def _lm_head(self, x_row, token, pos_inc, logits=True):
        self._chk(self.lib.sf_lm_head_argmax(
            self.head.data_ptr(), x_row.data_ptr(), _DT[x_row.dtype],
            self.logits.data_ptr() if logits else None, self.V, self.H, token.data_ptr(),
            pos_inc, self.hist.data_ptr() if pos_inc else None, self.head_ws.data_ptr(),
            self.head_ws.numel(), self._st()), "sf_lm_head_argmax")

    # --------------------------------------------------------------- prefill
    def reset(self) -> None:
        """Empty the KV cache (positions restart at 0; codes are overwritten)."""
        self.pos = 0
        self.pos_dev.zero_()

    def _bufs(self, T):
        if self._prefill_bufs is None or self._prefill_bufs["T"] < T:
            self._prefill_bufs = self._alloc_rows(T)
        return self._prefill_bufs

    def _alloc_rows(self, T):
        dev, a, f32 = self.device, self.act_dtype, torch.float32
        return dict(T=T, H=torch.empty((T, self.H), dtype=f32, device=dev),
                    Xn=torch.empty((T, self.H), dtype=a, device=dev),
                    QKV=torch.empty((T, self.qkv_n), dtype=f32, device=dev),
                    Q=torch.empty((T, self.Hq, self.D), dtype=a, device=dev),
                    A=torch.empty((T, self.Hq * self.D), dtype=a, device=dev),
                    Dl=torch.empty((T, self.H), dtype=f32, device=dev),
                    GU=torch.empty((T, 2 * self.I), dtype=f32, device=dev),
                    ACT=torch.empty((T, self.I), dtype=a, device=dev),
                    ids=torch.empty((T,), dtype=torch.int32, device=dev))

    def prefill(self, ids, want_logits: bool = True) -> int:
        """Run the prompt (appending to the cache) and return the greedy next
        token; `self.logits` holds the last row's logits."""
        ids = np.asarray(ids, dtype=np.int64).reshape(-1)
        T = int(ids.size)
        if T == 0:
            raise SFError("empty prompt")
        if ids.min() < 0 or ids.max() >= self.V:
            raise SFError("token id out of range")
        if self.pos + T > self.max_seq:
            raise SFError(f"prompt of {T} tokens exceeds the cache capacity {self.max_seq}")
        done = 0
        while done < T:  # chunks of at most max_prefill rows
            n = min(self.max_prefill, T - done)
            self._prefill_chunk(ids[done:done + n], want_logits and done + n == T)
            done += n
        return int(self.token.item())

    def set_position(self, n: int) -> None:
        """Trim the KV cache to its first n positions — QuantizedKVCache.trim
        (/root/reference/siliconfer/model/kv_cache.py:107-112) as speculative
        decoding uses it (engine/speculative.py:29-41). The codes past n stay
        in place and are overwritten by the next tokens."""
        n = int(n)
        if not 0 <= n <= self.pos:
            raise SFError(f"cannot trim the cache to {n} positions (it holds {self.pos})")
        self.pos = n
        self.pos_dev.fill_(n)

    def verify(self, ids, want_logits: bool = False) -> list[int]:
        """Append the B tokens `ids` at positions pos..pos+B-1 in one forward
        and return the greedy next token after each of them — the target's
        verify pass of speculative decoding (engine/speculative.py:277-283,
        `t_log = target(verify_ids)`, with the greedy pick of each row). For
        B <= 8 every projection is one batch GEMV over the B rows, so a
        verify streams the weights once, like one decode step, and after
        `capture_verify()` it is one graph replay. `want_logits` keeps the
        rows' logits in `self.vlogits[:B]` (B <= 8)."""
        ids = np.asarray(ids, dtype=np.int64).reshape(-1)
        B = int(ids.size)
        if B == 0:
            raise SFError("empty verify batch")
        if ids.min() < 0 or ids.max() >= self.V:
            raise SFError("token id out of range")
        if self.pos + B > self.max_seq:
            raise SFError(f"verify of {B} tokens at position {self.pos} exceeds the cache capacity "
                          f"{self.max_seq}")
        if want_logits and B > self.VERIFY_ROWS:
            raise SFError(f"verify logits are kept for at most {self.VERIFY_ROWS} rows")
        g = self._verify_graphs.get(B) if not want_logits else None
        if g is not None:
            self._vids_host[:B].copy_(torch.from_numpy(ids.astype(np.int32)))
            self._vbufs["ids"][:B].copy_(self._vids_host[:B], non_blocking=True)
            g.replay()
            self.pos += B  # the graph advanced pos_dev
            return self.vtok[:B].tolist()
        out = []
        done = 0
        while done < B:
            n = min(self.max_prefill, B - done)
            out += self._prefill_chunk(ids[done:done + n], want_logits, rows_head=True)
            done += n
        return out

    @property
    def verify_graph_sizes(self) -> set[int]:
        return set(self._verify_graphs)

    def capture_verify(self, sizes=range(1, 9)) -> None:
        """Record verify() of B rows as one HIP graph per B in `sizes` (B <=
        8): ids come from a fixed device buffer, positions from pos_dev (the
        graph advances it by B), tokens land in `self.vtok`. Verifies that
        ask for logits still run eagerly."""
        if self._vbufs is None:
            R = self.VERIFY_ROWS
            self._vbufs = self._alloc_rows(R)
            self._vids_host = torch.zeros((R,), dtype=torch.int32).pin_memory()
            wb = self.lib.sf_attn_workspace_bytes(R, self.Hq, self.D, self.attn_splits)
            self._vattn_ws = torch.zeros(max(wb, 256), dtype=torch.uint8, device=self.device)
        for B in sizes:
            if not 1 <= B <= self.VERIFY_ROWS:
                raise SFError(f"verify graphs hold 1..{self.VERIFY_ROWS} rows")
            torch.cuda.synchronize(self.device)
            s = torch.cuda.Stream(self.device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                self._rows_forward(self._vbufs, B, True)
                self._rows_head(self._vbufs["Xn"][:B], B, False)
                self.pos_dev.add_(B)
            torch.cuda.synchronize(self.device)
            self._verify_graphs[B] = g

    def _prefill_chunk(self, ids: np.ndarray, want_logits: bool, rows_head: bool = False):
        T = int(ids.size)
        b = self._bufs(T)
        b["ids"][:T].copy_(torch.from_numpy(ids.astype(np.int32)))
        self._rows_forward(b, T, False)
        Xn = b["Xn"][:T]
        toks = None
        if rows_head:  # every row's greedy token, 8 rows per lm_head pass
            R = self.VERIFY_ROWS
            toks = []
            for r0 in range(0, T, R):
                nr = min(R, T - r0)
                self._rows_head(Xn[r0:r0 + nr], nr, want_logits)
                toks += self.vtok[:nr].tolist()
        else:
            self._lm_head(Xn[T - 1], self.token, None, logits=want_logits)
        self.pos += T
        self.pos_dev.fill_(self.pos)
        return toks

    def _rows_head(self, Xn, nr, want_logits):
        self._chk(self.lib.sf_lm_head_argmax_rows(
            self.head.data_ptr(), Xn.data_ptr(), _DT[Xn.dtype],
            self.vlogits.data_ptr() if want_logits else None, self.V, self.H, nr,
            self.vtok.data_ptr(), self.rows_ws.data_ptr(), self.rows_ws.numel(), self._st()),
            "sf_lm_head_argmax_rows")

    def _rows_plan(self, T: int) -> tuple[bool, bool, bool, bool]:
        """How T rows run: (residual, fold_qkv, fold_gate_up, fold_down).
        residual: up to 8 rows every projection is a batch GEMV and the o /
        down projections add into the residual rows themselves (the norms then
        read them directly). fold_*: the RMSNorm / SwiGLU before that
        projection runs inside it where the GEMV can stage the rows'
        activations (sf_q4_gemv_fused_rows_supported) — each choice gives the
        same bits."""
        if T not in self._rows_plans:
            L0 = self.layers[0]
            residual = all(self._gemv_ok(T, w) for w in (L0.qkv, L0.o, L0.gate_up, L0.down))
            ok = lambda op, w: bool(self.fuse and residual and self.lib.sf_q4_gemv_fused_rows_supported(
                op, T, w.out_features, w.in_features, w.group_size, int(w.has_zeros),
                _DT[self.act_dtype]))
            self._rows_plans[T] = (residual, ok(_lib.SF_PRE_RMSNORM, L0.qkv),
                                   ok(_lib.SF_PRE_RMSNORM, L0.gate_up),
                                   ok(_lib.SF_PRE_SILU_MUL, L0.down))
        return self._rows_plans[T]

    def _gemv_fused_rows(self, w: Q4Weight, src, op: int, norm_w, y32, bias, T: int):
        self._chk(self.lib.sf_q4_gemv_fused_rows(
            w.blob.data_ptr(), src.data_ptr(), op, None if norm_w is None else norm_w.data_ptr(),
            float(self.config.rms_norm_eps), _DT[self.act_dtype], None, _lib.SF_F32, y32.data_ptr(),
            None if bias is None else bias.data_ptr(), _lib.SF_F32, T, w.out_features,
            w.in_features, w.group_size, int(w.has_zeros), self._st()), "sf_q4_gemv_fused_rows")

    def _rows_forward(self, b, T, dev_pos: bool):
        """Embed b["ids"][:T], run every layer over the T rows at positions
        pos.. (host `self.pos`, or pos_dev when dev_pos: graph-replayable) and
        leave the final-normed rows in b["Xn"][:T]. `_rows_plan(T)` says
        where the residual is added and which norms / SwiGLU fold into the
        next projection; every combination gives the same bits."""
        Hb, Xn, QKV, Q, A, Dl, GU, ACT = (b[k][:T] for k in ("H", "Xn", "QKV", "Q", "A", "Dl", "GU", "ACT"))
        lib, st = self.lib, self._st()
        self._chk(lib.sf_embed(b["ids"].data_ptr(), self.embed.data_ptr(), _lib.SF_BF16, Hb.data_ptr(),
                               T, self.H, self.V, st), "sf_embed")
        pos_dev = self.pos_dev.data_ptr() if dev_pos else None
        res, fq, fg, fd = self._rows_plan(T)
        RMS, SILU = _lib.SF_PRE_RMSNORM, _lib.SF_PRE_SILU_MUL
        # without the residual inside the projections, each norm adds the
        # previous projection's output (Dl) to the residual rows itself
        delta = lambda l: None if res or l < 0 else Dl
        parts = 0  # the previous projection's K-split partials still to add (see _gemm_delta)
        for l, L in enumerate(self.layers):
            qparts = 0  # q|k|v left as K-split partials for RoPE + append to sum
            if fq:
                self._gemv_fused_rows(L.qkv, Hb, RMS, L.w_in, QKV, L.qkv_bias, T)
            else:
                self._rmsnorm_delta(Hb, delta(l - 1), parts, L.w_in, Xn, T)
                qparts = self._gemm_parts(L.qkv, Xn)
                if not qparts:
                    self._gemm(L.qkv, Xn, QKV, L.qkv_bias)
            if qparts:
                self._rope_append_parts(l, qparts, L.qkv_bias, Q, T, pos_dev, 0 if dev_pos else self.pos)
            else:
                self._rope_append(l, QKV, Q, T, pos_dev, 0 if dev_pos else self.pos)
            args = (Q.data_ptr(), _DT[Q.dtype], self.k_codes[l].data_ptr(), self.k_scales[l].data_ptr(),
                    self.v_codes[l].data_ptr(), self.v_scales[l].data_ptr(), _lib.SF_F16, A.data_ptr(),
                    _DT[A.dtype])
            if dev_pos:
                self._chk(lib.sf_attn_prefill_i8kv_dev(
                    *args, self._vattn_ws.data_ptr(), self._vattn_ws.numel(), T, self.Hq, self.KVH,
                    pos_dev, self.max_seq, self.max_seq, self.D, self.scale, self.attn_splits, st),
                    "sf_attn_prefill_i8kv_dev")
            else:
                self._chk(lib.sf_attn_prefill_i8kv(*args, T, self.Hq, self.KVH, self.pos, self.max_seq,
                                                   self.D, self.scale, st), "sf_attn_prefill_i8kv")
            parts = 0
            if res:
                self._gemm(L.o, A, Hb, Hb)  # residual add as the bias (per row)
            else:
                parts = self._gemm_delta(L.o, A, Dl)
            if fg:
                assert parts == 0, "the folded RMSNorm reads no K-split partials"
                self._gemv_fused_rows(L.gate_up, Hb, RMS, L.w_post, GU, None, T)
            else:
                self._rmsnorm_delta(Hb, delta(l), parts, L.w_post, Xn, T)
                self._gemm(L.gate_up, Xn, GU, None)
            parts = 0  # consumed: the o projection's partials are in Hb now
            if fd:
                self._gemv_fused_rows(L.down, GU, SILU, None, Hb, Hb, T)
                continue
            self._chk(lib.sf_silu_mul(GU.data_ptr(), ACT.data_ptr(), _DT[ACT.dtype], T, self.I, st),
                      "sf_silu_mul")
            parts = 0
            if res:
                self._gemm(L.down, ACT, Hb, Hb)
            else:
                parts = self._gemm_delta(L.down, ACT, Dl)
        self._rmsnorm_delta(Hb, delta(len(self.layers) - 1), parts, self.norm_w, Xn, T)

    # ---------------------------------------------------------------- decode
    def decode_step(self, logits: bool = False) -> None:
        """One greedy decode step on the device: embeds `self.token` at
        position p = `pos_dev`, writes the next token to `self.token` and
        `self.hist[p]`, increments `pos_dev`. No host synchronisation."""
        lib, st = self.lib, self._st()
        pos = self.pos_dev.data_ptr()
        self._chk(lib.sf_embed(self.token.data_ptr(), self.embed.data_ptr(), _lib.SF_BF16,
                               self.h.data_ptr(), 1, self.H, self.V, st), "sf_embed")
        fuse = self.fuse
        for l, L in enumerate(self.layers):
            if self._qkv_rope:  # RMSNorm in the activation load, RoPE + append in the epilogue
                self._chk(lib.sf_q4_gemv_fused_rope(
                    L.qkv.blob.data_ptr(), self.h.data_ptr(), L.w_in.data_ptr(),
                    float(self.config.rms_norm_eps), _DT[self.act_dtype],
                    None if L.qkv_bias is None else L.qkv_bias.data_ptr(), _lib.SF_F32,
                    self.cos.data_ptr(), self.sin.data_ptr(), self.max_seq, self.q.data_ptr(),
                    _DT[self.q.dtype], self.k_codes[l].data_ptr(), self.k_scales[l].data_ptr(),
                    self.v_codes[l].data_ptr(), self.v_scales[l].data_ptr(), _lib.SF_F16, self.Hq,
                    self.KVH, self.D, self.max_seq, pos, L.qkv.out_features, L.qkv.in_features,
                    L.qkv.group_size, int(L.qkv.has_zeros), st), "sf_q4_gemv_fused_rope")
            else:
                if fuse:  # RMSNorm folded into the projection's activation load
                    self._gemv_fused(L.qkv, self.h, _lib.SF_PRE_RMSNORM, L.w_in, self.qkv,
                                     L.qkv_bias)
                else:
                    self._rmsnorm(self.h, None, L.w_in, self.xn, 1)
                    self._gemv(L.qkv, self.xn, self.qkv, L.qkv_bias)
                self._rope_append(l, self.qkv, self.q, 1, pos, 0)
            kv = (self.q.data_ptr(), _DT[self.q.dtype], self.k_codes[l].data_ptr(),
                  self.k_scales[l].data_ptr(), self.v_codes[l].data_ptr(), self.v_scales[l].data_ptr(),
                  _lib.SF_F16)
            if fuse and self._attn_fold:  # split partials; the merge rides in the o projection
                self._chk(lib.sf_attn_decode_i8kv_partials_dev(
                    *kv, self.attn_ws.data_ptr(), self.attn_ws.numel(), 1, self.Hq, self.KVH, pos, 1,
                    self.max_seq, self.max_seq, self.D, self.scale, self.decode_splits, st),
                    "sf_attn_decode_i8kv_partials_dev")
                self._chk(lib.sf_q4_gemv_attn_merge(
                    L.o.blob.data_ptr(), self.attn_ws.data_ptr(), self.attn_ws.numel(),
                    self.decode_splits, self.Hq, self.D, _DT[self.act_dtype], None, _lib.SF_F32,
                    self.h.data_ptr(), self.h.data_ptr(), _lib.SF_F32, 1, L.o.out_features,
                    L.o.group_size, int(L.o.has_zeros), st), "sf_q4_gemv_attn_merge")
            else:
                self._chk(lib.sf_attn_decode_i8kv_dev(
                    *kv, self.attn.data_ptr(), _DT[self.attn.dtype], self.attn_ws.data_ptr(),
                    self.attn_ws.numel(), 1, self.Hq, self.KVH, pos, 1, self.max_seq, self.max_seq,
                    self.D, self.scale, self.decode_splits, st), "sf_attn_decode_i8kv_dev")
                self._gemv(L.o, self.attn, self.h, self.h)    # residual add as the bias
            if fuse:  # RMSNorm, then SwiGLU, folded into the next projections
                self._gemv_fused(L.gate_up, self.h, _lib.SF_PRE_RMSNORM, L.w_post, self.gu, None)
                self._gemv_fused(L.down, self.gu, _lib.SF_PRE_SILU_MUL, None, self.h, self.h)
            else:
                self._rmsnorm(self.h, None, L.w_post, self.xn, 1)
                self._gemv(L.gate_up, self.xn, self.gu, None)
                self._chk(lib.sf_silu_mul(self.gu.data_ptr(), self.act.data_ptr(), _DT[self.act.dtype],
                                          1, self.I, st), "sf_silu_mul")
                self._gemv(L.down, self.act, self.h, self.h)
        if fuse:
            self._lm_head_norm(self.h, self.token, pos, logits=logits)
        else:
            self._rmsnorm(self.h, None, self.norm_w, self.xn, 1)
            self._lm_head(self.xn, self.token, pos, logits=logits)

    def capture(self, logits: bool = False) -> None:
        """Record one decode step as a HIP graph (positions and tokens are
        device-side, so every replay advances the sequence by one token).
        Capturing launches nothing; the step contains no memset."""
        torch.cuda.synchronize(self.device)
        s = torch.cuda.Stream(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            self.decode_step(logits=logits)
        torch.cuda.synchronize(self.device)
        self.graph = g

    def replay(self, n: int = 1) -> None:
        if self.graph is None:
            raise SFError("capture() first")
        if self.pos + n > self.max_seq:
            raise SFError("decode would exceed the cache capacity")
        for _ in range(n):
            self.graph.replay()
        self.pos += n

    # -------------------------------------------------------------- generate
    def generate(self, prompt_ids, max_tokens: int = 128, use_graph: bool = True) -> GenerationResult:
        """Greedy generation (the reference's `generate` at temperature 0,
        engine/generate.py:117-180): prefill, then max_tokens - 1 decode steps.
        Decode time covers the steps after the first token, as there."""
        import time
        self.reset()
        torch.cuda.synchronize(self.device)
        t0 = time.perf_counter()
        first = self.prefill(prompt_ids)
        t1 = time.perf_counter()
        n = max_tokens - 1
        if self.pos + n > self.max_seq:
            raise SFError("prompt + max_tokens exceeds the cache capacity")
        if use_graph and self.graph is None:
            raise SFError("capture() before generate(use_graph=True)")
        start = self.pos
        t2 = time.perf_counter()
        if use_graph:
            self.replay(n)
        else:
            for _ in range(n):
                self.decode_step()
            self.pos += n
        torch.cuda.synchronize(self.device)
        t3 = time.perf_counter()
        # the step at position p wrote its output token to hist[p]
        toks = [first] + (self.hist[start:start + n].cpu().tolist() if n > 0 else [])
        return GenerationResult(toks, t1 - t0, t3 - t2, int(np.asarray(prompt_ids).size), n)
