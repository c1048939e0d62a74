"""GPU: the module-level layers (siliconfer_amd/model/layers.py, the
reference's model/layers.py call surface) against the oracle of the
reference's forward pass (oracle/model.py) on a tiny checkpoint.

- A stack of TransformerBlocks with one QuantizedKVCache per layer (batch 1:
  the fused RoPE + int8 append, causal prefill attention for the prompt and
  for later chunks after the cached prefix, the split-T decode attention per
  token) gives the oracle's logits at every step, symmetric and asymmetric
  weights.
- The reference's other cache forms take the device's fp32 route: no cache
  equals the oracle's blocks with unquantized K / V, a (k, v) tuple fed token
  by token equals one causal call, and batch 2 over an int8 cache equals the
  batch-1 path row by row.
- RMSNorm, apply_rope and MLP against the oracle's rmsnorm, rope and swiglu.
"""

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle.linear import assert_close
from siliconfer_amd.engine.loader import load_model
from siliconfer_amd.engine.q4_loader import build_model, pack_and_replace_linears
from siliconfer_amd.model.config import rope_tables
from siliconfer_amd.model.kv_cache import QuantizedKVCache
from siliconfer_amd.model.layers import (MLP, RMSNorm, TransformerBlock, apply_rope,
                                         compute_rope_freqs)
from test_loader import TINY, tiny_checkpoint

pytestmark = pytest.mark.gpu
G = 64


def _setup(dev, tmp_path, sym, seed=11):
    tiny_checkpoint(tmp_path, cfg=TINY, seed=seed)
    cfg, w = load_model(tmp_path)
    pack_and_replace_linears(w, cfg, G, pack_sym=sym)
    m = build_model(cfg, dict(w), G, device=dev, max_seq=64, act_dtype=torch.float32)
    freqs = compute_rope_freqs(cfg, dev)
    blocks = [TransformerBlock.from_weights(cfg, w, i, freqs, G, dev) for i in range(cfg.num_hidden_layers)]
    return cfg, w, m, blocks


def _logits(m, blocks, cfg, ids, caches):
    """Embedding, the module blocks, final norm and the tied head (the test's
    own glue around the layers under test); last row's logits."""
    x = m.embed.float()[torch.as_tensor(ids, device=m.embed.device)][None]  # [1, T, H]
    for blk, c in zip(blocks, caches):
        x, _ = blk(x, c)
    norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps, x.device)
    with torch.no_grad():
        norm.weight.copy_(m.norm_w)
    xn = norm(x)[0, -1]
    return (m.head.float() @ xn).cpu().numpy()


@pytest.mark.parametrize("sym", [True, False])
def test_block_stack_int8_cache_matches_oracle(dev, tmp_path, sym):
    cfg, w, m, blocks = _setup(dev, tmp_path, sym)
    ids = np.random.default_rng(5).integers(0, cfg.vocab_size, 9)
    caches = [QuantizedKVCache(capacity=16) for _ in blocks]  # grows past 16 below
    W = m.export_weights()
    cos, sin = rope_tables(cfg, 64)
    oc = OM.KVCache(cfg.num_hidden_layers)
    got = [_logits(m, blocks, cfg, ids, caches)]
    ref = [OM.forward(W, cfg, ids, oc, cos, sin)[-1]]
    for step in range(9):
        t = int(np.argmax(ref[-1]))
        got.append(_logits(m, blocks, cfg, [t], caches))
        ref.append(OM.forward(W, cfg, [t], oc, cos, sin)[-1])
    assert caches[0].length() == 18 and caches[0].capacity >= 18
    # prompt chunks after a cached prefix: 5 rows (the decode kernel's causal
    # rows) and 17 rows (the flash prefill kernel), each from its offset
    rng = np.random.default_rng(6)
    for n in (5, 17):
        chunk = rng.integers(0, cfg.vocab_size, n)
        got.append(_logits(m, blocks, cfg, chunk, caches))
        ref.append(OM.forward(W, cfg, chunk, oc, cos, sin)[-1])
    assert caches[0].length() == 40
    for i, (g, r) in enumerate(zip(got, ref)):
        assert_close(g, r, 2e-3, f"sym={sym} step {i}")


def _float_block(L, cfg, x, pos0, cos, sin):
    """One block of the oracle's pieces with unquantized K / V (the reference's
    cache=None / tuple path): x [T, H] -> [T, H]."""
    T = x.shape[0]
    Hq, KVH, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    xn = OM.rmsnorm(x, L["w_in"], cfg.rms_norm_eps)
    qkv = OM.dense(L, "qkv", xn) + L["qkv_bias"]
    pos = np.arange(pos0, pos0 + T)
    q = OM.rope(qkv[:, :Hq * D].reshape(T, Hq, D), pos, cos, sin)
    k = OM.rope(qkv[:, Hq * D:(Hq + KVH) * D].reshape(T, KVH, D), pos, cos, sin)
    v = qkv[:, (Hq + KVH) * D:].reshape(T, KVH, D)
    a = OM.attend(q, np.transpose(k, (1, 0, 2)), np.transpose(v, (1, 0, 2)), pos0, D ** -0.5)
    x = x + OM.dense(L, "o", a.reshape(T, Hq * D))
    xn = OM.rmsnorm(x, L["w_post"], cfg.rms_norm_eps)
    return x + OM.dense(L, "down", OM.swiglu(OM.dense(L, "gate_up", xn), cfg.intermediate_size))


def test_no_cache_and_tuple_cache_match_float_oracle(dev, tmp_path):
    cfg, w, m, blocks = _setup(dev, tmp_path, True)
    W = m.export_weights()
    cos, sin = rope_tables(cfg, 64)
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, (7, cfg.hidden_size)).astype(np.float32)
    ref = _float_block(W["layers"][0], cfg, x, 0, cos, sin)
    xt = torch.as_tensor(x, device=dev)[None]
    got, kv = blocks[0](xt, None)
    assert_close(got[0].cpu().numpy(), ref, 2e-3, "no cache")
    assert kv[0].shape == (1, cfg.num_key_value_heads, 7, cfg.head_dim)
    # the same tokens through a (k, v) tuple: 4, then 1, then 2
    c = None
    outs = []
    for a, b in ((0, 4), (4, 5), (5, 7)):
        y, c = blocks[0](xt[:, a:b], c)
        outs.append(y[0])
    assert c[0].shape[2] == 7
    assert_close(torch.cat(outs).cpu().numpy(), ref, 2e-3, "tuple cache, fed in pieces")


def test_batch2_int8_cache_matches_batch1_rows(dev, tmp_path):
    cfg, w, m, blocks = _setup(dev, tmp_path, False)
    rng = np.random.default_rng(4)
    x = torch.as_tensor(rng.normal(0, 1, (2, 6, cfg.hidden_size)).astype(np.float32), device=dev)
    xn = torch.as_tensor(rng.normal(0, 1, (2, 1, cfg.hidden_size)).astype(np.float32), device=dev)
    blk = blocks[1]
    cb = QuantizedKVCache(capacity=8)
    y2, _ = blk(x, cb)
    z2, _ = blk(xn, cb)
    assert cb.length() == 7
    for b in range(2):
        c1 = QuantizedKVCache(capacity=8)
        y1, _ = blk(x[b:b + 1], c1)
        z1, _ = blk(xn[b:b + 1], c1)
        assert_close(y2[b].cpu().numpy(), y1[0].cpu().numpy(), 2e-3, f"batch row {b} prompt")
        assert_close(z2[b].cpu().numpy(), z1[0].cpu().numpy(), 2e-3, f"batch row {b} decode")


def test_rmsnorm_rope_mlp_match_oracle(dev, tmp_path):
    cfg, w, m, blocks = _setup(dev, tmp_path, True)
    W = m.export_weights()
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, (5, cfg.hidden_size)).astype(np.float32)
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        xt = torch.as_tensor(x, device=dev).to(dt)
        y = blocks[0].input_layernorm(xt)
        assert y.dtype == dt
        ref = OM.rmsnorm(xt.float().cpu().numpy(), W["layers"][0]["w_in"], cfg.rms_norm_eps)
        tol = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 8e-3}[dt]
        assert_close(y.float().cpu().numpy(), ref, tol, f"rmsnorm {dt}")
    cos, sin = rope_tables(cfg, 64)
    q = rng.normal(0, 1, (1, 3, 4, cfg.head_dim)).astype(np.float32)  # [B, heads, T, D]
    got = apply_rope(torch.as_tensor(q, device=dev), 10, compute_rope_freqs(cfg, dev)).cpu().numpy()
    ref = OM.rope(np.transpose(q[0], (1, 0, 2)), np.arange(10, 14), cos, sin)
    assert_close(np.transpose(got[0], (1, 0, 2)), ref, 1e-5, "apply_rope at offset 10")
    mlp: MLP = blocks[2].mlp
    got = mlp(torch.as_tensor(x, device=dev)).cpu().numpy()
    L = W["layers"][2]
    ref = OM.dense(L, "down", OM.swiglu(OM.dense(L, "gate_up", x), cfg.intermediate_size))
    assert_close(got, ref, 1e-3, "mlp")
