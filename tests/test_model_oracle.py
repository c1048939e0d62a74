"""CPU checks of the decoder oracle and the model configuration (no GPU).

Pins oracle/model.py against closed forms and invariants, and the config /
RoPE-frequency restatement against the reference's formulas
(/root/reference/siliconfer/model/config.py:52-90, model/layers.py:24-66).
"""

import math

import numpy as np
import pytest
import torch

from oracle import model as OM
from siliconfer_amd.model.config import ModelConfig, RoPEScalingConfig, rope_freqs, rope_tables


def test_rmsnorm_closed_form():
    rng = np.random.default_rng(0)
    x = rng.normal(0, 3, (4, 96)).astype(np.float32)
    w = rng.normal(1, 0.1, 96).astype(np.float32)
    got = OM.rmsnorm(x, w, 1e-6)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-6)
    # a constant row normalises to +-1 (times w)
    c = np.full((1, 8), -5.0, np.float32)
    np.testing.assert_allclose(OM.rmsnorm(c, np.ones(8, np.float32), 0.0), -np.ones((1, 8)), rtol=1e-6)


def test_rope_identity_at_zero_and_norm_preserving():
    cfg = ModelConfig(hidden_size=64, num_attention_heads=2, head_dim=32, rope_theta=10000.0)
    cos, sin = rope_tables(cfg, 64)
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (3, 2, 32)).astype(np.float32)
    np.testing.assert_array_equal(OM.rope(x[:1], np.array([0]), cos, sin), x[:1])
    y = OM.rope(x, np.array([5, 17, 63]), cos, sin)
    pairs_x = x[..., :16] ** 2 + x[..., 16:] ** 2
    pairs_y = y[..., :16] ** 2 + y[..., 16:] ** 2
    np.testing.assert_allclose(pairs_y, pairs_x, rtol=1e-5)
    # rotating by p then reading the angle back: position 1, pair 0 turns by freq 1 rad
    e = np.zeros((1, 1, 32), np.float32)
    e[0, 0, 0] = 1.0
    r = OM.rope(e, np.array([1]), cos, sin)
    assert abs(r[0, 0, 0] - math.cos(1.0)) < 1e-6 and abs(r[0, 0, 16] - math.sin(1.0)) < 1e-6


def test_rope_freqs_formula_and_llama3_scaling():
    cfg = ModelConfig(hidden_size=128, num_attention_heads=2, head_dim=64, rope_theta=1e6)
    f = rope_freqs(cfg)
    ref = 1.0 / (1e6 ** (np.arange(0, 64, 2) / 64.0))
    np.testing.assert_allclose(f, ref, rtol=1e-6)
    cfg.rope_scaling = RoPEScalingConfig(type="llama3", factor=8.0, low_freq_factor=1.0,
                                         high_freq_factor=4.0, original_max_position_embeddings=8192)
    g = rope_freqs(cfg)
    wl = 2 * math.pi / ref
    assert np.allclose(g[wl < 8192 / 4.0], ref[wl < 8192 / 4.0])       # high frequencies kept
    assert np.allclose(g[wl > 8192 / 1.0], ref[wl > 8192 / 1.0] / 8.0)  # low frequencies scaled
    mid = (wl >= 2048) & (wl <= 8192)
    smooth = (8192 / wl[mid] - 1.0) / 3.0
    np.testing.assert_allclose(g[mid], (1 - smooth) * ref[mid] / 8 + smooth * ref[mid], rtol=1e-5)


def test_config_from_dict_defaults_and_preset():
    c = ModelConfig.from_dict({"hidden_size": 896, "num_attention_heads": 14, "num_hidden_layers": 2})
    assert c.head_dim == 64 and c.num_key_value_heads == 14 and c.rms_norm_eps == 1e-5
    assert c.rope_theta == 500000.0 and c.attention_bias is False
    q = ModelConfig.qwen25_05b()
    assert (q.num_hidden_layers, q.hidden_size, q.intermediate_size, q.vocab_size) == (24, 896, 4864, 151936)
    assert (q.num_attention_heads, q.num_key_value_heads, q.head_dim, q.gqa_groups) == (14, 2, 64, 7)
    assert q.tie_word_embeddings and q.attention_bias and q.rope_theta == 1e6


def test_attend_single_token_returns_v():
    rng = np.random.default_rng(2)
    K = rng.normal(0, 1, (2, 1, 16)).astype(np.float32)
    V = rng.normal(0, 1, (2, 1, 16)).astype(np.float32)
    q = rng.normal(0, 1, (1, 4, 16)).astype(np.float32)
    out = OM.attend(q, K, V, 0, 0.25)
    for h in range(4):
        np.testing.assert_allclose(out[0, h], V[h // 2, 0], rtol=1e-6)


def tiny_weights(cfg, rng):
    H, I, D, Hq, KVH = (cfg.hidden_size, cfg.intermediate_size, cfg.head_dim,
                        cfg.num_attention_heads, cfg.num_key_value_heads)
    w = lambda *s: rng.normal(0, 0.05, s).astype(np.float32)
    layers = [dict(qkv=w((Hq + 2 * KVH) * D, H), qkv_bias=w((Hq + 2 * KVH) * D), o=w(H, Hq * D),
                   gate_up=w(2 * I, H), down=w(H, I), w_in=np.ones(H, np.float32),
                   w_post=np.ones(H, np.float32)) for _ in range(cfg.num_hidden_layers)]
    return dict(embed=w(cfg.vocab_size, H), norm=np.ones(H, np.float32), layers=layers)


def test_causal_block_equals_token_by_token():
    cfg = ModelConfig(hidden_size=32, intermediate_size=64, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=8, vocab_size=50,
                      rms_norm_eps=1e-6, rope_theta=10000.0, attention_bias=True)
    rng = np.random.default_rng(3)
    W = tiny_weights(cfg, rng)
    cos, sin = rope_tables(cfg, 32)
    ids = [3, 17, 5, 42, 9, 0]
    block = OM.forward(W, cfg, ids, OM.KVCache(2), cos, sin)
    cache = OM.KVCache(2)
    rows = [OM.forward(W, cfg, [t], cache, cos, sin)[0] for t in ids]
    np.testing.assert_allclose(block, np.stack(rows), rtol=1e-4, atol=1e-5)


def test_pack_sym_device_matches_numpy_packer():
    """The device-side packer (run here on CPU tensors) gives the numpy
    packer's codes and scales bit for bit."""
    from siliconfer_amd.kernels import pack_weights_sym
    from siliconfer_amd.model.llama import pack_sym_device

    rng = np.random.default_rng(4)
    W = rng.normal(0, 0.02, (48, 256)).astype(np.float32)
    W[3, :64] = 0.0  # an all-zero group
    pk, s = pack_weights_sym(W, 64)
    tpk, ts = pack_sym_device(torch.from_numpy(W), 64)
    np.testing.assert_array_equal(tpk.numpy(), pk)
    np.testing.assert_array_equal(ts.numpy(), s)
