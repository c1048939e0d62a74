"""CPU checks of the decoder oracle and the model configuration (no GPU).

Pins oracle/model.py against closed forms and invariants, and the config /
RoPE-frequency restatement against the reference's formulas
(/root/reference/siliconfer/model/config.py:52-90, model/layers.py:24-66).
"""

import math

import numpy as np
import pytest
import torch

from oracle import cpu, model as OM
from oracle import primitives as P
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


@pytest.mark.skipif(not cpu.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
def test_forward_through_reference_kernel_equals_dense():
    """The config-5 CPU baseline's path: every projection by the reference's
    q4_gemv_sym over the packed codes gives the dense forward over the same
    dequantized weights (fp32 sums in another order: 1e-4)."""
    cfg = ModelConfig(hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, vocab_size=50,
                      rms_norm_eps=1e-6, rope_theta=10000.0, attention_bias=True)
    rng = np.random.default_rng(5)
    W = tiny_weights(cfg, rng)
    for L in W["layers"]:
        for name in ("qkv", "o", "gate_up", "down"):
            pk, s = P.pack_weights_sym(L[name], 32)
            s32 = np.ascontiguousarray(s, np.float32)
            L[name + "_q4"] = (np.ascontiguousarray(pk), s32, 32)
            L[name] = P.dequant_packed(pk, s32, None, 32).astype(np.float32)
    cos, sin = rope_tables(cfg, 32)
    ids = [3, 17, 5, 42, 9, 0]
    def lin(L, name, x):
        pk, s32, g = L[name + "_q4"]
        return np.stack([cpu.gemv_sym_ref_rows(pk, s32, r, g, 3) for r in x])

    for f in (OM.dense, lin):
        cache = OM.KVCache(2)
        rows = [OM.forward(W, cfg, [t], cache, cos, sin, linear=f)[0] for t in ids]
        if f is OM.dense:
            dense = np.stack(rows)
    np.testing.assert_allclose(np.stack(rows), dense, rtol=1e-4, atol=1e-5)


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


# ---------------------------------------------------------------------------
# The whole forward pass against a scalar, per-element restatement of the
# reference's layers (/root/reference/siliconfer/model/layers.py:14-163,
# llama.py:55-79) on a tiny model, and planted mistakes that must fail it.
# ---------------------------------------------------------------------------

TINY = ModelConfig(hidden_size=8, intermediate_size=6, num_hidden_layers=2, num_attention_heads=4,
                   num_key_value_heads=2, head_dim=4, vocab_size=13, rms_norm_eps=1e-6,
                   rope_theta=10000.0)


def scalar_fixture_weights(seed=0):
    rng = np.random.default_rng(seed)
    c = TINY
    H, I, D = c.hidden_size, c.intermediate_size, c.head_dim
    rows = (c.num_attention_heads + 2 * c.num_key_value_heads) * D
    f = lambda *s, sd=0.5: rng.normal(0, sd, s).astype(np.float32)
    layers = [{"qkv": f(rows, H), "qkv_bias": f(rows, sd=0.2), "o": f(H, c.num_attention_heads * D),
               "gate_up": f(2 * I, H), "down": f(H, I), "w_in": 1 + f(H, sd=0.2),
               "w_post": 1 + f(H, sd=0.2)} for _ in range(c.num_hidden_layers)]
    return {"embed": f(c.vocab_size, H, sd=1.0), "norm": 1 + f(H, sd=0.2), "layers": layers}


def _cache_dequant(vec):
    """One cached vector as the int8 cache holds it (fp32 rule, fp16 scale)."""
    x = np.asarray(vec, np.float32)
    amax = np.float32(max(abs(float(v)) for v in x))
    s = np.float32(1.0) if amax == 0 else np.float32(amax / np.float32(127))
    codes = [max(-128, min(127, float(np.rint(np.float32(v / s))))) for v in x]
    s16 = float(np.float32(np.float16(s)))
    return [c * s16 for c in codes]


def scalar_forward(W, cfg, ids, cos, sin):
    """Token by token, element by element, in float64 (the logits of every token)."""
    H, Hq, KVH, D, I = (cfg.hidden_size, cfg.num_attention_heads, cfg.num_key_value_heads,
                        cfg.head_dim, cfg.intermediate_size)
    half, G, eps = D // 2, Hq // KVH, cfg.rms_norm_eps
    kcache = [[[] for _ in range(KVH)] for _ in W["layers"]]
    vcache = [[[] for _ in range(KVH)] for _ in W["layers"]]

    def rms(x, w):
        r = 1.0 / math.sqrt(sum(v * v for v in x) / len(x) + eps)
        return [x[i] * r * float(w[i]) for i in range(len(x))]

    def matvec(M, x):
        return [sum(float(M[r][i]) * x[i] for i in range(len(x))) for r in range(len(M))]

    def rot(v, p):
        out = list(v)
        for d in range(half):
            c, s = float(cos[p][d]), float(sin[p][d])
            out[d] = v[d] * c - v[d + half] * s
            out[d + half] = v[d + half] * c + v[d] * s
        return out

    logits = []
    for p, tok in enumerate(ids):
        x = [float(v) for v in W["embed"][tok]]
        for l, L in enumerate(W["layers"]):
            qkv = [a + float(b) for a, b in zip(matvec(L["qkv"], rms(x, L["w_in"])), L["qkv_bias"])]
            q = [rot(qkv[h * D:(h + 1) * D], p) for h in range(Hq)]
            for h in range(KVH):
                kcache[l][h].append(_cache_dequant(rot(qkv[(Hq + h) * D:(Hq + h + 1) * D], p)))
                vcache[l][h].append(_cache_dequant(qkv[(Hq + KVH + h) * D:(Hq + KVH + h + 1) * D]))
            attn = []
            for h in range(Hq):
                ks, vs = kcache[l][h // G], vcache[l][h // G]
                sc = [sum(q[h][d] * k[d] for d in range(D)) / math.sqrt(D) for k in ks]
                m = max(sc)
                e = [math.exp(s - m) for s in sc]
                attn += [sum(e[j] * vs[j][d] for j in range(len(e))) / sum(e) for d in range(D)]
            x = [a + b for a, b in zip(x, matvec(L["o"], attn))]
            gu = matvec(L["gate_up"], rms(x, L["w_post"]))
            act = [gu[j] / (1.0 + math.exp(-gu[j])) * gu[I + j] for j in range(I)]
            x = [a + b for a, b in zip(x, matvec(L["down"], act))]
        logits.append(matvec(W["embed"], rms(x, W["norm"])))
    return np.array(logits)


def oracle_logits(W, ids):
    cos, sin = rope_tables(TINY, 16)
    cache = OM.KVCache(TINY.num_hidden_layers)
    rows = [OM.forward(W, TINY, ids[:3], cache, cos, sin)]  # a causal block, then single tokens
    for t in ids[3:]:
        rows.append(OM.forward(W, TINY, [t], cache, cos, sin))
    return np.concatenate(rows)


def rel_err(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


IDS = [3, 11, 0, 7, 7, 2]


def test_forward_equals_scalar_restatement():
    W = scalar_fixture_weights(1)
    cos, sin = rope_tables(TINY, 16)
    ref = scalar_forward(W, TINY, IDS, cos, sin)
    assert rel_err(oracle_logits(W, IDS), ref) < 1e-5


def _rope_interleaved(x, positions, cos_t, sin_t):
    c, s = cos_t[positions][:, None, :], sin_t[positions][:, None, :]
    x1, x2 = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2], out[..., 1::2] = x1 * c - x2 * s, x2 * c + x1 * s
    return out


ORIG_ROPE, ORIG_ATTEND = OM.rope, OM.attend


def _attend_wrong_group(q, K, V, pos0, scale):
    """Head h reads kv head h % KVH instead of h // (H / KVH): permute the heads
    so the correct mapping sends each to the wrong kv head, then back."""
    H, KVH = q.shape[1], K.shape[0]
    G = H // KVH
    slot = [(h % KVH) * G + h // KVH for h in range(H)]
    qp = np.empty_like(q)
    qp[:, slot] = q
    return ORIG_ATTEND(qp, K, V, pos0, scale)[:, slot]


MISTAKES = {
    "gate_up_swapped": ("swiglu", lambda gu, I: (gu[:, I:] / (np.float32(1) + np.exp(-gu[:, I:]))) * gu[:, :I]),
    "sigmoid_not_silu": ("swiglu", lambda gu, I: (np.float32(1) / (np.float32(1) + np.exp(-gu[:, :I]))) * gu[:, I:]),
    "dropped_residual": ("residual", lambda x, d: d),
    "rope_interleaved": ("rope", _rope_interleaved),
    "rope_sin_sign": ("rope", lambda x, p, c, s: ORIG_ROPE(x, p, c, -s)),
    "wrong_gqa_head": ("attend", _attend_wrong_group),
}


@pytest.mark.parametrize("name", sorted(MISTAKES))
def test_planted_mistakes_fail_the_bar(monkeypatch, name):
    """Each mistake, planted in the oracle, moves the logits far past the
    decoder's 1e-2 bar against the scalar restatement."""
    W = scalar_fixture_weights(1)
    cos, sin = rope_tables(TINY, 16)
    ref = scalar_forward(W, TINY, IDS, cos, sin)
    attr, fn = MISTAKES[name]
    monkeypatch.setattr(OM, attr, fn)
    assert rel_err(oracle_logits(W, IDS), ref) > 1e-2


def test_attend_equals_per_row_loop():
    """The vectorised causal attention against a per-(row, head) loop with its
    own softmax, at a start offset (prefill after a cached prefix) and GQA 3:1."""
    rng = np.random.default_rng(7)
    T, H, KVH, D, pos0 = 5, 6, 2, 8, 4
    q = rng.normal(0, 1, (T, H, D)).astype(np.float32)
    K = rng.normal(0, 1, (KVH, pos0 + T, D)).astype(np.float32)
    V = rng.normal(0, 1, (KVH, pos0 + T, D)).astype(np.float32)
    got = OM.attend(q, K, V, pos0, 0.3)
    for t in range(T):
        for h in range(H):
            k, v = K[h // 3, :pos0 + t + 1].astype(np.float64), V[h // 3, :pos0 + t + 1].astype(np.float64)
            s = k @ q[t, h].astype(np.float64) * 0.3
            p = np.exp(s - s.max())
            np.testing.assert_allclose(got[t, h], p @ v / p.sum(), rtol=2e-6, atol=1e-7)
