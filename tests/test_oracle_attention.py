"""Pins the oracle's int8 KV quantization and decode attention (CPU only).

Reference: siliconfer/model/kv_cache.py:49-68, tests/test_kv_cache.py:24-81;
siliconfer/kernels/metal/q4_attention.py:63-70,183-261,
tests/test_metal_attention.py.
"""

import numpy as np
import pytest

from oracle import attention as A, cpu


def _inputs(rng, B, H, KVH, D, T):
    q = rng.normal(0, 1, (B, H, D))
    k = rng.normal(0, 1, (B, KVH, T, D)).astype(np.float32)
    v = rng.normal(0, 1, (B, KVH, T, D)).astype(np.float32)
    kc, ks = A.quantize_kv(k)
    vc, vs = A.quantize_kv(v)
    return q, kc, ks, vc, vs


def test_quantize_kv_closed_form():
    rng = np.random.default_rng(0)
    x = rng.normal(0, 1, (1, 2, 16, 64)).astype(np.float32)
    q, s = A.quantize_kv(x)
    assert q.dtype == np.int8 and s.shape == (1, 2, 16, 1) and s.dtype == np.float32
    np.testing.assert_array_equal(s, np.abs(x).max(-1, keepdims=True) / np.float32(127))
    assert q.min() >= -127          # -128 never produced: |x|/s <= 127
    assert np.all(np.abs(q).max(-1) == 127)
    err = np.abs(A.dequantize_kv(q, s) - x)
    assert err.max() < 0.05 * np.abs(x).max()     # test_kv_cache.py:33-45


def test_quantize_kv_zero_vector_and_ties():
    q, s = A.quantize_kv(np.zeros((1, 1, 1, 64), np.float32))
    assert np.all(q == 0) and s.item() == 1.0     # kv_cache.py:61 scale-1 fallback
    x = np.zeros((1, 1, 1, 8), np.float32)
    x[..., 0] = 127.0
    x[..., 1:4] = [2.5, 3.5, -0.5]
    q, s = A.quantize_kv(x)
    assert s.item() == 1.0 and q[0, 0, 0, :4].tolist() == [127, 2, 4, 0]


def test_incremental_equals_batch_quantization():
    rng = np.random.default_rng(1)
    k = rng.normal(0, 1, (1, 2, 5, 64)).astype(np.float32)
    qb, sb = A.quantize_kv(k)
    for t in range(5):
        qt, st = A.quantize_kv(k[:, :, t:t + 1])
        np.testing.assert_array_equal(qt[:, :, 0], qb[:, :, t])
        np.testing.assert_array_equal(st[:, :, 0], sb[:, :, t])


def test_single_token_returns_v():
    rng = np.random.default_rng(2)
    q, kc, ks, vc, vs = _inputs(rng, 1, 4, 4, 8, 1)
    out = A.attention_decode(q, kc, ks, vc, vs)
    np.testing.assert_allclose(out, A.dequantize_kv(vc, vs)[:, :, 0], rtol=1e-12)


def test_identical_keys_give_mean_of_v():
    rng = np.random.default_rng(3)
    B, H, KVH, D, T = 1, 2, 1, 16, 9
    kc = np.repeat(rng.integers(-100, 100, (B, KVH, 1, D), dtype=np.int8), T, axis=2)
    ks = np.full((B, KVH, T, 1), 0.01, np.float32)
    vc = rng.integers(-127, 128, (B, KVH, T, D)).astype(np.int8)
    vs = rng.uniform(0.001, 0.02, (B, KVH, T, 1)).astype(np.float32)
    out = A.attention_decode(rng.normal(0, 1, (B, H, D)), kc, ks, vc, vs)
    mean_v = A.dequantize_kv(vc, vs).mean(axis=2)
    np.testing.assert_allclose(out[:, 0], mean_v[:, 0], rtol=1e-12)
    np.testing.assert_allclose(out[:, 1], mean_v[:, 0], rtol=1e-12)


def test_gqa_equals_mha_with_repeated_heads():
    rng = np.random.default_rng(4)
    q, kc, ks, vc, vs = _inputs(rng, 2, 14, 2, 64, 37)
    out = A.attention_decode(q, kc, ks, vc, vs)
    rep = lambda a: np.repeat(a, 7, axis=1)
    out_mha = A.attention_decode(q, rep(kc), rep(ks), rep(vc), rep(vs))
    np.testing.assert_allclose(out, out_mha, rtol=1e-12)


@pytest.mark.parametrize("n_tiles", [1, 2, 3, 7, 16, 64, 200])
def test_split_combine_equals_unsplit(n_tiles):
    """test_metal_attention.py:124-139 — including uneven and > T tile counts."""
    rng = np.random.default_rng(11)
    q, kc, ks, vc, vs = _inputs(rng, 1, 14, 2, 64, 100)
    m, l, acc = A.split_partials(q, kc, ks, vc, vs, n_tiles)
    np.testing.assert_allclose(A.combine(m, l, acc), A.attention_decode(q, kc, ks, vc, vs),
                               rtol=1e-10, atol=1e-12)


def test_softmax_against_brute_force():
    rng = np.random.default_rng(5)
    q, kc, ks, vc, vs = _inputs(rng, 1, 1, 1, 8, 6)
    K = kc[0, 0].astype(np.float64) * ks[0, 0]
    V = vc[0, 0].astype(np.float64) * vs[0, 0]
    s = [float(np.dot(q[0, 0], K[t])) / np.sqrt(8) for t in range(6)]
    w = [np.exp(x) for x in s]
    ref = sum(w[t] * V[t] for t in range(6)) / sum(w)
    np.testing.assert_allclose(A.attention_decode(q, kc, ks, vc, vs)[0, 0], ref, rtol=1e-12)


def test_choose_n_tiles_heuristic():
    """test_metal_attention.py:160-165."""
    assert A.choose_n_tiles(8) == 1
    assert A.choose_n_tiles(128) > A.choose_n_tiles(32) > A.choose_n_tiles(8)
    assert A.choose_n_tiles(1_000_000) <= 256


def test_c_port_attention_matches_oracle():
    rng = np.random.default_rng(6)
    q, kc, ks, vc, vs = _inputs(rng, 1, 14, 2, 64, 300)
    out = cpu.attn_decode(q, kc, ks, vc, vs, nthreads=2)
    ref = A.attention_decode(q, kc, ks, vc, vs)
    assert np.abs(out - ref).max() <= 2e-5 * np.abs(ref).max()
