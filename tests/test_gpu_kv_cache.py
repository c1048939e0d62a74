"""GPU checks of the int8 KV cache: quantization bit-exact against the oracle,
and the QuantizedKVCache API. Reference tests restated:
tests/test_kv_cache.py:24-122.
"""

import numpy as np
import pytest
import torch

from oracle import attention as A
from siliconfer_amd.model.kv_cache import (QuantizedKVCache, dequantize_kv,
                                           make_quantized_cache, quantize_kv)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128, 8])
def test_quantize_kv_bit_exact(dev, dtype, D):
    rng = np.random.default_rng(D)
    x = torch.as_tensor(rng.normal(0, 2, (2, 3, 33, D)).astype(np.float32)).to(dtype)
    q, s = quantize_kv(x.to(dev))
    q_ref, s_ref = A.quantize_kv(x.float().numpy())
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    assert q.dtype == torch.int8 and tuple(s.shape) == (2, 3, 33, 1)


def test_fp16_scale_storage_is_rounded_fp32_scale(dev):
    rng = np.random.default_rng(1)
    k = torch.as_tensor(rng.normal(0, 1, (1, 2, 40, 64)).astype(np.float16))
    cache = QuantizedKVCache(capacity=64)
    cache.append(k.to(dev), k.to(dev))
    q_ref, s_ref = A.quantize_kv(k.float().numpy())
    np.testing.assert_array_equal(cache.q_k.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(cache.s_k.cpu().numpy(), s_ref.astype(np.float16))


def test_zero_vector_safe(dev):
    q, s = quantize_kv(torch.zeros((1, 1, 1, 64), device=dev))
    assert torch.all(q == 0) and float(s) == 1.0
    assert torch.all(dequantize_kv(q, s) == 0)


def test_incremental_matches_batch(dev):
    rng = np.random.default_rng(1)
    k = torch.as_tensor(rng.normal(0, 1, (1, 2, 5, 64)).astype(np.float32)).to(dev)
    v = torch.as_tensor(rng.normal(0, 1, (1, 2, 5, 64)).astype(np.float32)).to(dev)
    qb, sb = quantize_kv(k)
    cache = QuantizedKVCache(capacity=2, scale_dtype=torch.float32)   # also forces growth
    for t in range(5):
        cache.update(k[:, :, t:t + 1], v[:, :, t:t + 1])
    assert cache.length() == 5
    assert torch.equal(cache.q_k, qb)
    assert torch.equal(cache.s_k, sb)


def test_length_trim_and_update_return(dev):
    cache = QuantizedKVCache()
    assert cache.length() == 0
    k = torch.randn(1, 2, 3, 64, device=dev)
    kd, vd = cache.update(k, k)
    assert cache.length() == 3 and kd.shape == (1, 2, 3, 64)
    assert (kd - k).abs().max() <= 0.02 * k.abs().max()
    cache.update(torch.randn(1, 2, 2, 64, device=dev), torch.randn(1, 2, 2, 64, device=dev))
    assert cache.length() == 5
    cache.trim(4)
    assert cache.length() == 4 and cache.q_k.shape[2] == 4


def test_nbytes_roughly_half_of_fp16(dev):
    cache = QuantizedKVCache(scale_dtype=torch.float32)
    k = torch.randn(1, 2, 100, 64, device=dev)
    cache.update(k, k)
    ratio = cache.nbytes() / (2 * 1 * 2 * 100 * 64 * 2)
    assert 0.4 < ratio < 0.7


def test_make_quantized_cache():
    caches = make_quantized_cache(6)
    assert len(caches) == 6 and all(c.length() == 0 for c in caches)
