"""CPU checks of the generation loop's sampling rules (siliconfer_amd/engine/
generate.py), restating /root/reference/siliconfer/engine/generate.py:24-67:
temperature 0 is argmax; the repetition penalty divides positive and multiplies
negative logits of already generated ids; top-k keeps the k largest; top-p keeps
the smallest prefix of the sorted distribution whose mass before each kept token
is <= p. Sampling draws from the filtered softmax."""

import numpy as np
import pytest
import torch

from siliconfer_amd.engine.generate import SamplingParams, _prompt_array, sample_token


def test_temperature_zero_is_argmax():
    row = torch.tensor([0.1, 3.0, -2.0, 2.9])
    assert sample_token(row, SamplingParams(temperature=0)) == 1
    assert sample_token(row[None, None], SamplingParams(temperature=0)) == 1  # [B, T, V]: last row


def test_repetition_penalty_rule():
    row = torch.tensor([2.0, 1.9, -0.5, -0.6])
    # token 0 (positive) is divided by 2 -> 1.0 < 1.9: argmax moves to 1
    assert sample_token(row, SamplingParams(temperature=0, repetition_penalty=2.0), [0]) == 1
    # a negative logit is multiplied: -0.5 * 2 = -1.0, so -0.6 wins among the two
    r2 = torch.tensor([-0.5, -0.6])
    assert sample_token(r2, SamplingParams(temperature=0, repetition_penalty=2.0), [0]) == 1
    assert sample_token(row, SamplingParams(temperature=0, repetition_penalty=1.0), [0]) == 0


def test_top_k_one_and_tiny_top_p_are_greedy():
    g = torch.Generator().manual_seed(0)
    row = torch.randn(1000, generator=g)
    best = int(torch.argmax(row))
    for _ in range(20):
        assert sample_token(row, SamplingParams(temperature=1.0, top_k=1), generator=g) == best
        assert sample_token(row, SamplingParams(temperature=1.0, top_p=1e-6), generator=g) == best


def test_top_k_and_top_p_support():
    g = torch.Generator().manual_seed(1)
    row = torch.tensor([5.0, 4.0, 3.0, 0.0, -1.0])
    seen_k = {sample_token(row, SamplingParams(temperature=1.0, top_k=2), generator=g) for _ in range(200)}
    assert seen_k == {0, 1}
    # probabilities of [5, 4, 3] ~ [.66, .24, .09]: with p = 0.8 the mass before token 2 is 0.90 > 0.8
    seen_p = {sample_token(row, SamplingParams(temperature=1.0, top_p=0.8), generator=g) for _ in range(300)}
    assert seen_p == {0, 1}


def test_sampling_follows_softmax():
    g = torch.Generator().manual_seed(2)
    row = torch.tensor([1.0, 0.0, -1.0])
    n = 4000
    counts = np.bincount([sample_token(row, SamplingParams(temperature=1.0), generator=g) for _ in range(n)],
                         minlength=3) / n
    p = torch.softmax(row, 0).numpy()
    assert np.all(np.abs(counts - p) < 0.03)


def test_prompt_shapes():
    assert _prompt_array([[3, 4, 5]]).tolist() == [3, 4, 5]
    assert _prompt_array(torch.tensor([7, 8])).tolist() == [7, 8]
    from siliconfer_amd._lib import SFError
    with pytest.raises(SFError):
        _prompt_array([[1, 2], [3, 4]])
    with pytest.raises(SFError):
        _prompt_array([])


def test_reference_signatures():
    """generate / speculative_generate keep the reference's parameter order
    (engine/generate.py:117-125, engine/speculative.py:151-164); the KV-cache
    flag defaults to the int8 cache and refuses an explicit False."""
    import inspect

    from siliconfer_amd.engine import check_kv_cache_flag, generate, speculative_generate

    assert list(inspect.signature(generate).parameters)[:7] == [
        "model", "prompt_ids", "params", "eos_token_id", "stream", "on_token", "quantize_kv_cache"]
    sp = inspect.signature(speculative_generate).parameters
    assert list(sp) == ["draft", "target", "prompt_ids", "params", "K", "eos_token_id", "on_token",
                        "seed", "dynamic_K", "K_min", "K_max", "quantize_kv_cache"]
    assert sp["K"].default == 4 and sp["K_max"].default == 8 and sp["K_min"].default == 1
    check_kv_cache_flag(None)
    check_kv_cache_flag(True)
    with pytest.raises(RuntimeError, match="int8 KV cache only"):
        check_kv_cache_flag(False)
