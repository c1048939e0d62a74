"""The generation loop (siliconfer_amd/engine/generate.py) on the GPU against
the decoder's own greedy run, restating the reference's generate contract
(/root/reference/siliconfer/engine/generate.py:117-180): the tokens, the
on_token callback order, the stop after eos_token_id (the EOS token is the
last one returned and the cache holds every token but it), max_tokens, and
sampling rules that reduce to greedy (top_k = 1)."""

import numpy as np
import pytest
import torch

from siliconfer_amd.engine import SamplingParams, generate, warmup
from siliconfer_amd.model.config import ModelConfig
from siliconfer_amd.model.llama import LlamaModel

pytestmark = pytest.mark.gpu

SMALL = ModelConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                    num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=1000,
                    rms_norm_eps=1e-6, rope_theta=1e6, tie_word_embeddings=True)


@pytest.fixture(scope="module")
def model():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    dev = torch.device("cuda", 0)
    m = LlamaModel.random_init(SMALL, seed=31, device=dev, max_seq=160, act_dtype=torch.float16)
    warmup(m)
    return m


def test_greedy_tokens_and_callbacks(model):
    ids = np.random.default_rng(32).integers(0, SMALL.vocab_size, 9)
    ref = model.generate(ids, 40)
    seen = []
    r = generate(model, ids, SamplingParams(temperature=0, max_tokens=40), on_token=seen.append)
    assert r.token_ids == ref.token_ids == seen
    assert r.num_prefill_tokens == 9 and r.num_decode_tokens == 39
    r1 = generate(model, [ids.tolist()], SamplingParams(temperature=0, max_tokens=1))
    assert r1.token_ids == ref.token_ids[:1] and r1.num_decode_tokens == 0


@pytest.mark.parametrize("at", [0, 5, 22, 39])
def test_eos_stops_and_trims_the_cache(model, at):
    ids = np.random.default_rng(33).integers(0, SMALL.vocab_size, 12)
    ref = model.generate(ids, 40).token_ids
    eos = ref[at]
    k = ref.index(eos)  # first occurrence
    seen = []
    r = generate(model, ids, SamplingParams(temperature=0, max_tokens=40), eos_token_id=eos,
                 on_token=seen.append)
    assert r.token_ids == ref[:k + 1] == seen
    assert model.pos == 12 + k and int(model.pos_dev.item()) == 12 + k
    # a decode step from the trimmed state continues the uninterrupted sequence
    if k + 1 < len(ref):
        model.token.fill_(eos)
        model.replay(1)
        assert int(model.hist[12 + k].item()) == ref[k + 1]


def test_sampling_paths(model):
    ids = np.random.default_rng(34).integers(0, SMALL.vocab_size, 7)
    ref = model.generate(ids, 12).token_ids
    r = generate(model, ids, SamplingParams(temperature=1.0, top_k=1, max_tokens=12))
    assert r.token_ids == ref
    g1 = torch.Generator(device=model.device).manual_seed(5)
    g2 = torch.Generator(device=model.device).manual_seed(5)
    a = generate(model, ids, SamplingParams(temperature=0.8, top_p=0.9, max_tokens=12), generator=g1)
    b = generate(model, ids, SamplingParams(temperature=0.8, top_p=0.9, max_tokens=12), generator=g2)
    assert a.token_ids == b.token_ids and all(0 <= t < SMALL.vocab_size for t in a.token_ids)
    assert model.pos == 7 + 11
