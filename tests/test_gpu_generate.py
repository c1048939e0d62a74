"""The generation loop (siliconfer_amd/engine/generate.py) on the GPU against
the decoder's own greedy run, restating the reference's generate contract
(/root/reference/siliconfer/engine/generate.py:117-180): the tokens, the
on_token callback order, the stop after eos_token_id (the EOS token is the
last one returned and the cache holds every token but it), max_tokens, and
sampling rules that reduce to greedy (top_k = 1)."""

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle.linear import assert_close
from siliconfer_amd.engine import SamplingParams, generate, warmup
from siliconfer_amd.model.config import ModelConfig, rope_tables
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


def test_generate_against_oracle(model):
    """generate() pinned by the oracle, not only by the decoder's own runs:
    the tokens of a greedy generate() call, teacher-forced through
    oracle/model.py, are the oracle's argmax at every step whose top-2 margin
    clears 10x the logit tolerance (1e-2, fp16 activations), and the logits
    that generate() leaves for its last step meet that tolerance."""
    ids = np.random.default_rng(35).integers(0, SMALL.vocab_size, 10)
    r = generate(model, ids, SamplingParams(temperature=0, max_tokens=24))
    toks = r.token_ids
    W = model.export_weights()
    cos, sin = rope_tables(SMALL, model.max_seq)
    ref = OM.forward(W, SMALL, np.concatenate([ids, np.asarray(toks[:-1])]),
                     OM.KVCache(SMALL.num_hidden_layers), cos, sin, last_rows=len(toks))
    tol = 1e-2
    checked = 0
    for j, t in enumerate(toks):
        top2 = np.sort(ref[j])[-2:]
        if top2[1] - top2[0] > 10 * tol * np.linalg.norm(ref[j]) / np.sqrt(ref[j].size):
            assert t == OM.greedy(ref[j]), f"generate() token {j}"
            checked += 1
    print(f"generate(): {checked} of {len(toks)} tokens checked against the oracle's argmax")
    assert checked >= len(toks) // 2
    # the last step's logits, recomputed eagerly from the same state
    model.reset()
    model.prefill(np.concatenate([ids, np.asarray(toks[:-1])]))
    assert_close(model.logits.cpu().numpy(), ref[-1], tol, "generate() last-step logits")


def test_quantize_kv_cache_flag(model):
    """The reference's positional order (generate.py:117-125); the int8 cache
    is the only one here, so an explicit quantize_kv_cache=False is refused."""
    ids = np.random.default_rng(36).integers(0, SMALL.vocab_size, 5)
    p = SamplingParams(temperature=0, max_tokens=4)
    a = generate(model, ids, p, None, False, None, True)
    b = generate(model, ids, p)
    assert a.token_ids == b.token_ids
    with pytest.raises(RuntimeError, match="int8 KV cache only"):
        generate(model, ids, p, None, False, None, False)
