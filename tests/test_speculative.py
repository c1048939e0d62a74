"""Speculative decoding's round logic on the CPU (no GPU): greedy acceptance
and the cache bookkeeping of /root/reference/siliconfer/engine/speculative.py
:259-352, driven with stand-in decoders whose next token is a fixed function
of their cache contents. A cache trimmed to the wrong length, a draft that
skips its catch-up step or a wrong acceptance count changes what they
predict, so the output differs from the target's plain greedy sequence, which
the reference's test_speculative.py holds as the bar."""

import numpy as np
import pytest
import torch

from siliconfer_amd._lib import SFError
from siliconfer_amd.engine.speculative import accept_greedy, speculative_generate

V = 37


def target_next(prefix) -> int:
    h = 0
    for i, t in enumerate(prefix):
        h = (h * 131 + (t + 1) * (i % 7 + 3)) % 1000003
    return h % V


def draft_next(prefix, miss_every: int) -> int:
    t = target_next(prefix)
    # disagree with the target on a fixed pattern of prefixes
    if miss_every and (sum(prefix) + len(prefix)) % miss_every == 0:
        return (t + 1) % V
    return t


class FakeDecoder:
    """The LlamaModel surface speculative_generate uses, on a token cache:
    reset / prefill / verify / set_position / replay, token, hist, pos."""

    def __init__(self, next_fn, max_seq=512):
        self.next_fn, self.max_seq, self.V = next_fn, max_seq, V
        self.device = torch.device("cpu")
        self.graph = object()
        self.cache = np.full(max_seq, -1, dtype=np.int64)
        self.token = torch.zeros(1, dtype=torch.int32)
        self.hist = torch.zeros(max_seq + 1, dtype=torch.int32)
        self.pos = 0
        self.calls = []
        self.verify_graph_sizes = set(range(1, 9))

    def reset(self):
        self.pos = 0

    def _append(self, t):
        assert self.pos < self.max_seq
        self.cache[self.pos] = t
        self.pos += 1
        return self.next_fn(self.cache[:self.pos].tolist())

    def prefill(self, ids, want_logits=True):
        for t in ids:
            nxt = self._append(int(t))
        self.token.fill_(nxt)
        return nxt

    def verify(self, ids):
        self.calls.append(len(ids))
        return [self._append(int(t)) for t in ids]

    def set_position(self, n):
        assert 0 <= n <= self.pos
        self.pos = n

    def replay(self, n=1):
        for _ in range(n):
            p = self.pos
            nxt = self._append(int(self.token.item()))
            self.hist[p] = nxt
            self.token.fill_(nxt)


def greedy(prompt, n):
    seq, out = list(prompt), []
    for _ in range(n):
        t = target_next(seq)
        out.append(t)
        seq.append(t)
    return out


def test_accept_greedy():
    assert accept_greedy([1, 2, 3], [1, 2, 3, 9]) == (3, 9)   # all accepted + bonus
    assert accept_greedy([1, 2, 3], [5, 2, 3, 9]) == (0, 5)   # first rejected
    assert accept_greedy([1, 2, 3], [1, 7, 3, 9]) == (1, 7)
    assert accept_greedy([], [4]) == (0, 4)
    with pytest.raises(SFError):
        accept_greedy([1, 2], [1, 2])


@pytest.mark.parametrize("miss_every", [0, 2, 3, 5, 1])
@pytest.mark.parametrize("K,dynamic", [(1, False), (4, False), (7, False), (3, True)])
def test_output_is_target_greedy(miss_every, K, dynamic):
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    tgt = FakeDecoder(target_next)
    drf = FakeDecoder(lambda p: draft_next(p, miss_every))
    seen = []
    r = speculative_generate(drf, tgt, prompt, max_tokens=60, K=K, dynamic_K=dynamic,
                             on_token=seen.append)
    assert r.token_ids == greedy(prompt, 60)
    assert seen == r.token_ids
    assert r.num_prefill_tokens == len(prompt) and r.num_decode_tokens == 59
    assert r.total_accepted <= r.total_draft_tokens
    # the committed tokens: one per round plus every accepted draft token
    # (the last round may be clipped to max_tokens)
    assert r.total_rounds + r.total_accepted >= 59
    # both caches end at the committed length: prompt + every token but the last
    assert tgt.pos == drf.pos == len(prompt) + r.total_rounds + r.total_accepted
    if miss_every == 0:  # a draft that always agrees: every round accepts K (or K grows)
        assert r.acceptance_rate == 1.0
    if miss_every == 1:  # always disagrees: nothing accepted, one token per round
        assert r.total_accepted == 0 and r.total_rounds == 59
    if dynamic:
        assert max(tgt.calls) <= 7 + 1 and min(tgt.calls) >= 2
    else:
        assert set(tgt.calls) == {K + 1}


def test_dynamic_k_bounds():
    prompt = [7, 7, 7]
    tgt = FakeDecoder(target_next)
    drf = FakeDecoder(lambda p: draft_next(p, 0))
    r = speculative_generate(drf, tgt, prompt, max_tokens=80, K=2, dynamic_K=True, K_min=1, K_max=5)
    assert r.token_ids == greedy(prompt, 80)
    # a draft that always agrees grows K by one per round up to K_max
    assert tgt.calls[:4] == [3, 4, 5, 6] and set(tgt.calls[4:-1]) <= {6}


def test_eos_and_budget():
    prompt = [1, 2, 3]
    ref = greedy(prompt, 40)
    eos = ref[10]
    stop = ref.index(eos)
    tgt = FakeDecoder(target_next)
    drf = FakeDecoder(lambda p: draft_next(p, 4))
    r = speculative_generate(drf, tgt, prompt, max_tokens=40, K=4, eos_token_id=eos)
    # stops after the round that committed eos; never past max_tokens
    assert r.token_ids[:stop + 1] == ref[:stop + 1] and eos in r.token_ids
    assert r.token_ids == ref[:len(r.token_ids)] and len(r.token_ids) <= stop + 1 + 4
    r = speculative_generate(drf, tgt, prompt, max_tokens=5, K=7)
    assert r.token_ids == ref[:5]


def test_argument_checks():
    tgt, drf = FakeDecoder(target_next, max_seq=40), FakeDecoder(target_next, max_seq=40)
    with pytest.raises(SFError):
        speculative_generate(drf, tgt, [1, 2], max_tokens=60)          # cache too small
    with pytest.raises(SFError):
        speculative_generate(drf, tgt, [1, 2], max_tokens=8, temperature=0.7)
    with pytest.raises(SFError):
        speculative_generate(drf, tgt, [1, 2], max_tokens=8, K=0)
    drf.graph = None
    with pytest.raises(SFError):
        speculative_generate(drf, tgt, [1, 2], max_tokens=8)
