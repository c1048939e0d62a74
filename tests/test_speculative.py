"""Speculative decoding's round logic on the CPU (no GPU): greedy acceptance
and the cache bookkeeping of /root/reference/siliconfer/engine/speculative.py
:259-352, driven with stand-in decoders whose next token is a fixed function
of their cache contents. A cache trimmed to the wrong length, a draft that
skips its catch-up step or a wrong acceptance count changes what they
predict, so the output differs from the target's plain greedy sequence, which
the reference's test_speculative.py holds as the bar."""

import itertools

import numpy as np
import pytest
import torch

from siliconfer_amd._lib import SFError
from siliconfer_amd.engine import SamplingParams
from siliconfer_amd.engine.speculative import accept_greedy, speculative_generate

V = 37


def G(n):  # greedy parameters for n tokens
    return SamplingParams(temperature=0.0, max_tokens=n)


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


class FakeLogitDecoder(FakeDecoder):
    """A stand-in whose next-token logits are a fixed function of its cache
    (`logit_fn(prefix) -> [V]`), with the logits surface the sampled path
    uses: prefill / decode_step / verify with logits, sibling, capture."""

    def __init__(self, logit_fn, vocab, max_seq=64):
        self.logit_fn = logit_fn
        super().__init__(lambda p: int(np.argmax(logit_fn(p))), max_seq)
        self.V = vocab
        self.graph = None
        self.logits = torch.zeros(vocab, dtype=torch.float32)
        self.vlogits = torch.zeros((8, vocab), dtype=torch.float32)

    def _row(self):
        return torch.as_tensor(np.asarray(self.logit_fn(self.cache[:self.pos].tolist()), np.float32))

    def prefill(self, ids, want_logits=True):
        for t in ids:
            self._append(int(t))
        self.logits = self._row()
        self.token.fill_(int(torch.argmax(self.logits)))
        return int(self.token.item())

    def decode_step(self, logits=False):
        p = self.pos  # the caller advances the host position, as for LlamaModel
        self._append(int(self.token.item()))
        self.logits = self._row()
        self.pos = p
        nxt = int(torch.argmax(self.logits))
        self.hist[p] = nxt
        self.token.fill_(nxt)

    def verify(self, ids, want_logits=False):
        self.calls.append(len(ids))
        out = []
        for i, t in enumerate(ids):
            self._append(int(t))
            self.vlogits[i] = self._row()
            out.append(int(torch.argmax(self.vlogits[i])))
        return out

    def capture(self):
        self.graph = object()

    def sibling(self):
        return FakeLogitDecoder(self.logit_fn, self.V, self.max_seq)


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
    r = speculative_generate(drf, tgt, prompt, G(60), K=K, dynamic_K=dynamic,
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
    r = speculative_generate(drf, tgt, prompt, G(80), K=2, dynamic_K=True, K_min=1, K_max=5)
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
    r = speculative_generate(drf, tgt, prompt, G(40), K=4, eos_token_id=eos)
    # stops after the round that committed eos; never past max_tokens
    assert r.token_ids[:stop + 1] == ref[:stop + 1] and eos in r.token_ids
    assert r.token_ids == ref[:len(r.token_ids)] and len(r.token_ids) <= stop + 1 + 4
    r = speculative_generate(drf, tgt, prompt, G(5), K=7)
    assert r.token_ids == ref[:5]


def test_argument_checks():
    tgt, drf = FakeDecoder(target_next, max_seq=40), FakeDecoder(target_next, max_seq=40)
    with pytest.raises(SFError):
        speculative_generate(drf, tgt, [1, 2], G(60))          # cache too small
    with pytest.raises(SFError, match="at most 8 rows"):
        speculative_generate(drf, tgt, [1, 2], G(8), K=8)
    with pytest.raises(SFError):
        speculative_generate(drf, tgt, [1, 2], G(8), K=0)
    with pytest.raises(SFError, match="int8 KV cache only"):
        speculative_generate(drf, tgt, [1, 2], G(8), quantize_kv_cache=False)


def test_reference_argument_order():
    """The reference's positional order (speculative.py:151-164): params,
    K, eos_token_id, on_token, seed, dynamic_K, K_min, K_max,
    quantize_kv_cache; K_max defaults to 8 and dynamic_K then stops at 7."""
    prompt = [2, 7, 1, 8]
    tgt = FakeDecoder(target_next)
    drf = FakeDecoder(lambda p: draft_next(p, 0))
    seen = []
    r = speculative_generate(drf, tgt, prompt, G(50), 2, None, seen.append, 0, True, 1, 8, True)
    assert r.token_ids == greedy(prompt, 50) and seen == r.token_ids
    assert max(tgt.calls) == 8  # K grew to 7 (8 verify rows), not to K_max = 8


LOGIT_V = 4


def _logits(prefix, salt):
    h = 0
    for i, t in enumerate(prefix):
        h = (h * 1000003 + (t + 3) * (i + salt)) % 2147483647
    r = np.random.default_rng(h)
    return r.normal(0, 1.2, LOGIT_V)


def _target_seq_probs(prompt, n, temp):
    """Exact probability of each n-token continuation under the target."""
    probs = {}
    for seq in itertools.product(range(LOGIT_V), repeat=n):
        p, pre = 1.0, list(prompt)
        for t in seq:
            z = _logits(pre, 1) / temp
            e = np.exp(z - z.max())
            p *= e[t] / e.sum()
            pre.append(t)
        probs[seq] = p
    return probs


def test_sampled_output_follows_target_distribution():
    """Losslessness (speculative.py:1-10): at temperature > 0 the committed
    tokens are distributed as the target's own samples, whatever the draft.
    3-token continuations over a 4-token vocabulary, 3000 seeded runs against
    the exact target probabilities (chi-square). The draft's own distribution
    is far from the target's at this sample size, so always accepting the
    draft, or a wrong acceptance ratio, fails the bar."""
    from scipy.stats import chi2

    prompt, n, temp, runs = [1, 3], 3, 1.0, 3000
    want = _target_seq_probs(prompt, n, temp)
    tgt = FakeLogitDecoder(lambda p: _logits(p, 1), LOGIT_V)
    drf = FakeLogitDecoder(lambda p: _logits(p, 5), LOGIT_V)
    counts = dict.fromkeys(want, 0)
    params = SamplingParams(temperature=temp, max_tokens=n)
    for seed in range(runs):
        r = speculative_generate(drf, tgt, prompt, params, K=2, seed=seed)
        counts[tuple(r.token_ids)] += 1
    exp = np.array([want[k] * runs for k in want])
    obs = np.array([counts[k] for k in want])
    stat = float(((obs - exp) ** 2 / exp).sum())
    assert chi2.sf(stat, len(want) - 1) > 1e-4, f"chi-square {stat:.1f}"
    # power: the draft's sequence distribution against the target's at this n
    dq = {}
    for seq in want:
        p, pre = 1.0, list(prompt)
        for t in seq:
            z = _logits(pre, 5) / temp
            e = np.exp(z - z.max())
            p *= e[t] / e.sum()
            pre.append(t)
        dq[seq] = p
    d = np.array([dq[k] * runs for k in want])
    assert float(((d - exp) ** 2 / exp).sum()) > 10 * chi2.isf(1e-4, len(want) - 1)


def test_sampled_same_model_accepts_everything():
    """draft = target at temperature > 0: p_target / p_draft = 1 for every
    proposal, so every round accepts all K (test_speculative.py:149-152)."""
    tgt = FakeLogitDecoder(lambda p: _logits(p, 1), LOGIT_V)
    p = SamplingParams(temperature=0.7, max_tokens=25)
    r = speculative_generate(tgt, tgt, [2, 2], p, K=3, seed=11)
    assert r.acceptance_rate == 1.0 and len(r.token_ids) == 25
    r2 = speculative_generate(tgt, tgt, [2, 2], p, K=3, seed=11)
    assert r2.token_ids == r.token_ids
