"""Greedy speculative decoding over two int4 decoders on one GPU — the
reference's siliconfer.engine.speculative (/root/reference/siliconfer/engine/
speculative.py:151-365) at temperature 0.

Each round (speculative.py:259-352):
  1. the draft proposes K tokens from the last committed token: K decode
     steps, replayed from the draft's HIP graph without a host round trip;
  2. the target verifies [cur, d_0 .. d_{K-1}] in one forward
     (`LlamaModel.verify`: K + 1 <= 8 rows run every projection as one batch
     GEMV, so the verify streams the target's weights once; it replays the
     target's verify graph for K + 1 rows, recorded on first use);
  3. d_q is accepted while it equals the target's greedy token after row q
     (`_tok_prob` at temperature 0 gives 1 or 0, :44-51); the first mismatch
     is replaced by the target's token, and a fully accepted round adds the
     target's bonus token after row K (:286-303);
  4. both KV caches are trimmed to the committed length N + j + 1
     (`LlamaModel.set_position`, the cache `trim` of :29-41); when every draft
     token was accepted the draft runs d_{K-1} to catch up (:336-343);
  5. with `dynamic_K`, K grows by one after a fully accepted round and shrinks
     by one after a rejection, within [K_min, K_max] (:311-315).

The committed tokens are the target's own greedy choices at every position,
so the output is the target's greedy generation; the draft only decides how
many tokens one verify commits. Sampling at temperature > 0 is not part of
this build (the decoders pick greedily on the device)."""

from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Callable

import numpy as np
import torch

from .._lib import SFError


@dataclass
class SpeculativeResult:
    """The reference's SpeculativeResult (speculative.py:117-144)."""
    token_ids: list[int]
    prefill_time: float
    decode_time: float
    num_prefill_tokens: int
    num_decode_tokens: int
    total_rounds: int
    total_draft_tokens: int
    total_accepted: int

    @property
    def acceptance_rate(self) -> float:
        return self.total_accepted / self.total_draft_tokens if self.total_draft_tokens else 0.0

    @property
    def effective_tok_s(self) -> float:
        return self.num_decode_tokens / self.decode_time if self.decode_time else 0.0

    @property
    def prefill_tok_s(self) -> float:
        return self.num_prefill_tokens / self.prefill_time if self.prefill_time else 0.0


def accept_greedy(draft_tokens: list[int], target_tokens: list[int]) -> tuple[int, int]:
    """(j, replacement) of one greedy round: j = number of leading draft
    tokens equal to the target's choice at the same row; replacement = the
    target's token after row j (the correction, or the bonus when j = K)."""
    K = len(draft_tokens)
    if len(target_tokens) != K + 1:
        raise SFError(f"verify returned {len(target_tokens)} rows for {K} draft tokens")
    j = 0
    while j < K and draft_tokens[j] == target_tokens[j]:
        j += 1
    return j, target_tokens[j]


def speculative_generate(draft, target, prompt_ids, max_tokens: int = 128, K: int = 4,
                         eos_token_id: int | None = None,
                         on_token: Callable[[int], None] | None = None, dynamic_K: bool = False,
                         K_min: int = 1, K_max: int = 7, temperature: float = 0.0,
                         ) -> SpeculativeResult:
    """Greedy speculative generation with `draft` proposing and `target`
    verifying (both LlamaModel on the same device, same vocabulary).

    The draft must have a captured decode graph (`draft.capture()`); the
    target runs only prefill and verify. Both caches need room for the prompt,
    max_tokens and one round's K + 1 rows. `max_tokens` counts every generated
    token, the first (from the prefill) included, as SamplingParams.max_tokens
    does in the reference (speculative.py:259)."""
    if temperature > 0.0:
        raise SFError("speculative decoding here is greedy (temperature 0)")
    if draft.V != target.V:
        raise SFError("draft and target vocabularies differ")
    if draft.graph is None:
        raise SFError("capture() the draft's decode step first")
    if not 1 <= K_min <= K <= K_max:
        raise SFError(f"need 1 <= K_min <= K <= K_max (got {K_min}, {K}, {K_max})")
    ids = np.asarray(prompt_ids, dtype=np.int64).reshape(-1)
    T = int(ids.size)
    need = T + max_tokens + K_max + 1
    for m, name in ((draft, "draft"), (target, "target")):
        if need > m.max_seq:
            raise SFError(f"the {name} cache holds {m.max_seq} positions; prompt + max_tokens + "
                          f"K_max + 1 = {need}")
    dev = torch.device(target.device)
    # one verify graph per batch K+1 the rounds can use (recorded once)
    sizes = {k + 1 for k in range(K_min, K_max + 1) if k + 1 <= 8}
    missing = sorted(sizes - target.verify_graph_sizes)
    if missing:
        target.capture_verify(missing)

    def sync():
        if dev.type == "cuda":
            torch.cuda.synchronize(dev)

    draft.reset()
    target.reset()
    sync()
    t0 = time.perf_counter()
    cur = target.prefill(ids, want_logits=False)
    draft.prefill(ids, want_logits=False)
    sync()
    t_prefill = time.perf_counter()

    generated = [cur]
    if on_token is not None:
        on_token(cur)
    N = T
    rounds = drafted = accepted = 0
    cur_K = K
    t_dec = time.perf_counter()
    while len(generated) < max_tokens:
        round_K = cur_K
        # draft: round_K greedy steps from cur at positions N .. N+K-1 (each
        # step writes its token to hist[position] and feeds it to the next)
        draft.token.fill_(cur)
        draft.replay(round_K)
        d = draft.hist[N:N + round_K].tolist()
        drafted += round_K
        # target: one forward over [cur, d_0 .. d_{K-1}] at positions N .. N+K
        t = target.verify([cur] + d)
        j, replacement = accept_greedy(d, t)
        accepted += j
        if dynamic_K:
            cur_K = min(round_K + 1, K_max) if j == round_K else max(round_K - 1, K_min)
        new_batch = (d[:j] + [replacement])[:max_tokens - len(generated)]
        for tok in new_batch:
            generated.append(tok)
            if on_token is not None:
                on_token(tok)
        cur = generated[-1]
        # both caches cover positions 0 .. N+j (speculative.py:332-343)
        new_N = N + j + 1
        target.set_position(new_N)
        if j == round_K:  # the draft's last step left d_{K-1} as its input token
            draft.replay(1)
        else:
            draft.set_position(new_N)
        N = new_N
        rounds += 1
        if eos_token_id is not None and eos_token_id in new_batch:
            break
    sync()
    t_done = time.perf_counter()
    return SpeculativeResult(generated, t_prefill - t0, t_done - t_dec, T, len(generated) - 1,
                             rounds, drafted, accepted)
