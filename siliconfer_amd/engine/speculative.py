"""Speculative decoding over two int4 decoders on one GPU — the reference's
siliconfer.engine.speculative (/root/reference/siliconfer/engine/
speculative.py:151-365), same signature:

    speculative_generate(draft, target, prompt_ids, params=None, K=4,
                         eos_token_id=None, on_token=None, seed=None,
                         dynamic_K=False, K_min=1, K_max=8,
                         quantize_kv_cache=None)

Each round (speculative.py:259-352):
  1. the draft proposes K tokens from the last committed token;
  2. the target verifies [cur, d_0 .. d_{K-1}] in one forward
     (`LlamaModel.verify`: K + 1 <= 8 rows run every projection as one batch
     GEMV, so the verify streams the target's weights once);
  3. d_q is accepted with probability min(1, p_target(d_q) / p_draft(d_q))
     (:285-297); the first rejection is replaced by a draw from
     max(0, p_target - p_draft) / Z (`_sample_adjusted`, :62-84), and a fully
     accepted round adds a draw from the target's row K (:298-303);
  4. both KV caches are trimmed to the committed length N + j + 1
     (`LlamaModel.set_position`, the cache `trim` of :29-41); when every draft
     token was accepted the draft runs d_{K-1} to catch up (:336-343);
  5. with `dynamic_K`, K grows by one after a fully accepted round and shrinks
     by one after a rejection, within [K_min, K_max] (:311-315).

At temperature 0 (`params.temperature <= 0`) every probability is 1 or 0
(`_tok_prob`, :44-51), so d_q is accepted exactly when it equals the target's
greedy token: the draft's K steps replay its decode graph (each step feeds its
token to the next on the device) and the target's verify replays one graph per
K + 1, with the greedy pick of each row made on the device. At temperature > 0
the draft steps and the verify run eagerly and keep their fp32 logits; the
draws use torch on the device from a generator seeded with `seed` (the
reference seeds MLX's generator and draws its acceptance uniforms from
Python's `random`; both are replaced by the one seeded torch generator). As in
the reference, sampling here uses the temperature only (no top-k / top-p /
repetition penalty, :53-59).

Differences a caller can see:
  * K + 1 must fit the verify's 8 rows: K > 7 raises; with `dynamic_K`, K
    grows to at most min(K_max, 7) (K never enters the acceptance rule, so the
    output distribution is the same);
  * the decoders keep int8 KV caches: `quantize_kv_cache=False` raises
    (`True` and the default are the int8 cache);
  * `draft is target` runs the draft on `target.sibling()` (shared weights, a
    cache of its own), since a `LlamaModel` owns its cache where the
    reference's models take one as an argument.
"""

from __future__ import annotations

import time
from dataclasses import dataclass
from typing import Callable

import numpy as np
import torch

from .._lib import SFError
from .generate import SamplingParams, check_kv_cache_flag

VERIFY_MAX_ROWS = 8  # rows of one verify forward (LlamaModel.VERIFY_ROWS)


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


def _probs(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    return torch.softmax(logits.float() / temperature, dim=-1)


def _sample_logits(logits: torch.Tensor, temperature: float, gen: torch.Generator) -> int:
    """A draw from softmax(logits / T) (speculative.py:53-59)."""
    return int(torch.multinomial(_probs(logits, temperature), 1, generator=gen).item())


def _sample_adjusted(t_logits: torch.Tensor, d_logits: torch.Tensor, temperature: float,
                     gen: torch.Generator) -> int:
    """A draw from max(0, p_target - p_draft) / Z, or from p_target when Z
    vanishes (speculative.py:62-84)."""
    adj = torch.clamp(_probs(t_logits, temperature) - _probs(d_logits, temperature), min=0.0)
    total = float(adj.sum().item())
    if total < 1e-10:
        return _sample_logits(t_logits, temperature, gen)
    return int(torch.multinomial(adj / total, 1, generator=gen).item())


def accept_sampled(draft_tokens: list[int], draft_logits: list[torch.Tensor],
                   target_logits: torch.Tensor, temperature: float,
                   gen: torch.Generator) -> tuple[int, int]:
    """(j, replacement) of one sampled round (speculative.py:285-303): d_q is
    accepted with probability min(1, p_t(d_q) / (p_d(d_q) + 1e-12)); the
    first rejection is replaced from the adjusted distribution, a fully
    accepted round draws the bonus from the target's row K."""
    K = len(draft_tokens)
    if target_logits.shape[0] != K + 1:
        raise SFError(f"verify returned {target_logits.shape[0]} rows for {K} draft tokens")
    for q in range(K):
        tok = draft_tokens[q]
        p_t = float(_probs(target_logits[q], temperature)[tok].item())
        p_d = float(_probs(draft_logits[q], temperature)[tok].item())
        u = float(torch.rand((), generator=gen, device=gen.device).item())
        if u < min(1.0, p_t / (p_d + 1e-12)):
            continue
        return q, _sample_adjusted(target_logits[q], draft_logits[q], temperature, gen)
    return K, _sample_logits(target_logits[K], temperature, gen)


def speculative_generate(draft, target, prompt_ids, params: SamplingParams | None = None,
                         K: int = 4, eos_token_id: int | None = None,
                         on_token: Callable[[int], None] | None = None, seed: int | None = None,
                         dynamic_K: bool = False, K_min: int = 1, K_max: int = 8,
                         quantize_kv_cache: bool | None = None) -> SpeculativeResult:
    """Speculative generation with `draft` proposing and `target` verifying
    (both LlamaModel on the same device, same vocabulary). Argument meaning as
    in the reference (speculative.py:151-233); `params.max_tokens` counts
    every generated token, the first (from the prefill) included. Both caches
    need room for the prompt, max_tokens and one round's K + 1 rows."""
    params = params if params is not None else SamplingParams()
    check_kv_cache_flag(quantize_kv_cache)
    if K + 1 > VERIFY_MAX_ROWS:
        raise SFError(f"K={K}: the verify forward takes at most {VERIFY_MAX_ROWS} rows "
                      f"(K <= {VERIFY_MAX_ROWS - 1})")
    if not 1 <= K_min <= K <= K_max:
        raise SFError(f"need 1 <= K_min <= K <= K_max (got {K_min}, {K}, {K_max})")
    k_cap = min(K_max, VERIFY_MAX_ROWS - 1)
    if draft is target:
        draft = target.sibling()
    if draft.V != target.V:
        raise SFError("draft and target vocabularies differ")
    temp = float(params.temperature)
    greedy = temp <= 0.0
    if greedy and draft.graph is None:
        draft.capture()
    max_tokens = int(params.max_tokens)
    ids = np.asarray(prompt_ids.detach().cpu() if isinstance(prompt_ids, torch.Tensor) else prompt_ids,
                     dtype=np.int64).reshape(-1)
    T = int(ids.size)
    need = T + max_tokens + k_cap + 1
    for m, name in ((draft, "draft"), (target, "target")):
        if need > m.max_seq:
            raise SFError(f"the {name} cache holds {m.max_seq} positions; prompt + max_tokens + "
                          f"K_max + 1 = {need}")
    dev = torch.device(target.device)
    if greedy:  # one verify graph per batch K+1 the rounds can use (recorded once)
        sizes = {k + 1 for k in range(K_min, k_cap + 1)}
        missing = sorted(sizes - target.verify_graph_sizes)
        if missing:
            target.capture_verify(missing)
    gen = torch.Generator(device=dev)
    gen.manual_seed(int(seed) if seed is not None else int(torch.randint(0, 2 ** 62, ()).item()))

    def sync():
        if dev.type == "cuda":
            torch.cuda.synchronize(dev)

    draft.reset()
    target.reset()
    sync()
    t0 = time.perf_counter()
    cur = target.prefill(ids, want_logits=not greedy)
    draft.prefill(ids, want_logits=False)
    sync()
    t_prefill = time.perf_counter()
    if not greedy:
        cur = _sample_logits(target.logits, temp, gen)

    generated = [cur]
    if on_token is not None:
        on_token(cur)
    N = T
    rounds = drafted = accepted = 0
    cur_K = K
    t_dec = time.perf_counter()
    while len(generated) < max_tokens:
        round_K = cur_K
        draft.token.fill_(cur)
        if greedy:
            # round_K greedy steps from cur at positions N .. N+K-1 (each step
            # writes its token to hist[position] and feeds it to the next)
            draft.replay(round_K)
            d = draft.hist[N:N + round_K].tolist()
            # target: one forward over [cur, d_0 .. d_{K-1}] at positions N .. N+K
            j, replacement = accept_greedy(d, target.verify([cur] + d))
        else:
            d, d_logits = [], []
            for _ in range(round_K):
                p = draft.pos
                draft.decode_step(logits=True)
                draft.pos += 1
                row = draft.logits.clone()
                tok = _sample_logits(row, temp, gen)
                draft.token.fill_(tok)
                draft.hist[p] = tok
                d.append(tok)
                d_logits.append(row)
            target.verify([cur] + d, want_logits=True)
            j, replacement = accept_sampled(d, d_logits, target.vlogits[:round_K + 1], temp, gen)
        drafted += round_K
        accepted += j
        if dynamic_K:
            cur_K = min(round_K + 1, k_cap) if j == round_K else max(round_K - 1, K_min)
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
            if greedy:
                draft.replay(1)
            else:
                draft.token.fill_(d[-1])
                draft.decode_step()
                draft.pos += 1
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
