"""Generation loop over `LlamaModel` — the call surface of the reference's
`siliconfer.engine.generate` (/root/reference/siliconfer/engine/generate.py:15-180):
`SamplingParams`, `sample_token`, `GenerationResult`, `warmup` and
`generate(model, prompt_ids, params, eos_token_id, stream, on_token,
quantize_kv_cache)` with the same argument meaning and result fields.

How it runs on MI355X:
  * greedy (temperature <= 0, no repetition penalty), the benchmarked path:
    the prompt runs through `model.prefill`, then every decode step is one
    replay of the model's captured HIP graph. The step picks its token on the
    device and feeds it to the next step, so nothing returns to the host per
    token. Tokens come back in chunks (`CHUNK` steps) only when a caller
    needs them early: an `eos_token_id`, `on_token` or `stream`. A chunk that
    runs past the end-of-sequence token is cut there and the cache is trimmed
    back, so the tokens, the callbacks and the cache state equal a
    token-by-token loop's (generate.py:153-170);
  * sampling (temperature > 0 or a repetition penalty): eager decode steps
    that keep the fp32 logits; the next token is drawn on the device with
    torch (the reference's rules: penalty on previously generated ids,
    temperature, top-k, top-p nucleus, generate.py:24-67) and written back as
    the step's token.

KV cache: this decoder keeps the int8 cache (the reference's
`quantize_kv_cache=True` path, kv_cache.py:49-126) and has no full-precision one.
`quantize_kv_cache=True` and the default (None) run it; `False` raises, rather
than give int8-cache numerics to a caller who asked for the reference's fp16
cache. A call that leaves the flag out gets the int8 cache where the reference's
default is the fp16 one (generate.py:124, 135).
"""

from __future__ import annotations

import time
from collections.abc import Callable
from dataclasses import dataclass

import numpy as np
import torch

from .._lib import SFError
from ..model.llama import GenerationResult, LlamaModel

CHUNK = 16  # decode steps replayed between host reads when tokens are needed early

__all__ = ["SamplingParams", "sample_token", "GenerationResult", "warmup", "generate",
           "check_kv_cache_flag"]


def check_kv_cache_flag(quantize_kv_cache) -> None:
    """The decoders here keep an int8 KV cache only: refuse an explicit
    request for the reference's full-precision cache."""
    if quantize_kv_cache is not None and not quantize_kv_cache:
        raise SFError("quantize_kv_cache=False: this decoder keeps an int8 KV cache only "
                      "(pass True or leave it unset)")


@dataclass
class SamplingParams:
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0
    repetition_penalty: float = 1.0
    max_tokens: int = 128


def _is_greedy(p: SamplingParams) -> bool:
    return p.temperature <= 0 and p.repetition_penalty == 1.0


def sample_token(logits: torch.Tensor, params: SamplingParams,
                 generated_ids: list[int] | None = None,
                 generator: torch.Generator | None = None) -> int:
    """Next token from one row of logits ([V], or [..., V] whose last row is
    used), by the reference's rules (generate.py:24-67)."""
    row = logits.reshape(-1, logits.shape[-1])[-1].float().clone()
    if params.repetition_penalty != 1.0 and generated_ids:
        ids = torch.as_tensor(sorted(set(generated_ids)), device=row.device, dtype=torch.long)
        v = row[ids]
        row[ids] = torch.where(v > 0, v / params.repetition_penalty, v * params.repetition_penalty)
    if params.temperature <= 0:
        return int(torch.argmax(row).item())
    row = row / params.temperature
    if params.top_k > 0:
        kth = torch.topk(row, min(params.top_k, row.numel())).values[-1]
        row = torch.where(row < kth, torch.full_like(row, float("-inf")), row)
    if params.top_p < 1.0:
        srt, order = torch.sort(row, descending=True)
        probs = torch.softmax(srt, dim=-1)
        drop = (torch.cumsum(probs, dim=-1) - probs) > params.top_p
        srt = torch.where(drop, torch.full_like(srt, float("-inf")), srt)
        row = torch.empty_like(row).scatter_(0, order, srt)
    probs = torch.softmax(row, dim=-1)
    return int(torch.multinomial(probs, 1, generator=generator).item())


def warmup(model: LlamaModel, quantize_kv_cache: bool | None = None) -> None:
    """Record the decode-step graph and run a two-token prompt and one decode
    step, so the first timed `generate` pays no one-time set-up (the
    reference warms MLX's lazy compilation the same way, generate.py:89-114)."""
    check_kv_cache_flag(quantize_kv_cache)
    if model.graph is None:
        model.capture()
    model.reset()
    model.prefill([1, 2])
    model.replay(1)
    torch.cuda.synchronize(model.device)
    model.reset()


def _prompt_array(prompt_ids) -> np.ndarray:
    if isinstance(prompt_ids, torch.Tensor):
        prompt_ids = prompt_ids.detach().cpu().numpy()
    a = np.asarray(prompt_ids, dtype=np.int64)
    if a.ndim == 2:
        if a.shape[0] != 1:
            raise SFError(f"batch {a.shape[0]}: this decoder runs batch 1")
        a = a[0]
    if a.ndim != 1 or a.size == 0:
        raise SFError("prompt_ids must be a non-empty [T] or [1, T] array of token ids")
    return a


def generate(model: LlamaModel, prompt_ids, params: SamplingParams | None = None,
             eos_token_id: int | None = None, stream: bool = False,
             on_token: Callable[[int], None] | None = None,
             quantize_kv_cache: bool | None = None,
             generator: torch.Generator | None = None) -> GenerationResult:
    """Prefill the prompt, then decode up to `params.max_tokens - 1` more
    tokens, stopping after `eos_token_id`. `on_token` gets every token as it
    is produced (else `stream` prints it); `decode_tok_s` counts the tokens
    after the first over the time after prefill, as the reference does."""
    check_kv_cache_flag(quantize_kv_cache)
    params = params or SamplingParams()
    ids = _prompt_array(prompt_ids)
    if ids.size + params.max_tokens > model.max_seq + 1:
        raise SFError("prompt + max_tokens exceeds the cache capacity")
    emit_each = on_token is not None or stream
    out: list[int] = []

    def emit(tok: int) -> None:
        out.append(tok)
        if on_token is not None:
            on_token(tok)
        elif stream:
            print(tok, end=" ", flush=True)

    greedy = _is_greedy(params)
    if greedy and model.graph is None:
        model.capture()
    model.reset()
    torch.cuda.synchronize(model.device)
    t0 = time.perf_counter()
    first = model.prefill(ids, want_logits=not greedy)
    if not greedy:
        torch.cuda.synchronize(model.device)
    t1 = time.perf_counter()  # the prefill clock stops before the first draw (generate.py:139-141)
    if not greedy:
        first = sample_token(model.logits, params, out, generator)
        model.token.fill_(first)
    emit(first)
    t_dec = time.perf_counter()  # decode clock after the first token (generate.py:152)
    budget = params.max_tokens - 1
    done = eos_token_id is not None and first == eos_token_id
    while budget > 0 and not done:
        if greedy:
            n = min(budget, CHUNK) if (emit_each or eos_token_id is not None) else budget
            start = model.pos
            model.replay(n)
            toks = model.hist[start:start + n].cpu().tolist()
            for j, tok in enumerate(toks):
                emit(tok)
                if eos_token_id is not None and tok == eos_token_id:
                    done = True
                    model.set_position(start + j + 1)  # steps past the EOS are dropped
                    break
            budget -= n
        else:
            p = model.pos
            model.decode_step(logits=True)
            model.pos += 1
            tok = sample_token(model.logits, params, out, generator)
            model.token.fill_(tok)
            model.hist[p] = tok
            emit(tok)
            done = eos_token_id is not None and tok == eos_token_id
            budget -= 1
    torch.cuda.synchronize(model.device)
    t2 = time.perf_counter()
    if stream:
        print()
    return GenerationResult(out, t1 - t0, t2 - t_dec, int(ids.size), len(out) - 1)
