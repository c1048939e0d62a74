"""Speculative decoding on the GPU: the batched-row lm_head
(sf_lm_head_argmax_rows), the target's verify of K+1 rows
(LlamaModel.verify, every projection one batch GEMV), the cache trim
(LlamaModel.set_position) and speculative_generate against the target's own
greedy generation — the parity bar of the reference's
tests/test_speculative.py (speculative output equals target-only greedy
output) for /root/reference/siliconfer/engine/speculative.py:151-365.

Verify rows and decode steps compute the same function through different
kernels (batch GEMV and causal prefill attention vs the folded B=1 GEMV and
decode attention), so their logits agree to the decoder's tolerance (2e-3 at
fp32 activations, 1e-2 at fp16), not bit for bit; a greedy token may then
differ only where the top-2 margin is inside that tolerance, which the
token checks allow for and report."""

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle.linear import assert_close
from siliconfer_amd import _lib
from siliconfer_amd.engine import SamplingParams, speculative_generate
from siliconfer_amd.model.config import ModelConfig, rope_tables
from siliconfer_amd.model.llama import LlamaModel

pytestmark = pytest.mark.gpu

SMALL = ModelConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                    num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=1000,
                    rms_norm_eps=1e-6, rope_theta=1e6, tie_word_embeddings=True,
                    attention_bias=True)
TINY_DRAFT = ModelConfig(hidden_size=128, intermediate_size=256, num_hidden_layers=1,
                         num_attention_heads=2, num_key_value_heads=1, head_dim=64, vocab_size=1000,
                         rms_norm_eps=1e-6, rope_theta=1e6, tie_word_embeddings=True)


def st():
    return torch.cuda.current_stream().cuda_stream


def G(n):  # greedy parameters for n tokens
    return SamplingParams(temperature=0.0, max_tokens=n)


def near_tie(logits: np.ndarray, a: int, b: int, tol: float) -> bool:
    """Tokens a and b are both within tol (relative to the row's RMS) of the max."""
    scale = tol * 10 * np.linalg.norm(logits) / np.sqrt(logits.size)
    return abs(float(logits[a]) - float(logits[b])) <= scale


# ---------------------------------------------------------------- lm_head rows
ROW_CASES = [(1000, 256, 8, torch.float32), (1000, 256, 3, torch.float16),
             (5003, 896, 8, torch.bfloat16), (5003, 896, 1, torch.float32),
             (151936, 896, 8, torch.float16), (4099, 4096, 8, torch.bfloat16),
             (4099, 4096, 4, torch.float32), (777, 8192, 2, torch.float16),
             (3001, 2048, 8, torch.float16), (2000, 1536, 5, torch.bfloat16),
             (1000, 904, 4, torch.float16), (1000, 896, 2, torch.float16),
             (1000, 896, 3, torch.float16)]


def rows_on_mfma(H, B, xdt):
    """From 3 rows, fp16 / bf16 rows with H % 32 == 0 and H <= 2048 run on MFMA."""
    return B >= 3 and xdt != torch.float32 and H % 32 == 0 and H <= 2048


@pytest.mark.parametrize("V,H,B,xdt", ROW_CASES)
def test_lm_head_rows_equal_single_row(dev, V, H, B, xdt):
    lib = _lib.load()
    g = torch.Generator(device=dev).manual_seed(V + H + B)
    w = (torch.randn((V, H), generator=g, device=dev) * 0.05).to(torch.bfloat16)
    x = torch.randn((B, H), generator=g, device=dev).to(xdt)
    x[B - 1, :] = x[0, :]  # a repeated row gives the same logits and token
    logits = torch.full((B, V), float("nan"), device=dev)
    toks = torch.full((B,), -1, dtype=torch.int32, device=dev)
    ws = torch.zeros(lib.sf_lm_head_rows_workspace_bytes(V, B), dtype=torch.uint8, device=dev)
    for call in range(2):  # the workspace is left ready for the next call
        _lib.check(lib.sf_lm_head_argmax_rows(w.data_ptr(), x.data_ptr(), _lib.dt(x),
                                              logits.data_ptr(), V, H, B, toks.data_ptr(),
                                              ws.data_ptr(), ws.numel(), st()),
                   "sf_lm_head_argmax_rows")
    ws1 = torch.zeros(lib.sf_lm_head_workspace_bytes(V), dtype=torch.uint8, device=dev)
    one_l = torch.empty((V,), device=dev)
    one_t = torch.empty((1,), dtype=torch.int32, device=dev)
    ref = (x.double() @ w.double().T).cpu().numpy()
    lg = logits.cpu().numpy()
    for b in range(B):
        _lib.check(lib.sf_lm_head_argmax(w.data_ptr(), x[b].data_ptr(), _lib.dt(x), one_l.data_ptr(),
                                         V, H, one_t.data_ptr(), None, None, ws1.data_ptr(),
                                         ws1.numel(), st()), "sf_lm_head_argmax")
        torch.cuda.synchronize()
        assert int(toks[b]) == int(np.argmax(lg[b])), f"row {b}: token is not its logits' argmax"
        np.testing.assert_allclose(lg[b], ref[b], rtol=0, atol=1e-5 * np.abs(ref[b]).max() + 1e-6)
        if not rows_on_mfma(H, B, xdt):
            # the VALU kernel sums each row in the single-row kernel's order
            assert torch.equal(logits[b], one_l), f"row {b}: logits differ from the single-row kernel"
            assert int(toks[b]) == int(one_t[0]), f"row {b}: token"
        else:
            # MFMA: exact products, fp32 sums in another order
            one = one_l.cpu().numpy()
            np.testing.assert_allclose(lg[b], one, rtol=0, atol=2e-6 * np.abs(one).max())
            if int(toks[b]) != int(one_t[0]):
                assert near_tie(one, int(toks[b]), int(one_t[0]), 1e-5), f"row {b}: token"
    assert int(toks[0]) == int(toks[B - 1])
    # without logits: the same tokens
    toks2 = torch.full((B,), -1, dtype=torch.int32, device=dev)
    _lib.check(lib.sf_lm_head_argmax_rows(w.data_ptr(), x.data_ptr(), _lib.dt(x), None, V, H, B,
                                          toks2.data_ptr(), ws.data_ptr(), ws.numel(), st()),
               "sf_lm_head_argmax_rows")
    assert torch.equal(toks2, toks)


# ---------------------------------------------------------------- verify rows
def decode_logits(m: LlamaModel, prompt, feed) -> np.ndarray:
    """Logits after each token of `feed`, one eager decode step at a time."""
    m.reset()
    m.prefill(prompt)
    rows = []
    for t in feed:
        m.token.fill_(int(t))
        m.decode_step(logits=True)
        m.pos += 1
        rows.append(m.logits.cpu().numpy().copy())
    return np.stack(rows)


@pytest.mark.parametrize("act", [torch.float32, torch.float16])
@pytest.mark.parametrize("B", [1, 2, 5, 8, 11])
def test_verify_rows_match_decode_and_oracle(dev, act, B):
    m = LlamaModel.random_init(SMALL, seed=41, group_size=64, device=dev, max_seq=64, act_dtype=act)
    tol = 2e-3 if act == torch.float32 else 1e-2
    rng = np.random.default_rng(42 + B)
    prompt = rng.integers(0, SMALL.vocab_size, 9)
    feed = rng.integers(0, SMALL.vocab_size, B)
    m.reset()
    m.prefill(prompt)
    n0 = m.pos
    want = B <= m.VERIFY_ROWS
    toks = m.verify(feed, want_logits=want)
    assert m.pos == n0 + B and int(m.pos_dev.item()) == n0 + B and len(toks) == B
    W = m.export_weights()
    cos, sin = rope_tables(SMALL, m.max_seq)
    cache = OM.KVCache(SMALL.num_hidden_layers)
    OM.forward(W, SMALL, prompt, cache, cos, sin)
    ref = OM.forward(W, SMALL, feed, cache, cos, sin)
    dec = decode_logits(m, prompt, feed)
    for r in range(B):
        if want:
            got = m.vlogits[r].cpu().numpy()
            assert_close(got, ref[r], tol, f"verify row {r} vs oracle")
            assert_close(got, dec[r], tol, f"verify row {r} vs decode")
            assert toks[r] == int(np.argmax(got))
        if toks[r] != OM.greedy(ref[r]):
            assert near_tie(ref[r], toks[r], OM.greedy(ref[r]), tol), f"row {r}: token"


LLAMA_HD128 = ModelConfig(hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                          num_attention_heads=4, num_key_value_heads=1, head_dim=128, vocab_size=1000,
                          rms_norm_eps=1e-5, rope_theta=5e5, tie_word_embeddings=False,
                          attention_bias=False)


@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B", [3, 8])
def test_verify_rows_head_dim_128_match_oracle(dev, act, B):
    """Verify rows at head_dim 128 with GQA 4:1 and an untied lm_head against
    the oracle (the causal attention over the new rows and the batch GEMV at
    these shapes), bf16 activations included."""
    cfg = LLAMA_HD128
    m = LlamaModel.random_init(cfg, seed=47, group_size=64, device=dev, max_seq=64, act_dtype=act)
    tol = 1e-2 if act == torch.float16 else 3e-2
    rng = np.random.default_rng(48 + B)
    prompt = rng.integers(0, cfg.vocab_size, 13)
    feed = rng.integers(0, cfg.vocab_size, B)
    m.reset()
    m.prefill(prompt)
    toks = m.verify(feed, want_logits=True)
    W = m.export_weights()
    cos, sin = rope_tables(cfg, m.max_seq)
    cache = OM.KVCache(cfg.num_hidden_layers)
    OM.forward(W, cfg, prompt, cache, cos, sin)
    ref = OM.forward(W, cfg, feed, cache, cos, sin)
    for r in range(B):
        got = m.vlogits[r].cpu().numpy()
        assert_close(got, ref[r], tol, f"verify row {r} vs oracle")
        if toks[r] != OM.greedy(ref[r]):
            assert near_tie(ref[r], toks[r], OM.greedy(ref[r]), tol), f"row {r}: token"


@pytest.mark.parametrize("max_seq,prompt_len", [(64, 9), (2048, 1100)])
def test_verify_graph_equals_eager(dev, max_seq, prompt_len):
    """verify() replayed from its graph (positions read on the device) gives
    the eager verify's tokens and cache; at max_seq > 1024 the graph's causal
    attention runs split (the eager one is single-split), so tokens are
    compared up to near-ties and only the first layer's cache (written before
    any attention) bit for bit."""
    ms = [LlamaModel.random_init(SMALL, seed=45, group_size=64, device=dev, max_seq=max_seq,
                                 act_dtype=torch.float16) for _ in range(2)]
    g, e = ms
    g.capture_verify()
    assert g.verify_graph_sizes == set(range(1, 9))
    rng = np.random.default_rng(46)
    prompt = rng.integers(0, SMALL.vocab_size, prompt_len)
    for m in ms:
        m.reset()
        m.prefill(prompt)
    for B in (1, 3, 8, 2):
        feed = rng.integers(0, SMALL.vocab_size, B)
        tg = g.verify(feed)
        te = e.verify(feed, want_logits=True)
        assert g.pos == e.pos and int(g.pos_dev.item()) == g.pos
        if max_seq <= 1024:
            assert tg == te
        else:
            lg = e.vlogits[:B].cpu().numpy()
            for r in range(B):
                if tg[r] != te[r]:
                    assert near_tie(lg[r], tg[r], te[r], 1e-2), f"B={B} row {r}"
        n = g.pos
        for l in range(SMALL.num_hidden_layers if max_seq <= 1024 else 1):
            assert torch.equal(g.k_codes[l][:, :n], e.k_codes[l][:, :n])
            assert torch.equal(g.v_scales[l][:, :n], e.v_scales[l][:, :n])
        # trim back one row each time: the next verify overwrites it
        g.set_position(n - 1)
        e.set_position(n - 1)


@pytest.mark.parametrize("B", [1, 2, 3, 5, 8])
def test_fused_verify_equals_unfused(dev, B):
    """The verify forward with RMSNorm / SwiGLU folded into the batch GEMV and
    the residual added inside the o / down projections gives the same bits as
    the separate kernels (LlamaModel(fuse=False)), fp16 activations."""
    outs = []
    for fuse in (True, False):
        m = LlamaModel.random_init(SMALL, seed=47, group_size=64, device=dev, max_seq=64,
                                   act_dtype=torch.float16, fuse=fuse)
        g = torch.Generator(device=dev).manual_seed(3)
        for L in m.layers:  # non-unit norm weights
            L.w_in.mul_(1 + 0.2 * torch.randn(L.w_in.shape, generator=g, device=dev))
            L.w_post.mul_(1 + 0.2 * torch.randn(L.w_post.shape, generator=g, device=dev))
        res, fq, fg, fd = m._rows_plan(B)
        assert res and fq == fg == fuse
        rng = np.random.default_rng(48)
        m.reset()
        m.prefill(rng.integers(0, SMALL.vocab_size, 11))
        toks = m.verify(rng.integers(0, SMALL.vocab_size, B), want_logits=True)
        outs.append((toks, m.vlogits[:B].cpu().clone(), m.k_codes[1][:, :m.pos].cpu().clone()))
    (t0, l0, k0), (t1, l1, k1) = outs
    assert t0 == t1 and torch.equal(l0, l1) and torch.equal(k0, k1)


def test_trim_discards_stale_rows(dev):
    """After set_position(n) the cache behaves as if it held only n tokens:
    two runs whose first verify differs only in the rows past n give
    identical results from then on (a verify row depends only on the rows
    before it and the cache, so rows < n are the same bits in both)."""
    m = LlamaModel.random_init(SMALL, seed=43, group_size=64, device=dev, max_seq=64,
                               act_dtype=torch.float16)
    rng = np.random.default_rng(44)
    prompt = rng.integers(0, SMALL.vocab_size, 7)
    first = rng.integers(0, SMALL.vocab_size, 6)
    second = rng.integers(0, SMALL.vocab_size, 2)  # leaves stale rows past the new end
    outs = []
    for stale in (first[2:], rng.integers(0, SMALL.vocab_size, 4)):
        m.reset()
        m.prefill(prompt)
        n0 = m.pos
        t1 = m.verify(np.concatenate([first[:2], stale]), want_logits=True)
        m.set_position(n0 + 2)
        t2 = m.verify(second, want_logits=True)
        outs.append((t1[:2], t2, m.vlogits[:2].cpu().clone()))
        # then a decode step (graph-free) from the trimmed-and-extended cache
        m.token.fill_(int(t2[-1]))
        m.decode_step(logits=True)
        m.pos += 1
        outs[-1] += (m.logits.cpu().clone(),)
    a, b = outs
    assert a[0] == b[0] and a[1] == b[1]
    assert torch.equal(a[2], b[2]) and torch.equal(a[3], b[3])
    with pytest.raises(_lib.SFError):
        m.set_position(m.pos + 1)


# ---------------------------------------------------------- speculative decode
def check_greedy_equal(target: LlamaModel, prompt, got: list[int], tol: float, what: str):
    """got equals target.generate(prompt) token for token, except where the
    decode logits hold a near-tie (then the sequences may continue apart)."""
    want = target.generate(prompt, max_tokens=len(got)).token_ids
    if got == want:
        return
    i = next(k for k in range(len(got)) if got[k] != want[k])
    assert i > 0, f"{what}: the first token comes from the same prefill"
    lg = decode_logits(target, prompt, want[:i])[-1]
    assert near_tie(lg, got[i], want[i], tol), (
        f"{what}: token {i} is {got[i]}, greedy decode gives {want[i]} (margin "
        f"{abs(lg[got[i]] - lg[want[i]]):.3g})")


@pytest.mark.parametrize("act", [torch.float32, torch.float16])
@pytest.mark.parametrize("K,dynamic", [(1, False), (4, False), (7, False), (3, True)])
def test_speculative_equals_target_greedy(dev, act, K, dynamic):
    tol = 2e-3 if act == torch.float32 else 1e-2
    target = LlamaModel.random_init(SMALL, seed=51, group_size=64, device=dev, max_seq=128,
                                    act_dtype=act)
    target.capture()
    prompt = np.random.default_rng(52).integers(0, SMALL.vocab_size, 12)
    drafts = {"same weights": LlamaModel.random_init(SMALL, seed=51, group_size=64, device=dev,
                                                     max_seq=128, act_dtype=act),
              "other model": LlamaModel.random_init(TINY_DRAFT, seed=53, group_size=64, device=dev,
                                                    max_seq=128, act_dtype=act)}
    for name, draft in drafts.items():
        draft.capture()
        seen = []
        r = speculative_generate(draft, target, prompt, G(40), K=K, dynamic_K=dynamic,
                                 on_token=seen.append)
        assert len(r.token_ids) == 40 and seen == r.token_ids and r.num_decode_tokens == 39
        assert r.total_accepted <= r.total_draft_tokens
        assert target.pos == draft.pos == len(prompt) + r.total_rounds + r.total_accepted
        if name == "same weights":
            # a draft identical to the target proposes the target's own tokens
            assert r.acceptance_rate > 0.8, f"acceptance {r.acceptance_rate}"
        check_greedy_equal(target, prompt, r.token_ids, tol, f"{name} K={K}")


def test_speculative_eos_stops(dev):
    target = LlamaModel.random_init(SMALL, seed=55, group_size=64, device=dev, max_seq=128)
    draft = LlamaModel.random_init(TINY_DRAFT, seed=56, group_size=64, device=dev, max_seq=128)
    target.capture()
    draft.capture()
    prompt = np.random.default_rng(57).integers(0, SMALL.vocab_size, 10)
    full = speculative_generate(draft, target, prompt, G(30), K=4).token_ids
    # eos: the token whose first appearance after the prefill token comes last
    # (the prefill token itself is not checked for eos, speculative.py:243-351)
    first_at = {}
    for i in range(1, len(full)):
        first_at.setdefault(full[i], i)
    eos, stop = max(first_at.items(), key=lambda kv: kv[1])
    r = speculative_generate(draft, target, prompt, G(30), K=4, eos_token_id=eos)
    # stops after the round that committed eos: at most K tokens after it
    assert r.token_ids == full[:len(r.token_ids)] and stop < len(r.token_ids) <= stop + 1 + 4


def test_speculative_draft_is_target(dev):
    """draft=target, the reference tests' setting (test_speculative.py:125-137):
    the draft runs on a sibling decoder (same weights, own cache), so every
    greedy proposal is accepted and the output is the target's greedy one."""
    target = LlamaModel.random_init(SMALL, seed=58, group_size=64, device=dev, max_seq=128)
    target.capture()
    prompt = np.random.default_rng(59).integers(0, SMALL.vocab_size, 9)
    r = speculative_generate(target, target, prompt, G(24), 3, None, None, 0)  # reference order
    assert len(r.token_ids) == 24 and r.acceptance_rate == 1.0
    assert r.token_ids == target.generate(prompt, max_tokens=24).token_ids
    with pytest.raises(RuntimeError, match="at most 8 rows"):
        speculative_generate(target, target, prompt, G(8), K=8)
    with pytest.raises(RuntimeError, match="int8 KV cache only"):
        speculative_generate(target, target, prompt, G(8), quantize_kv_cache=False)


def test_speculative_sampled(dev):
    """Temperature > 0 (speculative.py:285-303): valid ids, max_tokens honoured,
    the same seed gives the same tokens, and a draft identical to the target
    has every proposal accepted (p_target / p_draft = 1 up to rounding)."""
    target = LlamaModel.random_init(SMALL, seed=60, group_size=64, device=dev, max_seq=128)
    draft = LlamaModel.random_init(TINY_DRAFT, seed=61, group_size=64, device=dev, max_seq=128)
    prompt = np.random.default_rng(62).integers(0, SMALL.vocab_size, 8)
    p = SamplingParams(temperature=0.8, max_tokens=20)
    a = speculative_generate(draft, target, prompt, p, K=3, seed=5, dynamic_K=True, K_max=6)
    b = speculative_generate(draft, target, prompt, p, K=3, seed=5, dynamic_K=True, K_max=6)
    assert len(a.token_ids) == 20 and all(0 <= t < SMALL.vocab_size for t in a.token_ids)
    assert a.token_ids == b.token_ids and a.total_rounds == b.total_rounds
    assert target.pos == draft.pos == len(prompt) + a.total_rounds + a.total_accepted
    same = speculative_generate(target, target, prompt, p, K=4, seed=7)
    assert same.acceptance_rate > 0.95 and len(same.token_ids) == 20
