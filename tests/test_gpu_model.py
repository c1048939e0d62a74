"""End-to-end decoder on the GPU against the numpy oracle
of the reference's forward pass (oracle/model.py, restating
/root/reference/siliconfer/model/layers.py, llama.py and the greedy branch of
engine/generate.py).

Tolerances: logits are compared norm-relative. The GPU path and the oracle
both compute in fp32 but sum in different orders; an int8 KV code can then
land on the other side of a rounding boundary (one code step, 1/127 of a
row's max), which moves scores by that much — hence 2e-3 for the 2-layer
model and 1e-2 after 24 layers. Greedy tokens must agree whenever the
oracle's top-2 margin exceeds the logit tolerance.
"""

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle.linear import assert_close
from siliconfer_amd.model.config import ModelConfig, RoPEScalingConfig, rope_tables
from siliconfer_amd.model.llama import LlamaModel, pack_sym_device

pytestmark = pytest.mark.gpu

SMALL = ModelConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                    num_attention_heads=4, num_key_value_heads=2, head_dim=64, vocab_size=1000,
                    rms_norm_eps=1e-6, rope_theta=1e6, tie_word_embeddings=True,
                    attention_bias=True)


def margin_ok(logits: np.ndarray, tol: float) -> bool:
    top2 = np.sort(logits)[-2:]
    return (top2[1] - top2[0]) > tol * np.linalg.norm(logits) / np.sqrt(logits.size) * 10


def check_against_oracle(m: LlamaModel, cfg, ids, n_decode, tol, what):
    W = m.export_weights()
    cos, sin = rope_tables(cfg, m.max_seq)
    cache = OM.KVCache(cfg.num_hidden_layers)
    m.reset()
    tok = m.prefill(ids)
    ref = OM.forward(W, cfg, ids, cache, cos, sin)[-1]
    got = m.logits.cpu().numpy()
    assert_close(got, ref, tol, f"{what} prefill logits")
    if margin_ok(ref, tol):
        assert tok == OM.greedy(ref), f"{what}: prefill token"
    for i in range(n_decode):
        m.decode_step(logits=True)
        torch.cuda.synchronize()
        ref = OM.forward(W, cfg, [tok], cache, cos, sin)[-1]
        got = m.logits.cpu().numpy()
        assert_close(got, ref, tol, f"{what} decode step {i} logits")
        nxt = int(m.token.item())
        if margin_ok(ref, tol):
            assert nxt == OM.greedy(ref), f"{what}: decode step {i} token"
        tok = nxt
        m.pos += 1
    assert int(m.pos_dev.item()) == m.pos


# logits tolerance by activation dtype: bf16 activations carry 8 mantissa bits
# against fp16's 11, so each rounding of a staged row is 8x coarser
ACT_TOL = {torch.float32: 2e-3, torch.float16: 1e-2, torch.bfloat16: 3e-2}


@pytest.mark.parametrize("act", [torch.float32, torch.float16, torch.bfloat16])
def test_small_model_matches_oracle(dev, act):
    m = LlamaModel.random_init(SMALL, seed=11, group_size=64, device=dev, max_seq=64, act_dtype=act)
    ids = np.random.default_rng(12).integers(0, SMALL.vocab_size, 13)
    tol = ACT_TOL[act]
    check_against_oracle(m, SMALL, ids, 6, tol, f"small/{act}")


GEOMETRIES = {
    # Llama-style: head_dim 128, one kv head per 4 query heads, no qkv bias, an
    # lm_head of its own, llama3 RoPE scaling
    "llama_hd128": ModelConfig(hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                               num_attention_heads=4, num_key_value_heads=1, head_dim=128,
                               vocab_size=1000, rms_norm_eps=1e-5, rope_theta=5e5,
                               rope_scaling=RoPEScalingConfig("llama3", 8.0, 1.0, 4.0, 64),
                               tie_word_embeddings=False, attention_bias=False),
    # multi-head attention (a kv head per query head) at head_dim 64
    "mha_hd64": ModelConfig(hidden_size=256, intermediate_size=640, num_hidden_layers=2,
                            num_attention_heads=4, num_key_value_heads=4, head_dim=64,
                            vocab_size=1000, rms_norm_eps=1e-6, rope_theta=1e6,
                            tie_word_embeddings=True, attention_bias=True),
}


@pytest.mark.parametrize("geom", sorted(GEOMETRIES))
@pytest.mark.parametrize("act", [torch.float32, torch.float16, torch.bfloat16])
def test_other_geometries_match_oracle(dev, geom, act):
    """The decoder is not specialised to config 5's shape: head_dim 128 with GQA
    4:1, untied lm_head and llama3 RoPE scaling, and MHA at head_dim 64, each
    through a 21-token prompt (the GEMM) and 8 decode steps against the oracle."""
    cfg = GEOMETRIES[geom]
    m = LlamaModel.random_init(cfg, seed=21, group_size=64, device=dev, max_seq=64, act_dtype=act)
    ids = np.random.default_rng(22).integers(0, cfg.vocab_size, 21)
    tol = ACT_TOL[act]
    check_against_oracle(m, cfg, ids, 8, tol, f"{geom}/{act}")


def test_prefill_in_chunks_equals_one_prefill(dev):
    a = LlamaModel.random_init(SMALL, seed=13, device=dev, max_seq=64)
    b = LlamaModel.random_init(SMALL, seed=13, device=dev, max_seq=64, max_prefill=5)
    ids = np.random.default_rng(14).integers(0, SMALL.vocab_size, 17)
    ta, tb = a.prefill(ids), b.prefill(ids)
    # chunks of <= 8 rows run the batch GEMV, the 17-row prompt the GEMM: the
    # two paths round differently, so an int8 KV code may differ by one step
    # (the module docstring's 2e-3)
    la = a.logits.cpu().numpy()
    assert_close(b.logits.cpu().numpy(), la, 2e-3, "chunked prefill")
    if margin_ok(la, 2e-3):
        assert ta == tb


def test_graph_replay_equals_eager(dev):
    m = LlamaModel.random_init(SMALL, seed=15, device=dev, max_seq=64)
    ids = np.random.default_rng(16).integers(0, SMALL.vocab_size, 9)
    m.prefill(ids)
    start = m.pos
    for _ in range(10):
        m.decode_step(logits=True)
    m.pos += 10
    torch.cuda.synchronize()
    eager_toks = m.hist[start:start + 10].cpu().clone()
    eager_logits = m.logits.cpu().clone()
    m.reset()
    m.prefill(ids)
    m.capture(logits=True)
    for r in range(10):  # replays with eager work and synchronisation between them
        m.replay(1)
        torch.cuda.synchronize()
        assert int(m.pos_dev.item()) == start + r + 1
    assert torch.equal(m.hist[start:start + 10].cpu(), eager_toks)
    assert torch.equal(m.logits.cpu(), eager_logits)


def test_generate_result(dev):
    m = LlamaModel.random_init(SMALL, seed=17, device=dev, max_seq=64)
    m.capture()
    ids = np.random.default_rng(18).integers(0, SMALL.vocab_size, 20)
    r = m.generate(ids, max_tokens=12)
    assert len(r.token_ids) == 12 and r.num_decode_tokens == 11 and r.num_prefill_tokens == 20
    assert r.decode_tok_s > 0 and r.prefill_tok_s > 0
    r2 = m.generate(ids, max_tokens=12, use_graph=False)
    assert r2.token_ids == r.token_ids
    # greedy continuation equals feeding the generated tokens back one at a time
    m.reset()
    m.prefill(ids)
    for t in r.token_ids[:-1]:
        m.token.fill_(t)
        m.decode_step()
        m.pos += 1
    assert int(m.token.item()) == r.token_ids[-1]


def test_capacity_and_id_checks(dev):
    from siliconfer_amd._lib import SFError

    m = LlamaModel.random_init(SMALL, seed=19, device=dev, max_seq=16)
    with pytest.raises(SFError):
        m.prefill(np.arange(17) % 100)
    with pytest.raises(SFError):
        m.prefill([SMALL.vocab_size])
    m.capture()
    m.prefill(np.arange(15))
    with pytest.raises(SFError):
        m.replay(2)


def test_device_packer_matches_numpy_packer(dev):
    from siliconfer_amd.kernels import pack_weights_sym

    rng = np.random.default_rng(20)
    W = rng.normal(0, 0.02, (64, 512)).astype(np.float32)
    pk, s = pack_weights_sym(W, 64)
    tpk, ts = pack_sym_device(torch.as_tensor(W).to(dev), 64)
    np.testing.assert_array_equal(tpk.cpu().numpy(), pk)
    np.testing.assert_array_equal(ts.cpu().numpy(), s)


def test_qwen05b_geometry_matches_oracle(dev):
    """BASELINE config 5 geometry (24 layers, 14/2 heads, vocab 151936): a
    32-token prompt and 3 decode steps against the oracle."""
    cfg = ModelConfig.qwen25_05b()
    m = LlamaModel.random_init(cfg, seed=4, group_size=64, device=dev, max_seq=64)
    ids = np.random.default_rng(4).integers(0, cfg.vocab_size, 32)
    check_against_oracle(m, cfg, ids, 3, 1e-2, "qwen0.5b")


@pytest.mark.parametrize("act", [torch.float32, torch.float16, torch.bfloat16])
def test_folded_decode_equals_unfolded(dev, act):
    """Decode with RMSNorm / SwiGLU folded into the projections gives the same
    bits as the separate kernels (non-unit norm weights, several steps)."""
    models = []
    for fuse in (True, False):
        m = LlamaModel.random_init(SMALL, seed=21, device=dev, max_seq=64, act_dtype=act, fuse=fuse)
        g = torch.Generator(device=dev)
        g.manual_seed(22)
        for L in m.layers:
            L.w_in.copy_(1 + 0.2 * torch.randn(L.w_in.shape, generator=g, device=dev))
            L.w_post.copy_(1 + 0.2 * torch.randn(L.w_post.shape, generator=g, device=dev))
        m.norm_w.copy_(1 + 0.2 * torch.randn(m.norm_w.shape, generator=g, device=dev))
        models.append(m)
    ids = np.random.default_rng(23).integers(0, SMALL.vocab_size, 11)
    for m in models:
        m.prefill(ids)
    for _ in range(5):
        outs = []
        for m in models:
            m.decode_step(logits=True)
            m.pos += 1
            torch.cuda.synchronize()
            outs.append((m.logits.cpu().clone(), int(m.token.item())))
        assert torch.equal(outs[0][0], outs[1][0]) and outs[0][1] == outs[1][1]


def test_config5_full_workload_against_oracle(dev):
    """BASELINE config 5 as the bench runs it (bench.py e2e_model): random-init
    Qwen2.5-0.5B geometry, seed 4, int4 sym g=64, fp16 activations, the 512-id
    prompt, then 255 decode steps replayed from the HIP graph. The oracle runs
    teacher-forced on the GPU's own tokens (prompt + generated, one causal
    block, pinned equal to token-by-token decoding). Every one of the 256
    steps is checked: its logits meet 1e-2 against the oracle's, its token is
    the argmax of its own logits (lowest index on ties), and the token is the
    oracle's argmax, or, where the oracle's top-2 margin is within twice that
    step's measured logit error (a near-tie that rounding may resolve either
    way), a logit within that distance of the oracle's maximum
    (reference harness: /root/reference/siliconfer/engine/generate.py:117-180)."""
    cfg = ModelConfig.qwen25_05b()
    m = LlamaModel.random_init(cfg, seed=4, group_size=64, device=dev, max_seq=512 + 256 + 256,
                               act_dtype=torch.float16)
    ids = np.random.default_rng(4).integers(0, cfg.vocab_size, 512)
    m.capture(logits=True)
    m.reset()
    first = m.prefill(ids)
    glog = [m.logits.cpu().numpy().copy()]
    for i in range(255):
        m.replay(1)
        torch.cuda.synchronize()
        glog.append(m.logits.cpu().numpy().copy())
    toks = [first] + m.hist[512:512 + 255].cpu().tolist()
    W = m.export_weights()
    cos, sin = rope_tables(cfg, m.max_seq)
    ref = OM.forward(W, cfg, np.concatenate([ids, np.asarray(toks[:-1])]), OM.KVCache(24), cos, sin,
                     last_rows=256)
    tol = 1e-2
    exact = ties = 0
    worst = 0.0
    for j in range(256):  # ref[j]: the logits after position 511 + j, which picked toks[j]
        got, r = glog[j], ref[j]
        assert_close(got, r, tol, f"config 5 logits of step {j}")
        worst = max(worst, float(np.abs(got - r).max() / np.abs(r).max()))
        assert toks[j] == int(np.argmax(got)), f"config 5 step {j}: token is not its logits' argmax"
        err = float(np.abs(got - r).max())
        best = OM.greedy(r)
        if toks[j] == best:
            exact += 1
        else:
            top2 = np.sort(r)[-2:]
            assert top2[1] - top2[0] <= 2 * err and r[toks[j]] >= r[best] - 2 * err, (
                f"config 5 step {j}: token {toks[j]}, oracle {best}, margin {top2[1] - top2[0]:.3g} "
                f"against twice the step's logit error {2 * err:.3g}")
            ties += 1
    print(f"config 5: 256 steps checked, {exact} tokens equal to the oracle's argmax, {ties} "
          f"near-ties resolved the other way; worst logit error {worst:.2e} of max |logit|")
    assert exact + ties == 256
