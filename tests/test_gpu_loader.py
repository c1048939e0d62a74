"""GPU: decoders built by the loader (siliconfer_amd/engine) from a checkpoint
and from the packed on-disk format, against the oracle of the reference's
forward pass (oracle/model.py) with the same weights, symmetric and
asymmetric, tied and untied lm_head.
"""

import numpy as np
import pytest
import torch

from oracle import model as OM
from oracle.linear import assert_close
from siliconfer_amd._lib import SFError
from siliconfer_amd.engine import load_q4_model
from siliconfer_amd.model.config import rope_tables
from test_loader import TINY, tiny_checkpoint

pytestmark = pytest.mark.gpu


def logits_run(m, ids, n_decode):
    """Prefill + n_decode greedy steps -> list of logits rows (fp32 numpy)."""
    m.reset()
    out = []
    m.prefill(ids)
    out.append(m.logits.cpu().numpy().copy())
    for _ in range(n_decode):
        m.decode_step(logits=True)
        m.pos += 1
        torch.cuda.synchronize()
        out.append(m.logits.cpu().numpy().copy())
    return out


def oracle_run(m, cfg, ids, n_decode, toks):
    W = m.export_weights()
    cos, sin = rope_tables(cfg, m.max_seq)
    cache = OM.KVCache(cfg.num_hidden_layers)
    rows = [OM.forward(W, cfg, ids, cache, cos, sin)[-1]]
    for t in toks:
        rows.append(OM.forward(W, cfg, [t], cache, cos, sin)[-1])
    return rows


@pytest.mark.parametrize("sym,tied", [(True, True), (False, True), (True, False)])
def test_loaded_decoder_matches_oracle(dev, tmp_path, sym, tied):
    cfg_raw = dict(TINY, tie_word_embeddings=tied)
    tiny_checkpoint(tmp_path, cfg=cfg_raw, seed=3)
    m, cfg = load_q4_model(tmp_path, group_size=64, sym=sym, device=dev, max_seq=64,
                           act_dtype=torch.float32)
    assert all(L.qkv.has_zeros != sym for L in m.layers)
    assert (m.head is m.embed) == tied
    ids = np.random.default_rng(5).integers(0, cfg.vocab_size, 9)
    got = logits_run(m, ids, 4)
    toks = [int(np.argmax(r)) for r in got[:-1]]
    ref = oracle_run(m, cfg, ids, 4, toks)
    for i, (g, r) in enumerate(zip(got, ref)):
        assert_close(g, r, 2e-3, f"sym={sym} tied={tied} step {i}")


def test_packed_file_gives_the_same_decoder(dev, tmp_path):
    src = tmp_path / "ckpt"
    src.mkdir()
    tiny_checkpoint(src, seed=4)
    a, _ = load_q4_model(src, group_size=64, sym=False, save_to=tmp_path / "packed", device=dev,
                         max_seq=64)
    b, _ = load_q4_model(tmp_path / "packed", device=dev, max_seq=64)
    for name in ("qkv", "o", "gate_up", "down"):
        for x, y in zip(getattr(a.layers[1], name).canonical(), getattr(b.layers[1], name).canonical()):
            assert torch.equal(x, y)
    ids = np.random.default_rng(6).integers(0, TINY["vocab_size"], 7)
    for ra, rb in zip(logits_run(a, ids, 3), logits_run(b, ids, 3)):
        np.testing.assert_array_equal(ra, rb)


def test_unquantized_projection_is_refused(dev, tmp_path):
    tiny_checkpoint(tmp_path, seed=7)
    with pytest.raises(SFError, match="int4 projections only"):
        load_q4_model(tmp_path, group_size=64, skip_layers={1}, device=dev, max_seq=64)
