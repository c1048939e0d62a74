"""CPU checks of the checkpoint loader and the int4 packing / packed file
(siliconfer_amd/engine), restating the reference's engine/loader.py:14-58 and
engine/q4_loader.py:26-193 behaviour: single-file and sharded checkpoints,
the tied lm_head, q_proj bias detection, the skip rules of
_pack_and_replace_linears (in_features < group_size; skip_layers), the HQQ ->
asymmetric rule, codes equal to the reference-named packers, and a bit-exact
save / load round trip of the packed format.
"""

import json

import numpy as np
import pytest
import torch

from siliconfer_amd.engine import (Checkpoint, load_model, load_q4_packed, pack_and_replace_linears,
                                   packing_symmetry, save_q4_model)
from siliconfer_amd.engine.q4_loader import PROJECTIONS, load_q4_model
from siliconfer_amd.kernels import pack_weights_asym, pack_weights_sym

TINY = {"architectures": ["Qwen2ForCausalLM"], "hidden_size": 128, "intermediate_size": 256,
        "num_hidden_layers": 3, "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 32,
        "vocab_size": 300, "rms_norm_eps": 1e-6, "rope_theta": 1e6, "tie_word_embeddings": True,
        "model_type": "qwen2"}


def tiny_checkpoint(tmp_path, cfg=TINY, bias=True, shards=1, seed=0, dtype=torch.float16):
    from safetensors.torch import save_file

    rng = np.random.default_rng(seed)
    H, I, D = cfg["hidden_size"], cfg["intermediate_size"], cfg["head_dim"]
    Hq, KVH = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    t = lambda *s: torch.from_numpy(rng.normal(0, 0.02, s).astype(np.float32)).to(dtype)
    w = {"model.embed_tokens.weight": t(cfg["vocab_size"], H), "model.norm.weight": t(H) + 1}
    if not cfg["tie_word_embeddings"]:
        w["lm_head.weight"] = t(cfg["vocab_size"], H)
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}"
        w |= {f"{p}.self_attn.q_proj.weight": t(Hq * D, H), f"{p}.self_attn.k_proj.weight": t(KVH * D, H),
              f"{p}.self_attn.v_proj.weight": t(KVH * D, H), f"{p}.self_attn.o_proj.weight": t(H, Hq * D),
              f"{p}.mlp.gate_proj.weight": t(I, H), f"{p}.mlp.up_proj.weight": t(I, H),
              f"{p}.mlp.down_proj.weight": t(H, I), f"{p}.input_layernorm.weight": t(H) + 1,
              f"{p}.post_attention_layernorm.weight": t(H) + 1}
        if bias:
            w |= {f"{p}.self_attn.q_proj.bias": t(Hq * D), f"{p}.self_attn.k_proj.bias": t(KVH * D),
                  f"{p}.self_attn.v_proj.bias": t(KVH * D)}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    names = sorted(w)
    if shards == 1:
        save_file(w, str(tmp_path / "model.safetensors"))
    else:
        parts = np.array_split(np.arange(len(names)), shards)
        wmap = {}
        for j, idx in enumerate(parts):
            fn = f"model-{j + 1:05d}-of-{shards:05d}.safetensors"
            save_file({names[k]: w[names[k]] for k in idx}, str(tmp_path / fn))
            wmap |= {names[k]: fn for k in idx}
        (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wmap}))
    return w


@pytest.mark.parametrize("shards", [1, 3])
def test_load_model_single_and_sharded(tmp_path, shards):
    w = tiny_checkpoint(tmp_path, shards=shards)
    cfg, got = load_model(tmp_path)
    assert cfg.hidden_size == 128 and cfg.num_hidden_layers == 3 and cfg.attention_bias
    assert got["lm_head.weight"] is got["model.embed_tokens.weight"]  # tied head filled in
    for k, v in w.items():
        assert torch.equal(got[k], v), k


@pytest.mark.parametrize("shards", [1, 3])
def test_checkpoint_index_reads_tensors_lazily(tmp_path, shards):
    w = tiny_checkpoint(tmp_path, shards=shards)
    ck = Checkpoint(tmp_path)
    assert len(ck.shards) == shards
    assert ck.names() == sorted(w) + ["lm_head.weight"]
    assert "lm_head.weight" in ck and "nope" not in ck
    assert torch.equal(ck.get("lm_head.weight"), w["model.embed_tokens.weight"])
    for k in ("model.layers.2.mlp.down_proj.weight", "model.norm.weight"):
        assert torch.equal(ck.get(k), w[k])
    assert dict(ck.items()).keys() == w.keys()
    with pytest.raises(KeyError):
        ck.get("model.layers.9.mlp.down_proj.weight")


def test_untied_head_is_read_as_stored(tmp_path):
    cfg = dict(TINY, tie_word_embeddings=False)
    w = tiny_checkpoint(tmp_path, cfg=cfg)
    c, got = load_model(tmp_path)
    assert not c.tie_word_embeddings
    assert got["lm_head.weight"] is not got["model.embed_tokens.weight"]
    assert torch.equal(got["lm_head.weight"], w["lm_head.weight"])


def test_no_bias_keeps_attention_bias_off(tmp_path):
    tiny_checkpoint(tmp_path, bias=False)
    cfg, _ = load_model(tmp_path)
    assert not cfg.attention_bias


def test_missing_checkpoint_raises(tmp_path):
    (tmp_path / "config.json").write_text(json.dumps(TINY))
    with pytest.raises(FileNotFoundError):
        load_model(tmp_path)


@pytest.mark.parametrize("sym", [True, False])
def test_packing_matches_reference_packers_and_skip_rules(tmp_path, sym):
    tiny_checkpoint(tmp_path)
    cfg, w = load_model(tmp_path)
    dense = {k: v.clone() for k, v in w.items()}
    # group 256: in_features 128 (every projection but down) is too small -> kept
    done = pack_and_replace_linears(w, cfg, group_size=256, skip_layers={1}, pack_sym=sym)
    assert done == ["model.layers.0.mlp.down_proj", "model.layers.2.mlp.down_proj"]
    for i in range(3):
        for parent, name in PROJECTIONS:
            p = f"model.layers.{i}.{parent}.{name}"
            if p in done:
                assert p + ".weight" not in w
                W = dense[p + ".weight"].float().numpy()
                if sym:
                    pk, s = pack_weights_sym(W, 256)
                    assert p + ".q4_zeros" not in w
                else:
                    pk, s, z = pack_weights_asym(W, 256)
                    np.testing.assert_array_equal(w[p + ".q4_zeros"].numpy(), z.astype(np.uint8))
                np.testing.assert_array_equal(w[p + ".q4_packed"].numpy(), pk)
                np.testing.assert_array_equal(w[p + ".q4_scales"].numpy(), s.astype(np.float16))
            else:
                assert torch.equal(w[p + ".weight"], dense[p + ".weight"])


def test_hqq_packs_asymmetric():
    assert packing_symmetry("hqq", True) is False and packing_symmetry("hqq", False) is False
    for m in ("rtn", "gptq", "awq", "sinq"):
        assert packing_symmetry(m, True) is True and packing_symmetry(m, False) is False


@pytest.mark.parametrize("sym", [True, False])
def test_packed_file_round_trip(tmp_path, sym):
    src = tmp_path / "ckpt"
    src.mkdir()
    tiny_checkpoint(src)
    cfg, w = load_model(src)
    pack_and_replace_linears(w, cfg, group_size=64, pack_sym=sym)
    out = save_q4_model(tmp_path / "packed", cfg, w, 64, sym, method="rtn")
    assert out.name == "model.q4.safetensors"
    cfg2, w2, meta = load_q4_packed(tmp_path / "packed")
    assert meta["group_size"] == 64 and meta["sym"] is sym and meta["method"] == "rtn"
    assert cfg2.to_dict() == cfg.to_dict()
    assert w2["lm_head.weight"] is w2["model.embed_tokens.weight"]
    assert set(w2) == set(w)
    for k, v in w.items():
        assert v.dtype == w2[k].dtype and torch.equal(v, w2[k]), k
    assert all(w2[k].dtype == torch.float16 for k in w2 if k.endswith(".q4_scales"))


def test_other_methods_need_prequantized_weights(tmp_path):
    tiny_checkpoint(tmp_path)
    with pytest.raises(ValueError, match="offline"):
        load_q4_model(tmp_path, method="gptq")
    with pytest.raises(ValueError, match="Unknown method"):
        load_q4_model(tmp_path, method="nope")


def test_not_a_packed_file(tmp_path):
    from siliconfer_amd._lib import SFError

    tiny_checkpoint(tmp_path)
    with pytest.raises(SFError, match="not a siliconfer_amd.q4 file"):
        load_q4_packed(tmp_path / "model.safetensors")
