"""CPU: the module-level layers (siliconfer_amd/model/layers.py) refuse host
tensors — every route of RMSNorm, Attention, MLP and TransformerBlock runs on
the GPU, none falls back to host arithmetic — and build the reference's
module tree (layers.py:69-163) with the projection shapes of the config."""

import pytest
import torch

from siliconfer_amd._lib import SFError
from siliconfer_amd.model.config import ModelConfig
from siliconfer_amd.model.layers import MLP, Attention, RMSNorm, TransformerBlock, compute_rope_freqs

CFG = ModelConfig(hidden_size=64, intermediate_size=128, num_hidden_layers=1, num_attention_heads=4,
                  num_key_value_heads=2, head_dim=16, vocab_size=50, attention_bias=True)


def test_module_tree_matches_reference_names_and_shapes():
    blk = TransformerBlock(CFG, compute_rope_freqs(CFG), device="cpu")
    a, m = blk.self_attn, blk.mlp
    assert (a.num_heads, a.num_kv_heads, a.head_dim) == (4, 2, 16)
    assert a.scale == 16 ** -0.5
    shapes = {n: tuple(getattr(a, n).weight.shape) for n in ("q_proj", "k_proj", "v_proj", "o_proj")}
    assert shapes == {"q_proj": (64, 64), "k_proj": (32, 64), "v_proj": (32, 64), "o_proj": (64, 64)}
    assert a.q_proj.bias is not None and a.o_proj.bias is None
    assert tuple(m.gate_proj.weight.shape) == (128, 64) and tuple(m.down_proj.weight.shape) == (64, 128)
    assert blk.input_layernorm.eps == CFG.rms_norm_eps
    assert compute_rope_freqs(CFG).shape == (8,)


@pytest.mark.parametrize("which", ["norm", "attn", "mlp", "block"])
def test_host_tensors_are_refused(which):
    blk = TransformerBlock(CFG, compute_rope_freqs(CFG), device="cpu")
    x = torch.zeros((1, 3, 64))
    call = {"norm": lambda: RMSNorm(64)(x), "attn": lambda: blk.self_attn(x, None),
            "mlp": lambda: blk.mlp(x), "block": lambda: blk(x, None)}[which]
    with pytest.raises(SFError):
        call()


def test_checkpoint_arrays_from_numpy_or_torch():
    """from_weights reads checkpoint entries given as numpy arrays or torch tensors."""
    import numpy as np

    from siliconfer_amd.model.layers import _f32, _host

    a = np.arange(6, dtype=np.uint8).reshape(2, 3)
    assert np.array_equal(_host(a), a) and np.array_equal(_host(torch.from_numpy(a)), a)
    h = np.array([1.5, -2.25], dtype=np.float16)
    for src in (h, torch.from_numpy(h)):
        t = _f32(src)
        assert t.dtype == torch.float32 and t.tolist() == [1.5, -2.25]
