"""int4 packing of a checkpoint's projections, the packed on-disk format, and
the decoder built from it — the reference's siliconfer.engine.q4_loader
(/root/reference/siliconfer/engine/q4_loader.py:26-193).

`pack_and_replace_linears` follows `_pack_and_replace_linears` (:26-82): the 7
attention / MLP projections of every layer are RTN-packed in place, symmetric or
asymmetric as the caller says; a projection with in_features < group_size
(synthetic tiny models, :70-72) and every projection of a layer in
`skip_layers` keep their dense weight. `packing_symmetry` is the rule of
load_q4_model (:178-183): HQQ is always asymmetric, every other method packs on
the grid its `sym` flag chose. Quantizers other than RTN run offline (they are
out of this build); their fake-quantized checkpoints load with
`prequantized=True` and are packed the same way.

Packed on-disk format (one safetensors file, read without executing anything
from it): the checkpoint's tensors with each packed projection `<p>.weight`
replaced by

    <p>.q4_packed  uint8 [N, K/2]   byte (n, j) = q[n, 2j] | q[n, 2j+1] << 4
                                    (two's-complement codes symmetric, unsigned
                                    asymmetric: the reference's canonical packing)
    <p>.q4_scales  fp16  [N, K/g]
    <p>.q4_zeros   uint8 [N, K/g]   asymmetric only: the integral zero-points

and metadata {"format": "siliconfer_amd.q4", "version": "1", "group_size",
"sym", "method", "config" (config.json as JSON)}. Scales are stored as fp16 and
zero-points as uint4 values in bytes, the kernels' storage (the reference keeps
fp32 arrays); a tied lm_head is not stored twice. Loading repacks each
projection into its device blob (`sf_q4_repack`) without re-quantizing.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

from .._lib import SFError
from ..kernels import pack_weights_asym, pack_weights_sym
from ..kernels.q4 import Q4Weight
from ..model.config import ModelConfig
from .loader import load_model

PROJECTIONS = [("self_attn", "q_proj"), ("self_attn", "k_proj"), ("self_attn", "v_proj"),
               ("self_attn", "o_proj"), ("mlp", "gate_proj"), ("mlp", "up_proj"),
               ("mlp", "down_proj")]
FORMAT = "siliconfer_amd.q4"
PACKED_FILE = "model.q4.safetensors"
QUANT_METHODS = ("rtn", "gptq", "awq", "hqq", "sinq")


def packing_symmetry(method: str, sym: bool) -> bool:
    """The grid the packer must use (q4_loader.py:178-183): HQQ fits a
    zero-point, so it is always asymmetric; the others follow `sym`."""
    return False if method == "hqq" else sym


def _prefix(i: int, parent: str, name: str) -> str:
    return f"model.layers.{i}.{parent}.{name}"


def pack_and_replace_linears(weights: dict[str, torch.Tensor], config: ModelConfig,
                             group_size: int = 128, skip_layers: set[int] | None = None,
                             pack_sym: bool = True) -> list[str]:
    """Pack every eligible projection of `weights` in place (see the module
    docstring); returns the prefixes that were packed."""
    packed_names = []
    for i in range(config.num_hidden_layers):
        if skip_layers and i in skip_layers:
            continue
        for parent, name in PROJECTIONS:
            p = _prefix(i, parent, name)
            W = weights[p + ".weight"]
            if W.shape[1] < group_size:  # too small to quantize (q4_loader.py:70-72)
                continue
            Wn = W.float().numpy()
            if pack_sym:
                packed, scales = pack_weights_sym(Wn, group_size)
                zeros = None
            else:
                packed, scales, zeros = pack_weights_asym(Wn, group_size)
            del weights[p + ".weight"]
            weights[p + ".q4_packed"] = torch.from_numpy(np.ascontiguousarray(packed))
            weights[p + ".q4_scales"] = torch.from_numpy(scales.astype(np.float16))
            if zeros is not None:
                weights[p + ".q4_zeros"] = torch.from_numpy(np.rint(zeros).astype(np.uint8))
            packed_names.append(p)
    return packed_names


def save_q4_model(path: str | Path, config: ModelConfig, weights: dict[str, torch.Tensor],
                  group_size: int, sym: bool, method: str = "rtn") -> Path:
    """Write `weights` (after pack_and_replace_linears) in the packed format.
    `path` is a file, or a directory that receives model.q4.safetensors."""
    from safetensors.torch import save_file

    path = Path(path)
    if path.is_dir() or not path.suffix:
        path.mkdir(parents=True, exist_ok=True)
        path = path / PACKED_FILE
    tensors = {}
    for k, t in weights.items():
        if (k == "lm_head.weight" and config.tie_word_embeddings
                and "model.embed_tokens.weight" in weights):
            continue  # the tied head is the embedding (restored on load)
        tensors[k] = t.detach().cpu().contiguous()
    meta = {"format": FORMAT, "version": "1", "group_size": str(group_size),
            "sym": "1" if sym else "0", "method": method, "config": json.dumps(config.to_dict())}
    save_file(tensors, str(path), metadata=meta)
    return path


def load_q4_packed(path: str | Path) -> tuple[ModelConfig, dict[str, torch.Tensor], dict]:
    """Read a packed file (or a directory holding model.q4.safetensors) ->
    (config, host tensors, metadata with group_size as int and sym as bool)."""
    from safetensors import safe_open
    from safetensors.torch import load_file

    path = Path(path)
    if path.is_dir():
        path = path / PACKED_FILE
    with safe_open(str(path), framework="pt") as f:
        meta = dict(f.metadata() or {})
    if meta.get("format") != FORMAT:
        raise SFError(f"{path}: not a {FORMAT} file (metadata format={meta.get('format')!r})")
    config = ModelConfig.from_dict(json.loads(meta["config"]))
    weights = load_file(str(path), device="cpu")
    if config.tie_word_embeddings and "lm_head.weight" not in weights:
        weights["lm_head.weight"] = weights["model.embed_tokens.weight"]
    meta["group_size"] = int(meta["group_size"])
    meta["sym"] = meta["sym"] == "1"
    return config, weights, meta


def _q4(weights: dict[str, torch.Tensor], prefixes: list[str], group_size: int,
        device: torch.device) -> Q4Weight:
    """One device weight from the packed projections `prefixes`, stacked by rows
    (packing is per row and per group, so stacking packed rows packs the stacked
    matrix)."""
    missing = [p for p in prefixes if p + ".q4_packed" not in weights]
    if missing:
        raise SFError(f"{missing[0]} is not packed int4 (in_features < group_size or a skipped "
                      "layer): this decoder runs int4 projections only")
    asym = [p + ".q4_zeros" in weights for p in prefixes]
    if any(asym) != all(asym):
        raise SFError(f"{prefixes}: fused projections must share one grid (all sym or all asym)")
    cat = lambda suf: torch.cat([weights[p + suf] for p in prefixes], dim=0)
    return Q4Weight(cat(".q4_packed"), cat(".q4_scales"), cat(".q4_zeros") if all(asym) else None,
                    group_size, device=device)


def build_model(config: ModelConfig, weights: dict[str, torch.Tensor], group_size: int,
                device=None, max_seq: int = 1024, act_dtype: torch.dtype = torch.float16,
                max_prefill: int = 512, fuse: bool = True):
    """The batch-1 decoder (LlamaModel) on the device from packed host tensors:
    q|k|v and gate|up are stacked into one projection each, biases and RMSNorm
    weights go to fp32, the embedding (and an untied lm_head) to bf16."""
    from ..model.llama import LayerWeights, LlamaModel

    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    f32 = lambda t: t.to(device=dev, dtype=torch.float32).contiguous()
    layers = []
    for i in range(config.num_hidden_layers):
        a, m = f"model.layers.{i}.self_attn", f"model.layers.{i}.mlp"
        qkv = _q4(weights, [f"{a}.q_proj", f"{a}.k_proj", f"{a}.v_proj"], group_size, dev)
        bias = None
        if config.attention_bias:
            bias = f32(torch.cat([weights[f"{a}.{n}.bias"] for n in ("q_proj", "k_proj", "v_proj")]))
        layers.append(LayerWeights(
            qkv, bias, _q4(weights, [f"{a}.o_proj"], group_size, dev),
            _q4(weights, [f"{m}.gate_proj", f"{m}.up_proj"], group_size, dev),
            _q4(weights, [f"{m}.down_proj"], group_size, dev),
            f32(weights[f"model.layers.{i}.input_layernorm.weight"]),
            f32(weights[f"model.layers.{i}.post_attention_layernorm.weight"])))
    bf16 = lambda t: t.to(device=dev, dtype=torch.bfloat16).contiguous()
    embed = bf16(weights["model.embed_tokens.weight"])
    head = weights.get("lm_head.weight")
    tied = head is None or head is weights["model.embed_tokens.weight"] or (
        config.tie_word_embeddings and head.data_ptr() == weights["model.embed_tokens.weight"].data_ptr())
    return LlamaModel(config, layers, embed, f32(weights["model.norm.weight"]), group_size, max_seq,
                      act_dtype, max_prefill, fuse, lm_head=None if tied else bf16(head))


def load_q4_model(model_dir: str | Path, method: str = "rtn", group_size: int = 128,
                  sym: bool = True, skip_layers: set[int] | None = None,
                  prequantized: bool = False, save_to: str | Path | None = None, **model_kw):
    """Load a decoder -> (LlamaModel, ModelConfig), like the reference's
    load_q4_model (q4_loader.py:85-193).

    A packed file (or a directory with model.q4.safetensors) loads as stored.
    Otherwise the HuggingFace checkpoint in `model_dir` is read and packed:
    `method="rtn"` quantizes here (round-to-nearest, symmetric or not per
    `sym`); for the other methods, which run offline, pass their
    fake-quantized checkpoint with `prequantized=True` — it is packed on the
    grid `packing_symmetry(method, sym)` names. `save_to` writes the packed file.
    `model_kw` go to build_model (device, max_seq, act_dtype, ...)."""
    path = Path(model_dir)
    if path.is_file() or (path / PACKED_FILE).exists():
        config, weights, meta = load_q4_packed(path)
        return build_model(config, weights, meta["group_size"], **model_kw), config
    if method not in QUANT_METHODS:
        raise ValueError(f"Unknown method {method!r}. Choose one of {', '.join(QUANT_METHODS)}.")
    if method != "rtn" and not prequantized:
        raise ValueError(f"method={method!r} runs offline in this build: quantize with it, save the "
                         "fake-quantized checkpoint and load that with prequantized=True")
    config, weights = load_model(path)
    pack_sym = packing_symmetry(method, sym)
    pack_and_replace_linears(weights, config, group_size, skip_layers, pack_sym)
    if save_to is not None:
        save_q4_model(save_to, config, weights, group_size, pack_sym, method)
    return build_model(config, weights, group_size, **model_kw), config
