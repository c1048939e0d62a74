"""HuggingFace safetensors checkpoints -> (ModelConfig, {name: tensor}), the
reference's siliconfer.engine.loader (/root/reference/siliconfer/engine/loader.py:14-58):
a single `model.safetensors` or the shards named by
`model.safetensors.index.json`; a tied `lm_head.weight` is filled from the
embedding; q_proj biases switch `attention_bias` on. Tensors stay on the host
(torch CPU tensors, read with safetensors, which executes nothing from the file).
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Any

import torch

from ..model.config import ModelConfig


def _find_safetensor_files(model_dir: Path) -> list[Path]:
    single = model_dir / "model.safetensors"
    if single.exists():
        return [single]
    index_path = model_dir / "model.safetensors.index.json"
    if index_path.exists():
        with open(index_path) as f:
            index: dict[str, Any] = json.load(f)
        return [model_dir / name for name in sorted(set(index["weight_map"].values()))]
    raise FileNotFoundError(f"No safetensors found in {model_dir}. "
                            "Expected model.safetensors or model.safetensors.index.json")


def load_weights(model_dir: str | Path) -> dict[str, torch.Tensor]:
    from safetensors.torch import load_file

    weights: dict[str, torch.Tensor] = {}
    for shard in _find_safetensor_files(Path(model_dir)):
        weights.update(load_file(str(shard), device="cpu"))
    return weights


def load_model(model_dir: str | Path) -> tuple[ModelConfig, dict[str, torch.Tensor]]:
    model_dir = Path(model_dir)
    config = ModelConfig.from_json(model_dir / "config.json")
    weights = load_weights(model_dir)
    if config.tie_word_embeddings and "lm_head.weight" not in weights:
        if "model.embed_tokens.weight" in weights:
            weights["lm_head.weight"] = weights["model.embed_tokens.weight"]
    if "model.layers.0.self_attn.q_proj.bias" in weights:
        config.attention_bias = True
    return config, weights


def weight_summary(weights: dict[str, torch.Tensor]) -> str:
    lines = []
    total_params = total_bytes = 0
    for name in sorted(weights):
        t = weights[name]
        total_params += t.numel()
        total_bytes += t.numel() * t.element_size()
        lines.append(f"  {name}: {list(t.shape)} {t.dtype}")
    lines.insert(0, f"Weights: {len(weights)} tensors, {total_params:,} params, "
                    f"{total_bytes / 1e9:.2f} GB")
    return "\n".join(lines)
