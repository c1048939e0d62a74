"""HuggingFace safetensors checkpoints on the host.

`Checkpoint` indexes a checkpoint directory without reading any tensor data: it
opens each safetensors shard's header once and keeps a map from tensor name to
the shard that holds it. Tensors are then read one at a time (`get`) or shard
by shard (`items`), so a caller that packs projections as it goes never holds
the whole dense checkpoint. Files are read with `safetensors`, which executes
nothing from them.

Which files make up the checkpoint, and two facts derived from its tensors,
follow the reference's loader (/root/reference/siliconfer/engine/loader.py:14-58),
because a drop-in caller relies on them:
  * `model.safetensors` alone, else the shards an
    `model.safetensors.index.json` weight map names, else FileNotFoundError;
  * with `tie_word_embeddings`, a missing `lm_head.weight` is the embedding
    (the same tensor object);
  * a `q_proj` bias in layer 0 switches `attention_bias` on.

`load_model` / `load_weights` return the reference's (config, {name: tensor})
shapes of result for callers that want everything at once.
"""

from __future__ import annotations

import json
from collections.abc import Iterator
from pathlib import Path

import torch

from ..model.config import ModelConfig

SINGLE_FILE = "model.safetensors"
INDEX_FILE = "model.safetensors.index.json"
EMBED = "model.embed_tokens.weight"
LM_HEAD = "lm_head.weight"


def _shard_paths(root: Path) -> list[Path]:
    if (root / SINGLE_FILE).exists():
        return [root / SINGLE_FILE]
    index = root / INDEX_FILE
    if index.exists():
        weight_map = json.loads(index.read_text())["weight_map"]
        return [root / f for f in sorted(set(weight_map.values()))]
    raise FileNotFoundError(f"No safetensors found in {root}. "
                            f"Expected {SINGLE_FILE} or {INDEX_FILE}")


class Checkpoint:
    """A checkpoint directory: `config` plus lazy access to its tensors."""

    def __init__(self, model_dir: str | Path):
        from safetensors import safe_open

        self.root = Path(model_dir)
        self.shards = _shard_paths(self.root)
        self._where: dict[str, Path] = {}
        for path in self.shards:
            with safe_open(str(path), framework="pt") as f:
                for name in f.keys():
                    self._where[name] = path
        self.config = ModelConfig.from_json(self.root / "config.json")
        if "model.layers.0.self_attn.q_proj.bias" in self._where:
            self.config.attention_bias = True

    def _tied_head(self) -> bool:
        return self.config.tie_word_embeddings and LM_HEAD not in self._where and EMBED in self._where

    def names(self) -> list[str]:
        """Stored tensor names, plus `lm_head.weight` when the head is tied."""
        return sorted(self._where) + ([LM_HEAD] if self._tied_head() else [])

    def __contains__(self, name: str) -> bool:
        return name in self._where or (name == LM_HEAD and self._tied_head())

    def get(self, name: str) -> torch.Tensor:
        """One tensor, read from its shard (a tied head reads the embedding)."""
        from safetensors import safe_open

        if name == LM_HEAD and self._tied_head():
            name = EMBED
        if name not in self._where:
            raise KeyError(name)
        with safe_open(str(self._where[name]), framework="pt") as f:
            return f.get_tensor(name)

    def items(self) -> Iterator[tuple[str, torch.Tensor]]:
        """(name, tensor) for every stored tensor, one shard open at a time."""
        from safetensors import safe_open

        for path in self.shards:
            with safe_open(str(path), framework="pt") as f:
                for name in f.keys():
                    yield name, f.get_tensor(name)

    def load_all(self) -> dict[str, torch.Tensor]:
        """Every tensor in one dict; a tied head is the embedding object itself."""
        out = dict(self.items())
        if self._tied_head():
            out[LM_HEAD] = out[EMBED]
        return out


def load_weights(model_dir: str | Path) -> dict[str, torch.Tensor]:
    return Checkpoint(model_dir).load_all()


def load_model(model_dir: str | Path) -> tuple[ModelConfig, dict[str, torch.Tensor]]:
    ckpt = Checkpoint(model_dir)
    return ckpt.config, ckpt.load_all()
