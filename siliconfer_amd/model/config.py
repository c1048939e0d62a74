"""Model configuration — the fields and defaults of the reference's
`siliconfer.model.config.ModelConfig`
(/root/reference/siliconfer/model/config.py:11-108), read from a HuggingFace
config.json the same way, plus the RoPE frequency rule of
`_compute_rope_freqs` (/root/reference/siliconfer/model/layers.py:24-55).
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import numpy as np


@dataclass
class RoPEScalingConfig:
    type: str = ""
    factor: float = 1.0
    low_freq_factor: float = 1.0
    high_freq_factor: float = 4.0
    original_max_position_embeddings: int = 8192


@dataclass
class ModelConfig:
    architectures: list[str] = field(default_factory=list)
    hidden_size: int = 0
    intermediate_size: int = 0
    num_hidden_layers: int = 0
    num_attention_heads: int = 0
    num_key_value_heads: int = 0
    head_dim: int = 0
    vocab_size: int = 0
    max_position_embeddings: int = 0
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_scaling: RoPEScalingConfig | None = None
    tie_word_embeddings: bool = False
    hidden_act: str = "silu"
    torch_dtype: str = "float16"
    bos_token_id: int | None = None
    eos_token_id: int | None = None
    attention_bias: bool = False
    model_type: str = ""

    def __post_init__(self) -> None:
        if self.head_dim == 0 and self.num_attention_heads > 0:
            self.head_dim = self.hidden_size // self.num_attention_heads
        if self.num_key_value_heads == 0:
            self.num_key_value_heads = self.num_attention_heads

    @property
    def gqa_groups(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    @classmethod
    def from_json(cls, path: str | Path) -> "ModelConfig":
        with open(path) as f:
            raw: dict[str, Any] = json.load(f)
        return cls.from_dict(raw)

    @classmethod
    def from_dict(cls, raw: dict[str, Any]) -> "ModelConfig":
        rope_scaling = None
        if raw_rope := raw.get("rope_scaling"):
            rope_scaling = RoPEScalingConfig(
                type=raw_rope.get("type", raw_rope.get("rope_type", "")),
                factor=raw_rope.get("factor", 1.0),
                low_freq_factor=raw_rope.get("low_freq_factor", 1.0),
                high_freq_factor=raw_rope.get("high_freq_factor", 4.0),
                original_max_position_embeddings=raw_rope.get(
                    "original_max_position_embeddings", 8192),
            )
        return cls(
            architectures=raw.get("architectures", []),
            hidden_size=raw.get("hidden_size", 0),
            intermediate_size=raw.get("intermediate_size", 0),
            num_hidden_layers=raw.get("num_hidden_layers", 0),
            num_attention_heads=raw.get("num_attention_heads", 0),
            num_key_value_heads=raw.get("num_key_value_heads", 0),
            head_dim=raw.get("head_dim", 0),
            vocab_size=raw.get("vocab_size", 0),
            max_position_embeddings=raw.get("max_position_embeddings", 0),
            rms_norm_eps=raw.get("rms_norm_eps", 1e-5),
            rope_theta=raw.get("rope_theta", 500000.0),
            rope_scaling=rope_scaling,
            tie_word_embeddings=raw.get("tie_word_embeddings", False),
            hidden_act=raw.get("hidden_act", "silu"),
            torch_dtype=raw.get("torch_dtype", "float16"),
            bos_token_id=raw.get("bos_token_id"),
            eos_token_id=raw.get("eos_token_id"),
            attention_bias=raw.get("attention_bias", False),
            model_type=raw.get("model_type", ""),
        )

    def to_dict(self) -> dict[str, Any]:
        """HF config.json fields (from_dict(to_dict()) round-trips)."""
        raw: dict[str, Any] = {k: getattr(self, k) for k in (
            "architectures", "hidden_size", "intermediate_size", "num_hidden_layers",
            "num_attention_heads", "num_key_value_heads", "head_dim", "vocab_size",
            "max_position_embeddings", "rms_norm_eps", "rope_theta", "tie_word_embeddings",
            "hidden_act", "torch_dtype", "bos_token_id", "eos_token_id", "attention_bias",
            "model_type")}
        if self.rope_scaling is not None:
            r = self.rope_scaling
            raw["rope_scaling"] = {"type": r.type, "factor": r.factor,
                                   "low_freq_factor": r.low_freq_factor,
                                   "high_freq_factor": r.high_freq_factor,
                                   "original_max_position_embeddings": r.original_max_position_embeddings}
        return raw

    @classmethod
    def qwen25_05b(cls) -> "ModelConfig":
        """Qwen2.5-0.5B geometry: 24 layers, hidden 896, 14 / 2 heads of 64,
        SwiGLU 4864, RMSNorm eps 1e-6, RoPE theta 1e6, vocab 151936, tied
        embeddings, q/k/v biases (Qwen2 attention)."""
        return cls(architectures=["Qwen2ForCausalLM"], hidden_size=896, intermediate_size=4864,
                   num_hidden_layers=24, num_attention_heads=14, num_key_value_heads=2,
                   head_dim=64, vocab_size=151936, max_position_embeddings=32768,
                   rms_norm_eps=1e-6, rope_theta=1000000.0, tie_word_embeddings=True,
                   torch_dtype="bfloat16", attention_bias=True, model_type="qwen2")


def rope_freqs(config: ModelConfig) -> np.ndarray:
    """fp32 inverse frequencies 1 / theta^(2i / D), with the reference's
    Llama-3 scaling when configured (layers.py:24-55)."""
    D = config.head_dim
    freqs = (1.0 / (np.float32(config.rope_theta)
                    ** (np.arange(0, D, 2, dtype=np.float32) / np.float32(D)))).astype(np.float32)
    sc = config.rope_scaling
    if sc and sc.type == "llama3":
        low_wl = sc.original_max_position_embeddings / sc.low_freq_factor
        high_wl = sc.original_max_position_embeddings / sc.high_freq_factor
        out = []
        for f in freqs.tolist():
            wl = 2.0 * math.pi / f
            if wl > low_wl:
                out.append(f / sc.factor)
            elif wl < high_wl:
                out.append(f)
            else:
                smooth = (sc.original_max_position_embeddings / wl - sc.low_freq_factor) / (
                    sc.high_freq_factor - sc.low_freq_factor)
                out.append((1 - smooth) * f / sc.factor + smooth * f)
        freqs = np.asarray(out, dtype=np.float32)
    return freqs


def rope_tables(config: ModelConfig, max_pos: int) -> tuple[np.ndarray, np.ndarray]:
    """fp32 cos / sin of position * freq for positions [0, max_pos): the angles
    of `apply_rope` (layers.py:58-62), [max_pos, head_dim / 2] each."""
    freqs = rope_freqs(config)
    angles = np.outer(np.arange(max_pos, dtype=np.float32), freqs).astype(np.float32)
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)
