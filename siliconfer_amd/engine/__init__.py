"""Model loading: HuggingFace safetensors checkpoints (the reference's
siliconfer.engine.loader), the int4 packing / packed on-disk format (its
siliconfer.engine.q4_loader), the generation loop (its siliconfer.engine.generate)
and speculative decoding (its siliconfer.engine.speculative)."""

from .generate import SamplingParams, check_kv_cache_flag, generate, sample_token, warmup
from .loader import Checkpoint, load_model, load_weights
from .q4_loader import (PROJECTIONS, build_model, load_q4_model, load_q4_packed,
                        pack_and_replace_linears, packing_symmetry, save_q4_model)
from .speculative import SpeculativeResult, accept_greedy, accept_sampled, speculative_generate

__all__ = ["Checkpoint", "load_model", "load_weights", "PROJECTIONS", "build_model",
           "load_q4_model", "load_q4_packed", "pack_and_replace_linears", "packing_symmetry",
           "save_q4_model", "SpeculativeResult", "accept_greedy", "accept_sampled",
           "speculative_generate", "SamplingParams", "check_kv_cache_flag", "generate",
           "sample_token", "warmup"]
