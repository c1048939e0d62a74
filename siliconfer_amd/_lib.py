"""ctypes binding of libsiliconfer_hip.so (the C ABI in include/siliconfer_hip.h).

torch is imported first so that the library binds to the HIP runtime torch has
already loaded (both are libamdhip64.so.7); device pointers and streams then
come straight from torch tensors.

There is no CPU fallback anywhere in siliconfer_amd: every compute call goes
through this library and raises if it cannot be loaded or no gfx950 device is
present.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsiliconfer_hip.so")

SF_F32, SF_F16, SF_BF16 = 0, 1, 2
SF_PRE_RMSNORM, SF_PRE_SILU_MUL = 1, 2
SF_CHAIN_IN_X0, SF_CHAIN_IN_PREV, SF_CHAIN_IN_SWIGLU = 0, 1, 2
SF_CHAIN_MAX_PHASES = 8
_DT = {torch.float32: SF_F32, torch.float16: SF_F16, torch.bfloat16: SF_BF16}

_c_i, _c_f, _c_sz, _c_p = ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/siliconfer_hip.h
_SIGS = {
    "sf_last_error": (ctypes.c_char_p, []),
    "sf_abi_version": (_c_i, []),
    "sf_device_arch_ok": (_c_i, [_c_i]),
    "sf_q4_blob_bytes": (_c_sz, [_c_i, _c_i, _c_i, _c_i]),
    "sf_q4_repack": (_c_i, [_c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_p, _c_sz, _c_p]),
    "sf_q4_unpack": (_c_i, [_c_p, _c_i, _c_i, _c_i, _c_i, _c_p, _c_p, _c_p, _c_p]),
    "sf_q4_gemv": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_p, _c_i,
                          _c_i, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "sf_q4_gemv_supported": (_c_i, [_c_i, _c_i, _c_i, _c_i, _c_i]),
    "sf_q4_gemv_fused": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_f, _c_i, _c_p, _c_i, _c_p, _c_p,
                                _c_i, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "sf_q4_gemv_fused_rows_supported": (_c_i, [_c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i]),
    "sf_q4_gemv_fused_rows": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_f, _c_i, _c_p, _c_i, _c_p, _c_p, _c_i,
                                     _c_i, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "sf_q4_gemv_fused_rope_supported": (_c_i, [_c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i]),
    "sf_q4_gemv_fused_rope": (_c_i, [_c_p, _c_p, _c_p, _c_f, _c_i, _c_p, _c_i, _c_p, _c_p, _c_i, _c_p,
                                     _c_i, _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i,
                                     _c_p, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "sf_q4_gemm_workspace_bytes": (_c_sz, [_c_i, _c_i, _c_i, _c_i]),
    "sf_q4_gemm": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_p, _c_i,
                          _c_i, _c_i, _c_i, _c_i, _c_i, _c_p, _c_sz, _c_p]),
    "sf_q4_gemm_splits": (_c_i, [_c_i, _c_i, _c_i, _c_i]),
    "sf_q4_gemm_partials": (_c_i, [_c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_p, _c_sz,
                                   _c_p]),
    "sf_kv_quant_append": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_p, _c_p, _c_p, _c_i,
                                  _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "sf_attn_workspace_bytes": (_c_sz, [_c_i, _c_i, _c_i, _c_i]),
    "sf_attn_default_splits": (_c_i, [_c_i, _c_i, _c_i]),
    "sf_attn_default_splits_d": (_c_i, [_c_i, _c_i, _c_i, _c_i]),
    "sf_attn_decode_i8kv": (_c_i, [_c_p, _c_i, _c_p, _c_p, _c_p, _c_p, _c_i, _c_p, _c_i,
                                   _c_p, _c_sz, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_f,
                                   _c_i, _c_p]),
    "sf_attn_noalloc_max_bytes": (_c_sz, []),
    "sf_attn_decode_i8kv_noalloc": (_c_i, [_c_p, _c_i, _c_p, _c_p, _c_p, _c_p, _c_i, _c_p, _c_i,
                                           _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_f, _c_i, _c_p]),
    "sf_attn_decode_i8kv_dev": (_c_i, [_c_p, _c_i, _c_p, _c_p, _c_p, _c_p, _c_i, _c_p, _c_i,
                                       _c_p, _c_sz, _c_i, _c_i, _c_i, _c_p, _c_i, _c_i, _c_i,
                                       _c_i, _c_f, _c_i, _c_p]),
    "sf_attn_decode_i8kv_partials_dev": (_c_i, [_c_p, _c_i, _c_p, _c_p, _c_p, _c_p, _c_i, _c_p, _c_sz,
                                                _c_i, _c_i, _c_i, _c_p, _c_i, _c_i, _c_i, _c_i, _c_f,
                                                _c_i, _c_p]),
    "sf_q4_gemv_attn_merge_supported": (_c_i, [_c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i]),
    "sf_q4_gemv_attn_merge": (_c_i, [_c_p, _c_p, _c_sz, _c_i, _c_i, _c_i, _c_i, _c_p, _c_i, _c_p, _c_p,
                                     _c_i, _c_i, _c_i, _c_i, _c_i, _c_p]),
    "sf_attn_prefill_i8kv": (_c_i, [_c_p, _c_i, _c_p, _c_p, _c_p, _c_p, _c_i, _c_p, _c_i,
                                    _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_f, _c_p]),
    "sf_attn_prefill_i8kv_dev": (_c_i, [_c_p, _c_i, _c_p, _c_p, _c_p, _c_p, _c_i, _c_p, _c_i, _c_p,
                                        _c_sz, _c_i, _c_i, _c_i, _c_p, _c_i, _c_i, _c_i, _c_f,
                                        _c_i, _c_p]),
    "sf_embed": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_i, _c_i, _c_i, _c_p]),
    "sf_rmsnorm": (_c_i, [_c_p, _c_p, _c_p, _c_i, _c_p, _c_i, _c_i, _c_i, _c_f, _c_p]),
    "sf_rmsnorm_partials": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_i, _c_i, _c_i, _c_f,
                                   _c_p]),
    "sf_rope_kv_append": (_c_i, [_c_p, _c_p, _c_p, _c_i, _c_p, _c_i, _c_p, _c_p, _c_p, _c_p,
                                 _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_p, _c_i, _c_p]),
    "sf_rope_kv_append_partials": (_c_i, [_c_p, _c_i, _c_p, _c_i, _c_p, _c_p, _c_i, _c_p, _c_i,
                                          _c_p, _c_p, _c_p, _c_p, _c_i, _c_i, _c_i, _c_i, _c_i,
                                          _c_i, _c_p, _c_i, _c_p]),
    "sf_silu_mul": (_c_i, [_c_p, _c_p, _c_i, _c_i, _c_i, _c_p]),
    "sf_lm_head_workspace_bytes": (_c_sz, [_c_i]),
    "sf_lm_head_argmax": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_i, _c_i, _c_p, _c_p, _c_p, _c_p,
                                 _c_sz, _c_p]),
    "sf_lm_head_argmax_rmsnorm": (_c_i, [_c_p, _c_p, _c_p, _c_f, _c_i, _c_p, _c_i, _c_i, _c_p,
                                         _c_p, _c_p, _c_p, _c_sz, _c_p]),
    "sf_lm_head_rows_workspace_bytes": (_c_sz, [_c_i, _c_i]),
    "sf_lm_head_argmax_rows": (_c_i, [_c_p, _c_p, _c_i, _c_p, _c_i, _c_i, _c_i, _c_p, _c_p, _c_sz,
                                      _c_p]),
    "sf_q4_chain_workspace_bytes": (_c_sz, [_c_p, _c_i]),
    "sf_q4_chain": (_c_i, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i, _c_p, _c_p, _c_p, _c_sz, _c_i, _c_i,
                           _c_p]),
    "sf_q4_chain_error": (_c_i, [_c_p, _c_p, _c_p]),
    "sf_floor_empty": (_c_i, [_c_p]),
    "sf_floor_read": (_c_i, [_c_p, _c_sz, _c_p, _c_p]),
}

_lock = threading.Lock()
_lib = None
_arch_ok: dict[int, bool] = {}


class SFError(RuntimeError):
    """A libsiliconfer_hip call failed (the reference raises RuntimeError too)."""


def load() -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise SFError(f"{LIB_PATH} is not built: run `python -m siliconfer_amd.build`")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def exported_symbols() -> list[str]:
    return sorted(_SIGS)


def last_error() -> str:
    return load().sf_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise SFError(f"{what}: {last_error()} (code {rc})")


def hip_available() -> bool:
    """True when the library loads and the current device is a gfx950 GPU."""
    try:
        lib = load()
    except SFError:
        return False
    if not torch.cuda.is_available():
        return False
    dev = torch.cuda.current_device()
    if dev not in _arch_ok:
        _arch_ok[dev] = lib.sf_device_arch_ok(dev) == 1
    return _arch_ok[dev]


def require_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise SFError(f"{name} must be a device tensor (got {t.device})")
    if not t.is_contiguous():
        raise SFError(f"{name} must be contiguous")


def dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise SFError(f"unsupported dtype {t.dtype}") from None


def stream(t: torch.Tensor | None = None) -> int:
    dev = t.device if t is not None else torch.device("cuda", torch.cuda.current_device())
    return torch.cuda.current_stream(dev).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
