"""C ABI checks that need no GPU: the library loads, exports every function
include/siliconfer_hip.h declares, sizes are computed on the host, and argument
validation rejects bad shapes with the reference's messages
(siliconfer/kernels/neon/bindings.cpp:24-40) before touching the device.
"""

import ctypes
import os
import re

import pytest

from siliconfer_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "siliconfer_hip.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sf_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_surface():
    names = declared_functions()
    for n in ("sf_q4_repack", "sf_q4_gemv", "sf_q4_gemm", "sf_kv_quant_append",
              "sf_attn_decode_i8kv", "sf_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"
    assert set(declared_functions()) == set(_lib.exported_symbols())


def test_abi_version():
    assert _lib.load().sf_abi_version() == 1


def test_blob_bytes_layout():
    lib = _lib.load()
    # sym 4096x4096 g128: weights 8 MiB, scales 512 octets x 32 groups x 8 x 2 B
    assert lib.sf_q4_blob_bytes(4096, 4096, 128, 0) == 8388608 + 512 * 32 * 16
    # asym adds 4 bytes per (octet, group) after a 256-byte aligned offset
    nb = lib.sf_q4_blob_bytes(4864, 896, 64, 1)
    w = 4864 * 448
    s_off = (w + 255) // 256 * 256
    z_off = (s_off + 608 * 14 * 16 + 255) // 256 * 256
    assert nb == z_off + 608 * 14 * 4
    # weights come in 1 KB units of 16 rows x 128 k: 10 x 96 pads to one unit
    assert lib.sf_q4_blob_bytes(10, 96, 32, 0) == 1024 + 2 * 3 * 16
    assert lib.sf_q4_blob_bytes(17, 160, 32, 0) == 2 * 2 * 1024 + 3 * 5 * 16
    assert lib.sf_q4_blob_bytes(10, 100, 64, 0) == 0      # K % g != 0
    assert lib.sf_q4_blob_bytes(0, 128, 64, 0) == 0


@pytest.mark.parametrize("K,g,code,msg", [
    (100, 64, -1, "in_features must be divisible by group_size"),
    (96, 48, -1, "null pointer argument"),   # any group size dividing K is a valid shape
    (6, 3, -1, "null pointer argument"),
])
def test_repack_rejects_bad_shapes(K, g, code, msg):
    lib = _lib.load()
    rc = lib.sf_q4_repack(None, None, None, 8, K, g, None, 0, None)
    assert rc == code
    assert msg in _lib.last_error()


def test_gemv_support_query():
    """sf_q4_gemv_supported: the MFMA GEMV's plans. Group sizes off the 32 grid
    and fp32 rows too long for the LDS staging run elsewhere (still computed)."""
    lib = _lib.load()
    F16, BF16, F32 = _lib.SF_F16, _lib.SF_BF16, _lib.SF_F32
    for B in (1, 2, 4, 8):
        for N, K in [(4096, 4096), (11008, 4096), (4096, 11008), (3584, 18944), (8192, 28672)]:
            assert lib.sf_q4_gemv_supported(B, N, K, 128, F16) == 1, (B, N, K)
            assert lib.sf_q4_gemv_supported(B, N, K, 128, BF16) == 1, (B, N, K)
        assert lib.sf_q4_gemv_supported(B, 896, 4864, 64, F16) == 1
        assert lib.sf_q4_gemv_supported(B, 4096, 9216, 96, F16) == 1
        assert lib.sf_q4_gemv_supported(B, 512, 768, 48, F16) == 0
        assert lib.sf_q4_gemv_supported(B, 512, 768, 16, F16) == 0
    assert lib.sf_q4_gemv_supported(1, 4096, 4096, 128, F32) == 1
    assert lib.sf_q4_gemv_supported(1, 8192, 28672, 128, F32) == 0
    assert lib.sf_q4_gemv_supported(9, 16, 128, 64, F16) == 0
    assert lib.sf_q4_gemv_supported(1, 16, 100, 64, F16) == 0


def test_gemv_rejects_batch_and_dtype():
    lib = _lib.load()
    rc = lib.sf_q4_gemv(None, None, 1, None, 1, None, None, 0, 9, 16, 128, 64, 0, None)
    assert rc == -1 and "batch must be 1..8" in _lib.last_error()
    rc = lib.sf_q4_gemv(None, None, 1, None, 1, None, None, 0, 1, 16, 100, 64, 0, None)
    assert rc == -1 and "in_features must be divisible by group_size" in _lib.last_error()


def test_gemm_workspace_and_validation():
    lib = _lib.load()
    assert lib.sf_q4_gemm_workspace_bytes(512, 4864, 896, 64) == 0      # 152 tiles: no split
    assert lib.sf_q4_gemm_workspace_bytes(512, 896, 4864, 64) > 0       # 28 tiles: split K
    assert lib.sf_q4_gemm_workspace_bytes(512, 896, 4848, 48) == 0      # group 48: VALU kernel
    rc = lib.sf_q4_gemm(None, None, 2, None, 2, None, None, 0, 4, 16, 96, 48, 0, None, 0, None)
    assert rc == -1 and "null pointer argument" in _lib.last_error()   # a valid shape
    rc = lib.sf_q4_gemm(None, None, 2, None, 2, None, None, 0, 4, 16, 96, 64, 0, None, 0, None)
    assert rc == -1 and "in_features must be divisible by group_size" in _lib.last_error()



def test_gemm_partials_splits_and_validation():
    """sf_q4_gemm_splits agrees with the workspace sizing (two or more splits
    exactly where sf_q4_gemm needs a workspace of splits x M x N floats);
    sf_q4_gemm_partials refuses an unsplit shape and sf_rmsnorm_partials bad
    arguments, before any launch."""
    lib = _lib.load()
    for M, N, K, g in ((512, 4864, 896, 64), (512, 896, 4864, 64), (512, 1152, 896, 64),
                       (512, 896, 896, 64), (16, 4096, 4096, 128), (9, 896, 4864, 32)):
        s = lib.sf_q4_gemm_splits(M, N, K, g)
        wsb = lib.sf_q4_gemm_workspace_bytes(M, N, K, g)
        assert s >= 1 and (s > 1) == (wsb > 0)
        assert s == 1 or wsb == s * M * N * 4
    assert lib.sf_q4_gemm_splits(512, 896, 4864, 64) == 8   # 28 tiles: split 8 ways
    assert lib.sf_q4_gemm_splits(512, 896, 4848, 48) == 0   # group 48: the VALU kernel
    assert lib.sf_q4_gemm_splits(512, 896, 4864, 0) == 0
    blob, x = 256 * 1024, 4096  # fake addresses: validation fails before any use
    rc = lib.sf_q4_gemm_partials(blob, x, 2, 512, 4864, 896, 64, 0, None, 0, None)
    assert rc == -1 and "runs unsplit" in _lib.last_error()
    rc = lib.sf_q4_gemm_partials(blob, x, 2, 512, 896, 4864, 64, 0, None, 0, None)
    assert rc == -1 and "workspace too small" in _lib.last_error()
    rc = lib.sf_rmsnorm_partials(None, None, 2, None, 0, None, 0, 4, 896, 1e-6, None)
    assert rc == -1 and "null pointer argument" in _lib.last_error()
    rc = lib.sf_rmsnorm_partials(x, x, 0, x, 0, x, 0, 4, 896, 1e-6, None)
    assert rc == -1 and "n_parts=0" in _lib.last_error()
    rope = lambda n, bdt: lib.sf_rope_kv_append_partials(x, n, x, bdt, x, x, 64, x, 1, x, x, x, x, 1,
                                                          4, 14, 2, 64, 64, None, 0, None)
    assert rope(0, _lib.SF_F32) == -1 and "n_parts=0" in _lib.last_error()
    assert rope(2, 7) == -1 and "bad bias dtype 7" in _lib.last_error()


def test_attention_validation_and_sizes():
    lib = _lib.load()
    acc = 14 * 256 * 64 * 4  # split acc, then (m, l) at the next 256-byte boundary
    assert lib.sf_attn_workspace_bytes(1, 14, 64, 256) == acc + 14 * 256 * 2 * 4
    assert lib.sf_attn_workspace_bytes(1, 14, 64, 3) == 10752 + 14 * 3 * 2 * 4
    rc = lib.sf_attn_decode_i8kv_partials_dev(None, 0, None, None, None, None, 1, None, 0, 1, 14, 2,
                                              None, 0, 16, 16, 64, 0.1, 1, None)
    assert rc == -1 and "null pointer" in _lib.last_error()
    rc = lib.sf_attn_decode_i8kv(None, 0, None, None, None, None, 1, None, 0, None, 0,
                                 1, 14, 2, 16, 16, 512, 0.1, 1, None)
    assert rc == -1 and "exceeds kernel's compile-time max 256" in _lib.last_error()
    rc = lib.sf_attn_decode_i8kv(None, 0, None, None, None, None, 1, None, 0, None, 0,
                                 1, 14, 3, 16, 16, 64, 0.1, 1, None)
    assert rc == -1 and "not a multiple" in _lib.last_error()
    assert lib.sf_attn_default_splits(1, 2, 16384) == 128
    assert lib.sf_attn_default_splits(1, 2, 4096) == 64
    assert lib.sf_attn_default_splits(1, 2, 100) == 1
    assert lib.sf_attn_default_splits(1, 2, 160) == 1 and lib.sf_attn_default_splits(1, 2, 161) == 8
    assert lib.sf_attn_default_splits_d(1, 2, 512, 64) == 16
    assert lib.sf_attn_default_splits_d(1, 2, 1024, 128) == 32
    assert lib.sf_attn_default_splits_d(1, 2, 2048, 64) == 64
    assert lib.sf_attn_default_splits_d(1, 2, 2049, 64) == 33
    assert lib.sf_attn_default_splits_d(1, 2, 4096, 128) == 64
    assert lib.sf_attn_default_splits_d(1, 2, 8192, 128) == 128


def test_kv_append_validation():
    lib = _lib.load()
    rc = lib.sf_kv_quant_append(None, None, 1, None, None, None, None, 1, 1, 2, 4, 10, 12, 64, None)
    assert rc == -1 and "overflow" in _lib.last_error()


def test_python_layer_raises_without_device():
    """No CPU fallback: on a host without a GPU the product refuses to compute."""
    import numpy as np
    import torch

    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from siliconfer_amd import kernels as K

    assert K.HIP_AVAILABLE is False
    W = np.random.default_rng(0).normal(0, 1, (16, 64)).astype(np.float32)
    pk, s = K.pack_weights_sym(W, 64)
    with pytest.raises(RuntimeError):
        K.gemv_sym(pk, s, np.ones(64, np.float32), 64)


def test_fused_gemv_rejects_bad_op_and_missing_norm_weight():
    lib = _lib.load()
    blob, src, y = 256 * 1024, 4096, 8192  # fake addresses: validation fails before any use
    args = lambda op, nw, K=256: (blob, src, op, nw, 1e-6, _lib.SF_F16, None, _lib.SF_F32, y, None,
                                  _lib.SF_F32, 64, K, 64, 0, None)
    assert lib.sf_q4_gemv_fused(*args(7, 4096)) == -1
    assert "fused op" in _lib.last_error()
    assert lib.sf_q4_gemv_fused(*args(_lib.SF_PRE_RMSNORM, None)) == -1
    assert "null pointer" in _lib.last_error()
    assert lib.sf_q4_gemv_fused(*args(_lib.SF_PRE_SILU_MUL, None, K=100)) == -1
    assert "divisible by group_size" in _lib.last_error()


def test_lm_head_rows_validation_and_sizes():
    lib = _lib.load()
    assert lib.sf_lm_head_rows_workspace_bytes(151936, 8) == 256 + 8 * 1024 * 8
    assert lib.sf_lm_head_rows_workspace_bytes(1000, 9) == 0
    w, x, tok, ws = 256 * 1024, 4096, 8192, 512 * 1024  # fake addresses: validation fails first
    big = 1 << 20
    args = lambda xdt, H, B, wsb=big: (w, x, xdt, None, 1000, H, B, tok, ws, wsb, None)
    assert lib.sf_lm_head_argmax_rows(*args(_lib.SF_F16, 896, 0)) == -1
    assert lib.sf_lm_head_argmax_rows(*args(_lib.SF_F16, 896, 9)) == -1
    assert "must be 1..8" in _lib.last_error()
    assert lib.sf_lm_head_argmax_rows(*args(_lib.SF_F32, 4096, 8)) == -2   # 128 KB of rows
    assert lib.sf_lm_head_argmax_rows(*args(_lib.SF_F16, 900, 2)) == -2    # not a multiple of 8
    assert lib.sf_lm_head_argmax_rows(*args(_lib.SF_F16, 896, 8, wsb=1024)) == -1
    assert "workspace too small" in _lib.last_error()
    assert lib.sf_lm_head_argmax_rows(*args(7, 896, 2)) == -1


def test_fused_rows_support_and_validation():
    lib = _lib.load()
    F16, F32, RMS, SILU = _lib.SF_F16, _lib.SF_F32, _lib.SF_PRE_RMSNORM, _lib.SF_PRE_SILU_MUL
    ok = lib.sf_q4_gemv_fused_rows_supported
    # config-5 verify shapes: the two RMSNorm folds run at every batch; the down
    # projection's activations (4864 per row, two 8-k pieces per thread of a
    # 10-wave plan) fit the LDS staging up to two rows
    for B in (1, 2, 3, 4, 5, 8):
        assert ok(RMS, B, 1152, 896, 64, 0, F16) == 1
        assert ok(RMS, B, 9728, 896, 64, 0, F16) == 1
        assert ok(SILU, B, 896, 4864, 64, 0, F16) == (B <= 2)
    assert ok(SILU, 4, 1152, 896, 64, 0, F16) == 1
    assert ok(RMS, 4, 1152, 896, 64, 0, F32) == 1          # fp32: high + low rows staged
    assert ok(RMS, 1, 1152, 896, 64, 0, F32) == 1
    assert ok(RMS, 1, 4096, 16384, 128, 0, F16) == 0       # 16 waves of 8 units: over the cap
    assert ok(7, 4, 1152, 896, 64, 0, F16) == 0
    blob, src, y = 256 * 1024, 4096, 8192  # fake addresses: validation fails before any use
    args = lambda B, op=RMS, N=1152, K=896: (blob, src, op, src, 1e-6, F16, None, F32, y, None,
                                             F32, B, N, K, 64, 0, None)
    assert lib.sf_q4_gemv_fused_rows(*args(9)) == -1
    assert lib.sf_q4_gemv_fused_rows(*args(5, SILU, 896, 4864)) == -2
    assert "run sf_rmsnorm" in _lib.last_error()


def test_attn_merge_fold_support_and_validation():
    """sf_q4_gemv_attn_merge: 2..8 splits, head_dim a multiple of 8, the GEMV's
    plans with at most four units per wave; everything else is refused before
    any launch."""
    lib = _lib.load()
    ok = lib.sf_q4_gemv_attn_merge_supported
    F16, BF16, F32 = _lib.SF_F16, _lib.SF_BF16, _lib.SF_F32
    for S in range(2, 9):
        for act in (F16, BF16, F32):
            assert ok(1, 896, 14, 64, S, 64, act) == 1, (S, act)   # the 0.5B o projection
    assert ok(1, 896, 14, 64, 1, 64, F16) == 0 and ok(1, 896, 14, 64, 9, 64, F16) == 0
    assert ok(1, 1024, 8, 128, 5, 128, BF16) == 1
    assert ok(1, 4096, 32, 128, 8, 128, F16) == 1                 # 7B: K = 4096
    assert ok(2, 896, 14, 64, 4, 64, F16) == 1
    assert ok(1, 896, 14, 60, 4, 60, F16) == 0                    # head_dim % 8
    assert ok(9, 896, 14, 64, 4, 64, F16) == 0
    assert ok(1, 896, 14, 64, 4, 48, F16) == 0                    # group size off the 32 grid
    blob = ws = 1 << 20  # never dereferenced: every call below fails its checks first
    rc = lib.sf_q4_gemv_attn_merge(blob, ws, 1 << 20, 9, 14, 64, F16, None, F32, ws, None, F32, 1,
                                   896, 64, 0, None)
    assert rc == -2 and "run sf_attn_decode_i8kv and sf_q4_gemv instead" in _lib.last_error()
    rc = lib.sf_q4_gemv_attn_merge(blob, ws, 256, 4, 14, 64, F16, None, F32, ws, None, F32, 1,
                                   896, 64, 0, None)
    assert rc == -1 and "workspace too small" in _lib.last_error()
    rc = lib.sf_q4_gemv_attn_merge(blob, ws + 16, 1 << 20, 4, 14, 64, F16, None, F32, ws, None,
                                   F32, 1, 896, 64, 0, None)
    assert rc == -1 and "256-byte aligned" in _lib.last_error()
    rc = lib.sf_attn_decode_i8kv_partials_dev(ws, 1, ws, ws, ws, ws, 1, ws, 1 << 20, 1, 14, 2, ws,
                                              0, 16, 16, 64, 0.1, 1, None)
    assert rc == -1 and "partials need 2..512 splits" in _lib.last_error()


def test_fused_rope_support():
    lib = _lib.load()
    ok = lib.sf_q4_gemv_fused_rope_supported
    # config 5 (hidden 896, 14/2 heads of 64): one 64-row head per workgroup
    for act in (_lib.SF_F16, _lib.SF_BF16, _lib.SF_F32):
        assert ok(1152, 896, 64, 14, 2, 64, act) == 1
    assert ok(512, 256, 64, 4, 2, 64, _lib.SF_F16) == 1
    assert ok(6144, 4096, 128, 32, 8, 128, _lib.SF_F16) == 0   # 7B: head_dim 128
    assert ok(1000, 896, 64, 14, 2, 64, _lib.SF_F16) == 0      # N != (H + 2 KVH) D
    rc = lib.sf_q4_gemv_fused_rope(256 * 1024, 4096, 4096, 1e-6, _lib.SF_F16, None, _lib.SF_F32,
                                   4096, 4096, 64, 4096, _lib.SF_F16, 4096, 4096, 4096, 4096,
                                   _lib.SF_F16, 32, 8, 128, 64, 4096, 6144, 4096, 128, 0, None)
    assert rc == -2 and "sf_rope_kv_append instead" in _lib.last_error()
