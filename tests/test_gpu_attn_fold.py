"""The decode attention's split merge folded into the o projection
(sf_q4_gemv_attn_merge over the partials of sf_attn_decode_i8kv_partials_dev)
against the same attention with its merge launch (sf_attn_decode_i8kv_dev
writing an act-dtype output) followed by the plain GEMV: bit for bit, on both
decode kernels. The merged attention itself is checked against the oracle
(float64 dequantize-then-softmax, 2e-3 relative plus the output dtype's
rounding)."""

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle.linear import assert_close
from siliconfer_amd import _lib
from test_gpu_fused import make_weight, st

pytestmark = pytest.mark.gpu
F32 = _lib.SF_F32
TOL = {torch.float32: 2e-3, torch.float16: 3e-3, torch.bfloat16: 1.2e-2}


@pytest.fixture(params=["mfma", "valu"])
def kernel_choice(request, monkeypatch):
    monkeypatch.setenv("SF_ATTN_MFMA", "1" if request.param == "mfma" else "0")
    return request.param


def cache(dev, rng, B, KVH, T_cap, D):
    k = rng.normal(0, 1, (B, KVH, T_cap, D)).astype(np.float32)
    v = rng.normal(0, 1, (B, KVH, T_cap, D)).astype(np.float32)
    kc, ks = A.quantize_kv(k)
    vc, vs = A.quantize_kv(v)
    ks, vs = ks.astype(np.float16), vs.astype(np.float16)
    t = lambda a: torch.as_tensor(a).to(dev).contiguous()
    return (kc, ks, vc, vs), (t(kc), t(ks), t(vc), t(vs))


def fold_and_reference(lib, dev, q, kv, B, H, KVH, D, T, T_cap, S, w, act, ws1=None):
    """(fold output, merged attention, attention + GEMV output); ws1: the
    fold's workspace (default: a new one)."""
    kcd, ksd, vcd, vsd = kv
    N = w.out_features
    T_dev = torch.tensor([T], dtype=torch.int32, device=dev)
    scale = float(D ** -0.5)
    wsb = lib.sf_attn_workspace_bytes(B, H, D, S)
    # workspaces start as NaN bytes: nothing may read what a split did not write
    if ws1 is None:
        ws1 = torch.full((wsb,), 0xFF, dtype=torch.uint8, device=dev)
    assert ws1.numel() >= wsb
    ws2 = torch.full((wsb,), 0xFF, dtype=torch.uint8, device=dev)
    kvp = (q.data_ptr(), _lib.dt(q), kcd.data_ptr(), ksd.data_ptr(), vcd.data_ptr(), vsd.data_ptr(),
           _lib.SF_F16)
    y_fold = torch.empty((B, N), dtype=torch.float32, device=dev)
    _lib.check(lib.sf_attn_decode_i8kv_partials_dev(*kvp, ws1.data_ptr(), ws1.numel(), B, H, KVH,
                                                     T_dev.data_ptr(), 0, T_cap, T_cap, D, scale, S,
                                                     st()), "sf_attn_decode_i8kv_partials_dev")
    _lib.check(lib.sf_q4_gemv_attn_merge(w.blob.data_ptr(), ws1.data_ptr(), ws1.numel(), S, H, D,
                                         _lib._DT[act], None, F32, y_fold.data_ptr(), None, F32, B,
                                         N, w.group_size, int(w.has_zeros), st()),
               "sf_q4_gemv_attn_merge")
    attn = torch.empty((B, H, D), dtype=act, device=dev)
    _lib.check(lib.sf_attn_decode_i8kv_dev(*kvp, attn.data_ptr(), _lib.dt(attn), ws2.data_ptr(), wsb,
                                           B, H, KVH, T_dev.data_ptr(), 0, T_cap, T_cap, D, scale, S,
                                           st()), "sf_attn_decode_i8kv_dev")
    y_ref = torch.empty((B, N), dtype=torch.float32, device=dev)
    _lib.check(lib.sf_q4_gemv(w.blob.data_ptr(), attn.data_ptr(), _lib.dt(attn), None, F32,
                              y_ref.data_ptr(), None, F32, B, N, H * D, w.group_size,
                              int(w.has_zeros), st()), "sf_q4_gemv")
    torch.cuda.synchronize()
    return y_fold, attn, y_ref


# (B, H, KVH, D, T, T_cap, S, N, g, asym)
CASES = [
    (1, 14, 2, 64, 700, 768, 6, 896, 64, False),   # the 0.5B decoder at a 768-token cache
    (1, 14, 2, 64, 1, 768, 6, 896, 64, True),      # one token: five empty splits
    (1, 14, 2, 64, 40, 64, 2, 896, 64, True),
    (1, 14, 2, 64, 1000, 1024, 8, 896, 128, False),
    (1, 8, 2, 128, 333, 512, 5, 1024, 128, True),  # head_dim 128
    (1, 20, 1, 64, 150, 256, 3, 300, 64, False),   # 20 heads per kv head: the VALU kernel
    (2, 14, 2, 64, 100, 128, 3, 896, 64, True),    # two rows
]


@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,H,KVH,D,T,T_cap,S,N,g,asym", CASES)
def test_fold_equals_attention_then_gemv(dev, kernel_choice, act, B, H, KVH, D, T, T_cap, S, N,
                                         g, asym):
    lib = _lib.load()
    assert lib.sf_q4_gemv_attn_merge_supported(B, N, H, D, S, g, _lib._DT[act]) == 1
    rng = np.random.default_rng(1000 + T + S)
    (kc, ks, vc, vs), kv = cache(dev, rng, B, KVH, T_cap, D)
    qn = rng.normal(0, 1, (B, H, D)).astype(np.float32)
    q = torch.as_tensor(qn).to(dev).to(act)
    w = make_weight(dev, N, H * D, g, asym, seed=T + 7)[0]
    y_fold, attn, y_ref = fold_and_reference(lib, dev, q, kv, B, H, KVH, D, T, T_cap, S, w, act)
    assert torch.equal(y_fold, y_ref), (y_fold - y_ref).abs().max().item()
    # the merged attention (the GEMV's input) against the oracle
    qa = q.float().cpu().numpy()
    ref = A.attention_decode(qa, kc, ks.astype(np.float64), vc, vs.astype(np.float64),
                             scale=float(D ** -0.5), T=T)
    assert_close(attn.float().cpu().numpy(), ref, TOL[act], f"merged attention T={T} S={S}")


def test_fold_reuses_workspace_across_calls(dev):
    """Two folds in a row on one workspace, the second over a shorter cache and
    fewer splits: each reads only what its own attention launch wrote."""
    lib = _lib.load()
    rng = np.random.default_rng(5)
    (_, _, _, _), kv = cache(dev, rng, 1, 2, 768, 64)
    w = make_weight(dev, 896, 896, 64, True, seed=3)[0]
    q = torch.as_tensor(rng.normal(0, 1, (1, 14, 64)).astype(np.float16)).to(dev)
    ws = torch.full((lib.sf_attn_workspace_bytes(1, 14, 64, 8),), 0xFF, dtype=torch.uint8,
                    device=dev)
    for T, S in ((760, 8), (65, 2)):
        y_fold, _, y_ref = fold_and_reference(lib, dev, q, kv, 1, 14, 2, 64, T, 768, S, w,
                                              torch.float16, ws1=ws)
        assert torch.equal(y_fold, y_ref), (T, S)
