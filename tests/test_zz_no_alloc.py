"""sf_attn_decode_i8kv_noalloc — decode attention that allocates nothing — through
the C ABI against sf_attn_decode_i8kv with a caller-provided workspace: the same
kernels and split count give the same bits, on several calls in a row with
shrinking inputs (the fixed scratch keeps the previous call's contents), and
both stay within the 2e-3 attention bar against the oracle. A shape whose
workspace exceeds the fixed scratch is refused with SF_EINVAL."""

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle.linear import assert_close
from siliconfer_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(rng, B, H, KVH, D, T):
    q = rng.normal(0, 1, (B, H, D)).astype(np.float16)
    kc, ks = A.quantize_kv(rng.normal(0, 1, (B, KVH, T, D)).astype(np.float32))
    vc, vs = A.quantize_kv(rng.normal(0, 1, (B, KVH, T, D)).astype(np.float32))
    return q, kc, ks[..., 0].astype(np.float16), vc, vs[..., 0].astype(np.float16)


def _run(dev, lib, noalloc, q, kc, ks, vc, vs, n_splits):
    t = lambda a: torch.as_tensor(np.ascontiguousarray(a)).to(dev)
    qd, kcd, ksd, vcd, vsd = t(q), t(kc), t(ks), t(vc), t(vs)
    B, H, D = q.shape
    KVH, T = kc.shape[1], kc.shape[2]
    out = torch.full((B, H, D), float("nan"), dtype=torch.float32, device=dev)
    st = _lib.stream(qd)
    F16, F32 = _lib.SF_F16, _lib.SF_F32
    if noalloc:
        rc = lib.sf_attn_decode_i8kv_noalloc(qd.data_ptr(), F16, kcd.data_ptr(), ksd.data_ptr(),
                                             vcd.data_ptr(), vsd.data_ptr(), F16, out.data_ptr(), F32,
                                             B, H, KVH, T, T, D, D ** -0.5, n_splits, st)
    else:
        nb = lib.sf_attn_workspace_bytes(B, H, D, n_splits or lib.sf_attn_default_splits_d(B, KVH, T, D))
        ws = torch.zeros(max(nb, 1 << 16), dtype=torch.uint8, device=dev)
        rc = lib.sf_attn_decode_i8kv(qd.data_ptr(), F16, kcd.data_ptr(), ksd.data_ptr(),
                                     vcd.data_ptr(), vsd.data_ptr(), F16, out.data_ptr(), F32,
                                     ws.data_ptr(), ws.numel(), B, H, KVH, T, T, D, D ** -0.5,
                                     n_splits, st)
    _lib.check(rc, "noalloc" if noalloc else "workspace")
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("order", ["large_first", "small_first"])
def test_noalloc_matches_workspace_entry_point(dev, order):
    lib = _lib.load()
    cases = [(1, 14, 2, 64, 16384, 0), (1, 14, 2, 64, 4096, 0), (2, 14, 2, 64, 777, 5),
             (1, 14, 2, 64, 300, 0)]  # config 4 at both lengths, then smaller inputs
    if order == "small_first":
        cases = cases[::-1]
    for i, (B, H, KVH, D, T, S) in enumerate(cases):
        rng = np.random.default_rng(100 + i)
        inp = _inputs(rng, B, H, KVH, D, T)
        a = _run(dev, lib, True, *inp, S)
        b = _run(dev, lib, False, *inp, S)
        assert torch.equal(a, b), f"noalloc differs from the workspace call at {B, H, KVH, D, T, S}"
        q, kc, ks, vc, vs = inp
        ref = A.attention_decode(q.astype(np.float64), kc, ks.astype(np.float64), vc,
                                 vs.astype(np.float64))
        assert_close(a.numpy(), ref, 2e-3, f"noalloc T={T}")


def test_noalloc_refuses_shapes_beyond_its_scratch(dev):
    lib = _lib.load()
    cap = lib.sf_attn_noalloc_max_bytes()
    assert cap == 4 << 20
    B, H, KVH, D, T, S = 8, 32, 8, 128, 2048, 64
    assert lib.sf_attn_workspace_bytes(B, H, D, S) > cap
    rc = lib.sf_attn_decode_i8kv_noalloc(None, _lib.SF_F16, None, None, None, None, _lib.SF_F16,
                                         None, _lib.SF_F32, B, H, KVH, T, T, D, 0.1, S, None)
    assert rc == -1 and "more than its fixed" in _lib.last_error()
