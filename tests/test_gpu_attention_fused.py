"""GPU checks of the one-launch decode attention (sf_attn_decode_i8kv_fused)
through the C ABI: bit for bit equal to the two-launch call
(sf_attn_decode_i8kv: split partials, then the merge launch) on the same
inputs, across shapes, split counts, repeated calls and graph replays on one
workspace, and the bounded poll: a split that publishes nothing (host test
hook) makes every waiting workgroup give up, write NaN and set the error word.
Parity with the oracle is covered through attention_decode
(tests/test_gpu_attention.py), which runs this entry point.
"""

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle.linear import assert_close
from siliconfer_amd import _lib

pytestmark = pytest.mark.gpu


def inputs(dev, B, H, KVH, T, D, seed=0):
    rng = np.random.default_rng(seed)
    q = rng.normal(0, 1, (B, H, D)).astype(np.float16)
    kc, ks = A.quantize_kv(rng.normal(0, 1, (B, KVH, T, D)).astype(np.float32))
    vc, vs = A.quantize_kv(rng.normal(0, 1, (B, KVH, T, D)).astype(np.float32))
    t = lambda a: torch.as_tensor(np.ascontiguousarray(a)).to(dev)
    return (t(q), t(kc), t(ks.reshape(B, KVH, T).astype(np.float16)), t(vc),
            t(vs.reshape(B, KVH, T).astype(np.float16)))


def two_launch(dev, q, kc, ks, vc, vs, S):
    lib = _lib.load()
    B, H, D = q.shape
    KVH, T = kc.shape[1], kc.shape[2]
    out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    nb = lib.sf_attn_workspace_bytes(B, H, D, S)
    ws = torch.empty(max(nb, 256), dtype=torch.uint8, device=dev)
    _lib.check(lib.sf_attn_decode_i8kv(q.data_ptr(), _lib.SF_F16, kc.data_ptr(), ks.data_ptr(),
                                       vc.data_ptr(), vs.data_ptr(), _lib.SF_F16, out.data_ptr(),
                                       _lib.SF_F32, ws.data_ptr(), nb, B, H, KVH, T, T, D, 0.125,
                                       S, _lib.stream(q)), "sf_attn_decode_i8kv")
    return out


def fused(q, kc, ks, vc, vs, S, ws, out, spin_cap=0, drop=-1, T=None):
    lib = _lib.load()
    B, H, D = q.shape
    KVH, T_cap = kc.shape[1], kc.shape[2]
    _lib.check(lib.sf_attn_decode_i8kv_fused(q.data_ptr(), _lib.SF_F16, kc.data_ptr(), ks.data_ptr(),
                                             vc.data_ptr(), vs.data_ptr(), _lib.SF_F16, out.data_ptr(),
                                             _lib.SF_F32, ws.data_ptr(), ws.numel(), B, H, KVH,
                                             T_cap if T is None else T, T_cap, D, 0.125, S, spin_cap,
                                             drop, _lib.stream(q)), "sf_attn_decode_i8kv_fused")
    return out


def fresh_ws(dev, B, H, D, S):
    return torch.zeros(_lib.load().sf_attn_fused_workspace_bytes(B, H, D, S), dtype=torch.uint8,
                       device=dev)


def error_word(ws):
    import ctypes

    v = ctypes.c_int(-1)
    _lib.check(_lib.load().sf_attn_fused_error(ws.data_ptr(), ctypes.addressof(v), _lib.stream(ws)),
               "sf_attn_fused_error")
    return v.value


@pytest.mark.parametrize("B,H,KVH,T,D,S", [
    (1, 14, 2, 4096, 64, 32),     # config 4, default splits
    (1, 14, 2, 16384, 64, 64),
    (1, 14, 2, 1000, 64, 3),      # a ragged last split, merge slices of 150 outputs
    (1, 14, 2, 4096, 64, 128),    # splits of one tile: a tree span over 64, two launches
    (2, 8, 1, 700, 128, 31),      # batch 2, head_dim 128, merge slices over two heads
    (1, 16, 1, 2048, 128, 16),    # 16 heads per kv head: a merge slice past the poll limit, two launches
    (1, 4, 4, 300, 64, 7),        # MHA
])
def test_fused_equals_two_launches_bitwise(dev, B, H, KVH, T, D, S):
    q, kc, ks, vc, vs = inputs(dev, B, H, KVH, T, D, seed=T + S)
    ref = two_launch(dev, q, kc, ks, vc, vs, S)
    ws = fresh_ws(dev, B, H, D, S)
    out = torch.empty_like(ref)
    for _ in range(3):  # the group counters advance: every call stays exact
        out.fill_(7.0)
        fused(q, kc, ks, vc, vs, S, ws, out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    assert error_word(ws) == 0
    o = A.attention_decode(q.float().cpu().numpy(), kc.cpu().numpy(),
                           ks.float().cpu().numpy().astype(np.float64), vc.cpu().numpy(),
                           vs.float().cpu().numpy().astype(np.float64), scale=0.125)
    assert_close(out.cpu().numpy(), o, 2e-3, "fused attention vs oracle")


def test_one_workspace_across_split_counts_and_lengths(dev):
    """Calls with other split counts, cache lengths and shapes in between
    leave stale words of older tags behind; none is taken for a new one."""
    B, H, KVH, D, T = 1, 14, 2, 64, 4096
    q, kc, ks, vc, vs = inputs(dev, B, H, KVH, T, D, seed=3)
    ws = fresh_ws(dev, B, H, D, 128)
    out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    for S, Tv in ((32, 4096), (64, 4096), (16, 1000), (128, 4096), (32, 2500), (2, 64)):
        ref = two_launch(dev, q[:, :, :], kc[:, :, :Tv].contiguous(), ks[:, :, :Tv].contiguous(),
                         vc[:, :, :Tv].contiguous(), vs[:, :, :Tv].contiguous(), S)
        fused(q, kc[:, :, :Tv].contiguous(), ks[:, :, :Tv].contiguous(), vc[:, :, :Tv].contiguous(),
              vs[:, :, :Tv].contiguous(), S, ws, out)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (S, Tv)
    assert error_word(ws) == 0


def test_graph_replays_advance_the_tag(dev):
    """One captured call replayed several times, eager calls and new inputs
    between the replays: each replay's output equals the two-launch call."""
    B, H, KVH, D, T, S = 1, 14, 2, 64, 4096, 32
    q, kc, ks, vc, vs = inputs(dev, B, H, KVH, T, D, seed=5)
    ws = fresh_ws(dev, B, H, D, S)
    out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    s = torch.cuda.Stream(dev)
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=s):
        fused(q, kc, ks, vc, vs, S, ws, out)
    rng = np.random.default_rng(9)
    for r in range(4):
        q.copy_(torch.as_tensor(rng.normal(0, 1, q.shape).astype(np.float16)).to(dev))
        ref = two_launch(dev, q, kc, ks, vc, vs, S)
        out.fill_(-1.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), r
        eager = torch.empty_like(out)
        fused(q, kc, ks, vc, vs, S, ws, eager)  # an eager call on the same workspace
        torch.cuda.synchronize()
        assert torch.equal(eager, ref), r
    assert error_word(ws) == 0


def test_dropped_split_gives_up_with_error_then_recovers(dev):
    """The host makes one split publish nothing: every workgroup's bounded
    poll gives up (64 rounds), the outputs are NaN and the error word is set.
    The next call on the same workspace (new tag) is exact again."""
    B, H, KVH, D, T, S = 1, 14, 2, 64, 4096, 32
    q, kc, ks, vc, vs = inputs(dev, B, H, KVH, T, D, seed=11)
    ref = two_launch(dev, q, kc, ks, vc, vs, S)
    ws = fresh_ws(dev, B, H, D, S)
    out = torch.empty_like(ref)
    fused(q, kc, ks, vc, vs, S, ws, out, spin_cap=64, drop=5)
    torch.cuda.synchronize()
    assert error_word(ws) == 1
    assert torch.isnan(out).all()
    ws[:4].zero_()
    fused(q, kc, ks, vc, vs, S, ws, out)
    torch.cuda.synchronize()
    assert error_word(ws) == 0
    assert torch.equal(out, ref)
