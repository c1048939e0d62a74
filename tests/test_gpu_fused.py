"""Folded producers of the decode step, through the C ABI: the GEMV with the
RMSNorm or SwiGLU of its input folded into the activation load
(sf_q4_gemv_fused) and the lm_head with the final RMSNorm folded in
(sf_lm_head_argmax_rmsnorm) against the unfused sequence (sf_rmsnorm /
sf_silu_mul into an activation buffer, then sf_q4_gemv / sf_lm_head_argmax).
The contract is bit-identity with that sequence, and through it the oracle
(layers.py:14-21, 143-144 of /root/reference/siliconfer/model, then the
q4 GEMV of kernels/neon/q4_gemv.cpp) at the GEMV tolerance.
"""

import numpy as np
import pytest
import torch

from oracle import linear
from oracle import model as OM
from oracle import primitives as P
from siliconfer_amd import _lib
from siliconfer_amd.kernels import Q4Weight

pytestmark = pytest.mark.gpu
SF_EUNSUPPORTED = -2  # include/siliconfer_hip.h
F32, F16, BF16 = _lib.SF_F32, _lib.SF_F16, _lib.SF_BF16
ACTS = [torch.float16, torch.bfloat16, torch.float32]


def st():
    return torch.cuda.current_stream().cuda_stream


def make_weight(dev, N, K, g, asym, seed):
    rng = np.random.default_rng(seed)
    W = rng.normal(0.01 if asym else 0, 0.02, (N, K)).astype(np.float32)
    if asym:
        pk, s, z = P.pack_weights_asym(W, g)
    else:
        (pk, s), z = P.pack_weights_sym(W, g), None
    return Q4Weight(pk, s, z, g, device=dev), pk, s, z


def gemv(lib, w, x, bias=None):
    y = torch.empty((1, w.out_features), dtype=torch.float32, device=x.device)
    _lib.check(lib.sf_q4_gemv(w.blob.data_ptr(), x.data_ptr(), _lib.dt(x), None, F32, y.data_ptr(),
                              None if bias is None else bias.data_ptr(), F32, 1, w.out_features,
                              w.in_features, w.group_size, int(w.has_zeros), st()), "sf_q4_gemv")
    return y


def fused(lib, w, src, op, norm_w, act, bias=None, eps=1e-6):
    y = torch.empty((1, w.out_features), dtype=torch.float32, device=src.device)
    _lib.check(lib.sf_q4_gemv_fused(w.blob.data_ptr(), src.data_ptr(), op,
                                    None if norm_w is None else norm_w.data_ptr(), eps,
                                    _lib._DT[act],
                                    None, F32, y.data_ptr(), None if bias is None else bias.data_ptr(),
                                    F32, w.out_features, w.in_features, w.group_size,
                                    int(w.has_zeros), st()), "sf_q4_gemv_fused")
    return y


SHAPES = [(1152, 896, 64, False), (4864, 896, 64, True), (96, 4096, 128, False),
          (40, 96, 32, True), (300, 8192, 128, True)]


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("N,K,g,asym", SHAPES)
def test_rmsnorm_gemv_equals_rmsnorm_then_gemv(dev, act, N, K, g, asym):
    lib = _lib.load()
    w, pk, s, z = make_weight(dev, N, K, g, asym, N + K)
    rng = np.random.default_rng(K)
    h = torch.as_tensor(rng.normal(0, 2, (1, K)).astype(np.float32)).to(dev)
    nw = torch.as_tensor(rng.normal(1, 0.1, K).astype(np.float32)).to(dev)
    bias = torch.as_tensor(rng.normal(0, 1, N).astype(np.float32)).to(dev)
    xn = torch.empty((1, K), dtype=act, device=dev)
    _lib.check(lib.sf_rmsnorm(h.data_ptr(), None, nw.data_ptr(), F32, xn.data_ptr(), _lib.dt(xn), 1,
                              K, 1e-6, st()), "sf_rmsnorm")
    ref = gemv(lib, w, xn, bias)
    got = fused(lib, w, h, _lib.SF_PRE_RMSNORM, nw, act, bias)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())
    # and the oracle: rmsnorm in fp32, the activation rounded to act, the GEMV
    xo = OM.rmsnorm(h.cpu().numpy(), nw.cpu().numpy(), 1e-6)
    xo = torch.as_tensor(xo).to(act).float().numpy().astype(np.float64)
    exp = linear.gemv(pk, s.astype(np.float16).astype(np.float64), xo, g, zeros=z) + bias.cpu().numpy()
    linear.assert_close(got.cpu().numpy(), exp, 2e-3 if act == torch.bfloat16 else 1e-3,
                        f"rmsnorm-gemv {act}")


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("N,K,g,asym", SHAPES)
def test_silu_gemv_equals_silu_then_gemv(dev, act, N, K, g, asym):
    lib = _lib.load()
    w, pk, s, z = make_weight(dev, N, K, g, asym, N * 3 + K)
    rng = np.random.default_rng(K + 1)
    gu = torch.as_tensor(rng.normal(0, 3, (1, 2 * K)).astype(np.float32)).to(dev)
    a = torch.empty((1, K), dtype=act, device=dev)
    _lib.check(lib.sf_silu_mul(gu.data_ptr(), a.data_ptr(), _lib.dt(a), 1, K, st()), "sf_silu_mul")
    ref = gemv(lib, w, a)
    got = fused(lib, w, gu, _lib.SF_PRE_SILU_MUL, None, act)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())
    g64 = gu.cpu().numpy().astype(np.float64)
    xo = g64[:, :K] / (1 + np.exp(-g64[:, :K])) * g64[:, K:]
    xo = torch.as_tensor(xo.astype(np.float32)).to(act).float().numpy().astype(np.float64)
    exp = linear.gemv(pk, s.astype(np.float16).astype(np.float64), xo, g, zeros=z)
    linear.assert_close(got.cpu().numpy(), exp, 2e-3 if act == torch.bfloat16 else 1e-3,
                        f"silu-gemv {act}")


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("V,H", [(151936, 896), (1000, 64), (5000, 1600)])
def test_lm_head_rmsnorm_equals_rmsnorm_then_lm_head(dev, act, V, H):
    lib = _lib.load()
    rng = np.random.default_rng(V + H)
    Wt = torch.as_tensor(rng.normal(0, 0.02, (V, H)).astype(np.float32)).to(dev).to(torch.bfloat16)
    h = torch.as_tensor(rng.normal(0, 2, H).astype(np.float32)).to(dev)
    nw = torch.as_tensor(rng.normal(1, 0.1, H).astype(np.float32)).to(dev)
    outs = []
    for fold in (False, True):
        logits = torch.empty(V, dtype=torch.float32, device=dev)
        tok = torch.zeros(1, dtype=torch.int32, device=dev)
        pos = torch.tensor([2], dtype=torch.int32, device=dev)
        hist = torch.full((4,), -1, dtype=torch.int32, device=dev)
        ws = torch.zeros(lib.sf_lm_head_workspace_bytes(V), dtype=torch.uint8, device=dev)
        if fold:
            _lib.check(lib.sf_lm_head_argmax_rmsnorm(
                Wt.data_ptr(), h.data_ptr(), nw.data_ptr(), 1e-6, _lib._DT[act], logits.data_ptr(), V,
                H, tok.data_ptr(), pos.data_ptr(), hist.data_ptr(), ws.data_ptr(), ws.numel(), st()),
                "sf_lm_head_argmax_rmsnorm")
        else:
            xn = torch.empty(H, dtype=act, device=dev)
            _lib.check(lib.sf_rmsnorm(h.data_ptr(), None, nw.data_ptr(), F32, xn.data_ptr(),
                                      _lib.dt(xn), 1, H, 1e-6, st()), "sf_rmsnorm")
            _lib.check(lib.sf_lm_head_argmax(Wt.data_ptr(), xn.data_ptr(), _lib.dt(xn),
                                             logits.data_ptr(), V, H, tok.data_ptr(), pos.data_ptr(),
                                             hist.data_ptr(), ws.data_ptr(), ws.numel(), st()),
                       "sf_lm_head_argmax")
        torch.cuda.synchronize()
        assert int(ws[:256].count_nonzero()) == 0
        outs.append((logits.cpu(), int(tok.item()), int(pos.item()), hist.cpu()))
    (l0, t0, p0, h0), (l1, t1, p1, h1) = outs
    assert torch.equal(l0, l1) and t0 == t1 and p0 == p1 == 3 and torch.equal(h0, h1)
    assert int(h1[2]) == t1


@pytest.mark.parametrize("act", [torch.float16, torch.bfloat16])
def test_many_rows_round_like_the_unfolded_path(dev, act):
    """Rows whose normalised values sit next to an fp16 / bf16 rounding
    boundary: the folded kernels must round the fp32 product exactly like
    sf_rmsnorm (fp32 product, then one conversion), not as one fused
    multiply-and-round. 96 random rows of 256 values cover many such cases."""
    lib = _lib.load()
    V, H = 512, 256
    rng = np.random.default_rng(77)
    Wt = torch.as_tensor(rng.normal(0, 0.02, (V, H)).astype(np.float32)).to(dev).to(torch.bfloat16)
    w, *_ = make_weight(dev, 64, H, 64, False, 78)
    ws = torch.zeros(lib.sf_lm_head_workspace_bytes(V), dtype=torch.uint8, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    for r in range(96):
        h = torch.as_tensor(rng.normal(0, 10 ** rng.uniform(-1, 1), (1, H)).astype(np.float32)).to(dev)
        nw = torch.as_tensor(rng.normal(1, 0.3, H).astype(np.float32)).to(dev)
        xn = torch.empty((1, H), dtype=act, device=dev)
        _lib.check(lib.sf_rmsnorm(h.data_ptr(), None, nw.data_ptr(), F32, xn.data_ptr(), _lib.dt(xn), 1,
                                  H, 1e-6, st()), "sf_rmsnorm")
        l0 = torch.empty(V, dtype=torch.float32, device=dev)
        l1 = torch.empty(V, dtype=torch.float32, device=dev)
        _lib.check(lib.sf_lm_head_argmax(Wt.data_ptr(), xn.data_ptr(), _lib.dt(xn), l0.data_ptr(), V, H,
                                         tok.data_ptr(), None, None, ws.data_ptr(), ws.numel(), st()),
                   "sf_lm_head_argmax")
        _lib.check(lib.sf_lm_head_argmax_rmsnorm(Wt.data_ptr(), h.data_ptr(), nw.data_ptr(), 1e-6,
                                                 _lib._DT[act], l1.data_ptr(), V, H, tok.data_ptr(),
                                                 None, None, ws.data_ptr(), ws.numel(), st()),
                   "sf_lm_head_argmax_rmsnorm")
        y0 = gemv(lib, w, xn)
        y1 = fused(lib, w, h, _lib.SF_PRE_RMSNORM, nw, act)
        torch.cuda.synchronize()
        assert torch.equal(l0, l1), f"lm_head row {r}"
        assert torch.equal(y0, y1), f"gemv row {r}"


# ------------------------------------------------------------------ batch rows
def gemv_rows(lib, w, x, y32, bias=None):
    B = x.shape[0]
    _lib.check(lib.sf_q4_gemv(w.blob.data_ptr(), x.data_ptr(), _lib.dt(x), None, F32, y32.data_ptr(),
                              None if bias is None else bias.data_ptr(), F32, B, w.out_features,
                              w.in_features, w.group_size, int(w.has_zeros), st()), "sf_q4_gemv")


def fused_rows(lib, w, src, op, norm_w, B, y32, bias=None, eps=1e-6):
    _lib.check(lib.sf_q4_gemv_fused_rows(
        w.blob.data_ptr(), src.data_ptr(), op, None if norm_w is None else norm_w.data_ptr(), eps,
        F16, None, F32, y32.data_ptr(), None if bias is None else bias.data_ptr(), F32, B,
        w.out_features, w.in_features, w.group_size, int(w.has_zeros), st()), "sf_q4_gemv_fused_rows")


# config-5 verify shapes (qkv, gate_up with four tiles per wave, down) and 7B ones
ROW_SHAPES = [(1152, 896, 64, False), (9728, 896, 64, True), (896, 4864, 64, False),
              (4096, 4096, 128, False), (11008, 4096, 128, True), (96, 4096, 128, False)]


@pytest.mark.parametrize("B", [3, 5, 8])
@pytest.mark.parametrize("N,K,g,asym", ROW_SHAPES)
@pytest.mark.parametrize("op", [_lib.SF_PRE_RMSNORM, _lib.SF_PRE_SILU_MUL])
def test_fused_rows_equal_separate_kernels(dev, B, N, K, g, asym, op):
    """sf_q4_gemv_fused_rows == sf_rmsnorm / sf_silu_mul then sf_q4_gemv, bit
    for bit, with an [N] bias and with the per-row residual (bias = y_f32).
    Where the folded kernels have no plan for the shape, the entry point
    refuses it with SF_EUNSUPPORTED before launching anything, and the
    separate kernels that callers run instead meet the oracle."""
    lib = _lib.load()
    supported = bool(lib.sf_q4_gemv_fused_rows_supported(op, B, N, K, g, int(asym), F16))
    w, pk, s, z = make_weight(dev, N, K, g, asym, N + K + B)
    rng = np.random.default_rng(N * B + op)
    rms = op == _lib.SF_PRE_RMSNORM
    src = torch.as_tensor(rng.normal(0, 2, (B, K if rms else 2 * K)).astype(np.float32)).to(dev)
    nw = torch.as_tensor(rng.normal(1, 0.1, K).astype(np.float32)).to(dev) if rms else None
    bias = torch.as_tensor(rng.normal(0, 1, N).astype(np.float32)).to(dev)
    xn = torch.empty((B, K), dtype=torch.float16, device=dev)
    if rms:
        _lib.check(lib.sf_rmsnorm(src.data_ptr(), None, nw.data_ptr(), F32, xn.data_ptr(), F16, B, K,
                                  1e-6, st()), "sf_rmsnorm")
    else:
        _lib.check(lib.sf_silu_mul(src.data_ptr(), xn.data_ptr(), F16, B, K, st()), "sf_silu_mul")
    ref = torch.empty((B, N), device=dev)
    got = torch.empty((B, N), device=dev)
    gemv_rows(lib, w, xn, ref, bias)
    if not supported:
        sentinel = torch.full((B, N), 7.0, device=dev)
        rc = lib.sf_q4_gemv_fused_rows(
            w.blob.data_ptr(), src.data_ptr(), op, None if nw is None else nw.data_ptr(), 1e-6, F16, None,
            F32, sentinel.data_ptr(), bias.data_ptr(), F32, B, N, K, g, int(asym), st())
        torch.cuda.synchronize()
        assert rc == SF_EUNSUPPORTED and "LDS staging" in _lib.last_error(), (rc, _lib.last_error())
        assert bool((sentinel == 7.0).all()), "a refused call wrote its output"
        exp = linear.gemv(pk, s.astype(np.float16).astype(np.float64),
                          xn.float().cpu().numpy().astype(np.float64), g, zeros=z) + bias.cpu().numpy()
        linear.assert_close(ref.cpu().numpy(), exp, 1e-3, f"separate kernels op={op} B={B}")
        return
    fused_rows(lib, w, src, op, nw, B, got, bias)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    # per-row residual: y = y_old + W x, each row its own y_old
    old = torch.as_tensor(rng.normal(0, 1, (B, N)).astype(np.float32)).to(dev)
    ref2, got2 = old.clone(), old.clone()
    gemv_rows(lib, w, xn, ref2, ref2)
    fused_rows(lib, w, src, op, nw, B, got2, got2)
    torch.cuda.synchronize()
    assert torch.equal(got2, ref2)
    plain = torch.empty((B, N), device=dev)
    gemv_rows(lib, w, xn, plain)
    torch.cuda.synchronize()
    assert torch.equal(ref2, plain + old)
    # and the oracle on the rounded activations
    exp = linear.gemv(pk, s.astype(np.float16).astype(np.float64),
                      xn.float().cpu().numpy().astype(np.float64), g, zeros=z) + bias.cpu().numpy()
    linear.assert_close(got.cpu().numpy(), exp, 1e-3, f"fused rows op={op} B={B}")


@pytest.mark.parametrize("B,K", [(1, 512), (2, 512), (4, 512), (4, 8192)])
def test_residual_bias_alias(dev, B, K):
    """bias = y_f32 adds each row's own previous value: fp16 activations, and
    fp32 ones (staged as high and low bf16 rows; at K = 8192 four such rows
    exceed the LDS budget and the batch runs in slices of two)."""
    lib = _lib.load()
    w, pk, s, z = make_weight(dev, 640, K, 64, False, 7)
    for xdt in (torch.float16, torch.float32):
        x = torch.randn((B, K), device=dev).to(xdt)
        old = torch.randn((B, 640), device=dev)
        y = old.clone()
        plain = torch.empty((B, 640), device=dev)
        gemv_rows(lib, w, x, y, y)
        gemv_rows(lib, w, x, plain)
        torch.cuda.synchronize()
        assert torch.equal(y, plain + old), f"{xdt} B={B}"
        exp = linear.gemv(pk, s.astype(np.float16).astype(np.float64),
                          x.float().cpu().numpy().astype(np.float64), 64, zeros=z)
        linear.assert_close(plain.cpu().numpy(), exp, 1e-3, f"{xdt} B={B} K={K}")


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("H,KVH,K,asym,pos", [(14, 2, 896, False, 517), (4, 2, 256, True, 0),
                                              (14, 2, 896, True, 63)])
def test_qkv_rope_append_equals_separate_kernels(dev, act, H, KVH, K, asym, pos):
    """sf_q4_gemv_fused_rope == sf_q4_gemv_fused (RMSNorm folded) then
    sf_rope_kv_append: q_out, the cache codes and scales at *pos_dev, bit for bit."""
    lib = _lib.load()
    D, T_cap = 64, 64 if pos < 64 else 1024
    N = (H + 2 * KVH) * D
    assert lib.sf_q4_gemv_fused_rope_supported(N, K, 64, H, KVH, D, _lib._DT[act])
    w, *_ = make_weight(dev, N, K, 64, asym, N + K + pos)
    rng = np.random.default_rng(pos + K)
    h = torch.as_tensor(rng.normal(0, 2, (1, K)).astype(np.float32)).to(dev)
    nw = torch.as_tensor(rng.normal(1, 0.1, K).astype(np.float32)).to(dev)
    bias = torch.as_tensor(rng.normal(0, 1, N).astype(np.float32)).to(dev)
    from siliconfer_amd.model.config import ModelConfig, rope_tables
    cfg = ModelConfig(hidden_size=K, intermediate_size=K, num_hidden_layers=1,
                      num_attention_heads=H, num_key_value_heads=KVH, head_dim=D,
                      vocab_size=100, rope_theta=1e6)
    cos, sin = (torch.from_numpy(t).to(dev) for t in rope_tables(cfg, T_cap))
    pos_dev = torch.tensor([pos], dtype=torch.int32, device=dev)
    outs = []
    for fold in (False, True):
        q = torch.zeros((H, D), dtype=act, device=dev)
        kc = torch.zeros((KVH, T_cap, D), dtype=torch.int8, device=dev)
        vc = torch.zeros_like(kc)
        ks = torch.zeros((KVH, T_cap), dtype=torch.float16, device=dev)
        vs = torch.zeros_like(ks)
        cache = (kc.data_ptr(), ks.data_ptr(), vc.data_ptr(), vs.data_ptr())
        if fold:
            _lib.check(lib.sf_q4_gemv_fused_rope(
                w.blob.data_ptr(), h.data_ptr(), nw.data_ptr(), 1e-6, _lib._DT[act], bias.data_ptr(),
                F32, cos.data_ptr(), sin.data_ptr(), T_cap, q.data_ptr(), _lib.dt(q), *cache, F16,
                H, KVH, D, T_cap, pos_dev.data_ptr(), N, K, 64, int(asym), st()),
                "sf_q4_gemv_fused_rope")
        else:
            qkv = fused(lib, w, h, _lib.SF_PRE_RMSNORM, nw, act, bias)
            _lib.check(lib.sf_rope_kv_append(
                qkv.data_ptr(), cos.data_ptr(), sin.data_ptr(), T_cap, q.data_ptr(), _lib.dt(q),
                *cache, F16, 1, H, KVH, D, T_cap, pos_dev.data_ptr(), 0, st()), "sf_rope_kv_append")
        torch.cuda.synchronize()
        outs.append([t.cpu() for t in (q, kc, ks, vc, vs)])
    for a, b, name in zip(*outs, ("q", "k codes", "k scales", "v codes", "v scales")):
        assert torch.equal(a, b), name
    assert int(outs[1][2][:, pos].count_nonzero()) == KVH   # the row at pos was written
