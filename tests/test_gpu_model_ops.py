"""GPU parity of the decoder-step operations (csrc/model_ops.hip) and of the
attention's device-length and causal-prefill modes, through the C ABI, against
the oracle / numpy restatements of the reference's layers
(/root/reference/siliconfer/model/layers.py:14-163, llama.py:55-79).
"""

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import model as OM
from oracle.linear import assert_close
from siliconfer_amd import _lib
from siliconfer_amd.model.config import ModelConfig, rope_tables

pytestmark = pytest.mark.gpu
F32, F16, BF16 = _lib.SF_F32, _lib.SF_F16, _lib.SF_BF16


def st():
    return torch.cuda.current_stream().cuda_stream


def test_embed_gather_exact(dev):
    lib = _lib.load()
    rng = np.random.default_rng(0)
    table = torch.as_tensor(rng.normal(0, 1, (300, 96)).astype(np.float32)).to(dev).to(torch.bfloat16)
    ids = np.array([0, 299, 17, 17, 5], np.int32)
    ids_d = torch.as_tensor(ids).to(dev)  # device tensors stay referenced until the kernel ran
    out = torch.empty((5, 96), dtype=torch.float32, device=dev)
    _lib.check(lib.sf_embed(ids_d.data_ptr(), table.data_ptr(), BF16, out.data_ptr(), 5, 96, 300,
                            st()), "sf_embed")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), table.float().cpu().numpy()[ids])


@pytest.mark.parametrize("odt", [torch.float32, torch.float16])
def test_rmsnorm_and_residual_add(dev, odt):
    lib = _lib.load()
    rng = np.random.default_rng(1)
    x = rng.normal(0, 2, (7, 896)).astype(np.float32)
    d = rng.normal(0, 1, (7, 896)).astype(np.float32)
    w = rng.normal(1, 0.1, 896).astype(np.float32)
    xt, dt, wt = torch.as_tensor(x).to(dev), torch.as_tensor(d).to(dev), torch.as_tensor(w).to(dev)
    out = torch.empty((7, 896), dtype=odt, device=dev)
    _lib.check(lib.sf_rmsnorm(xt.data_ptr(), dt.data_ptr(), wt.data_ptr(), F32, out.data_ptr(),
                              _lib.dt(out), 7, 896, 1e-6, st()), "sf_rmsnorm")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(xt.cpu().numpy(), x + d)          # in-place residual add
    ref = OM.rmsnorm(x + d, w, 1e-6)
    tol = 2e-6 if odt == torch.float32 else 1e-3
    assert_close(out.float().cpu().numpy(), ref, tol, "rmsnorm")


def test_rope_kv_append_matches_oracle(dev):
    """q rotated within fp32 rounding; k (after RoPE) and v codes bit-exact
    with the oracle's quantize_kv on the same fp32 inputs; scales fp16."""
    lib = _lib.load()
    cfg = ModelConfig(hidden_size=896, num_attention_heads=14, num_key_value_heads=2, head_dim=64,
                      rope_theta=1e6)
    Hq, KVH, D, T_cap = 14, 2, 64, 64
    cos, sin = rope_tables(cfg, T_cap)
    rng = np.random.default_rng(2)
    rows, pos0 = 5, 9
    qkv = rng.normal(0, 1, (rows, (Hq + 2 * KVH) * D)).astype(np.float32)
    kc = torch.zeros((KVH, T_cap, D), dtype=torch.int8, device=dev)
    vc = torch.zeros_like(kc)
    ks = torch.zeros((KVH, T_cap), dtype=torch.float16, device=dev)
    vs = torch.zeros_like(ks)
    q_out = torch.empty((rows, Hq, D), dtype=torch.float32, device=dev)
    qkv_d, cos_d, sin_d = (torch.as_tensor(a).to(dev) for a in (qkv, cos, sin))
    _lib.check(lib.sf_rope_kv_append(
        qkv_d.data_ptr(), cos_d.data_ptr(), sin_d.data_ptr(), T_cap, q_out.data_ptr(), F32,
        kc.data_ptr(), ks.data_ptr(), vc.data_ptr(), vs.data_ptr(), F16, rows, Hq, KVH, D, T_cap,
        None, pos0, st()), "sf_rope_kv_append")
    torch.cuda.synchronize()
    pos = np.arange(pos0, pos0 + rows)
    q = OM.rope(qkv[:, :Hq * D].reshape(rows, Hq, D), pos, cos, sin)
    k = OM.rope(qkv[:, Hq * D:(Hq + KVH) * D].reshape(rows, KVH, D), pos, cos, sin)
    v = qkv[:, (Hq + KVH) * D:].reshape(rows, KVH, D)
    np.testing.assert_array_equal(q_out.cpu().numpy(), q)
    for got_c, got_s, x in ((kc, ks, k), (vc, vs, v)):
        codes, s = A.quantize_kv(np.transpose(x, (1, 0, 2)))
        np.testing.assert_array_equal(got_c.cpu().numpy()[:, pos0:pos0 + rows], codes)
        np.testing.assert_array_equal(got_s.cpu().numpy()[:, pos0:pos0 + rows], s[..., 0].astype(np.float16))
        assert not got_c.cpu().numpy()[:, :pos0].any()          # nothing written outside the rows


def test_rope_kv_append_device_position(dev):
    lib = _lib.load()
    cfg = ModelConfig(hidden_size=128, num_attention_heads=2, num_key_value_heads=1, head_dim=64)
    cos, sin = rope_tables(cfg, 32)
    rng = np.random.default_rng(3)
    qkv = torch.as_tensor(rng.normal(0, 1, (1, 4 * 64)).astype(np.float32)).to(dev)
    cos_d, sin_d = torch.as_tensor(cos).to(dev), torch.as_tensor(sin).to(dev)
    outs = []
    for mode in ("host", "dev"):
        kc = torch.zeros((1, 32, 64), dtype=torch.int8, device=dev)
        ks = torch.zeros((1, 32), dtype=torch.float16, device=dev)
        vc, vs = torch.zeros_like(kc), torch.zeros_like(ks)
        q = torch.empty((1, 2, 64), dtype=torch.float16, device=dev)
        pos = torch.tensor([11], dtype=torch.int32, device=dev)
        _lib.check(lib.sf_rope_kv_append(
            qkv.data_ptr(), cos_d.data_ptr(), sin_d.data_ptr(), 32, q.data_ptr(), F16, kc.data_ptr(),
            ks.data_ptr(), vc.data_ptr(), vs.data_ptr(), F16, 1, 2, 1, 64, 32,
            pos.data_ptr() if mode == "dev" else None, 11, st()), "rope")
        torch.cuda.synchronize()
        outs.append((q.cpu(), kc.cpu(), ks.cpu(), vc.cpu(), vs.cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert outs[0][1][0, 11].abs().sum() > 0


def test_silu_mul(dev):
    lib = _lib.load()
    rng = np.random.default_rng(4)
    gu = rng.normal(0, 3, (3, 2 * 200)).astype(np.float32)
    out = torch.empty((3, 200), dtype=torch.float32, device=dev)
    gu_d = torch.as_tensor(gu).to(dev)
    _lib.check(lib.sf_silu_mul(gu_d.data_ptr(), out.data_ptr(), F32, 3, 200, st()), "sf_silu_mul")
    torch.cuda.synchronize()
    g, u = gu[:, :200].astype(np.float64), gu[:, 200:].astype(np.float64)
    np.testing.assert_allclose(out.cpu().numpy(), g / (1 + np.exp(-g)) * u, rtol=2e-6, atol=1e-7)


def lm_head(dev, W, x, with_pos=False):
    lib = _lib.load()
    V, H = W.shape
    Wt = torch.as_tensor(W).to(dev).to(torch.bfloat16)
    xt = torch.as_tensor(x).to(dev)
    logits = torch.empty(V, dtype=torch.float32, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = torch.zeros(lib.sf_lm_head_workspace_bytes(V), dtype=torch.uint8, device=dev)
    pos = torch.tensor([3], dtype=torch.int32, device=dev) if with_pos else None
    hist = torch.full((8,), -1, dtype=torch.int32, device=dev) if with_pos else None
    _lib.check(lib.sf_lm_head_argmax(Wt.data_ptr(), xt.data_ptr(), _lib.dt(xt), logits.data_ptr(), V, H,
                                     tok.data_ptr(), None if pos is None else pos.data_ptr(),
                                     None if hist is None else hist.data_ptr(), ws.data_ptr(),
                                     ws.numel(), st()), "sf_lm_head_argmax")
    assert int(ws[:256].count_nonzero()) == 0  # counter back at zero
    return logits.cpu().numpy(), int(tok.item()), Wt.float().cpu().numpy(), pos, hist


@pytest.mark.parametrize("V,H", [(151936, 896), (1000, 64), (5000, 1600)])
def test_lm_head_logits_and_argmax(dev, V, H):
    rng = np.random.default_rng(5)
    W = rng.normal(0, 0.02, (V, H)).astype(np.float32)
    x = rng.normal(0, 1, H).astype(np.float32)
    logits, tok, Wb, _, _ = lm_head(dev, W, x)
    ref = Wb.astype(np.float64) @ x.astype(np.float64)
    assert_close(logits, ref, 1e-5, f"logits V={V}")
    assert tok == int(np.argmax(logits))


def test_lm_head_ties_pick_lowest_index_and_position(dev):
    rng = np.random.default_rng(6)
    W = rng.normal(0, 0.02, (3000, 128)).astype(np.float32)
    W[2900] = W[1234] = W[2000] = 0.5  # identical best rows
    x = np.ones(128, np.float32)
    logits, tok, _, pos, hist = lm_head(dev, W, x, with_pos=True)
    assert tok == 1234
    assert int(pos.item()) == 4 and int(hist[3].item()) == 1234 and int(hist[2].item()) == -1


def make_cache(rng, KVH, T, D):
    k = rng.normal(0, 1, (1, KVH, T, D)).astype(np.float32)
    v = rng.normal(0, 1, (1, KVH, T, D)).astype(np.float32)
    kc, ks = A.quantize_kv(k)
    vc, vs = A.quantize_kv(v)
    return kc, ks[..., 0], vc, vs[..., 0]


def test_attention_device_length_equals_host_length(dev):
    lib = _lib.load()
    rng = np.random.default_rng(7)
    kc, ks, vc, vs = make_cache(rng, 2, 300, 64)
    t = lambda a: torch.as_tensor(np.ascontiguousarray(a)).to(dev)
    kct, kst, vct, vst = t(kc), t(ks), t(vc), t(vs)
    q = t(rng.normal(0, 1, (1, 14, 64)).astype(np.float32))
    S = 8
    ws = torch.zeros(lib.sf_attn_workspace_bytes(1, 14, 64, S), dtype=torch.uint8, device=dev)
    for T in (1, 77, 300):
        o1 = torch.empty((1, 14, 64), dtype=torch.float32, device=dev)
        o2 = torch.empty_like(o1)
        _lib.check(lib.sf_attn_decode_i8kv(q.data_ptr(), F32, kct.data_ptr(), kst.data_ptr(),
                                           vct.data_ptr(), vst.data_ptr(), F32, o1.data_ptr(), F32,
                                           ws.data_ptr(), ws.numel(), 1, 14, 2, T, 300, 64, 0.125,
                                           min(S, T), st()), "host T")
        Td = torch.tensor([T - 1], dtype=torch.int32, device=dev)
        _lib.check(lib.sf_attn_decode_i8kv_dev(q.data_ptr(), F32, kct.data_ptr(), kst.data_ptr(),
                                               vct.data_ptr(), vst.data_ptr(), F32, o2.data_ptr(), F32,
                                               ws.data_ptr(), ws.numel(), 1, 14, 2, Td.data_ptr(), 1,
                                               300, 300, 64, 0.125, S, st()), "device T")
        ref = A.attention_decode(q.cpu().numpy(), kc, ks[..., None], vc, vs[..., None], scale=0.125, T=T)
        assert_close(o2.cpu().numpy(), ref, 2e-3, f"device T={T}")
        assert_close(o1.cpu().numpy(), o2.cpu().numpy(), 1e-5, f"host vs device T={T}")


@pytest.mark.parametrize("T0,Tq", [(0, 1), (0, 37), (20, 16), (0, 512), (100, 300)])
def test_causal_prefill_attention(dev, T0, Tq):
    """Causal prompt attention over the int8 cache, up to config 5's 512-row
    prompt and a prompt chunk after a cached prefix."""
    lib = _lib.load()
    rng = np.random.default_rng(8 + Tq)
    T_cap = max(64, T0 + Tq)
    kc, ks, vc, vs = make_cache(rng, 2, T_cap, 64)
    t = lambda a: torch.as_tensor(np.ascontiguousarray(a)).to(dev)
    q = rng.normal(0, 1, (Tq, 14, 64)).astype(np.float32)
    out = torch.empty((Tq, 14, 64), dtype=torch.float32, device=dev)
    qd, kcd, ksd, vcd, vsd = t(q), t(kc), t(ks), t(vc), t(vs)
    _lib.check(lib.sf_attn_prefill_i8kv(qd.data_ptr(), F32, kcd.data_ptr(), ksd.data_ptr(),
                                        vcd.data_ptr(), vsd.data_ptr(), F32, out.data_ptr(), F32,
                                        Tq, 14, 2, T0, T_cap, 64, 0.125, st()), "prefill")
    torch.cuda.synchronize()
    K = (kc[0].astype(np.float32) * ks[0][..., None])
    V = (vc[0].astype(np.float32) * vs[0][..., None])
    ref = OM.attend(q, K, V, T0, 0.125)
    assert_close(out.cpu().numpy(), ref, 2e-3, f"prefill T0={T0} Tq={Tq}")


@pytest.mark.parametrize("kernel", ["mfma", "valu"])
@pytest.mark.parametrize("D,H,KVH,T0,Tq,T_cap", [
    (64, 14, 2, 0, 16, 16),       # the smallest flash chunk, cache exactly full
    (64, 14, 2, 0, 24, 64),       # first workgroups see one key tile: three of their waves have none
    (64, 14, 2, 5, 333, 341),     # T_cap % 4 != 0 (per-token scale loads)
    (128, 32, 2, 0, 100, 128),    # 16 query heads per kv head, head_dim 128
    (128, 8, 8, 40, 70, 112),     # MHA
    (64, 16, 2, 7, 257, 300),     # 8 heads per kv head, rows not a multiple of 16
])
@pytest.mark.parametrize("qdt,sdt", [(torch.float32, np.float32), (torch.float16, np.float16),
                                     (torch.bfloat16, np.float16)])
def test_prefill_attention_shapes(dev, monkeypatch, kernel, D, H, KVH, T0, Tq, T_cap, qdt, sdt):
    """Causal prefill attention (the flash MFMA kernel for prompt chunks of 16+
    rows at head_dim 64 / 128; SF_ATTN_MFMA=0 keeps the split-T decode kernel)
    against the oracle's causal attention over the dequantized int8 cache."""
    monkeypatch.setenv("SF_ATTN_MFMA", "1" if kernel == "mfma" else "0")
    lib = _lib.load()
    rng = np.random.default_rng(D + H + Tq)
    kc, ks, vc, vs = make_cache(rng, KVH, T_cap, D)
    ks, vs = ks.astype(sdt), vs.astype(sdt)
    t = lambda a: torch.as_tensor(np.ascontiguousarray(a)).to(dev)
    q = t(rng.normal(0, 1, (Tq, H, D)).astype(np.float32)).to(qdt)
    out = torch.empty((Tq, H, D), dtype=torch.float32, device=dev)
    kcd, ksd, vcd, vsd = t(kc), t(ks), t(vc), t(vs)
    sdt_code = F16 if sdt == np.float16 else F32
    _lib.check(lib.sf_attn_prefill_i8kv(q.data_ptr(), _lib.dt(q), kcd.data_ptr(), ksd.data_ptr(),
                                        vcd.data_ptr(), vsd.data_ptr(), sdt_code, out.data_ptr(), F32,
                                        Tq, H, KVH, T0, T_cap, D, D ** -0.5, st()), "prefill")
    torch.cuda.synchronize()
    K = kc[0].astype(np.float32) * ks[0].astype(np.float32)[..., None]
    V = vc[0].astype(np.float32) * vs[0].astype(np.float32)[..., None]
    ref = OM.attend(q.float().cpu().numpy(), K, V, T0, D ** -0.5)
    assert_close(out.cpu().numpy(), ref, 2e-3, f"prefill {kernel} D={D} H={H}/{KVH} T0={T0} Tq={Tq}")


def test_rope_append_from_gemm_partials(dev):
    """The prompt path's qkv projection: sf_q4_gemm_partials + sf_rope_kv_append_partials
    (partials summed in split order, bias added) store the same q rows, KV codes and
    scales, bit for bit, as sf_q4_gemm(..., bias) into a qkv buffer + sf_rope_kv_append."""
    from oracle import primitives as P
    from siliconfer_amd.kernels import Q4Weight

    lib = _lib.load()
    rng = np.random.default_rng(11)
    M, H, KVH, D, K, T_cap = 512, 14, 2, 64, 896, 600
    N = (H + 2 * KVH) * D
    pk, s = P.pack_weights_sym(rng.normal(0, 0.02, (N, K)).astype(np.float32), 64)
    w = Q4Weight(pk, s, None, 64, device=dev)
    S = lib.sf_q4_gemm_splits(M, N, K, 64)
    assert S > 1
    X = torch.as_tensor(rng.normal(0, 1, (M, K)).astype(np.float32)).to(dev).half().contiguous()
    bias = torch.as_tensor(rng.normal(0, 0.1, N).astype(np.float32)).to(dev)
    pos = np.arange(T_cap)[:, None] * (1e6 ** (-np.arange(0, D, 2) / D))[None, :]
    cos = torch.as_tensor(np.cos(pos).astype(np.float32)).to(dev)
    sin = torch.as_tensor(np.sin(pos).astype(np.float32)).to(dev)
    wsb = lib.sf_q4_gemm_workspace_bytes(M, N, K, 64)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream

    def cache():
        return (torch.zeros((M, H, D), dtype=torch.float16, device=dev),
                torch.zeros((KVH, T_cap, D), dtype=torch.int8, device=dev),
                torch.zeros((KVH, T_cap), dtype=torch.float16, device=dev),
                torch.zeros((KVH, T_cap, D), dtype=torch.int8, device=dev),
                torch.zeros((KVH, T_cap), dtype=torch.float16, device=dev))

    def ptrs(c):
        q, kc, ks, vc, vs = c
        return (cos.data_ptr(), sin.data_ptr(), T_cap, q.data_ptr(), F16, kc.data_ptr(), ks.data_ptr(),
                vc.data_ptr(), vs.data_ptr(), F16, M, H, KVH, D, T_cap, None, 40)

    qkv = torch.empty((M, N), dtype=torch.float32, device=dev)
    c1, c2 = cache(), cache()
    _lib.check(lib.sf_q4_gemm(w.blob.data_ptr(), X.data_ptr(), F16, None, F32, qkv.data_ptr(),
                              bias.data_ptr(), F32, M, N, K, 64, 0, ws.data_ptr(), wsb, st), "sf_q4_gemm")
    _lib.check(lib.sf_rope_kv_append(qkv.data_ptr(), *ptrs(c1), st), "sf_rope_kv_append")
    ws.fill_(0x7F)
    _lib.check(lib.sf_q4_gemm_partials(w.blob.data_ptr(), X.data_ptr(), F16, M, N, K, 64, 0,
                                       ws.data_ptr(), wsb, st), "sf_q4_gemm_partials")
    _lib.check(lib.sf_rope_kv_append_partials(ws.data_ptr(), S, bias.data_ptr(), F32, *ptrs(c2), st),
               "sf_rope_kv_append_partials")
    torch.cuda.synchronize()
    for a, b in zip(c1, c2):
        assert torch.equal(a.view(torch.uint8) if a.dtype == torch.int8 else a.view(torch.int16),
                           b.view(torch.uint8) if b.dtype == torch.int8 else b.view(torch.int16))
    assert bool((c2[2][:, 40:40 + M] > 0).all())  # every appended row has its scale
