"""GPU parity of the split-T decode attention over the int8 KV cache against the
oracle (float64 dequantize-then-softmax), through the C ABI
(sf_attn_decode_i8kv). Bar: 2e-3 relative.
Reference tests restated: tests/test_metal_attention.py:45-183. Each test runs
on both kernels (the `kernel_choice` fixture).
"""

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle.linear import assert_close
from siliconfer_amd.kernels.attention import (_choose_n_tiles, attention_decode, default_splits,
                                              fused_quantized_attention_decode)

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.fixture(params=["mfma", "valu"], autouse=True)
def kernel_choice(request, monkeypatch):
    """Every test runs on both decode kernels: the MFMA one (up to 16 query
    heads per kv head, head_dim 64 / 128) and the VALU one (SF_ATTN_MFMA=0,
    read by the library on every call)."""
    monkeypatch.setenv("SF_ATTN_MFMA", "1" if request.param == "mfma" else "0")
    return request.param


def make_inputs(rng, B, H, KVH, D, T, scale_dtype=np.float32):
    q = rng.normal(0, 1, (B, H, D)).astype(np.float32)
    k = rng.normal(0, 1, (B, KVH, T, D)).astype(np.float32)
    v = rng.normal(0, 1, (B, KVH, T, D)).astype(np.float32)
    kc, ks = A.quantize_kv(k)
    vc, vs = A.quantize_kv(v)
    return q, kc, ks.astype(scale_dtype), vc, vs.astype(scale_dtype)


def run(dev, q, kc, ks, vc, vs, n_tiles=None):
    t = lambda a: torch.as_tensor(a).to(dev)
    out = fused_quantized_attention_decode(t(q), t(kc), t(ks), t(vc), t(vs), n_tiles=n_tiles)
    assert out.dtype == torch.float32 and tuple(out.shape) == q.shape
    return out.cpu().numpy()


def check(dev, q, kc, ks, vc, vs, n_tiles=None, what=""):
    out = run(dev, q, kc, ks, vc, vs, n_tiles)
    ref = A.attention_decode(q, kc, ks.astype(np.float64), vc, vs.astype(np.float64))
    assert_close(out, ref, TOL, what)
    return out


@pytest.mark.parametrize("T", [1, 3, 5, 128])
def test_mha(dev, T):
    rng = np.random.default_rng(0)
    check(dev, *make_inputs(rng, 1, 4, 4, 8, T), what=f"MHA T={T}")


@pytest.mark.parametrize("T", [1, 3, 128, 512])
def test_gqa_qwen_geometry(dev, T):
    rng = np.random.default_rng(3)
    check(dev, *make_inputs(rng, 1, 14, 2, 64, T), what=f"GQA T={T}")


def test_output_finite_and_shape(dev):
    rng = np.random.default_rng(5)
    out = run(dev, *make_inputs(rng, 2, 8, 4, 32, 64))
    assert out.shape == (2, 8, 32) and np.isfinite(out).all()


def test_batch_dimension(dev):
    rng = np.random.default_rng(9)
    check(dev, *make_inputs(rng, 3, 4, 2, 16, 32), what="B=3")


@pytest.mark.parametrize("n_tiles", [1, 2, 3, 7, 16, 64, 200])
def test_explicit_n_tiles(dev, n_tiles):
    rng = np.random.default_rng(11)
    check(dev, *make_inputs(rng, 1, 14, 2, 64, 100), n_tiles=n_tiles, what=f"n_tiles={n_tiles}")


def test_different_n_tiles_agree(dev):
    rng = np.random.default_rng(13)
    inp = make_inputs(rng, 1, 14, 2, 64, 300)
    a, b = run(dev, *inp, n_tiles=1), run(dev, *inp, n_tiles=37)
    assert np.abs(a - b).max() <= 1e-5 * np.abs(a).max()


def test_choose_n_tiles_heuristic():
    assert _choose_n_tiles(8) == 1
    assert _choose_n_tiles(128) > _choose_n_tiles(32) > _choose_n_tiles(8)
    assert _choose_n_tiles(1_000_000) <= 256


@pytest.mark.parametrize("T", [256, 2048])
def test_repeated_calls_bitwise_identical(dev, T):
    rng = np.random.default_rng(17)
    inp = make_inputs(rng, 1, 14, 2, 64, T)
    first = run(dev, *inp)
    for _ in range(10):
        assert np.array_equal(run(dev, *inp), first)


@pytest.mark.parametrize("T", [4096, 16384])
def test_config4_fp16_cache(dev, T):
    """Qwen2.5-0.5B geometry, K/V ~ N(0,1) fp16 -> int8 with fp16
    per-token scales, q fp16 [1, 14, 64], scale 1/8."""
    rng = np.random.default_rng(3)
    k = rng.normal(0, 1, (1, 2, T, 64)).astype(np.float16).astype(np.float32)
    v = rng.normal(0, 1, (1, 2, T, 64)).astype(np.float16).astype(np.float32)
    kc, ks = A.quantize_kv(k)
    vc, vs = A.quantize_kv(v)
    ks16, vs16 = ks[..., 0].astype(np.float16), vs[..., 0].astype(np.float16)
    q = rng.normal(0, 1, (1, 14, 64)).astype(np.float16)
    t = lambda a: torch.as_tensor(a).to(dev)
    out = attention_decode(t(q), t(kc), t(ks16), t(vc), t(vs16), scale=0.125)
    ref = A.attention_decode(q.astype(np.float64), kc, ks16.astype(np.float64), vc,
                             vs16.astype(np.float64), scale=0.125)
    assert_close(out.cpu().numpy(), ref, TOL, f"config4 T={T}")


def test_partial_cache_prefix(dev):
    """Only the first T of T_cap positions are read."""
    rng = np.random.default_rng(21)
    q, kc, ks, vc, vs = make_inputs(rng, 1, 14, 2, 64, 500)
    t = lambda a: torch.as_tensor(a).to(dev)
    out = attention_decode(t(q), t(kc), t(ks), t(vc), t(vs), T=321)
    ref = A.attention_decode(q, kc, ks, vc, vs, T=321)
    assert_close(out.cpu().numpy(), ref, TOL, "prefix")


@pytest.mark.parametrize("sdtype", [np.float16, np.float32])
@pytest.mark.parametrize("T,S", [(1, 8), (31, 8), (100, 8), (520, 8), (1000, 32), (321, 1),
                                 (700, 0)])
def test_rows_past_length_never_read_into_the_result(dev, sdtype, T, S):
    """The cache rows at and past the length T hold anything (here random codes
    and NaN scales): the result equals the one over a cache whose rows past T
    are zeros, bit for bit, on the host-length and the device-length paths. The
    split kernel loads a wave's first tiles before the length is known, so these
    rows are read and must be masked (S = 0: the default split count)."""
    from siliconfer_amd import _lib

    lib = _lib.load()
    T_cap, B, H, KVH, D = 1024, 1, 14, 2, 64
    rng = np.random.default_rng(T + S)
    q, kc, ks, vc, vs = make_inputs(rng, B, H, KVH, D, T_cap, sdtype)
    clean = [a.copy() for a in (kc, ks, vc, vs)]
    dirty = [a.copy() for a in (kc, ks, vc, vs)]
    for a in clean:
        a[:, :, T:] = 0 if a.dtype == np.int8 else 1
    for a in dirty:
        if a.dtype == np.int8:
            a[:, :, T:] = rng.integers(-127, 128, a[:, :, T:].shape, dtype=np.int8)
        else:
            a[:, :, T:] = np.nan
    t = lambda a: torch.as_tensor(a).to(dev).contiguous()
    st = torch.cuda.current_stream().cuda_stream
    nsp = S if S > 0 else int(lib.sf_attn_default_splits_d(B, KVH, T_cap, D))
    ws = torch.empty((max(lib.sf_attn_workspace_bytes(B, H, D, max(nsp, 2)), 256),),
                     dtype=torch.uint8, device=dev)
    T_dev = torch.tensor([T], dtype=torch.int32, device=dev)
    outs = []
    for kc_, ks_, vc_, vs_ in (clean, dirty):
        kcd, ksd, vcd, vsd, qd = t(kc_), t(ks_), t(vc_), t(vs_), t(q)
        args = (qd.data_ptr(), _lib.SF_F32, kcd.data_ptr(), ksd.data_ptr(), vcd.data_ptr(),
                vsd.data_ptr(), _lib.dt(ksd))
        host = attention_decode(qd, kcd, ksd, vcd, vsd, T=T, n_splits=S or None)
        devo = torch.empty((B, H, D), dtype=torch.float32, device=dev)
        _lib.check(lib.sf_attn_decode_i8kv_dev(*args, devo.data_ptr(), _lib.SF_F32, ws.data_ptr(),
                                               ws.numel(), B, H, KVH, T_dev.data_ptr(), 0, T_cap,
                                               T_cap, D, float(D ** -0.5), nsp, st),
                   "sf_attn_decode_i8kv_dev")
        torch.cuda.synchronize()
        outs.append((host.cpu(), devo.cpu()))
    for i in range(2):
        assert torch.isfinite(outs[1][i]).all()
        assert torch.equal(outs[0][i], outs[1][i]), ("host", "device")[i]
    ref = A.attention_decode(q, kc, ks.astype(np.float64), vc, vs.astype(np.float64), T=T)
    assert_close(outs[1][1].numpy(), ref, TOL, f"device length T={T} S={nsp}")


@pytest.mark.parametrize("D", [16, 128, 256])
def test_head_dims(dev, D):
    rng = np.random.default_rng(D)
    check(dev, *make_inputs(rng, 1, 8, 2, D, 77), what=f"D={D}")


def test_head_group_larger_than_block(dev):
    """GQA groups of more than 8 query heads span several head blocks."""
    rng = np.random.default_rng(22)
    check(dev, *make_inputs(rng, 2, 20, 2, 64, 150), what="G=10")


def test_max_splits(dev):
    """512 splits (the kernel's maximum) over a 4096-token cache."""
    rng = np.random.default_rng(23)
    check(dev, *make_inputs(rng, 1, 14, 2, 64, 4096), n_tiles=512, what="512 splits")


def test_workspace_reused_across_shapes(dev):
    """One workspace serves calls of different shapes in a row, and nothing in
    it needs clearing: it starts filled with 0xFF bytes (NaN floats), which
    every split's partial overwrites before the merge launch reads it."""
    from siliconfer_amd import _lib

    lib = _lib.load()
    ws = torch.full((8 << 20,), 0xFF, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    t = lambda a: torch.as_tensor(a).to(dev).contiguous()
    cases = [(2, 20, 2, 64, 1000, 300), (1, 14, 2, 64, 100, 7), (2, 20, 2, 64, 1000, 300),
             (1, 8, 8, 128, 333, 64)]
    for i, (B, H, KVH, D, T, S) in enumerate(cases):
        rng = np.random.default_rng(100 + i)
        q, kc, ks, vc, vs = make_inputs(rng, B, H, KVH, D, T)
        out = torch.empty((B, H, D), dtype=torch.float32, device=dev)
        qd, kcd, ksd, vcd, vsd = t(q), t(kc), t(ks), t(vc), t(vs)
        assert lib.sf_attn_workspace_bytes(B, H, D, S) <= ws.numel()
        rc = lib.sf_attn_decode_i8kv(qd.data_ptr(), _lib.SF_F32, kcd.data_ptr(), ksd.data_ptr(),
                                     vcd.data_ptr(), vsd.data_ptr(), _lib.SF_F32, out.data_ptr(),
                                     _lib.SF_F32, ws.data_ptr(), ws.numel(), B, H, KVH, T, T, D,
                                     float(D ** -0.5), S, st)
        _lib.check(rc, "sf_attn_decode_i8kv")
        torch.cuda.synchronize()
        ref = A.attention_decode(q, kc, ks, vc, vs)
        assert_close(out.cpu().numpy(), ref, TOL, f"case {i}")


@pytest.mark.parametrize("dtype,tol", [(torch.float16, 2e-3), (torch.bfloat16, 8e-3)])
def test_half_precision_q_and_out(dev, dtype, tol):
    """q and the output in fp16 / bf16; the tolerance adds the output's own
    rounding (bf16 keeps 8 significant bits)."""
    rng = np.random.default_rng(24)
    q, kc, ks, vc, vs = make_inputs(rng, 1, 14, 2, 64, 700)
    qh = torch.as_tensor(q).to(dtype)
    t = lambda a: torch.as_tensor(a).to(dev)
    out = attention_decode(qh.to(dev), t(kc), t(ks), t(vc), t(vs), out_dtype=dtype)
    assert out.dtype == dtype
    ref = A.attention_decode(qh.float().numpy().astype(np.float64), kc, ks, vc, vs)
    assert_close(out.float().cpu().numpy(), ref, tol, f"{dtype}")


@pytest.mark.parametrize("G", [3, 5, 6, 7, 8, 12, 16])
def test_gqa_group_widths(dev, G):
    """Every head-block width the kernel is built for (exact and padded blocks,
    and groups split over several blocks)."""
    rng = np.random.default_rng(30 + G)
    check(dev, *make_inputs(rng, 2, 2 * G, 2, 64, 333), what=f"G={G}")


@pytest.mark.parametrize("T,S", [(1, 1), (31, 1), (33, 2), (1000, 3), (777, 100)])
def test_sixteen_heads_d128(dev, T, S):
    """A full 16-head group at head_dim 128: partial 32-token tiles, splits
    shorter than a tile, and many splits."""
    rng = np.random.default_rng(40 + T)
    check(dev, *make_inputs(rng, 1, 32, 2, 128, T), n_tiles=S, what=f"G=16 D=128 T={T} S={S}")


@pytest.mark.parametrize("T", [480, 512, 513, 545, 1024, 1100, 1280])
def test_one_split_wave_rounds(dev, T):
    """One split at head_dim 64 runs 16 waves, one 32-token tile each per round:
    15, 16 and 17 tiles (one wave takes a second tile), a partial last tile, and
    two full rounds."""
    rng = np.random.default_rng(50 + T)
    check(dev, *make_inputs(rng, 1, 14, 2, 64, T), n_tiles=1, what=f"one split T={T}")
    check(dev, *make_inputs(rng, 2, 14, 2, 64, T, np.float16), n_tiles=1,
          what=f"one split B=2 fp16 scales T={T}")


@pytest.mark.parametrize("H", [14, 32])
@pytest.mark.parametrize("T", [257, 513, 640])
def test_one_split_head_dim_128(dev, H, T):
    """One split at head_dim 128 (8 waves, two tiles each in flight): several
    tile rotations, beyond the default one-split limit of 320 tokens."""
    rng = np.random.default_rng(60 + T + H)
    check(dev, *make_inputs(rng, 1, H, 2, 128, T), n_tiles=1, what=f"D=128 H={H} one split T={T}")
    check(dev, *make_inputs(rng, 1, H, 2, 128, T, np.float16), n_tiles=1,
          what=f"D=128 H={H} one split fp16 scales T={T}")


@pytest.mark.parametrize("D,T", [(64, 160), (64, 161), (128, 160), (128, 161), (64, 2048), (64, 2049),
                                 (64, 16384), (128, 8192)])
def test_default_split_switch(dev, D, T):
    """The default split count on either side of the one-split limit and of
    the 32 -> 64 tokens-per-split step, and at 128 splits (a merge span of two
    splits per lane), through attention_decode's own pick
    (fp32 and fp16 scales); default_splits reports the count it uses."""
    assert (default_splits(1, 2, T, D) == 1) == (T <= 160)
    for sdt in (np.float32, np.float16):
        rng = np.random.default_rng(70 + T + D)
        q, kc, ks, vc, vs = make_inputs(rng, 1, 14, 2, D, T, sdt)
        t = lambda a: torch.as_tensor(a).to(dev)
        out = attention_decode(t(q), t(kc), t(ks), t(vc), t(vs)).cpu().numpy()
        ref = A.attention_decode(q, kc, ks.astype(np.float64), vc, vs.astype(np.float64))
        assert_close(out, ref, TOL, f"default splits D={D} T={T} {sdt.__name__}")
