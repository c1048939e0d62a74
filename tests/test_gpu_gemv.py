"""GPU parity of the int4 decode GEMV (B = 1..8) against the oracle and the
reference's golden vectors, through the C ABI (sf_q4_repack / sf_q4_gemv).

Bar: fp32-accumulated output within 1e-3 relative —
norm-relative max error AND elementwise |y - y*| <= 1e-3 |y*| + 1e-3 max|y*|
(oracle.linear.assert_close). The oracle uses exactly the values the kernel is
given: fp16-rounded scales, and activations as rounded to the kernel's dtype.
Reference tests restated: tests/test_kernel.py:38-129, 167-178.
"""

import numpy as np
import pytest
import torch

from conftest import golden_cases, load_golden
from oracle import linear, primitives as P
from siliconfer_amd.kernels import Q4Weight

pytestmark = pytest.mark.gpu
TOL = 1e-3


def run_gemv(dev, packed, scales, zeros, x, g, xdtype=torch.float16, bias=None,
             out_dtype=torch.float16):
    """-> (y_f32 numpy [B, N], y in out_dtype as numpy float64, x as the kernel saw it)."""
    w = Q4Weight(packed, scales, zeros, g, device=dev)
    xt = torch.as_tensor(np.atleast_2d(x), dtype=torch.float32).to(dev).to(xdtype).contiguous()
    B, N = xt.shape[0], packed.shape[0]
    y32 = torch.empty((B, N), dtype=torch.float32, device=dev)
    y = torch.empty((B, N), dtype=out_dtype, device=dev)
    bt = None if bias is None else torch.as_tensor(bias).to(dev)
    w.matmul(xt, bias=bt, out=y, out_f32=y32)
    torch.cuda.synchronize()
    return y32.cpu().numpy(), y.float().cpu().numpy().astype(np.float64), xt.float().cpu().numpy()


def s16(s):
    return np.asarray(s, np.float32).astype(np.float16).astype(np.float64)


@pytest.mark.parametrize("name", golden_cases("gemv_"))
def test_golden_reference_vectors(dev, name):
    c = load_golden(name)
    g = int(c["g"])
    y32, _, _ = run_gemv(dev, c["packed"], c["scales"], None, c["x"], g)
    linear.assert_close(y32[0], c["y_ref16"], TOL, name)


@pytest.mark.parametrize("name", golden_cases("gemm_"))
def test_golden_reference_gemm_vectors(dev, name):
    """T = 4 goes through the GEMV (<= 8 rows), T = 32 through the MFMA GEMM."""
    c = load_golden(name)
    g = int(c["g"])
    w = Q4Weight(c["packed"], c["scales"], None, g, device=dev)
    X = torch.as_tensor(c["x"]).to(dev)
    for dt in (torch.float16, torch.float32):
        Y = w.matmul(X.to(dt).contiguous(), out_dtype=torch.float32)
        linear.assert_close(Y.cpu().numpy(), c["y_ref16"], TOL, f"{name}/{dt}")


def test_config1_decode_gemv(dev):
    """W [4864, 896] ~ N(0, 0.02), RTN sym g=64, x fp16 [1, 896]."""
    rng = np.random.default_rng(0)
    W = rng.normal(0, 0.02, (4864, 896)).astype(np.float32)
    x = rng.normal(0, 1, (1, 896)).astype(np.float16)
    pk, s = P.pack_weights_sym(W, 64)
    y32, y16, xk = run_gemv(dev, pk, s, None, x, 64)
    ref = linear.gemv(pk, s16(s), xk, 64)
    linear.assert_close(y32, ref, TOL, "config1 f32")
    linear.assert_close(y16, ref, TOL, "config1 fp16 out")


@pytest.fixture(scope="module")
def config3_cases():
    out = []
    for i, (N, K) in enumerate([(4096, 4096), (11008, 4096), (4096, 11008)]):
        rng = np.random.default_rng(2 + i)
        W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
        x = rng.normal(0, 1, (8, K)).astype(np.float16)
        pk, s = P.pack_weights_sym(W, 128)
        ref = linear.gemv(pk, s16(s), x.astype(np.float64), 128)   # [8, N]
        out.append((N, K, pk, s, x, ref))
    return out


@pytest.mark.parametrize("shape_idx", [0, 1, 2])
def test_config3_7b_shapes_all_batches(dev, config3_cases, shape_idx):
    """7B shapes, sym g=128, batch 1, 2, 4, 8 (plus 3, 5, 6, 7)."""
    N, K, pk, s, x, ref = config3_cases[shape_idx]
    w = Q4Weight(pk, s, None, 128, device=dev)
    xt = torch.as_tensor(x).to(dev)
    for B in range(1, 9):
        y32 = torch.empty((B, N), dtype=torch.float32, device=dev)
        w.matmul(xt[:B].contiguous(), out_f32=y32)
        linear.assert_close(y32.cpu().numpy(), ref[:B], TOL, f"[{N},{K}] B={B}")


def _laplace_with_outliers(rng, shape, b=0.015):
    W = rng.laplace(0, b, shape).astype(np.float32)
    n_out = max(1, round(W.size / 1e6))
    idx = rng.choice(W.size, n_out, replace=False)
    W.reshape(-1)[idx] = (40 * b * np.sqrt(2) * rng.choice([-1, 1], n_out)).astype(np.float32)
    return W


@pytest.mark.parametrize("N,K", [(4864, 896), (896, 4864)])
def test_asym_gemv_config2_weights(dev, N, K):
    """Asymmetric (HQQ-style) codes with zero-points, the config-2 weights, B = 1..8."""
    rng = np.random.default_rng(1)
    W = _laplace_with_outliers(rng, (N, K))
    pk, s, z = P.pack_weights_asym(W, 64)
    x = rng.normal(0, 1, (8, K)).astype(np.float16)
    ref = linear.gemv(pk, s16(s), x.astype(np.float64), 64, zeros=z)
    w = Q4Weight(pk, s, z, 64, device=dev)
    xt = torch.as_tensor(x).to(dev)
    for B in (1, 2, 3, 8):
        y = w.matmul(xt[:B].contiguous(), out_dtype=torch.float32)
        linear.assert_close(y.cpu().numpy(), ref[:B], TOL, f"asym [{N},{K}] B={B}")


@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("asym", [False, True])
def test_bf16_and_f32_activations(dev, xdtype, asym):
    rng = np.random.default_rng(21)
    N, K = 1000, 2048
    W = rng.normal(0.01 if asym else 0, 0.02, (N, K)).astype(np.float32)
    if asym:
        pk, s, z = P.pack_weights_asym(W, 128)
    else:
        (pk, s), z = P.pack_weights_sym(W, 128), None
    x = rng.normal(0, 3, (5, K)).astype(np.float32)
    for B in (1, 2, 5):
        y32, _, xk = run_gemv(dev, pk, s, z, x[:B], 128, xdtype=xdtype)
        ref = linear.gemv(pk, s16(s), xk.astype(np.float64), 128, zeros=z)
        linear.assert_close(y32, ref, TOL, f"{xdtype} asym={asym} B={B}")


@pytest.mark.parametrize("xdtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,K,g,asym", [
    (130, 160, 32, True),      # K past the last whole unit; a scale group per MFMA
    (64, 1344, 96, False),     # groups of 96 (not a power of two), half a unit at the end
    (4100, 4096, 64, True),    # wide: four row tiles per workgroup at batch > 4
    (48, 12288, 64, True),     # 96 units, two scale groups per unit, zero-points
    (300, 8192, 128, False),   # fp32: four rows' high and low parts exceed the LDS budget
])
def test_activation_dtypes_and_batches(dev, xdtype, N, K, g, asym):
    """Every activation dtype at batch 1..8 over the GEMV's paths: LDS-staged
    and directly loaded activations, fp32 rows in batch slices, group sizes
    that fold per unit, per two MFMAs and per MFMA, K not a multiple of the
    128-k unit. Against the oracle on the activations as the kernel saw them."""
    rng = np.random.default_rng(N * 7 + K)
    W = rng.normal(0.01 if asym else 0, 0.02, (N, K)).astype(np.float32)
    if asym:
        pk, s, z = P.pack_weights_asym(W, g)
    else:
        (pk, s), z = P.pack_weights_sym(W, g), None
    x = rng.normal(0, 2, (8, K)).astype(np.float32)
    for B in (1, 3, 6, 8):
        y32, _, xk = run_gemv(dev, pk, s, z, x[:B], g, xdtype=xdtype)
        ref = linear.gemv(pk, s16(s), xk.astype(np.float64), g, zeros=z)
        linear.assert_close(y32, ref, TOL, f"{xdtype} N={N} K={K} g={g} asym={asym} B={B}")


@pytest.mark.parametrize("N,K,g", [
    (1, 128, 128),      # single row (test_kernel.py:121-129)
    (13, 128, 64),      # rows not a multiple of 8; 4 lanes per row
    (77, 1024, 32),     # 32 lanes per row, group 32
    (130, 2048, 64),    # one full wave per row
    (129, 4864, 64),    # 3 waves per row (down projection width)
    (33, 16384, 256),   # widest supported row: 8 waves
])
def test_edge_shapes(dev, N, K, g):
    rng = np.random.default_rng(N * 7 + K)
    W = rng.normal(0, 1, (N, K)).astype(np.float32)
    pk, s = P.pack_weights_sym(W, g)
    x = rng.normal(0, 1, (3, K)).astype(np.float16)
    for B in (1, 3):
        y32, _, xk = run_gemv(dev, pk, s, None, x[:B], g)
        linear.assert_close(y32, linear.gemv(pk, s16(s), xk, g), TOL, f"N={N} K={K} B={B}")


def test_zero_input_gives_zero(dev):
    rng = np.random.default_rng(0)
    pk, s = P.pack_weights_sym(rng.normal(0, 1, (32, 128)).astype(np.float32), 128)
    y32, _, _ = run_gemv(dev, pk, s, None, np.zeros((1, 128), np.float32), 128)
    assert np.all(y32 == 0)


def test_bias_and_output_dtypes(dev):
    rng = np.random.default_rng(4)
    W = rng.normal(0, 1, (64, 256)).astype(np.float32)
    b = rng.normal(0, 0.1, 64).astype(np.float32)
    pk, s = P.pack_weights_sym(W, 64)
    x = rng.normal(0, 1, (2, 256)).astype(np.float16)
    ref = linear.gemv(pk, s16(s), x.astype(np.float64), 64) + b
    for od in (torch.float16, torch.bfloat16, torch.float32):
        y32, y, _ = run_gemv(dev, pk, s, None, x, 64, bias=b, out_dtype=od)
        linear.assert_close(y32, ref, TOL, "bias f32")
        rounding = {torch.float16: 2 ** -11, torch.bfloat16: 2 ** -8, torch.float32: 1e-7}[od]
        linear.assert_close(y, ref, TOL + rounding, f"bias {od}")


def test_bf16_output_rounding_bits(dev):
    """The bf16 output conversion (sf_f32_to_bf16: gfx950's v_cvt_pk_bf16_f32)
    pinned bit for bit against torch's round-to-nearest-even cast: zero
    weights make each output exactly its fp32 bias, which holds ties (both
    ways to even), values just off a tie, bf16 subnormals and their ties,
    the largest finite values (one rounds to infinity), infinities and NaN."""
    N = 64
    pk = np.zeros((N, 64), np.uint8)
    s = np.ones((N, 2), np.float32)
    u = lambda bits: np.uint32(bits).view(np.float32)
    vals = [1.0, u(0x3F808000), u(0x3F818000), u(0x3F808001), u(0x3F817FFF), -u(0x3F808000),
            u(0x00008000), u(0x00018000), u(0x00000001), u(0x00010000), u(0x0000FFFF),
            -u(0x00008000), u(0x7F7FFFFF), u(0x7F7F7FFF), u(0x7F7F8000), np.inf, -np.inf,
            np.nan, u(0x3EAAAAAB), 65504.0, 1e-40, -3.0e38]
    b = np.zeros(N, np.float32)
    b[:len(vals)] = np.asarray(vals, np.float32)
    x = np.random.default_rng(9).normal(0, 1, (1, 128)).astype(np.float16)
    _, y, _ = run_gemv(dev, pk, s, None, x, 64, bias=b, out_dtype=torch.bfloat16)
    want = torch.from_numpy(b).to(torch.bfloat16).view(torch.int16).numpy()
    got = torch.from_numpy(y[0].astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy()
    nan = np.isnan(b)
    assert np.array_equal(got[~nan], want[~nan]), np.nonzero(got != want)
    assert np.all(np.isnan(y[0][nan]))


def test_repeated_launches_bitwise_identical(dev):
    """The reduction order is fixed: repeated calls give identical bits
    (the reference's race check, tests/test_metal_attention.py:87-103)."""
    rng = np.random.default_rng(7)
    pk, s = P.pack_weights_sym(rng.normal(0, 0.02, (4096, 4096)).astype(np.float32), 128)
    w = Q4Weight(pk, s, None, 128, device=dev)
    x = torch.as_tensor(rng.normal(0, 1, (4, 4096)).astype(np.float16)).to(dev)
    first = w.matmul(x, out_dtype=torch.float32).clone()
    for _ in range(10):
        assert torch.equal(w.matmul(x, out_dtype=torch.float32), first)


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("N,K,g", [(37, 384, 128), (21, 96, 32), (16, 160, 32), (50, 640, 64)])
def test_repack_round_trip_bit_exact(dev, asym, N, K, g):
    """canonical -> unit-order blob -> canonical, bit for bit; N not a multiple
    of the 16-row tile and K not a multiple of the 128-k unit exercise the
    padding."""
    rng = np.random.default_rng(5)
    W = rng.normal(0, 1, (N, K)).astype(np.float32)
    if asym:
        pk, s, z = P.pack_weights_asym(W, g)
    else:
        (pk, s), z = P.pack_weights_sym(W, g), None
    w = Q4Weight(pk, s, z, g, device=dev)
    pk2, s2, z2 = w.canonical()
    np.testing.assert_array_equal(pk2.cpu().numpy(), pk)
    np.testing.assert_array_equal(s2.cpu().numpy(), s.astype(np.float16))
    if asym:
        np.testing.assert_array_equal(z2.cpu().numpy(), z.astype(np.uint8))


@pytest.mark.parametrize("xdtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,K,g", [(24, 64, 32), (40, 256, 64), (16, 2048, 128)])
def test_unit_vector_activations_pin_row_and_k_mapping(dev, xdtype, N, K, g):
    """x = e_k picks column k: y[n] = (q[n,k] - z) * s[n, k/g] exactly (one product),
    with a distinct scale per (row, group). Any mix-up of rows, k positions,
    batch rows or scale cells shows up as an exact mismatch."""
    rng = np.random.default_rng(K)
    q = rng.integers(-8, 8, (N, K)).astype(np.int8)
    pk = P.pack_rows(q)
    s = (np.arange(N * (K // g)).reshape(N, K // g) % 61 + 1).astype(np.float32) / 8
    w = Q4Weight(pk, s, None, g, device=dev)
    ks = sorted(set([0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 15, 16, 31, K - 1] + list(rng.integers(0, K, 10))))
    for b0 in range(0, len(ks), 8):
        kk = ks[b0:b0 + 8]
        X = np.zeros((len(kk), K), np.float32)
        X[np.arange(len(kk)), kk] = 1.0
        y = w.matmul(torch.as_tensor(X).to(dev).to(xdtype), out_dtype=torch.float32).cpu().numpy()
        exp = (q[:, kk].astype(np.float64) * s[:, np.array(kk) // g]).T
        np.testing.assert_array_equal(y, exp.astype(np.float32))


@pytest.mark.parametrize("N,K,g,asym", [
    (13, 64, 64, False),       # half a 128-k unit, rows far below a 16-row tile
    (1000, 896, 64, True),     # 7 units over 7 waves, ragged last tile
    (77, 4864, 64, False),     # 38 units: 10 waves of 4 (the last of 2)
    (4100, 11008, 128, True),  # 86 units, wide: four row tiles per workgroup at batch > 4
    (64, 12288, 128, False),   # 96 units: 16 waves of 8 at batch > 4
    (48, 12288, 64, True),     # 96 units at g = 64: two scale groups per unit
    (40, 2048, 256, False),    # groups of 256: one group over two units
])
def test_batch3to8_shapes(dev, N, K, g, asym):
    """Batch 3..8 with fp16 activations: ragged row tiles, uneven K splits over
    waves, LDS-staged (batch <= 4) and directly loaded (batch > 4)
    activations, groups spanning half, one and two units."""
    rng = np.random.default_rng(N + K)
    W = rng.normal(0.01 if asym else 0, 0.02, (N, K)).astype(np.float32)
    if asym:
        pk, s, z = P.pack_weights_asym(W, g)
    else:
        (pk, s), z = P.pack_weights_sym(W, g), None
    x = rng.normal(0, 1, (8, K)).astype(np.float16)
    for B in (3, 4, 5, 6, 7, 8):
        y32, y, xk = run_gemv(dev, pk, s, z, x[:B], g)
        ref = linear.gemv(pk, s16(s), xk.astype(np.float64), g, zeros=z)
        linear.assert_close(y32, ref, TOL, f"N={N} K={K} g={g} asym={asym} B={B}")
        linear.assert_close(y, ref, TOL, f"fp16 out N={N} K={K} B={B}")


# ---------------------------------------------------------------------------
# The reference GEMV takes any K with K % g == 0 and any group size (vector
# path plus scalar tail, /root/reference/siliconfer/kernels/neon/q4_gemv.cpp:
# 124-134; validation only in bindings.cpp:24-40): long K runs the MFMA GEMV
# in per-wave chunks, group sizes off the 32 grid (and fp32 rows too long for
# the LDS) the VALU kernel. Both directly through the C ABI and through
# Q4Weight.matmul (Q4Linear's route).
# ---------------------------------------------------------------------------

def _rand_case(rng, N, K, g, asym):
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    if asym:
        pk, s, z = P.pack_weights_asym(W, g)
    else:
        (pk, s), z = P.pack_weights_sym(W, g), None
    return pk, s, z


def _capi_gemv(dev, pk, s, z, x, g, xdtype):
    from siliconfer_amd import _lib

    w = Q4Weight(pk, s, z, g, device=dev)
    xt = torch.as_tensor(x, dtype=torch.float32).to(dev).to(xdtype).contiguous()
    B, N, K = xt.shape[0], pk.shape[0], 2 * pk.shape[1]
    y32 = torch.empty((B, N), dtype=torch.float32, device=dev)
    lib = _lib.load()
    _lib.check(lib.sf_q4_gemv(w.blob.data_ptr(), xt.data_ptr(), _lib.dt(xt), None, _lib.SF_F32,
                              y32.data_ptr(), None, 0, B, N, K, g, int(z is not None),
                              _lib.stream(xt)), "sf_q4_gemv")
    torch.cuda.synchronize()
    return y32.cpu().numpy(), xt.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("xdtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("K", [18944, 28672])
@pytest.mark.parametrize("B", [1, 8])
def test_long_k_gemv(dev, xdtype, K, B):
    """K past 16 waves x the unit cap (Qwen2.5-7B down_proj 18944, Llama-70B
    MLP 28672; g = 128): chunked MFMA GEMV (fp32 at 28672: VALU kernel)."""
    rng = np.random.default_rng(K + B)
    for asym in (False, True):
        pk, s, z = _rand_case(rng, 160, K, 128, asym)
        x = rng.normal(0, 1, (B, K)).astype(np.float32)
        y, xk = _capi_gemv(dev, pk, s, z, x, 128, xdtype)
        ref = linear.gemv(pk, s16(s), xk, 128, zeros=z)
        linear.assert_close(y, ref, TOL, f"K={K} B={B} {xdtype} asym={asym}")


@pytest.mark.parametrize("xdtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,K,g", [(96, 768, 16), (70, 480, 48), (40, 9216, 96), (33, 90, 6),
                                   (20, 12, 2), (17, 1000, 8)])
def test_any_group_size(dev, xdtype, N, K, g):
    """Group sizes that are not a multiple of 32 (a group boundary inside an
    MFMA's 32 k), including K not a multiple of 8: GEMV at 1..8 rows through
    the C ABI, and GEMV / GEMM rows through Q4Weight.matmul."""
    rng = np.random.default_rng(N * K + g)
    for asym in (False, True):
        pk, s, z = _rand_case(rng, N, K, g, asym)
        for B in (1, 3, 8):
            x = rng.normal(0, 1, (B, K)).astype(np.float32)
            y, xk = _capi_gemv(dev, pk, s, z, x, g, xdtype)
            linear.assert_close(y, linear.gemv(pk, s16(s), xk, g, zeros=z), TOL,
                                f"N={N} K={K} g={g} B={B} {xdtype} asym={asym}")
        w = Q4Weight(pk, s, z, g, device=dev)
        for M in (2, 40):
            X = torch.as_tensor(rng.normal(0, 1, (M, K)).astype(np.float32)).to(dev).to(xdtype)
            Y = w.matmul(X.contiguous(), out_dtype=torch.float32)
            xk = X.float().cpu().numpy().astype(np.float64)
            linear.assert_close(Y.cpu().numpy(), linear.gemm(pk, s16(s), xk, g, zeros=z), TOL,
                                f"matmul M={M} g={g} {xdtype} asym={asym}")


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("N,K,g", [(70, 480, 48), (33, 90, 6), (20, 12, 2), (9, 1000, 8)])
def test_repack_round_trip_any_group(dev, asym, N, K, g):
    rng = np.random.default_rng(N + K + g)
    pk, s, z = _rand_case(rng, N, K, g, asym)
    w = Q4Weight(pk, s, z, g, device=dev)
    pk2, s2, z2 = w.canonical()
    np.testing.assert_array_equal(pk2.cpu().numpy(), pk)
    np.testing.assert_array_equal(s2.cpu().numpy(), np.asarray(s, np.float32).astype(np.float16))
    if asym:
        np.testing.assert_array_equal(z2.cpu().numpy(), z.astype(np.uint8))
