"""GPU parity of the int4 prefill GEMM (MFMA) against the oracle, through the C
ABI (sf_q4_gemm). Bar: 1e-3 relative (oracle.linear.assert_close).
Reference tests restated: tests/test_kernel.py:136-151, 181-210.
"""

import numpy as np
import pytest
import torch

from oracle import linear, primitives as P
from siliconfer_amd.kernels import Q4Weight

pytestmark = pytest.mark.gpu
TOL = 1e-3


def s16(s):
    return np.asarray(s, np.float32).astype(np.float16).astype(np.float64)


def laplace_outliers(rng, shape, b=0.015):
    W = rng.laplace(0, b, shape).astype(np.float32)
    n_out = max(1, round(W.size / 1e6))
    idx = rng.choice(W.size, n_out, replace=False)
    W.reshape(-1)[idx] = (40 * b * np.sqrt(2) * rng.choice([-1, 1], n_out)).astype(np.float32)
    return W


def gemm_dev(dev, pk, s, z, X, g, xdtype, out_dtype=torch.float32, bias=None):
    w = Q4Weight(pk, s, z, g, device=dev)
    xt = torch.as_tensor(X, dtype=torch.float32).to(dev).to(xdtype).contiguous()
    bt = None if bias is None else torch.as_tensor(bias).to(dev)
    y = w.matmul(xt, out_dtype=out_dtype, bias=bt)
    torch.cuda.synchronize()
    return y.float().cpu().numpy().astype(np.float64), xt.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("N,K", [(4864, 896), (896, 4864)])
def test_config2_asym_prefill(dev, N, K):
    """X bf16 [512, K] ~ N(0,1); W ~ Laplace(0, 0.015) with 40-sigma
    outliers; asym g=64, fp16 scales, uint4 zero-points. Up/gate and down shapes."""
    rng = np.random.default_rng(1)
    W = laplace_outliers(rng, (N, K))
    pk, s, z = P.pack_weights_asym(W, 64)
    X = rng.normal(0, 1, (512, K)).astype(np.float32)
    y, xk = gemm_dev(dev, pk, s, z, X, 64, torch.bfloat16)
    linear.assert_close(y, linear.gemm(pk, s16(s), xk, 64, zeros=z), TOL, f"config2 [{N},{K}]")


@pytest.mark.parametrize("N,K", [(4864, 896), (896, 4864)])
def test_config2_hqq_packed_prefill(dev, N, K):
    """Config 2 through the HQQ producer (siliconfer_amd/quant/hqq.py; the
    reference packs HQQ projections with pack_weights_asym, q4_loader.py:178-183):
    the HQQ-packed tensors differ from min-max RTN only in fp32 scale rounding
    (one fp16-stored scale on the down shape), and the GEMM on them meets the bar."""
    from siliconfer_amd.quant.hqq import hqq_pack

    rng = np.random.default_rng(1)
    if K == 4864:
        laplace_outliers(rng, (4864, 896))  # the down shape is the second draw (tests/test_hqq.py)
    W = laplace_outliers(rng, (N, K))
    pk, s, z = hqq_pack(W, 64)
    X = np.random.default_rng(5).normal(0, 1, (512, K)).astype(np.float32)
    y, xk = gemm_dev(dev, pk, s, z, X, 64, torch.bfloat16)
    linear.assert_close(y, linear.gemm(pk, s16(s), xk, 64, zeros=z), TOL, f"config2 hqq [{N},{K}]")


@pytest.mark.parametrize("xdtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M,N,K,g", [(33, 100, 256, 64), (200, 257, 512, 128), (130, 640, 96, 32),
                                     # groups of 96 (a group boundary inside a K step) and
                                     # 256 (four steps); split-K starting mid-group
                                     (130, 200, 288, 96), (70, 300, 1024, 256),
                                     (64, 96, 1152, 128), (40, 50, 1152, 96),
                                     # 7B / 8B MLP depths: K split over many 64-k steps
                                     (96, 384, 14336, 128), (144, 136, 11008, 64)])
def test_gemm_shapes_and_dtypes_sym(dev, xdtype, M, N, K, g):
    rng = np.random.default_rng(M + N + K)
    W = rng.normal(0, 1, (N, K)).astype(np.float32)
    pk, s = P.pack_weights_sym(W, g)
    X = rng.normal(0, 1, (M, K)).astype(np.float32)
    y, xk = gemm_dev(dev, pk, s, None, X, g, xdtype)
    linear.assert_close(y, linear.gemm(pk, s16(s), xk, g), TOL, f"{M}x{N}x{K} {xdtype}")


def test_gemm_asym_matches_fake_quant_matmul(dev):
    """tests/test_kernel.py:198-210 (T = 8 goes to the GEMV; 64 to the GEMM)."""
    rng = np.random.default_rng(3)
    W = rng.normal(0, 1, (32, 128)).astype(np.float32)
    pk, s, z = P.pack_weights_asym(W, 128)
    Wq = P.dequant_packed(pk, s16(s), z, 128)
    for T in (8, 64):
        X = rng.normal(0, 1, (T, 128)).astype(np.float32)
        y, xk = gemm_dev(dev, pk, s, z, X, 128, torch.float32)
        linear.assert_close(y, xk @ Wq.T, TOL, f"T={T}")


@pytest.mark.parametrize("asym", [False, True])
def test_gemm_equals_gemv_loop(dev, asym):
    """tests/test_kernel.py:136-151, 181-195: rows of the GEMM equal single-row GEMVs."""
    rng = np.random.default_rng(99)
    W = rng.normal(0, 1, (64, 128)).astype(np.float32)
    if asym:
        pk, s, z = P.pack_weights_asym(W, 64)
    else:
        (pk, s), z = P.pack_weights_sym(W, 64), None
    w = Q4Weight(pk, s, z, 64, device=dev)
    X = torch.as_tensor(rng.normal(0, 1, (32, 128)).astype(np.float16)).to(dev)
    Y = w.matmul(X, out_dtype=torch.float32)
    rows = torch.cat([w.matmul(X[t:t + 1].contiguous(), out_dtype=torch.float32) for t in range(32)])
    linear.assert_close(Y.cpu().numpy(), rows.cpu().numpy(), 1e-5, "gemm vs gemv loop")


def test_gemm_bias_and_split_k_determinism(dev):
    rng = np.random.default_rng(12)
    N, K = 896, 4864                       # 28 output tiles at M=512: split-K path
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    b = rng.normal(0, 0.1, N).astype(np.float32)
    pk, s = P.pack_weights_sym(W, 64)
    X = rng.normal(0, 1, (512, K)).astype(np.float32)
    y, xk = gemm_dev(dev, pk, s, None, X, 64, torch.bfloat16, bias=b)
    linear.assert_close(y, linear.gemm(pk, s16(s), xk, 64) + b, TOL, "split-K + bias")
    w = Q4Weight(pk, s, None, 64, device=dev)
    xt = torch.as_tensor(X).to(dev).to(torch.bfloat16)
    first = w.matmul(xt, out_dtype=torch.float32).clone()
    for _ in range(5):
        assert torch.equal(w.matmul(xt, out_dtype=torch.float32), first)


@pytest.mark.parametrize("xdtype", [torch.float16, torch.bfloat16, torch.float32])
def test_gemm_unit_vector_rows_pin_mapping(dev, xdtype):
    """Row m of X = e_{k(m)}: Y[m, n] = q[n, k(m)] * s[n, k(m)/g] exactly (one product)."""
    rng = np.random.default_rng(31)
    N, K, g, M = 136, 320, 64, 150
    q = rng.integers(-8, 8, (N, K)).astype(np.int8)
    s = (np.arange(N * (K // g)).reshape(N, K // g) % 53 + 1).astype(np.float32) / 16
    w = Q4Weight(P.pack_rows(q), s, None, g, device=dev)
    kk = rng.integers(0, K, M)
    X = np.zeros((M, K), np.float32)
    X[np.arange(M), kk] = 1.0
    Y = w.matmul(torch.as_tensor(X).to(dev).to(xdtype), out_dtype=torch.float32).cpu().numpy()
    exp = (q[:, kk].astype(np.float64) * s[:, kk // g]).T
    np.testing.assert_array_equal(Y, exp.astype(np.float32))


@pytest.mark.parametrize("N,K,has_zeros", [(896, 4864, True), (896, 896, False), (896, 896, True)])
def test_gemm_partials_fold_into_rmsnorm(dev, N, K, has_zeros):
    """The prompt path's o / down projections: sf_q4_gemm_partials leaves the
    K-split partials and sf_rmsnorm_partials adds them to the residual rows and
    normalizes. Residual rows and normed outputs equal, bit for bit, the reduce
    into a delta buffer followed by sf_rmsnorm (the path they replace)."""
    from siliconfer_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(N + K)
    W = laplace_outliers(rng, (N, K))
    if has_zeros:
        pk, s, z = P.pack_weights_asym(W, 64)
    else:
        (pk, s), z = P.pack_weights_sym(W, 64), None
    w = Q4Weight(pk, s, z, 64, device=dev)
    M = 512
    S = lib.sf_q4_gemm_splits(M, N, K, 64)
    assert S > 1
    X = torch.as_tensor(rng.normal(0, 1, (M, K)).astype(np.float32)).to(dev).half().contiguous()
    h0 = torch.as_tensor(rng.normal(0, 1, (M, N)).astype(np.float32)).to(dev)
    nw = torch.as_tensor(rng.uniform(0.5, 1.5, N).astype(np.float32)).to(dev)
    wsb = lib.sf_q4_gemm_workspace_bytes(M, N, K, 64)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    F32, F16 = _lib.SF_F32, _lib.SF_F16
    # the reduce path
    Dl = torch.empty((M, N), dtype=torch.float32, device=dev)
    x1, o1 = h0.clone(), torch.empty((M, N), dtype=torch.float16, device=dev)
    _lib.check(lib.sf_q4_gemm(w.blob.data_ptr(), X.data_ptr(), F16, None, F32, Dl.data_ptr(), None, F32,
                              M, N, K, 64, int(has_zeros), ws.data_ptr(), wsb, st), "sf_q4_gemm")
    _lib.check(lib.sf_rmsnorm(x1.data_ptr(), Dl.data_ptr(), nw.data_ptr(), F32, o1.data_ptr(), F16, M, N,
                              1e-6, st), "sf_rmsnorm")
    # the partials path (the workspace first filled with something else)
    ws.fill_(0x7F)
    x2, o2 = h0.clone(), torch.empty((M, N), dtype=torch.float16, device=dev)
    _lib.check(lib.sf_q4_gemm_partials(w.blob.data_ptr(), X.data_ptr(), F16, M, N, K, 64, int(has_zeros),
                                       ws.data_ptr(), wsb, st), "sf_q4_gemm_partials")
    _lib.check(lib.sf_rmsnorm_partials(x2.data_ptr(), ws.data_ptr(), S, nw.data_ptr(), F32, o2.data_ptr(),
                                       F16, M, N, 1e-6, st), "sf_rmsnorm_partials")
    torch.cuda.synchronize()
    assert torch.equal(x1.view(torch.int32), x2.view(torch.int32))
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    # and the delta itself against the oracle's GEMM
    ref = linear.gemm(pk, s16(s), X.float().cpu().numpy().astype(np.float64), 64,
                      zeros=z)
    linear.assert_close((x2 - h0).double().cpu().numpy(), ref, 1e-3, f"partials delta [{N},{K}]")


@pytest.mark.parametrize("xdtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("M", [1, 5, 8, 9, 12, 16, 17])
def test_few_rows_run_as_batch_gemvs(dev, xdtype, M):
    """sf_q4_gemm at up to 16 rows runs as 8-row sf_q4_gemv slices: the same
    bits as those calls (the bias and the fp32 copy included); 17 rows take the
    tile kernel. Every case against the oracle."""
    from siliconfer_amd import _lib

    lib = _lib.load()
    F16, F32 = _lib.SF_F16, _lib.SF_F32
    rng = np.random.default_rng(300 + M)
    N, K, g = 1000, 768, 64
    pk, s, z = P.pack_weights_asym(rng.normal(0, 0.02, (N, K)).astype(np.float32), g)
    w = Q4Weight(pk, s, z, g, device=dev)
    bias = rng.normal(0, 0.1, N).astype(np.float32)
    X = torch.as_tensor(rng.normal(0, 1, (M, K)).astype(np.float32)).to(dev).to(xdtype).contiguous()
    b = torch.as_tensor(bias).to(dev)
    wsb = lib.sf_q4_gemm_workspace_bytes(M, N, K, g)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    xd = _lib.dt(X)
    Y = torch.full((M, N), 7.0, dtype=torch.float16, device=dev)
    Y32 = torch.full((M, N), 7.0, dtype=torch.float32, device=dev)
    _lib.check(lib.sf_q4_gemm(w.blob.data_ptr(), X.data_ptr(), xd, Y.data_ptr(), F16, Y32.data_ptr(),
                              b.data_ptr(), F32, M, N, K, g, 1, ws.data_ptr() if wsb else None, wsb, st),
               "sf_q4_gemm")
    if M <= 16:
        R = torch.empty_like(Y)
        R32 = torch.empty_like(Y32)
        for m0 in range(0, M, 8):
            mb = min(8, M - m0)
            _lib.check(lib.sf_q4_gemv(w.blob.data_ptr(), X[m0:].data_ptr(), xd, R[m0:].data_ptr(), F16,
                                      R32[m0:].data_ptr(), b.data_ptr(), F32, mb, N, K, g, 1, st),
                       "sf_q4_gemv")
        torch.cuda.synchronize()
        assert torch.equal(Y, R) and torch.equal(Y32, R32)
    torch.cuda.synchronize()
    xk = X.float().cpu().numpy().astype(np.float64)
    ref = linear.gemm(pk, s16(s), xk, g, zeros=z) + bias[None, :]
    linear.assert_close(Y32.cpu().numpy().astype(np.float64), ref, TOL, f"gemm M={M} {xdtype}")
    linear.assert_close(Y.float().cpu().numpy().astype(np.float64), ref, TOL, f"gemm fp16 out M={M} {xdtype}")
