"""Q4Linear on the GPU — the reference's tests/test_integration.py:81-171
restated against the oracle (fp16-stored scales; 1e-3 bar)."""

import numpy as np
import pytest
import torch

from oracle import linear, primitives as P
from siliconfer_amd.kernels import pack_weights_asym, pack_weights_sym
from siliconfer_amd.model import Q4Linear

pytestmark = pytest.mark.gpu
TOL = 1e-3


def s16(s):
    return np.asarray(s, np.float32).astype(np.float16).astype(np.float64)


def test_q4linear_matches_fake_quant(dev):
    rng = np.random.default_rng(1)
    W = rng.normal(0, 1, (32, 64)).astype(np.float32)
    x = rng.normal(0, 1, (1, 64)).astype(np.float32)
    pk, s = pack_weights_sym(W, group_size=64)
    layer = Q4Linear(pk, s, group_size=64)
    y = layer(torch.as_tensor(x).to(dev)).cpu().numpy()
    linear.assert_close(y[0], linear.gemv(pk, s16(s), x[0], 64), TOL, "q4linear")
    y_fq = P.fake_quantize(W, 64, True) @ x[0]
    assert np.abs(y[0] - y_fq).max() <= 2e-3 * np.abs(y_fq).max()   # fp16 scale storage


def test_q4linear_with_bias(dev):
    rng = np.random.default_rng(2)
    W = rng.normal(0, 1, (16, 64)).astype(np.float32)
    b = rng.normal(0, 0.1, 16).astype(np.float32)
    x = torch.as_tensor(rng.normal(0, 1, (1, 64)).astype(np.float32)).to(dev)
    pk, s = pack_weights_sym(W, group_size=64)
    y0 = Q4Linear(pk, s, group_size=64)(x)
    yb = Q4Linear(pk, s, bias=b, group_size=64)(x)
    np.testing.assert_allclose(yb.cpu().numpy(), y0.cpu().numpy() + b, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_q4linear_batch_and_seq(dev, dtype):
    rng = np.random.default_rng(3)
    W = rng.normal(0, 1, (32, 64)).astype(np.float32)
    x = torch.as_tensor(rng.normal(0, 1, (2, 5, 64)).astype(np.float32)).to(dev).to(dtype)
    pk, s = pack_weights_sym(W, group_size=64)
    y = Q4Linear(pk, s, group_size=64)(x)
    # fp32 out whatever x's dtype, as the reference's layer (q4_linear.py:55-63)
    assert y.shape == (2, 5, 32) and y.dtype == torch.float32
    ref = linear.gemm(pk, s16(s), x.float().reshape(10, 64).cpu().numpy().astype(np.float64), 64)
    linear.assert_close(y.reshape(10, 32).cpu().numpy(), ref, TOL, str(dtype))


def test_q4linear_asym_matches_fake_quant(dev):
    rng = np.random.default_rng(4)
    W = (rng.normal(0, 1, (32, 64)) + 1.0).astype(np.float32)
    x = rng.normal(0, 1, (1, 64)).astype(np.float32)
    pk, s, z = pack_weights_asym(W, group_size=64)
    y = Q4Linear(pk, s, zeros=z, group_size=64)(torch.as_tensor(x).to(dev)).cpu().numpy()[0]
    linear.assert_close(y, linear.gemv(pk, s16(s), x[0], 64, zeros=z), TOL, "asym")


def test_q4linear_asym_differs_from_sym_on_skewed(dev):
    rng = np.random.default_rng(5)
    W = (rng.normal(0, 1, (16, 64)) + 2.0).astype(np.float32)
    x = torch.as_tensor(rng.normal(0, 1, (1, 64)).astype(np.float32)).to(dev)
    pa, sa, za = pack_weights_asym(W, group_size=64)
    ps, ss = pack_weights_sym(W, group_size=64)
    ya = Q4Linear(pa, sa, zeros=za, group_size=64)(x).cpu().numpy()
    ys = Q4Linear(ps, ss, group_size=64)(x).cpu().numpy()
    assert not np.allclose(ya, ys, atol=1e-3)


def test_functional_api_numpy_in_numpy_out(dev):
    """siliconfer.kernels.neon-style calls with numpy arrays (test_kernel.py:68-80)."""
    from siliconfer_amd.kernels import gemm_asym, gemm_sym, gemv_asym, gemv_scalar, gemv_sym

    rng = np.random.default_rng(42)
    W = rng.normal(0, 1, (128, 256)).astype(np.float32)
    x = rng.normal(0, 1, 256).astype(np.float32)
    X = rng.normal(0, 1, (32, 256)).astype(np.float32)
    pk, s = pack_weights_sym(W, 64)
    y = gemv_sym(pk, s, x, 64)
    assert isinstance(y, np.ndarray) and y.dtype == np.float32 and y.shape == (128,)
    linear.assert_close(y, linear.gemv(pk, s16(s), x, 64), TOL, "gemv_sym")
    np.testing.assert_array_equal(gemv_scalar(pk, s, x, 64), y)
    linear.assert_close(gemm_sym(pk, s, X, 64), linear.gemm(pk, s16(s), X, 64), TOL, "gemm_sym")
    pa, sa, za = pack_weights_asym(W, 64)
    linear.assert_close(gemv_asym(pa, sa, za, x, 64), linear.gemv(pa, s16(sa), x, 64, zeros=za),
                        TOL, "gemv_asym")
    linear.assert_close(gemm_asym(pa, sa, za, X, 64), linear.gemm(pa, s16(sa), X, 64, zeros=za),
                        TOL, "gemm_asym")
    with pytest.raises(RuntimeError, match="x length mismatch"):
        gemv_sym(pk, s, x[:128], 64)
    with pytest.raises(RuntimeError, match="scales shape mismatch"):
        gemv_sym(pk, s[:, :2], x, 64)
