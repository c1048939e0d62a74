"""Pins the oracle's GEMV / GEMM (CPU only).

Against: golden vectors from the reference's compiled q4_gemv.cpp / q4_gemm.cpp
(tests/golden/, made by make_golden.py); the reference's live compiled kernels
when oracle/_ref is built; the literal group-wise loop of q4_gemv.cpp:272-296;
and mathematical invariants (zero input, linearity, GEMM == GEMV loop,
asym factorised form == direct form).
"""

import numpy as np
import pytest

from conftest import golden_cases, load_golden
from oracle import cpu, linear, primitives as P

# fp32 accumulation in the reference vs float64 here: a few ulps of the output scale
F32_TOL = 2e-6


@pytest.mark.parametrize("name", golden_cases())
def test_oracle_matches_reference_golden(name):
    c = load_golden(name)
    g = int(c["g"])
    for sk, yk in (("scales", "y_ref"), ("scales16", "y_ref16")):
        s = c[sk].astype(np.float32)
        y = linear.gemm(c["packed"], s, c["x"], g) if int(c["T"]) else linear.gemv(c["packed"], s, c["x"], g)
        linear.assert_close(y, c[yk], F32_TOL, f"{name}/{sk}")


def test_golden_inputs_are_oracle_quantized():
    """The fixtures' packed tensors are what the oracle's quantizer produces."""
    c = load_golden("gemv_128x256_g64")
    rng = np.random.default_rng(int(c["seed"]))
    W = rng.normal(0, 1, (128, 256)).astype(np.float32)
    pk, s = P.pack_weights_sym(W, 64)
    np.testing.assert_array_equal(pk, c["packed"])
    np.testing.assert_array_equal(s, c["scales"])


@pytest.mark.skipif(not cpu.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("N,K,g", [(4864, 896, 64), (512, 4096, 128), (300, 11008, 128)])
def test_oracle_matches_live_reference_at_config_widths(N, K, g):
    rng = np.random.default_rng(N + K)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    x = rng.normal(0, 1, K).astype(np.float16).astype(np.float32)
    pk, s = P.pack_weights_sym(W, g)
    y_ref = cpu.gemv_sym(pk, s, x, g, impl="reference")
    linear.assert_close(linear.gemv(pk, s, x, g), y_ref, 1e-5, "live reference")


@pytest.mark.skipif(not cpu.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("parts", [1, 3, 7])
def test_reference_row_split_equals_whole_call(parts):
    """The CPU baseline's all-cores leg deals rows of the reference's own
    kernel to threads: every row's bits equal the single call's."""
    rng = np.random.default_rng(parts)
    W = rng.normal(0, 0.02, (1157, 896)).astype(np.float32)
    x = rng.normal(0, 1, 896).astype(np.float32)
    pk, s = P.pack_weights_sym(W, 64)
    s = np.ascontiguousarray(s, np.float32)
    whole = cpu.gemv_sym(pk, s, x, 64, impl="reference")
    split = cpu.gemv_sym_ref_rows(np.ascontiguousarray(pk), s, x, 64, parts)
    np.testing.assert_array_equal(split, whole)


def test_oracle_matches_literal_loop():
    rng = np.random.default_rng(2)
    W = rng.normal(0, 1, (6, 128)).astype(np.float32)
    x = rng.normal(0, 1, 128)
    pk, s = P.pack_weights_sym(W, 64)
    np.testing.assert_allclose(linear.gemv(pk, s, x, 64), linear.gemv_groupwise_loops(pk, s, x, 64),
                               rtol=1e-12, atol=1e-12)
    pa, sa, za = P.pack_weights_asym(W, 32)
    np.testing.assert_allclose(linear.gemv(pa, sa, x, 32, zeros=za),
                               linear.gemv_groupwise_loops(pa, sa, x, 32, zeros=za),
                               rtol=1e-12, atol=1e-12)


def test_oracle_gemv_equals_fake_quant_matmul():
    """The reference tests' oracle form (test_kernel.py:28-31, 161-164)."""
    rng = np.random.default_rng(42)
    W = rng.normal(0, 1, (128, 256)).astype(np.float32)
    x = rng.normal(0, 1, 256).astype(np.float32)
    for sym in (True, False):
        if sym:
            pk, s = P.pack_weights_sym(W, 64)
            y = linear.gemv(pk, s, x, 64)
        else:
            pk, s, z = P.pack_weights_asym(W, 64)
            y = linear.gemv(pk, s, x, 64, zeros=z)
        y_fq = P.fake_quantize(W, 64, sym).astype(np.float64) @ x.astype(np.float64)
        np.testing.assert_allclose(y, y_fq, rtol=1e-5, atol=1e-5)


def test_oracle_zero_input_and_linearity():
    rng = np.random.default_rng(0)
    W = rng.normal(0, 1, (32, 128)).astype(np.float32)
    pk, s = P.pack_weights_sym(W, 128)
    assert np.all(linear.gemv(pk, s, np.zeros(128), 128) == 0)
    a, b = rng.normal(0, 1, 128), rng.normal(0, 1, 128)
    np.testing.assert_allclose(linear.gemv(pk, s, 2 * a - 3 * b, 128),
                               2 * linear.gemv(pk, s, a, 128) - 3 * linear.gemv(pk, s, b, 128),
                               rtol=1e-12, atol=1e-12)


def test_oracle_gemm_is_gemv_loop():
    rng = np.random.default_rng(99)
    W = rng.normal(0, 1, (64, 128)).astype(np.float32)
    X = rng.normal(0, 1, (7, 128))
    pk, s, z = P.pack_weights_asym(W, 64)
    Y = linear.gemm(pk, s, X, 64, zeros=z)
    for t in range(7):
        np.testing.assert_allclose(Y[t], linear.gemv(pk, s, X[t], 64, zeros=z), rtol=1e-13, atol=1e-13)


def test_c_port_matches_oracle():
    """The C restatement used as the timed CPU baseline computes the same thing."""
    rng = np.random.default_rng(5)
    W = rng.normal(0, 0.02, (200, 896)).astype(np.float32)
    x = rng.normal(0, 1, 896).astype(np.float32)
    pk, s = P.pack_weights_sym(W, 64)
    for nt in (1, 4):
        linear.assert_close(cpu.gemv_sym(pk, s, x, 64, nthreads=nt), linear.gemv(pk, s, x, 64), 1e-5, "port sym")
    pa, sa, za = P.pack_weights_asym(W, 64)
    linear.assert_close(cpu.gemv_asym(pa, sa, za, x, 64, nthreads=2),
                        linear.gemv(pa, sa, x, 64, zeros=za), 1e-5, "port asym")
    X = rng.normal(0, 1, (3, 896)).astype(np.float32)
    linear.assert_close(cpu.gemm_asym(pa, sa, za, X, 64), linear.gemm(pa, sa, X, 64, zeros=za), 1e-5, "port gemm")


def test_planted_mistakes_are_caught():
    """A dropped zero-point, a swapped nibble order or a wrong sign fails the bar."""
    rng = np.random.default_rng(8)
    W = rng.normal(0.3, 1, (16, 128)).astype(np.float32)
    x = rng.normal(0, 1, 128)
    pa, sa, za = P.pack_weights_asym(W, 64)
    good = linear.gemv(pa, sa, x, 64, zeros=za)
    with pytest.raises(AssertionError):
        linear.assert_close(linear.gemv(pa, sa, x, 64, zeros=np.zeros_like(za)), good, 1e-3)
    swapped = ((pa >> 4) | (pa << 4)).astype(np.uint8)
    with pytest.raises(AssertionError):
        linear.assert_close(linear.gemv(swapped, sa, x, 64, zeros=za), good, 1e-3)
    pk, s = P.pack_weights_sym(W, 64)
    unsigned_read = linear.gemv(pk, s, x, 64, zeros=np.zeros_like(s))  # codes as unsigned
    with pytest.raises(AssertionError):
        linear.assert_close(unsigned_read, linear.gemv(pk, s, x, 64), 1e-3)
