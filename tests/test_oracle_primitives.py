"""Pins the oracle's quantize / pack / unpack restatement, and checks the
product's offline quantizers against it (CPU only).

Reference: siliconfer/quant/primitives.py, siliconfer/kernels/neon/__init__.py:42-81,
tests/test_primitives.py, tests/test_kernel.py:38-61.
"""

import itertools

import numpy as np
import pytest

from oracle import primitives as P
from siliconfer_amd import kernels as K
from siliconfer_amd.quant import primitives as QP


# ---- unpack: exhaustive known answers --------------------------------------

def test_unpack_all_256_bytes_signed_and_unsigned():
    b = np.arange(256, dtype=np.uint8)
    u = P.unpack_int4(b, 512, signed=False).reshape(256, 2)
    s = P.unpack_int4(b, 512, signed=True).reshape(256, 2)
    for v in range(256):
        lo, hi = v & 15, v >> 4
        assert (u[v, 0], u[v, 1]) == (lo, hi)
        assert (s[v, 0], s[v, 1]) == (lo - 16 * (lo >= 8), hi - 16 * (hi >= 8))
    assert s.min() == -8 and s.max() == 7


def test_reference_literal_boundary_vector():
    values = np.array([-8, -1, 0, 1, 7, -8, 7, -1], dtype=np.int8)  # test_primitives.py:148
    packed = P.pack_int4(values)
    assert packed.tolist() == [0xF8, 0x10, 0x87, 0xF7]
    np.testing.assert_array_equal(P.unpack_int4(packed, 8, signed=True), values)


def test_pack_lo_even_hi_odd_round_trip():
    rng = np.random.default_rng(7)
    q = rng.integers(-8, 8, size=(5, 64), dtype=np.int8)
    pk = P.pack_rows(q)
    assert pk.shape == (5, 32)
    np.testing.assert_array_equal(pk & 15, (q[:, 0::2] & 15).astype(np.uint8))
    np.testing.assert_array_equal(pk >> 4, (q[:, 1::2] & 15).astype(np.uint8))
    np.testing.assert_array_equal(P.unpack_rows(pk, signed=True), q)


def test_pack_odd_count_raises():
    with pytest.raises(ValueError, match="even"):
        P.pack_int4(np.array([1, 2, 3], dtype=np.int8))


# ---- quantize_sym ------------------------------------------------------------

def test_quantize_sym_invariants():
    rng = np.random.default_rng(0)
    w = rng.normal(0, 10, (32, 256)).astype(np.float32)
    q, s = P.quantize_sym(w, 64)
    assert q.dtype == np.int8 and s.shape == (32, 4)
    assert q.min() >= -7 and q.max() <= 7       # -8 is never produced (|w|/s <= 7)
    # the max-|w| element of every group maps to +-7 exactly
    g = np.abs(w.reshape(32, 4, 64)).argmax(-1)
    qa = np.take_along_axis(np.abs(q.reshape(32, 4, 64)), g[..., None], -1)
    assert np.all(qa == 7)
    np.testing.assert_array_equal(s, (np.abs(w.reshape(32, 4, 64)).max(-1) / np.float32(7)))


def test_quantize_sym_is_nearest_code_brute_force():
    """Each code is the argmin over the 16 codes of |w - q*s| in float32 (ties -> even)."""
    rng = np.random.default_rng(3)
    w = rng.normal(0, 1, (4, 32)).astype(np.float32)
    q, s = P.quantize_sym(w, 32)
    codes = np.arange(-8, 8, dtype=np.float32)
    for i, j in itertools.product(range(4), range(32)):
        r = np.float32(w[i, j]) / s[i, 0]
        best = codes[np.argmin(np.abs(codes - r))]
        assert q[i, j] == best


def test_quantize_round_half_even_ties():
    # group max 7 -> s = 1; w = 2.5 -> 2, 3.5 -> 4, -0.5 -> -0 (even)
    w = np.array([[7.0, 2.5, 3.5, -0.5] + [0.0] * 28], dtype=np.float32)
    q, s = P.quantize_sym(w, 32)
    assert s[0, 0] == 1.0
    assert q[0, :4].tolist() == [7, 2, 4, 0]


def test_zero_group_scale_zero_codes_zero():
    w = np.zeros((8, 128), dtype=np.float32)
    q, s = P.quantize_sym(w, 128)
    assert np.all(q == 0) and np.all(s == 0)
    qa, sa, za = P.quantize_asym(w, 128)
    assert np.all(qa == 0) and np.all(sa == 0) and np.all(za == 0)


# ---- quantize_asym -------------------------------------------------------------

def test_quantize_asym_invariants():
    rng = np.random.default_rng(1)
    w = rng.uniform(-5, 3, (16, 256)).astype(np.float32)
    q, s, z = P.quantize_asym(w, 128)
    assert q.dtype == np.uint8 and q.max() <= 15
    assert np.all(z == np.rint(z)) and z.min() >= 0 and z.max() <= 15
    deq = P.dequantize_asym(q, s, z, 128)
    assert np.abs(deq - w).max() <= s.max() + 1e-5   # test_primitives.py:79-89 bound


def test_asym_beats_sym_on_skewed():
    rng = np.random.default_rng(99)
    w = rng.uniform(0, 4, (32, 128)).astype(np.float32)
    e_sym = np.sqrt(np.mean((w - P.fake_quantize(w, 128, True)) ** 2))
    e_asym = np.sqrt(np.mean((w - P.fake_quantize(w, 128, False)) ** 2))
    assert e_asym < e_sym


def test_group_size_not_divisible_raises():
    with pytest.raises(ValueError, match="not divisible"):
        P.quantize_sym(np.zeros((8, 100), np.float32), 128)


# ---- dequant value exactness (fp16 scales) -----------------------------------------

def test_dequant_product_exact_in_fp32_for_fp16_scales():
    """q*s and (q-z)*s with an fp16 scale need <= 15 significant bits: exact in fp32.
    Enumerates all 16 codes x all finite positive fp16 scales."""
    s16 = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    for code in range(-15, 16):
        exact = code * s16
        assert np.array_equal(exact.astype(np.float32).astype(np.float64), exact)


# ---- product quantizers == oracle (bit-exact) ----------------------------------------

@pytest.mark.parametrize("g", [32, 64, 128])
def test_product_pack_weights_match_oracle(g):
    rng = np.random.default_rng(g)
    W = rng.normal(0, 0.02, (48, 256)).astype(np.float32)
    pk, s = K.pack_weights_sym(W, g)
    pk_o, s_o = P.pack_weights_sym(W, g)
    np.testing.assert_array_equal(pk, pk_o)
    np.testing.assert_array_equal(s, s_o)
    pa, sa, za = K.pack_weights_asym(W + 0.01, g)
    pa_o, sa_o, za_o = P.pack_weights_asym(W + 0.01, g)
    np.testing.assert_array_equal(pa, pa_o)
    np.testing.assert_array_equal(sa, sa_o)
    np.testing.assert_array_equal(za, za_o)


def test_product_pack_unpack_match_oracle():
    rng = np.random.default_rng(13)
    u = rng.integers(0, 16, size=128, dtype=np.uint8)
    np.testing.assert_array_equal(QP.pack_int4(u), P.pack_int4(u))
    np.testing.assert_array_equal(QP.unpack_int4(QP.pack_int4(u), 128, signed=False), u)
    s = rng.integers(-8, 8, size=64, dtype=np.int8)
    np.testing.assert_array_equal(QP.unpack_int4(QP.pack_int4(s), 64, signed=True), s)
    w = rng.normal(0, 1, (16, 128)).astype(np.float32)
    for sym in (True, False):
        np.testing.assert_array_equal(QP.fake_quantize(w, 64, sym), P.fake_quantize(w, 64, sym))
