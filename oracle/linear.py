"""Oracle for the int4 GEMV / GEMM (decode and prefill through `Q4Linear`).

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`).

What the reference computes (/root/reference):
  sym GEMV   siliconfer/kernels/neon/q4_gemv.cpp:262-297 (scalar, what runs on x86)
             and :37-140 (NEON): y[i] = sum_g s[i,g] * sum_{k in g} q[i,k] * x[k]
  asym GEMV  siliconfer/kernels/neon/q4_gemv.cpp:145-238:
             y[i] = sum_g s[i,g] * (sum_{k in g} q[i,k] x[k] - z[i,g] * sum_{k in g} x[k])
             (the reference's numpy twin is kernels/neon/__init__.py:109-124)
  GEMM       siliconfer/kernels/neon/q4_gemm.cpp:12-51: Y[t,:] = GEMV(X[t,:]) for t < T
  Q4Linear   siliconfer/model/q4_linear.py:49-68: [...,K] -> [T,K] -> GEMM -> [...,N] (+bias)

The oracle evaluates the same real-valued quantity in float64: dequantize the
packed weights exactly (q*s and (q-z)*s are exact in float64) and take the
matrix product with the float64-upcast activations. The reference tests use this
very form as their own oracle (tests/test_kernel.py:28-31, 161-164, 207-208).

Pinning (tests/test_oracle_linear.py):
  * golden vectors from the reference's own compiled `q4_gemv_sym_scalar` /
    `q4_gemm_sym_neon` (tests/golden/, made by tests/golden/make_golden.py from
    oracle/_ref), within float32 accumulation error;
  * brute-force scalar loops on tiny inputs (the group-wise sum order of
    q4_gemv.cpp:276-293), zero input -> 0, single row, linearity in x,
    GEMM == loop of GEMVs;
  * asym: the factorised form (q4_gemv.cpp:234) equals the direct (q-z)*s form.
"""

from __future__ import annotations

import numpy as np

from .primitives import dequant_packed, unpack_rows


def gemv(packed: np.ndarray, scales: np.ndarray, x: np.ndarray, group_size: int,
         zeros: np.ndarray | None = None) -> np.ndarray:
    """y = dequant(W) @ x in float64. x: [K] or [B, K] -> [N] or [B, N]."""
    w = dequant_packed(packed, scales, zeros, group_size, np.float64)
    x64 = np.asarray(x, dtype=np.float64)
    return x64 @ w.T


def gemm(packed: np.ndarray, scales: np.ndarray, X: np.ndarray, group_size: int,
         zeros: np.ndarray | None = None) -> np.ndarray:
    """Y[T, N] = X[T, K] @ dequant(W).T in float64."""
    X = np.asarray(X)
    if X.ndim != 2:
        raise ValueError("X must be 2-D [T, in_f]")
    return gemv(packed, scales, X, group_size, zeros)


def gemv_groupwise_loops(packed: np.ndarray, scales: np.ndarray, x: np.ndarray,
                         group_size: int, zeros: np.ndarray | None = None) -> np.ndarray:
    """Pure-Python loop form following q4_gemv.cpp:272-296 literally: per row,
    per group, integer-code dot product, then one multiply by the group scale.
    For tiny inputs only; used to pin `gemv` against the reference's sum order."""
    signed = zeros is None
    q = unpack_rows(np.asarray(packed), signed=signed).astype(np.int64)
    n, k = q.shape
    g = group_size
    y = np.zeros(n, dtype=np.float64)
    xs = [float(v) for v in np.asarray(x, dtype=np.float64)]
    for i in range(n):
        acc = 0.0
        for gi in range(k // g):
            dot = 0.0
            xsum = 0.0
            for kk in range(gi * g, (gi + 1) * g):
                dot += int(q[i, kk]) * xs[kk]
                xsum += xs[kk]
            if zeros is not None:
                dot -= float(zeros[i, gi]) * xsum
            acc += dot * float(scales[i, gi])
        y[i] = acc
    return y


def assert_close(y: np.ndarray, y_ref: np.ndarray, tol: float, what: str = "") -> None:
    """Parity assertion: norm-relative AND elementwise (rtol + atol floor)."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    assert y.shape == y_ref.shape, f"{what}: shape {y.shape} != {y_ref.shape}"
    assert np.all(np.isfinite(y)), f"{what}: non-finite output"
    scale = max(float(np.max(np.abs(y_ref))), 1e-30) if y_ref.size else 1.0
    err = np.abs(y - y_ref)
    if err.size == 0:
        return
    norm_rel = float(err.max()) / scale
    bound = tol * np.abs(y_ref) + tol * scale
    worst = float(np.max(err - bound))
    assert norm_rel <= tol and worst <= 0.0, (
        f"{what}: norm-relative err {norm_rel:.3e} (tol {tol:g}); "
        f"elementwise excess {worst:.3e}; max|ref| {scale:.3e}")
