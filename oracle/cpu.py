"""ctypes bindings for the CPU checker libraries. TEST INFRASTRUCTURE ONLY.

* `port`      — oracle/liboracle_cpu.so built from oracle/q4_cpu.c (the C
                restatement of the reference's scalar CPU kernels).
* `reference` — oracle/_ref/libref_q4.so built by oracle/Makefile from the
                reference's own q4_gemv.cpp / q4_gemm.cpp (symmetric path only;
                see oracle/ref_glue.cpp). Absent where /root/reference is absent
                and the library was not carried over.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
PORT_PATH = os.path.join(_HERE, "liboracle_cpu.so")
REF_PATH = os.path.join(_HERE, "_ref", "libref_q4.so")

_u8p = ctypes.POINTER(ctypes.c_uint8)
_i8p = ctypes.POINTER(ctypes.c_int8)
_f32p = ctypes.POINTER(ctypes.c_float)
_i = ctypes.c_int

_port = None
_ref = None


def build() -> None:
    """Run oracle/Makefile (C restatement, plus _ref when the reference is present)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def port_lib():
    global _port
    if _port is None:
        if not os.path.exists(PORT_PATH):
            raise FileNotFoundError(f"{PORT_PATH} not built (run `make -C oracle`)")
        lib = ctypes.CDLL(PORT_PATH)
        lib.oc_gemv_sym.argtypes = [_u8p, _f32p, _f32p, _f32p, _i, _i, _i, _i]
        lib.oc_gemv_asym.argtypes = [_u8p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i]
        lib.oc_gemm_sym.argtypes = [_u8p, _f32p, _f32p, _f32p, _i, _i, _i, _i, _i]
        lib.oc_gemm_asym.argtypes = [_u8p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i, _i]
        lib.oc_attn_decode.argtypes = [_f32p, _i8p, _f32p, _i8p, _f32p, _f32p,
                                       _i, _i, _i, _i, _i, _i, ctypes.c_float, _i]
        lib.oc_attn_decode.restype = _i
        lib.oc_max_threads.restype = _i
        for f in ("oc_gemv_sym", "oc_gemv_asym", "oc_gemm_sym", "oc_gemm_asym"):
            getattr(lib, f).restype = None
        _port = lib
    return _port


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref_lib():
    global _ref
    if _ref is None:
        if not ref_available():
            raise FileNotFoundError(f"{REF_PATH} not built (needs /root/reference)")
        lib = ctypes.CDLL(REF_PATH)
        lib.ref_q4_gemv_sym_scalar.argtypes = [_u8p, _f32p, _f32p, _f32p, _i, _i, _i]
        lib.ref_q4_gemv_sym.argtypes = [_u8p, _f32p, _f32p, _f32p, _i, _i, _i]
        lib.ref_q4_gemm_sym.argtypes = [_u8p, _f32p, _f32p, _f32p, _i, _i, _i, _i]
        lib.ref_q4_gemv_sym_rows.argtypes = [_u8p, _f32p, _f32p, _f32p, _i, _i, _i, _i]
        _ref = lib
    return _ref


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def gemv_sym(packed, scales, x, group_size, nthreads=1, impl="port"):
    packed, scales, x = _c(packed, np.uint8), _c(scales, np.float32), _c(x, np.float32)
    N, Kh = packed.shape
    y = np.empty(N, dtype=np.float32)
    if impl == "port":
        port_lib().oc_gemv_sym(_ptr(packed, _u8p), _ptr(scales, _f32p), _ptr(x, _f32p),
                               _ptr(y, _f32p), N, 2 * Kh, group_size, nthreads)
    elif impl == "reference":
        ref_lib().ref_q4_gemv_sym(_ptr(packed, _u8p), _ptr(scales, _f32p), _ptr(x, _f32p),
                                  _ptr(y, _f32p), N, 2 * Kh, group_size)
    elif impl == "reference_scalar":
        ref_lib().ref_q4_gemv_sym_scalar(_ptr(packed, _u8p), _ptr(scales, _f32p), _ptr(x, _f32p),
                                         _ptr(y, _f32p), N, 2 * Kh, group_size)
    else:
        raise ValueError(impl)
    return y


def gemv_sym_ref_rows(packed, scales, x, group_size, parts=1):
    """The reference's q4_gemv_sym (q4_gemv.cpp:240-247, scalar on x86) over
    `parts` row slices on an OpenMP team of `parts` threads (ref_glue.cpp).
    Each row's sum is the reference's own; only the rows are dealt out.
    packed/scales must already be contiguous u8 / fp32."""
    N, Kh = packed.shape
    x = _c(x, np.float32).reshape(-1)
    y = np.empty(N, dtype=np.float32)
    ref_lib().ref_q4_gemv_sym_rows(_ptr(packed, _u8p), _ptr(scales, _f32p), _ptr(x, _f32p),
                                   _ptr(y, _f32p), N, 2 * Kh, group_size, parts)
    return y


def gemv_asym(packed, scales, zeros, x, group_size, nthreads=1):
    packed, scales = _c(packed, np.uint8), _c(scales, np.float32)
    zeros, x = _c(zeros, np.float32), _c(x, np.float32)
    N, Kh = packed.shape
    y = np.empty(N, dtype=np.float32)
    port_lib().oc_gemv_asym(_ptr(packed, _u8p), _ptr(scales, _f32p), _ptr(zeros, _f32p),
                            _ptr(x, _f32p), _ptr(y, _f32p), N, 2 * Kh, group_size, nthreads)
    return y


def gemm_sym(packed, scales, X, group_size, nthreads=1, impl="port"):
    packed, scales, X = _c(packed, np.uint8), _c(scales, np.float32), _c(X, np.float32)
    N, Kh = packed.shape
    T = X.shape[0]
    Y = np.empty((T, N), dtype=np.float32)
    if impl == "port":
        port_lib().oc_gemm_sym(_ptr(packed, _u8p), _ptr(scales, _f32p), _ptr(X, _f32p),
                               _ptr(Y, _f32p), T, N, 2 * Kh, group_size, nthreads)
    elif impl == "reference":
        ref_lib().ref_q4_gemm_sym(_ptr(packed, _u8p), _ptr(scales, _f32p), _ptr(X, _f32p),
                                  _ptr(Y, _f32p), N, 2 * Kh, T, group_size)
    else:
        raise ValueError(impl)
    return Y


def gemm_asym(packed, scales, zeros, X, group_size, nthreads=1):
    packed, scales = _c(packed, np.uint8), _c(scales, np.float32)
    zeros, X = _c(zeros, np.float32), _c(X, np.float32)
    N, Kh = packed.shape
    T = X.shape[0]
    Y = np.empty((T, N), dtype=np.float32)
    port_lib().oc_gemm_asym(_ptr(packed, _u8p), _ptr(scales, _f32p), _ptr(zeros, _f32p),
                            _ptr(X, _f32p), _ptr(Y, _f32p), T, N, 2 * Kh, group_size, nthreads)
    return Y


def attn_decode(q, k_codes, k_scales, v_codes, v_scales, T=None, scale=None, nthreads=1):
    q = _c(q, np.float32)
    B, H, D = q.shape
    KVH, Tcap = k_codes.shape[1], k_codes.shape[2]
    if T is None:
        T = Tcap
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    kc, vc = _c(k_codes, np.int8), _c(v_codes, np.int8)
    ks = _c(np.asarray(k_scales).reshape(B, KVH, Tcap), np.float32)
    vs = _c(np.asarray(v_scales).reshape(B, KVH, Tcap), np.float32)
    out = np.empty((B, H, D), dtype=np.float32)
    rc = port_lib().oc_attn_decode(_ptr(q, _f32p), _ptr(kc, _i8p), _ptr(ks, _f32p), _ptr(vc, _i8p),
                                   _ptr(vs, _f32p), _ptr(out, _f32p), B, H, KVH, T, Tcap, D,
                                   float(scale), nthreads)
    if rc != 0:
        raise ValueError("H must be a multiple of KVH")
    return out


def max_threads() -> int:
    return int(port_lib().oc_max_threads())
