"""Device int4 weights and the GEMV / GEMM calls on them.

`Q4Weight` owns the device blob that `sf_q4_repack` builds from the reference's
canonical packed tensors (siliconfer/kernels/neon/__init__.py:42-81). Its
`matmul` routes rows <= 8 to the decode GEMV where its MFMA plan takes the
shape (sf_q4_gemv_supported) and everything else to the prefill GEMM — the
roles of q4_gemv_* and q4_gemm_* in the reference
(siliconfer/kernels/neon/bindings.cpp:45-150). Every K and group size the
reference takes (K % group_size == 0) computes.
"""

from __future__ import annotations

import numpy as np
import torch

from .. import _lib
from .._lib import SFError

GEMV_MAX_ROWS = 8


def _as_tensor(a, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    if isinstance(a, np.ndarray):
        a = torch.from_numpy(np.ascontiguousarray(a))
    if not isinstance(a, torch.Tensor):
        a = torch.as_tensor(a)
    return a.to(device=device, dtype=dtype).contiguous()


def _zeros_u8(zeros, device: torch.device) -> torch.Tensor:
    """Zero-points arrive as the reference's float32 [N, G] array of integers."""
    z = zeros.detach().cpu().numpy() if isinstance(zeros, torch.Tensor) else np.asarray(zeros)
    zr = np.rint(z)
    if not np.array_equal(zr, z) or zr.min(initial=0) < 0 or zr.max(initial=0) > 15:
        raise SFError("zeros must be integers in [0, 15] (uint4 zero-points)")
    return torch.from_numpy(zr.astype(np.uint8)).to(device)


class Q4Weight:
    """An N x K int4 matrix resident in HBM in the kernels' blob layout.

    Args mirror Q4Linear's (siliconfer/model/q4_linear.py:32-47): `packed`
    uint8 [N, K/2]; `scales` [N, K/g] (stored as fp16); `zeros` [N, K/g]
    integral zero-points or None for symmetric codes.
    """

    def __init__(self, packed, scales, zeros=None, group_size: int = 128, device=None):
        dev = torch.device(device) if device is not None else torch.device(
            "cuda", torch.cuda.current_device() if torch.cuda.is_available() else 0)
        pk_shape = tuple(packed.shape)
        if len(pk_shape) != 2:
            raise SFError("W must be 2-D [out, in/2]")
        N, Kh = pk_shape
        K = 2 * Kh
        if group_size <= 0 or K % group_size != 0:
            raise SFError("in_features must be divisible by group_size")
        G = K // group_size
        if tuple(scales.shape) != (N, G):
            raise SFError("scales shape mismatch")
        if zeros is not None and tuple(zeros.shape) != (N, G):
            raise SFError("zeros shape mismatch")
        self.out_features, self.in_features, self.group_size = N, K, group_size
        self.has_zeros = zeros is not None
        self.device = dev
        lib = _lib.load()
        nbytes = lib.sf_q4_blob_bytes(N, K, group_size, int(self.has_zeros))
        if nbytes == 0:
            raise SFError("invalid int4 weight shape")
        pk = _as_tensor(packed, torch.uint8, dev)
        sc = _as_tensor(scales, torch.float16, dev)
        zu = _zeros_u8(zeros, dev) if self.has_zeros else None
        self.blob = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _lib.check(lib.sf_q4_repack(pk.data_ptr(), sc.data_ptr(), _lib.ptr(zu), N, K, group_size,
                                    self.blob.data_ptr(), nbytes, _lib.stream(self.blob)),
                   "sf_q4_repack")

    @property
    def nbytes(self) -> int:
        return self.blob.numel()

    def canonical(self):
        """(packed u8 [N,K/2], scales f16 [N,G], zeros u8 [N,G] or None) on the device."""
        N, K, g = self.out_features, self.in_features, self.group_size
        dev = self.device
        pk = torch.empty((N, K // 2), dtype=torch.uint8, device=dev)
        sc = torch.empty((N, K // g), dtype=torch.float16, device=dev)
        zu = torch.empty((N, K // g), dtype=torch.uint8, device=dev) if self.has_zeros else None
        _lib.check(_lib.load().sf_q4_unpack(self.blob.data_ptr(), N, K, g, int(self.has_zeros),
                                            pk.data_ptr(), sc.data_ptr(), _lib.ptr(zu),
                                            _lib.stream(self.blob)), "sf_q4_unpack")
        return pk, sc, zu

    def matmul(self, x: torch.Tensor, out_dtype: torch.dtype | None = None,
               bias: torch.Tensor | None = None, out: torch.Tensor | None = None,
               out_f32: torch.Tensor | None = None) -> torch.Tensor:
        """x [M, K] (fp16 / bf16 / fp32, on the device) -> [M, N] of out_dtype (default x.dtype)."""
        _lib.require_device(x, "x")
        if x.dim() != 2 or x.shape[1] != self.in_features:
            raise SFError("X/W in_features mismatch")
        M = x.shape[0]
        N, K, g = self.out_features, self.in_features, self.group_size
        if out_dtype is None:
            out_dtype = x.dtype
        if out is None and out_f32 is None:
            out = torch.empty((M, N), dtype=out_dtype, device=x.device)
        if M == 0:
            return out if out is not None else out_f32
        if bias is not None:
            _lib.require_device(bias, "bias")
        lib = _lib.load()
        st = _lib.stream(x)
        ydt = _lib.dt(out) if out is not None else _lib.SF_F32
        bdt = _lib.dt(bias) if bias is not None else 0
        if M <= GEMV_MAX_ROWS and lib.sf_q4_gemv_supported(M, N, K, g, _lib.dt(x)):
            rc = lib.sf_q4_gemv(self.blob.data_ptr(), x.data_ptr(), _lib.dt(x), _lib.ptr(out), ydt,
                                _lib.ptr(out_f32), _lib.ptr(bias), bdt, M, N, K, g,
                                int(self.has_zeros), st)
            _lib.check(rc, "sf_q4_gemv")
        else:
            ws_bytes = lib.sf_q4_gemm_workspace_bytes(M, N, K, g)
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device) if ws_bytes else None
            rc = lib.sf_q4_gemm(self.blob.data_ptr(), x.data_ptr(), _lib.dt(x), _lib.ptr(out), ydt,
                                _lib.ptr(out_f32), _lib.ptr(bias), bdt, M, N, K, g,
                                int(self.has_zeros), _lib.ptr(ws), ws_bytes, st)
            _lib.check(rc, "sf_q4_gemm")
        return out if out is not None else out_f32
