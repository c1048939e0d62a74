"""Q4Linear: drop-in replacement for a linear layer backed by the int4 HIP kernels.

Same constructor and call contract as the reference's
`siliconfer.model.q4_linear.Q4Linear` (/root/reference/siliconfer/model/q4_linear.py:12-68):
`Q4Linear(packed, scales, zeros=None, bias=None, group_size=128)`; `layer(x)`
maps [..., in_features] -> [..., out_features] and adds `bias`.

Where the reference evaluates the MLX graph, copies x to the host and runs the
CPU GEMM on every call (q4_linear.py:51-63), this layer keeps the weights in
HBM as a repacked blob and runs entirely on the device stream: rows <= 8 go to
the decode GEMV, more rows to the MFMA prefill GEMM. The output is fp32 like
the reference's (it casts x to fp32 and its GEMM returns fp32, q4_linear.py:55-63);
fp16 / bf16 x are read as they are, which equals the reference's upcast since
every fp16 / bf16 value is exact in fp32. The bias is added in fp32.
"""

from __future__ import annotations

import numpy as np
import torch

from ..kernels.q4 import Q4Weight


class Q4Linear(torch.nn.Module):
    """Holds `_packed` uint8 [out, in/2], `_scales` [out, n_groups], `_zeros`
    [out, n_groups] or None (host copies, as the reference keeps them), plus the
    device `weight` (Q4Weight) the kernels read."""

    def __init__(self, packed, scales, zeros=None, bias=None, group_size: int = 128,
                 device=None) -> None:
        super().__init__()
        self._packed = packed
        self._scales = scales
        self._zeros = zeros
        self.group_size = group_size
        self.out_features = packed.shape[0]
        self.in_features = packed.shape[1] * 2
        self.weight = Q4Weight(packed, scales, zeros, group_size, device=device)
        if bias is not None:
            if isinstance(bias, np.ndarray):
                bias = torch.from_numpy(bias)
            bias = torch.as_tensor(bias).to(self.weight.device).contiguous()
        self.bias = bias

    @property
    def device(self) -> torch.device:
        return self.weight.device

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        orig = x.shape
        x2 = x.reshape(-1, self.in_features)
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        if x2.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            x2 = x2.float()
        y = self.weight.matmul(x2, out_dtype=torch.float32, bias=self.bias)
        return y.reshape(*orig[:-1], self.out_features)

    __call__ = torch.nn.Module.__call__

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"group_size={self.group_size}, asym={self._zeros is not None}, "
                f"bias={self.bias is not None}")
