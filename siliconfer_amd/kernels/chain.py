"""A chain of dependent batch-1 int4 GEMVs in one persistent launch
(sf_q4_chain): the projections of a decoder layer, each consuming the
previous one's output, as one kernel whose workgroups fetch each phase's
weights before they wait for its input. No counterpart in the reference,
which runs every Q4Linear as its own call
(/root/reference/siliconfer/model/layers.py:93-95, 133, 139-144)."""

from __future__ import annotations

import ctypes

import torch

from .. import _lib
from .._lib import SFError
from .q4 import Q4Weight

IN_X0, IN_PREV, IN_SWIGLU = _lib.SF_CHAIN_IN_X0, _lib.SF_CHAIN_IN_PREV, _lib.SF_CHAIN_IN_SWIGLU
SPIN_CAP = 1 << 20


class Q4Chain:
    """Phases `weights[p]` (symmetric Q4Weight), phase p > 0 fed by phase
    p-1 through `in_kinds[p]` (IN_PREV: its first K outputs; IN_SWIGLU:
    silu(gate) * up of its 2K outputs), each intermediate rounded to fp16.
    Owns the workspace (the launch counter and the tagged hand-off words)."""

    def __init__(self, weights: list[Q4Weight], in_kinds: list[int]):
        if not weights or len(weights) != len(in_kinds) or len(weights) > _lib.SF_CHAIN_MAX_PHASES:
            raise SFError("a chain takes 1..8 phases, one input kind each")
        if any(w.has_zeros for w in weights):
            raise SFError("the chain runs symmetric weights")
        self.weights, self.in_kinds = weights, list(in_kinds)
        self.device = weights[0].device
        n = len(weights)
        self._N = (ctypes.c_int * n)(*[w.out_features for w in weights])
        self._K = (ctypes.c_int * n)(*[w.in_features for w in weights])
        self._g = (ctypes.c_int * n)(*[w.group_size for w in weights])
        self._kind = (ctypes.c_int * n)(*self.in_kinds)
        self._blobs = (ctypes.c_void_p * n)(*[w.blob.data_ptr() for w in weights])
        lib = _lib.load()
        nb = lib.sf_q4_chain_workspace_bytes(self._N, n)
        if nb == 0:
            raise SFError("invalid chain")
        self.workspace = torch.zeros(nb, dtype=torch.uint8, device=self.device)

    def __call__(self, x0: torch.Tensor, out: torch.Tensor | None = None, spin_cap: int = SPIN_CAP,
                 drop_phase: int = -1) -> torch.Tensor:
        """x0 fp16 [K0] on the device -> fp32 [N_last], enqueued on the current stream."""
        _lib.require_device(x0, "x0")
        if x0.dtype != torch.float16 or x0.numel() != self.weights[0].in_features:
            raise SFError("x0 must be fp16 with in_features of the first phase")
        if out is None:
            out = torch.empty(self.weights[-1].out_features, dtype=torch.float32, device=x0.device)
        lib = _lib.load()
        _lib.check(lib.sf_q4_chain(self._blobs, self._N, self._K, self._g, self._kind,
                                   len(self.weights), x0.data_ptr(), out.data_ptr(),
                                   self.workspace.data_ptr(), self.workspace.numel(), spin_cap,
                                   drop_phase, _lib.stream(x0)), "sf_q4_chain")
        return out

    def error(self) -> int:
        """The first failed wait recorded in the workspace (0: none); synchronous."""
        v = ctypes.c_int(0)
        _lib.check(_lib.load().sf_q4_chain_error(self.workspace.data_ptr(), ctypes.addressof(v),
                                                 _lib.stream(self.workspace)), "sf_q4_chain_error")
        return v.value
