"""HQQ int4 producer (offline, CPU, float64) — the reference's
`hqq_quantize_weight` (/root/reference/siliconfer/quant/hqq.py:84-164).

For every quantization group the search tries a few clip ranges and keeps the
one whose real (round + clip + dequantize) reconstruction has the smallest
mean L_p error, p < 1:

  * the group's robust spread is sigma = 1.4826 * MAD (median absolute
    deviation from the median; an eps stands in for a zero MAD);
  * candidate k (from `k_grid`) clips to [max(min, med - k sigma),
    min(max, med + k sigma)]; `None` is the untrimmed min-max range, which
    makes the result never worse than asymmetric RTN under the same loss;
  * a range gives scale = (hi - lo) / (2^bits - 1) (1 when not positive) and
    zero = clip(round(-lo / scale), 0, 2^bits - 1); codes are
    clip(round(w / scale + zero), 0, 2^bits - 1) and the loss is
    mean((|w - scale (q - zero)| + eps)^p) over the group;
  * the first candidate with the smallest loss wins (a later one must be
    strictly better to replace it).

The result is fake-quantized fp32 weights, as in the reference; the loader
then packs them on the asymmetric grid (`hqq_pack`, the reference's
HQQ -> `pack_weights_asym` rule, engine/q4_loader.py:178-183). Rounding is
numpy's round-half-to-even throughout, as the reference's.

This module computes candidates one at a time and keeps only their [N, G]
losses, scales and zero-points, then re-derives the winning codes once; the
reference carries running best arrays through the loop. Both pick the same
candidate (argmin returns the first minimum).
"""

from __future__ import annotations

import numpy as np

EPS = 1e-8
MAD_TO_SIGMA = 1.4826
DEFAULT_K_GRID = (150.0, 100.0, 80.0, None)


def _range_params(lo: np.ndarray, hi: np.ndarray, qmax: float):
    scale = (hi - lo) / qmax
    scale = np.where(scale <= 0, 1.0, scale)
    zero = np.clip(np.round(-lo / scale), 0, qmax)
    return scale, zero


def _codes(Wg: np.ndarray, scale: np.ndarray, zero: np.ndarray, qmax: float) -> np.ndarray:
    return np.clip(np.round(Wg / scale + zero), 0, qmax)


def hqq_search(W: np.ndarray, group_size: int = 128, p: float = 0.7,
               k_grid=DEFAULT_K_GRID, bits: int = 4):
    """The per-group choice: (scale f64 [N,G], zero f64 [N,G], winner index
    into k_grid int [N,G], loss f64 [C,N,G] of every candidate)."""
    W = np.asarray(W)
    N, K = W.shape
    if K % group_size:
        raise ValueError(f"in_features={K} not divisible by group_size={group_size}")
    qmax = float(2 ** bits - 1)
    Wg = W.reshape(N, K // group_size, group_size).astype(np.float64)
    wmin, wmax = Wg.min(axis=-1), Wg.max(axis=-1)
    med = np.median(Wg, axis=-1)
    mad = np.median(np.abs(Wg - med[..., None]), axis=-1)
    sigma = np.where(mad == 0.0, EPS, mad) * MAD_TO_SIGMA
    scales, zeros, losses = [], [], []
    for k in k_grid:
        if k is None:
            lo, hi = wmin, wmax
        else:
            lo = np.maximum(wmin, med - k * sigma)
            hi = np.minimum(wmax, med + k * sigma)
        scale, zero = _range_params(lo, hi, qmax)
        q = _codes(Wg, scale[..., None], zero[..., None], qmax)
        err = np.abs(Wg - scale[..., None] * (q - zero[..., None]))
        losses.append(((err + EPS) ** p).mean(axis=-1))
        scales.append(scale)
        zeros.append(zero)
    loss = np.stack(losses)
    win = np.argmin(loss, axis=0)
    pick = lambda a: np.take_along_axis(np.stack(a), win[None], axis=0)[0]
    return pick(scales), pick(zeros), win, loss


def hqq_quantize_weight(W: np.ndarray, group_size: int = 128, p: float = 0.7,
                        k_grid=DEFAULT_K_GRID, bits: int = 4) -> np.ndarray:
    """Fake-quantized fp32 weights [N, K] from the HQQ search. A matrix with
    in_features < group_size is one group per row, plain asymmetric RTN
    (the reference's fallback, hqq.py:116-120)."""
    W = np.asarray(W)  # the search runs in float64 from the caller's values (hqq.py:122)
    N, K = W.shape
    if K < group_size:
        if bits != 4:
            raise NotImplementedError("the small-matrix fallback is 4-bit RTN")
        from .primitives import fake_quantize

        return fake_quantize(W, group_size=K, sym=False)
    scale, zero, _, _ = hqq_search(W, group_size, p, k_grid, bits)
    qmax = float(2 ** bits - 1)
    Wg = W.reshape(N, K // group_size, group_size).astype(np.float64)
    q = _codes(Wg, scale[..., None], zero[..., None], qmax)
    return (scale[..., None] * (q - zero[..., None])).reshape(N, K).astype(np.float32)


def hqq_pack(W: np.ndarray, group_size: int = 128, p: float = 0.7, k_grid=DEFAULT_K_GRID):
    """What the loader stores for an HQQ projection: the fake-quantized
    weights packed on the asymmetric int4 grid -> (packed u8 [N, K/2],
    scales f32 [N, G], zeros f32 [N, G])."""
    from ..kernels import pack_weights_asym

    return pack_weights_asym(hqq_quantize_weight(W, group_size, p, k_grid), group_size)
