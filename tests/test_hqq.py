"""The HQQ producer (siliconfer_amd/quant/hqq.py), restating
/root/reference/siliconfer/quant/hqq.py:84-164.

Pins:
  * a per-group brute force (each group searched on its own, candidates in
    order, strictly-better replacement) gives the same winner, scale and
    zero-point as the vectorised search; planted mistakes in that brute force
    (no 1.4826 factor, the last equal candidate winning, clip bounds taken
    around the mean instead of the median) change the result on the same
    outlier fixture, so the fixture can tell them apart;
  * with k_grid = (None,) the search is min-max asymmetric RTN (closed form);
  * the reference's own tests (tests/test_hqq.py:75-192) restated: shape,
    boundedness, beats RTN on the bulk with an aggressive grid, several
    groups, p sweep, never worse than RTN in its own L_p loss, the small
    fallback;
  * BASELINE config 2 (Laplace(0, 0.015) with 40-sigma outliers, g = 64): no
    group clips at the default grid, and the HQQ-packed codes and zero-points
    equal min-max RTN's (the GPU GEMM parity on the HQQ-packed tensors is in
    tests/test_gpu_gemm.py).
"""

import numpy as np
import pytest

from siliconfer_amd.kernels import pack_weights_asym
from siliconfer_amd.quant import fake_quantize
from siliconfer_amd.quant.hqq import DEFAULT_K_GRID, hqq_pack, hqq_quantize_weight, hqq_search

AGGRESSIVE = (30.0, 20.0, 15.0, None)


def outlier_weight(N, K, seed):
    """Gaussian core with two +-50 outliers per row (the reference tests' fixture)."""
    rng = np.random.default_rng(seed)
    W = rng.normal(0, 1, (N, K)).astype(np.float32)
    mask = np.zeros_like(W, dtype=bool)
    for i in range(N):
        idx = rng.choice(K, size=2, replace=False)
        W[i, idx] = rng.choice([-1, 1], size=2) * 50.0
        mask[i, idx] = True
    return W, mask


def brute(W, g, p, k_grid, mistake=None):
    """Each group on its own; returns (win, scale, zero) arrays [N, G]."""
    N, K = W.shape
    G = K // g
    win = np.zeros((N, G), int)
    sc = np.zeros((N, G))
    zr = np.zeros((N, G))
    for n in range(N):
        for j in range(G):
            w = W[n, j * g:(j + 1) * g].astype(np.float64)
            center = w.mean() if mistake == "mean" else np.median(w)
            mad = np.median(np.abs(w - np.median(w)))
            sigma = (mad if mad != 0 else 1e-8) * (1.0 if mistake == "no_factor" else 1.4826)
            best = None
            for c, k in enumerate(k_grid):
                lo, hi = (w.min(), w.max()) if k is None else (max(w.min(), center - k * sigma),
                                                             min(w.max(), center + k * sigma))
                s = (hi - lo) / 15.0
                s = 1.0 if s <= 0 else s
                z = min(max(np.round(-lo / s), 0), 15)
                q = np.clip(np.round(w / s + z), 0, 15)
                loss = ((np.abs(w - s * (q - z)) + 1e-8) ** p).mean()
                take = best is None or (loss <= best[0] if mistake == "last_wins" else loss < best[0])
                if take:
                    best = (loss, c, s, z)
            win[n, j], sc[n, j], zr[n, j] = best[1], best[2], best[3]
    return win, sc, zr


def test_search_matches_per_group_brute_force():
    W, _ = outlier_weight(12, 256, seed=3)
    for grid in (AGGRESSIVE, DEFAULT_K_GRID, (None,)):
        s, z, win, loss = hqq_search(W, 64, 0.7, grid)
        bw, bs, bz = brute(W, 64, 0.7, grid)
        np.testing.assert_array_equal(win, bw)
        np.testing.assert_array_equal(s, bs)
        np.testing.assert_array_equal(z, bz)
        assert loss.shape == (len(grid), 12, 4)


@pytest.mark.parametrize("mistake", ["no_factor", "last_wins", "mean"])
def test_planted_mistakes_change_the_choice(mistake):
    W, _ = outlier_weight(12, 256, seed=3)
    # duplicate candidates make the tie rule visible: (20, 20, None) ties on every group
    grid = (20.0, 20.0, 15.0, None) if mistake == "last_wins" else AGGRESSIVE
    s, z, win, _ = hqq_search(W, 64, 0.7, grid)
    bw, bs, bz = brute(W, 64, 0.7, grid, mistake=mistake)
    assert not (np.array_equal(win, bw) and np.array_equal(s, bs) and np.array_equal(z, bz))


def test_untrimmed_grid_is_min_max_rtn():
    rng = np.random.default_rng(4)
    W = rng.normal(0, 0.02, (64, 512)).astype(np.float32)
    s, z, win, _ = hqq_search(W, 128, 0.7, (None,))
    Wg = W.reshape(64, 4, 128).astype(np.float64)
    lo, hi = Wg.min(-1), Wg.max(-1)
    np.testing.assert_array_equal(s, (hi - lo) / 15.0)
    np.testing.assert_array_equal(z, np.clip(np.round(-lo / ((hi - lo) / 15.0)), 0, 15))
    Wq = hqq_quantize_weight(W, 128, k_grid=(None,))
    np.testing.assert_allclose(Wq, fake_quantize(W, 128, sym=False), rtol=0, atol=2e-7)


def test_output_shape_and_bounds():
    rng = np.random.default_rng(0)
    W = rng.normal(0, 1, (64, 128)).astype(np.float32)
    Wq = hqq_quantize_weight(W, 128)
    assert Wq.shape == W.shape and Wq.dtype == np.float32
    W, _ = outlier_weight(32, 128, seed=11)
    Wq = hqq_quantize_weight(W, 128)
    assert np.abs(Wq).max() <= 55.0 and np.isfinite(Wq).all()


def _mse(a, b, mask):
    return float(((a.astype(np.float64) - b.astype(np.float64)) ** 2)[mask].mean())


@pytest.mark.parametrize("N,K,seed", [(64, 128, 1), (32, 256, 99)])
def test_beats_rtn_on_the_bulk(N, K, seed):
    W, mask = outlier_weight(N, K, seed)
    rtn = fake_quantize(W, 128, sym=False)
    hqq = hqq_quantize_weight(W, 128, 0.7, AGGRESSIVE)
    assert _mse(W, hqq, ~mask) < _mse(W, rtn, ~mask)


@pytest.mark.parametrize("p", [0.5, 0.7, 1.0])
def test_p_sweep(p):
    W, mask = outlier_weight(32, 128, seed=5)
    rtn = _mse(W, fake_quantize(W, 128, sym=False), ~mask)
    hqq = _mse(W, hqq_quantize_weight(W, 128, p, AGGRESSIVE), ~mask)
    assert hqq <= rtn + 1e-6
    if p < 1.0:
        assert hqq < rtn


def test_never_worse_than_rtn_in_its_loss():
    W = np.random.default_rng(42).normal(0, 1, (32, 128)).astype(np.float32)
    lp = lambda Wq: float((np.abs(W.astype(np.float64) - Wq.astype(np.float64)) ** 0.7).mean())
    assert lp(hqq_quantize_weight(W, 128, 0.7, AGGRESSIVE)) <= lp(fake_quantize(W, 128, sym=False)) + 1e-6


def test_small_matrix_fallback():
    W = np.random.default_rng(0).normal(0, 1, (8, 32)).astype(np.float32)
    np.testing.assert_array_equal(hqq_quantize_weight(W, 128), fake_quantize(W, 32, sym=False))


def laplace_outliers(rng, shape, b=0.015):
    """BASELINE config 2's weights (the generator tests/test_gpu_gemm.py uses)."""
    W = rng.laplace(0, b, shape).astype(np.float32)
    n_out = max(1, round(W.size / 1e6))
    idx = rng.choice(W.size, n_out, replace=False)
    W.reshape(-1)[idx] = (40 * b * np.sqrt(2) * rng.choice([-1, 1], n_out)).astype(np.float32)
    return W


def test_config2_weights_do_not_clip():
    rng = np.random.default_rng(1)
    for N, K in [(4864, 896), (896, 4864)]:
        W = laplace_outliers(rng, (N, K))
        s, z, win, loss = hqq_search(W, 64)
        # every group's winner is an untrimmed range: its bounds are the group's min and max
        Wg = W.reshape(N, K // 64, 64).astype(np.float64)
        np.testing.assert_allclose(s, (Wg.max(-1) - Wg.min(-1)) / 15.0, rtol=1e-12)
        pk_h, s_h, z_h = hqq_pack(W, 64)
        pk_r, s_r, z_r = pack_weights_asym(W, 64)
        np.testing.assert_array_equal(pk_h, pk_r)
        np.testing.assert_array_equal(z_h, z_r)
        # re-deriving the scale from fake-quantized weights moves it by fp32 rounding only
        np.testing.assert_allclose(s_h, s_r, rtol=5e-7)
