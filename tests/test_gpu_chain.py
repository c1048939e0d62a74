"""The persistent GEMV chain (sf_q4_chain) on the GPU against the oracle:
each phase is the reference's symmetric GEMV (q4_gemv.cpp:37-140 via
oracle.linear.gemv) on the previous phase's output rounded to fp16 (or
silu(gate) * up of it, layers.py:143-144, rounded to fp16), as the kernel
hands activations on. Plus: repeated launches are bitwise identical (the
launch counter advances, the sums keep their order), graph replays equal the
eager result, and a forced wait timeout comes back as an error while the
kernel still exits."""

import numpy as np
import pytest
import torch

from oracle import linear, primitives as P
from siliconfer_amd.kernels import Q4Weight
from siliconfer_amd.kernels.chain import IN_PREV, IN_SWIGLU, IN_X0, Q4Chain

pytestmark = pytest.mark.gpu


def s16(s):
    return np.asarray(s, np.float32).astype(np.float16).astype(np.float64)


def silu_mul(g, u):
    return g / (1.0 + np.exp(-g)) * u


def make_chain(dev, shapes, g, kinds, seed):
    rng = np.random.default_rng(seed)
    mats = []
    for N, K in shapes:
        pk, s = P.pack_weights_sym(rng.normal(0, 0.02, (N, K)).astype(np.float32), g)
        mats.append((pk, s))
    ws = [Q4Weight(pk, s, None, g, device=dev) for pk, s in mats]
    return mats, Q4Chain(ws, kinds)


def oracle_chain(mats, kinds, x0, g):
    x = x0.astype(np.float64)
    for p, (pk, s) in enumerate(mats):
        K = pk.shape[1] * 2
        if p > 0:
            x = silu_mul(y[:K], y[K:2 * K]) if kinds[p] == IN_SWIGLU else y[:K]
            x = x.astype(np.float32).astype(np.float16).astype(np.float64)
        y = linear.gemv(pk, s16(s), x, g)
    return y


@pytest.mark.parametrize("g", [64, 128])
def test_one_phase_equals_gemv_oracle(dev, g):
    mats, ch = make_chain(dev, [(1000, 1024)], g, [IN_X0], 1)
    x0 = np.random.default_rng(2).normal(0, 1, 1024).astype(np.float16)
    y = ch(torch.as_tensor(x0).to(dev)).cpu().numpy()
    linear.assert_close(y, linear.gemv(mats[0][0], s16(mats[0][1]), x0.astype(np.float64), g), 1e-3,
                        f"chain of one, g={g}")
    assert ch.error() == 0


@pytest.mark.parametrize("g", [64, 128])
def test_layer_shaped_chain_against_oracle(dev, g):
    """q|k|v -> o (the first H outputs stand in for the attention output) ->
    gate|up -> SwiGLU -> down at a small hidden size, rows not a multiple of 16."""
    H, I = 512, 1408
    shapes = [(3 * H, H), (H, H), (2 * I, H), (H - 8, I)]
    kinds = [IN_X0, IN_PREV, IN_PREV, IN_SWIGLU]
    mats, ch = make_chain(dev, shapes, g, kinds, 3)
    x0 = np.random.default_rng(4).normal(0, 1, H).astype(np.float16)
    xt = torch.as_tensor(x0).to(dev)
    y = ch(xt).cpu().numpy()
    assert ch.error() == 0
    linear.assert_close(y, oracle_chain(mats, kinds, x0, g), 2e-3, f"layer chain g={g}")
    # repeated launches: same bits (the launch counter advances every call)
    for _ in range(3):
        assert np.array_equal(ch(xt).cpu().numpy(), y)


def test_graph_replays_equal_eager(dev):
    H, I = 256, 640
    shapes = [(2 * H, H), (2 * I, H), (H, I)]
    kinds = [IN_X0, IN_PREV, IN_SWIGLU]
    mats, ch = make_chain(dev, shapes, 128, kinds, 5)
    x0 = torch.as_tensor(np.random.default_rng(6).normal(0, 1, H).astype(np.float16)).to(dev)
    eager = ch(x0).clone()
    out = torch.zeros_like(eager)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr, stream=s):
        ch(x0, out=out)
    for r in range(6):  # replays with eager work and synchronisation between them
        out.zero_()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        ch(x0)
    assert ch.error() == 0


def test_wait_timeout_reports_error(dev):
    """The host withholds phase 0's outputs (test hook) with a small wait
    bound: phase 1's wait expires, the launch completes, the error names the
    waiting phase; a new workspace runs clean afterwards."""
    shapes = [(256, 256), (256, 256), (128, 256)]
    kinds = [IN_X0, IN_PREV, IN_PREV]
    mats, ch = make_chain(dev, shapes, 128, kinds, 7)
    x0 = torch.as_tensor(np.random.default_rng(8).normal(0, 1, 256).astype(np.float16)).to(dev)
    ch(x0, spin_cap=64, drop_phase=0)
    torch.cuda.synchronize()
    assert ch.error() == 2  # 1 + the phase whose wait expired
    ok = Q4Chain(ch.weights, kinds)
    y = ok(x0).cpu().numpy()
    assert ok.error() == 0
    linear.assert_close(y, oracle_chain(mats, kinds, x0.cpu().numpy(), 128), 2e-3, "after timeout")


def test_7b_layer_chain_b1(dev):
    """The 7B decoder layer's projections at batch 1, g = 128: q|k|v [12288,
    4096] -> o [4096, 4096] -> gate|up [22016, 4096] -> SwiGLU -> down
    [4096, 11008], against the oracle."""
    shapes = [(12288, 4096), (4096, 4096), (22016, 4096), (4096, 11008)]
    kinds = [IN_X0, IN_PREV, IN_PREV, IN_SWIGLU]
    mats, ch = make_chain(dev, shapes, 128, kinds, 9)
    x0 = np.random.default_rng(10).normal(0, 1, 4096).astype(np.float16)
    y = ch(torch.as_tensor(x0).to(dev)).cpu().numpy()
    assert ch.error() == 0
    linear.assert_close(y, oracle_chain(mats, kinds, x0, 128), 2e-3, "7B layer chain")
