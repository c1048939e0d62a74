"""Benchmark: int4 decode GEMV achieved HBM GB/s at 7B shapes.

One step = one pass over config 3's sweep on one GPU: symmetric int4 RTN, group
128, W in {[4096,4096], [11008,4096], [4096,11008]} x batch {1, 2, 4, 8}, fp16
activations, fp32 accumulation — 12 GEMV launches. Every launch reads a
different copy of its weight blob: >= 512 MB of copies per shape (twice the
256 MB last-level cache), the four batch cases of a shape read four different
copies and the next step the next four, so the weights come from HBM. The steps
are replayed from HIP graphs, eight steps (96 launches) per graph where the
step count allows.

Printed JSON (one line):
  value         whole-job algorithmic GB/s: sum of per-launch algorithmic bytes
                over the K timed steps / time between HIP events bracketing
                them (inputs resident in HBM);
  roofline      the GEMV kernel: achieved = average algorithmic bytes per
                launch / average launch duration of the timed region (the HIP
                events around the K steps, on the stream the launches run on;
                so achieved equals `value`); `frac_of_floor` sets the step
                against this GPU's own plain read of each case's bytes
                (sf_floor_read), and `floor.empty_launch_us` is an empty launch,
                both timed as graphs of back-to-back cold launches in the same
                run; `cases` times each case alone the same way (an event pair
                around one launch has a ~6 us floor of its own); `traffic` is
                the HBM bytes per launch
                that rocprofv3 FETCH_SIZE + WRITE_SIZE counters measured
                (profiles/gemv_sweep_pmc.json, calibrated on a copy of known
                size), when that file is present;
  decode_tok_s  BASELINE config 5, the metric's second half: greedy decode on a
                random-init Qwen2.5-0.5B-geometry model (all projections int4
                sym g=64, int8 KV, bf16 tied embedding), 512 random prompt ids,
                256 tokens, batch 1; fp32 residual stream, projections fed
                fp16 activations (RNE from fp32: each projection stays within
                the 1e-3 bar against the reference's fp32 Q4Linear); decode
                steps are HIP-graph replays; median of 3. `e2e_config5` has
                the details (fp32-activation projections too, prefill time,
                the lm_head's share, bytes per token and the HBM roofline,
                and the reference's CPU path on the host cores: its own
                q4_gemv_sym for every projection, numpy for the rest, one
                thread and then every core);
  secondary     the other hot-path kernels at their BASELINE configs, timed the
                same way: config-1 GEMV, config-2 prefill GEMM, config-4
                decode attention, the KV-cache append;
  cpu_baseline  the reference's own CPU kernel (q4_gemv.cpp / q4_gemm.cpp,
                compiled from /root/reference into oracle/_ref) or, when that
                library is absent, the C restatement oracle/q4_cpu.c, on a
                bounded sample of the same sweep, single-threaded as the
                reference runs; `all_cores` adds the restatement on every core.

Algorithmic bytes per launch (B = batch): N*K/2 (int4) + 2*N*K/128 (fp16
scales) + 2*B*K (fp16 x) + 2*B*N (fp16 y).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-e2e]
       python bench.py --profile-kernels   (the sweep's graph replays, for rocprofv3 runs)
       python bench.py --profile-e2e       (config-5 decode-graph replays for rocprofv3)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008)]
BATCHES = [1, 2, 4, 8]
GROUP = 128
COLD_BYTES = 512 << 20
ROOT = os.path.dirname(os.path.abspath(__file__))
PMC_FILE = os.path.join(ROOT, "profiles", "gemv_sweep_pmc.json")


def alg_bytes(N: int, K: int, B: int, g: int = GROUP, zeros: bool = False) -> int:
    z = N * (K // g) // 2 if zeros else 0
    return N * K // 2 + 2 * N * (K // g) + z + 2 * B * K + 2 * B * N


def quantize_shape(N, K, seed, g=GROUP):
    """Config-3 synthetic weights: W ~ N(0, 0.02) RTN-quantized, symmetric."""
    from siliconfer_amd.kernels import pack_weights_sym

    rng = np.random.default_rng(seed)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    return pack_weights_sym(W, g)


def cold_copies(t, nbytes):
    """t plus clones so that the set spans >= COLD_BYTES."""
    n = max(2, -(-COLD_BYTES // max(nbytes, 1)))
    return [t] + [t.clone() for _ in range(n - 1)]


class Timer:
    """Average duration of a launch sequence: HIP events around graph replays.
    With eager=True it only launches each call once (profiling runs)."""

    def __init__(self, torch, stream, eager=False):
        self.torch, self.stream, self.eager = torch, stream, eager

    def per_call_us(self, fns, reps=4):
        torch = self.torch
        if self.eager:
            with torch.cuda.stream(self.stream):
                for f in fns:
                    f()
            torch.cuda.synchronize()
            return float("nan")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            for f in fns:
                f()
        with torch.cuda.stream(self.stream):
            g.replay()
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(self.stream)
            for _ in range(reps):
                g.replay()
            b.record(self.stream)
            torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / (reps * len(fns))


class GpuSweep:
    def __init__(self, dev):
        import torch

        from siliconfer_amd import _lib
        from siliconfer_amd.kernels import Q4Weight

        self.torch = torch
        self.lib = _lib.load()
        self.dev = dev
        self.stream = torch.cuda.Stream(dev)   # default priority; all work runs on it
        self.cases = []       # (N, K, B, blob_ptrs[], x_ptr, y_ptr)
        self.keep = []
        rng = np.random.default_rng(123)
        self.n_rot = 1
        for i, (N, K) in enumerate(SHAPES):
            pk, s = quantize_shape(N, K, 2 + i)
            w = Q4Weight(pk, s, None, GROUP, device=dev)
            blobs = cold_copies(w.blob, w.nbytes)
            self.keep += blobs
            self.n_rot = max(self.n_rot, len(blobs))
            x = torch.as_tensor(rng.normal(0, 1, (8, K)).astype(np.float16)).to(dev)
            self.keep.append(x)
            for bi, B in enumerate(BATCHES):
                y = torch.empty((B, N), dtype=torch.float16, device=dev)
                self.keep.append(y)
                self.cases.append((N, K, B, bi, [b.data_ptr() for b in blobs], x.data_ptr(), y.data_ptr()))
        self.step_bytes = sum(alg_bytes(N, K, B) for N, K, B, *_ in self.cases)
        self.graphs = None

    def launch_copy(self, ci: int, copy: int) -> None:
        N, K, B, bi, blobs, xp, yp = self.cases[ci]
        rc = self.lib.sf_q4_gemv(blobs[copy % len(blobs)], xp, 1, yp, 1, None, None, 0, B, N, K,
                                 GROUP, 0, self.torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(self.lib.sf_last_error().decode())

    def launch(self, ci: int, rot: int) -> None:
        """Case ci in step `rot`: the four batch cases of a shape read four
        different copies of its blob, and the next step the next four, so no
        copy is read again before >= COLD_BYTES of other copies have been."""
        self.launch_copy(ci, rot * len(BATCHES) + self.cases[ci][3])

    def eager_step(self, rot: int) -> None:
        for ci in range(len(self.cases)):
            self.launch(ci, rot)

    GROUP_STEPS = 8  # steps per group graph (one replay launches 96 GEMVs)

    def capture(self) -> None:
        """One graph per step rotation, and one per run of GROUP_STEPS aligned
        rotations, so the timed loop pays one graph launch per 8 steps."""
        torch = self.torch
        self.graphs, self.group_graphs = [], {}
        for rot in range(self.n_rot):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.stream):
                self.eager_step(rot)
            self.graphs.append(g)
        S = self.GROUP_STEPS
        for r0 in range(0, self.n_rot - S + 1, S):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.stream):
                for rot in range(r0, r0 + S):
                    self.eager_step(rot)
            self.group_graphs[r0] = g
        torch.cuda.synchronize()

    def step(self, i: int) -> None:
        if self.graphs is not None:
            self.graphs[i % self.n_rot].replay()
        else:
            self.eager_step(i)

    def run(self, start: int, count: int) -> None:
        """Steps start .. start + count - 1 (rotation i % n_rot each), through
        the group graphs where a whole aligned group fits."""
        i, end = start, start + count
        while i < end:
            g = self.group_graphs.get(i % self.n_rot) if self.graphs is not None else None
            if g is not None and end - i >= self.GROUP_STEPS:
                g.replay()
                i += self.GROUP_STEPS
            else:
                self.step(i)
                i += 1

    def per_case_us(self):
        timer = Timer(self.torch, self.stream)
        out = []
        for ci, (N, K, B, bi, blobs, *_) in enumerate(self.cases):
            fns = [(lambda r=r, ci=ci: self.launch_copy(ci, r)) for r in range(len(blobs))]
            out.append(timer.per_call_us(fns))
        return out


def floor_us(dev, stream, byte_counts):
    """This GPU's per-launch floor, timed like the GEMV cases (graphs of
    back-to-back launches between HIP events, every launch on memory no launch
    of the last >= COLD_BYTES touched): an empty launch, and a plain read of
    each byte count (sf_floor_read)."""
    import torch

    from siliconfer_amd import _lib

    lib = _lib.load()
    timer = Timer(torch, stream)
    cur = lambda: torch.cuda.current_stream().cuda_stream
    empty = timer.per_call_us([lambda: lib.sf_floor_empty(cur())] * 64)
    pool_bytes = COLD_BYTES + (128 << 20)
    pool = torch.randint(0, 256, (pool_bytes,), dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    reads = {}
    for nb in sorted(set(byte_counts)):
        nb16 = nb // 16 * 16
        step = -(-nb16 // 4096) * 4096
        n = max(2, -(-COLD_BYTES // step))
        fns = [(lambda o=(i * step) % (pool_bytes - nb16): lib.sf_floor_read(
            pool.data_ptr() + o, nb16, sink.data_ptr(), cur())) for i in range(n)]
        reads[nb] = timer.per_call_us(fns)
    del pool
    return empty, reads


SECONDARY_CASES = ("config1", "config2_up", "config2_down", "config4_T4096", "config4_T16384",
                   "kv_append", "chain7b")


def secondary(dev, stream, eager=False, only=None):
    """The other hot-path kernels at their BASELINE configs (cold HBM,
    graph-timed); `only`: a subset of SECONDARY_CASES (the per-case rocprofv3
    runs time one case alone)."""
    import torch

    want = lambda name: only is None or name in only

    from siliconfer_amd import _lib
    from siliconfer_amd.kernels import Q4Weight, pack_weights_asym

    lib = _lib.load()
    timer = Timer(torch, stream, eager)
    cur = lambda: torch.cuda.current_stream().cuda_stream
    out = {}
    rng = np.random.default_rng(0)

    # config 1: [4864, 896] sym g=64, B=1
    if want("config1"):
        _config1(dev, lib, timer, cur, rng, out)
    # config 2: asym prefill GEMM, X bf16 [512, K], up/gate [4864, 896] and down [896, 4864]
    for name, (N, K) in (("config2_up", (4864, 896)), ("config2_down", (896, 4864))):
        W = laplace_outliers(rng, (N, K))
        if want(name):
            _config2(dev, lib, timer, cur, rng, out, N, K, W)
    # config 4: decode attention over an int8 cache, fp16 scales, q fp16 [1, 14, 64]
    for T in (4096, 16384):
        if want(f"config4_T{T}"):
            _config4(dev, lib, timer, cur, out, T)
    if want("kv_append"):
        _kv_append(dev, lib, timer, cur, out)
    if want("chain7b"):
        _chain7b(dev, lib, timer, cur, out)
    return out


def laplace_outliers(rng, shape, b=0.015):
    """BASELINE config 2's weights: Laplace(0, b) with one outlier of 40 sigma
    (sigma = b sqrt 2) per 10^6 weights, random sign."""
    W = rng.laplace(0, b, shape).astype(np.float32)
    n_out = max(1, round(W.size / 1e6))
    idx = rng.choice(W.size, n_out, replace=False)
    W.reshape(-1)[idx] = (40 * b * np.sqrt(2) * rng.choice([-1, 1], n_out)).astype(np.float32)
    return W


def _config1(dev, lib, timer, cur, rng, out):
    import torch

    from siliconfer_amd.kernels import Q4Weight

    pk, s = quantize_shape(4864, 896, 0, g=64)
    w = Q4Weight(pk, s, None, 64, device=dev)
    blobs = cold_copies(w.blob, w.nbytes)
    x = torch.as_tensor(rng.normal(0, 1, (1, 896)).astype(np.float16)).to(dev)
    y = torch.empty((1, 4864), dtype=torch.float16, device=dev)
    us = timer.per_call_us([(lambda b=b: lib.sf_q4_gemv(b.data_ptr(), x.data_ptr(), 1, y.data_ptr(), 1,
                                                        None, None, 0, 1, 4864, 896, 64, 0, cur()))
                            for b in blobs])
    nb = alg_bytes(4864, 896, 1, 64)
    out["config1_gemv_4864x896_g64_b1"] = {"us": round(us, 3), "GBps": round(nb / us / 1e3, 1),
                                           "bytes": nb}


def _config2(dev, lib, timer, cur, rng, out, N, K, W):
    import torch

    from siliconfer_amd.kernels import Q4Weight, pack_weights_asym

    pa, sa, za = pack_weights_asym(W, 64)
    wq = Q4Weight(pa, sa, za, 64, device=dev)
    X = torch.as_tensor(rng.normal(0, 1, (512, K)).astype(np.float32)).to(dev).to(torch.bfloat16)
    Y = torch.empty((512, N), dtype=torch.bfloat16, device=dev)
    wsb = lib.sf_q4_gemm_workspace_bytes(512, N, K, 64)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    blobs = cold_copies(wq.blob, wq.nbytes)
    fns = [(lambda b=b: lib.sf_q4_gemm(b.data_ptr(), X.data_ptr(), 2, Y.data_ptr(), 2, None, None,
                                       0, 512, N, K, 64, 1, ws.data_ptr() if wsb else None, wsb,
                                       cur())) for b in blobs]
    us = timer.per_call_us(fns, reps=2)
    flops = 2.0 * 512 * N * K
    out[f"config2_gemm_asym_m512_{N}x{K}"] = {
        "us": round(us, 3), "TFLOPs": round(flops / us / 1e6, 1),
        "mfma_frac_of_bf16_peak": round(flops / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4)}
    if wsb:  # split K: the GEMM launch alone (its partials), timed the same way
        part = [(lambda b=b: lib.sf_q4_gemm_partials(b.data_ptr(), X.data_ptr(), 2, 512, N, K, 64, 1,
                                                     ws.data_ptr(), wsb, cur())) for b in blobs]
        up = timer.per_call_us(part, reps=2)
        out[f"config2_gemm_asym_m512_{N}x{K}"].update(
            gemm_launch_us=round(up, 3), reduce_launch_us_by_difference=round(us - up, 3))


def _config4(dev, lib, timer, cur, out, T):
    import torch

    kc = torch.randint(-127, 128, (1, 2, T, 64), dtype=torch.int8, device=dev)
    vc = torch.randint(-127, 128, (1, 2, T, 64), dtype=torch.int8, device=dev)
    ks = (torch.rand((1, 2, T), device=dev) * 0.02 + 0.005).half()
    vs = (torch.rand((1, 2, T), device=dev) * 0.02 + 0.005).half()
    q = torch.randn((1, 14, 64), device=dev).half()
    o = torch.empty((1, 14, 64), dtype=torch.float16, device=dev)
    per = kc.numel() * 2 + ks.numel() * 4
    n = max(2, -(-COLD_BYTES // per))
    sets = [(kc, ks, vc, vs)] + [(kc.clone(), ks.clone(), vc.clone(), vs.clone())
                                 for _ in range(n - 1)]
    nsp = lib.sf_attn_default_splits_d(1, 2, T, 64)
    ws_bytes = lib.sf_attn_workspace_bytes(1, 14, 64, nsp)
    wsp = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)  # split partials
    fns = [(lambda a=a: lib.sf_attn_decode_i8kv(q.data_ptr(), 1, a[0].data_ptr(), a[1].data_ptr(),
                                                a[2].data_ptr(), a[3].data_ptr(), 1, o.data_ptr(),
                                                1, wsp.data_ptr(), ws_bytes, 1, 14, 2, T, T, 64,
                                                0.125, nsp, cur())) for a in sets]
    us = timer.per_call_us(fns)
    nb = 2 * 2 * T * 64 + 2 * 2 * 2 * T + 2 * 2 * 14 * 64
    out[f"config4_attn_T{T}"] = {"us": round(us, 3), "GBps": round(nb / us / 1e3, 1),
                                 "bytes": nb, "splits": nsp,
                                 "launches": "one" if nsp == 1 else "two (split partials, merge)"}
    if nsp > 1:  # the split launch alone (partials, no merge), timed the same way
        t0 = torch.zeros((1,), dtype=torch.int32, device=dev)
        part = [(lambda a=a: lib.sf_attn_decode_i8kv_partials_dev(
            q.data_ptr(), 1, a[0].data_ptr(), a[1].data_ptr(), a[2].data_ptr(), a[3].data_ptr(), 1,
            wsp.data_ptr(), ws_bytes, 1, 14, 2, t0.data_ptr(), T, T, T, 64, 0.125, nsp, cur())) for a in sets]
        up = timer.per_call_us(part)
        out[f"config4_attn_T{T}"].update(split_launch_us=round(up, 3),
                                         merge_launch_us_by_difference=round(us - up, 3))


def sweep_attn_splits(dev, head_dim=64, Ts=(128, 512, 1024, 4096, 16384),
                      splits=(1, 2, 8, 16, 32, 64)) -> dict:
    """Config-4-shaped decode attention (14 / 2 heads, fp16 q, scales and
    output) over T x split count, graph-timed over cold copies of the cache
    (up to 256 copies): the measurements behind sf_attn_default_splits_d."""
    import torch

    from siliconfer_amd import _lib

    lib = _lib.load()
    stream = torch.cuda.Stream(dev)
    timer = Timer(torch, stream)
    cur = lambda: torch.cuda.current_stream().cuda_stream
    q = torch.randn((1, 14, head_dim), device=dev).half()
    o = torch.empty((1, 14, head_dim), dtype=torch.float16, device=dev)
    table = {}
    for T in Ts:
        kc = torch.randint(-127, 128, (1, 2, T, head_dim), dtype=torch.int8, device=dev)
        vc = torch.randint(-127, 128, (1, 2, T, head_dim), dtype=torch.int8, device=dev)
        ks = (torch.rand((1, 2, T), device=dev) * 0.02 + 0.005).half()
        vs = (torch.rand((1, 2, T), device=dev) * 0.02 + 0.005).half()
        per = kc.numel() * 2 + ks.numel() * 4
        n = min(256, max(2, -(-(256 << 20) // per)))
        sets = [(kc, ks, vc, vs)] + [(kc.clone(), ks.clone(), vc.clone(), vs.clone()) for _ in range(n - 1)]
        row = {}
        for S in splits:
            if S > T:
                continue
            wsb = lib.sf_attn_workspace_bytes(1, 14, head_dim, S)
            ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev)
            fns = [(lambda a=a, S=S, ws=ws, wsb=wsb: lib.sf_attn_decode_i8kv(
                q.data_ptr(), 1, a[0].data_ptr(), a[1].data_ptr(), a[2].data_ptr(), a[3].data_ptr(), 1,
                o.data_ptr(), 1, ws.data_ptr(), wsb, 1, 14, 2, T, T, head_dim, 0.125, S, cur()))
                for a in sets]
            row[S] = round(min(timer.per_call_us(fns), timer.per_call_us(fns)), 3)
        table[T] = row
        del sets
    return {"attn_split_sweep_us": table, "head_dim": head_dim,
            "default_splits": {T: int(lib.sf_attn_default_splits_d(1, 2, T, head_dim)) for T in Ts}}


def _kv_append(dev, lib, timer, cur, out):
    """KV append: one decode token, [1, 2, 1, 64] fp16 K and V into a 4096-slot cache."""
    import torch

    qk = torch.empty((1, 2, 4096, 64), dtype=torch.int8, device=dev)
    sk = torch.empty((1, 2, 4096), dtype=torch.float16, device=dev)
    qv, sv = torch.empty_like(qk), torch.empty_like(sk)
    kn = torch.randn((1, 2, 1, 64), device=dev).half()
    vn = torch.randn((1, 2, 1, 64), device=dev).half()
    fns = [(lambda t=t: lib.sf_kv_quant_append(kn.data_ptr(), vn.data_ptr(), 1, qk.data_ptr(),
                                               sk.data_ptr(), qv.data_ptr(), sv.data_ptr(), 1, 1, 2,
                                               1, t, 4096, 64, cur())) for t in range(64)]
    out["kv_append_1tok_2heads_d64"] = {"us": round(timer.per_call_us(fns), 3)}


CHAIN7B = [(12288, 4096), (4096, 4096), (22016, 4096), (4096, 11008)]


def _chain7b(dev, lib, timer, cur, out):
    """A 7B decoder layer's four int4 projections at batch 1 (sym g=128):
    q|k|v [12288, 4096] -> o [4096, 4096] (first 4096 outputs) -> gate|up
    [22016, 4096] -> down [4096, 11008] (silu(gate) * up folded), fp16
    between phases. Timed two ways over cold weight copies: one persistent
    launch (sf_q4_chain) and four GEMV launches (the last with the SwiGLU
    folded). Algorithmic bytes: every phase's codes and scales, x0 and the
    fp32 output."""
    import torch

    from siliconfer_amd import _lib
    from siliconfer_amd.kernels import Q4Weight
    from siliconfer_amd.kernels.chain import IN_PREV, IN_SWIGLU, IN_X0, Q4Chain
    from siliconfer_amd.model.llama import pack_sym_device

    per_set = sum(N * K // 2 + 2 * N * K // 128 for N, K in CHAIN7B)
    nset = max(2, -(-COLD_BYTES // per_set))
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    sets = []
    for _ in range(nset):
        ws = []
        for N, K in CHAIN7B:
            W = torch.randn((N, K), generator=g, device=dev) * 0.02
            pk, sc = pack_sym_device(W, 128)
            ws.append(Q4Weight(pk, sc, None, 128, device=dev))
            del W, pk, sc
        sets.append(ws)
    chains = [Q4Chain(ws, [IN_X0, IN_PREV, IN_PREV, IN_SWIGLU]) for ws in sets]
    x0 = torch.randn(4096, generator=g, device=dev).half()
    y = torch.empty(4096, device=dev)
    y16 = torch.empty((1, 12288), device=dev, dtype=torch.float16)
    o16 = torch.empty((1, 4096), device=dev, dtype=torch.float16)
    gu = torch.empty((1, 22016), device=dev)

    def separate(ws):
        ws[0].matmul(x0.view(1, -1), out=y16)
        ws[1].matmul(y16[:, :4096], out=o16)
        ws[2].matmul(o16, out_f32=gu)
        w = ws[3]
        _lib.check(lib.sf_q4_gemv_fused(w.blob.data_ptr(), gu.data_ptr(), _lib.SF_PRE_SILU_MUL, None, 0.0,
                                        _lib.SF_F16, None, 0, y.data_ptr(), None, 0, w.out_features,
                                        w.in_features, w.group_size, 0, cur()), "sf_q4_gemv_fused")

    t_chain = timer.per_call_us([(lambda c=c: c(x0, out=y)) for c in chains])
    t_sep = timer.per_call_us([(lambda ws=ws: separate(ws)) for ws in sets])
    errs = [c.error() for c in chains]
    if any(errs):
        raise RuntimeError(f"sf_q4_chain reported a failed wait: {errs}")
    nb = per_set + 2 * 4096 + 4 * 4096
    out["chain7b_layer_b1"] = {
        "bytes": nb,
        "one_launch_us": round(t_chain, 3), "one_launch_GBps": round(nb / t_chain / 1e3, 1),
        "one_launch_frac_of_8TBps": round(nb / t_chain / 1e3 / HBM_PEAK_GBS, 4),
        "four_launches_us": round(t_sep, 3), "four_launches_GBps": round(nb / t_sep / 1e3, 1),
        "four_launches_frac_of_8TBps": round(nb / t_sep / 1e3 / HBM_PEAK_GBS, 4)}
    del chains, sets
    torch.cuda.empty_cache()


E2E_PROMPT, E2E_TOKENS = 512, 256


def e2e_model(dev, act):
    from siliconfer_amd.model.config import ModelConfig
    from siliconfer_amd.model.llama import LlamaModel

    cfg = ModelConfig.qwen25_05b()
    m = LlamaModel.random_init(cfg, seed=4, group_size=64, device=dev,
                               max_seq=E2E_PROMPT + E2E_TOKENS + 256, act_dtype=act)
    ids = np.random.default_rng(4).integers(0, cfg.vocab_size, E2E_PROMPT)
    return cfg, m, ids


def e2e_decode(dev, runs: int = 3):
    """random-init Qwen2.5-0.5B geometry, every projection
    int4 sym g=64, int8 KV, 512 uniformly random prompt ids, 256 greedy tokens,
    batch 1; decode tok/s = 255 decode steps (HIP-graph replays) / their time,
    median of `runs` after a warmup generation (the reference's
    GenerationResult.decode_tok_s)."""
    import torch

    out = {}
    m_rope = False
    for name, act in (("fp16", torch.float16), ("fp32", torch.float32)):
        cfg, m, ids = e2e_model(dev, act)
        m_rope = m._qkv_rope
        m.capture()
        m.generate(ids, 16)
        rs = [m.generate(ids, E2E_TOKENS) for _ in range(runs)]
        order = sorted(range(runs), key=lambda i: rs[i].decode_tok_s)
        med = rs[order[runs // 2]]
        timer = Timer(torch, torch.cuda.Stream(dev))
        head_us = timer.per_call_us([lambda: m._lm_head_norm(m.h, m.token, None, logits=False)] * 32)
        # the prompt's causal attention alone: every layer's call on its own cache
        from siliconfer_amd import _lib
        lib = _lib.load()
        Qp = torch.randn((E2E_PROMPT, m.Hq, m.D), device=dev).to(act)
        Ap = torch.empty((E2E_PROMPT, m.Hq * m.D), dtype=act, device=dev)
        cur = lambda: torch.cuda.current_stream().cuda_stream
        pf_fns = [(lambda l=l: lib.sf_attn_prefill_i8kv(
            Qp.data_ptr(), _lib.dt(Qp), m.k_codes[l].data_ptr(), m.k_scales[l].data_ptr(),
            m.v_codes[l].data_ptr(), m.v_scales[l].data_ptr(), _lib.SF_F16, Ap.data_ptr(), _lib.dt(Ap),
            E2E_PROMPT, m.Hq, m.KVH, 0, m.max_seq, m.D, m.scale, cur()))
            for l in range(cfg.num_hidden_layers)]
        pf_attn_ms = timer.per_call_us(pf_fns) * cfg.num_hidden_layers * 1e-3
        w_bytes = sum(getattr(L, n).nbytes for L in m.layers for n in ("qkv", "o", "gate_up", "down"))
        head_bytes = m.embed.numel() * 2
        T_mean = E2E_PROMPT + E2E_TOKENS / 2
        kv_bytes = cfg.num_hidden_layers * 2 * cfg.num_key_value_heads * T_mean * (cfg.head_dim + 2)
        per_tok = w_bytes + head_bytes + kv_bytes
        ms = 1e3 / med.decode_tok_s
        out[name] = {
            "decode_tok_s": round(med.decode_tok_s, 1),
            "runs_tok_s": [round(r.decode_tok_s, 1) for r in rs],
            "ms_per_token": round(ms, 4),
            "prefill_ms_512": round(med.prefill_time * 1e3, 3),
            "prefill_attention_ms_512": round(pf_attn_ms, 3),
            "prefill_attention_share": round(pf_attn_ms / (med.prefill_time * 1e3), 4),
            "lm_head_us": round(head_us, 2),
            "lm_head_share": round(head_us * 1e-3 / ms, 4),
            "hbm_bytes_per_token": int(per_tok),
            "hbm_GBps": round(per_tok / (ms * 1e-3) / 1e9, 1),
            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / per_tok, 1),
            "first_tokens": med.token_ids[:8],
        }
        del m
        torch.cuda.empty_cache()
    # embed; per layer qkv (norm folded; RoPE + KV append folded into its
    # epilogue where the plan allows), attention, o, gate_up (norm folded), down
    # (SwiGLU folded); lm_head (final norm folded)
    per_layer = 5 if m_rope else 6
    out["launches_per_token"] = 1 + per_layer * cfg.num_hidden_layers + 1
    return out


SPEC_DRAFT = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                  num_attention_heads=4, num_key_value_heads=2, head_dim=64)


def spec_draft(dev, cfg, act):
    """A 2-layer draft with the target's vocabulary (random weights)."""
    from siliconfer_amd.model.config import ModelConfig
    from siliconfer_amd.model.llama import LlamaModel

    dcfg = ModelConfig(vocab_size=cfg.vocab_size, rms_norm_eps=cfg.rms_norm_eps,
                       rope_theta=cfg.rope_theta, tie_word_embeddings=True, **SPEC_DRAFT)
    return LlamaModel.random_init(dcfg, seed=5, group_size=64, device=dev,
                                  max_seq=E2E_PROMPT + E2E_TOKENS + 256, act_dtype=act)


def e2e_speculative(dev, reps: int = 20):
    """Config-5 target (fp16 activations) after the 512-token prompt: device
    time of one verify of B = K+1 rows (its HIP graph replayed between HIP
    events, the position reset by a one-element fill each time) against one
    decode step, and greedy speculative generation of 256 tokens with a
    2-layer random draft (tok/s, acceptance). Random weights make greedy
    text repetitive, so the acceptance rate here says nothing about a real
    draft; the verify / decode cost ratio is the figure that carries over."""
    import torch

    from siliconfer_amd.engine import SamplingParams, speculative_generate

    def G(n):  # greedy, n tokens
        return SamplingParams(temperature=0.0, max_tokens=n)

    cfg, t, ids = e2e_model(dev, torch.float16)
    t.capture()
    t.capture_verify()
    t.reset()
    t.prefill(ids)
    N = t.pos
    ev = lambda: torch.cuda.Event(enable_timing=True)

    def dev_ms(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = ev(), ev()
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    def one_verify(B):
        t.pos_dev.fill_(N)
        t._verify_graphs[B].replay()

    def one_decode():
        t.pos_dev.fill_(N)
        t.graph.replay()

    decode_ms = dev_ms(one_decode)
    verify = {B: round(dev_ms(lambda: one_verify(B)), 4) for B in (1, 2, 4, 8)}
    t.set_position(N)
    draft = spec_draft(dev, cfg, torch.float16)
    draft.capture()
    out = {"decode_step_ms": round(decode_ms, 4), "verify_ms": verify,
           "verify8_over_decode": round(verify[8] / decode_ms, 3)}
    for K in (3, 7):
        speculative_generate(draft, t, ids, G(32), K=K)
        r = speculative_generate(draft, t, ids, G(E2E_TOKENS), K=K)
        out[f"K{K}"] = {"tok_s": round(r.effective_tok_s, 1),
                        "acceptance": round(r.acceptance_rate, 3), "rounds": r.total_rounds}
    return out


E2E_PROFILE_STEPS = 32


def profile_e2e(dev) -> dict:
    """Kernel-trace workload for config 5, timed as the bench times it: the
    decode step's HIP graph captured, the 512-token prompt, then
    E2E_PROFILE_STEPS graph replays (one token each) between HIP events."""
    import torch

    _, m, ids = e2e_model(dev, torch.float16)
    m.capture()
    m.reset()
    m.prefill(ids)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    m.replay(E2E_PROFILE_STEPS)
    b.record()
    torch.cuda.synchronize()
    return {"profile_e2e": f"prefill 512 + {E2E_PROFILE_STEPS} decode-graph replays, fp16 activations",
            "us_per_token_events_under_this_run": round(a.elapsed_time(b) * 1e3 / E2E_PROFILE_STEPS, 2)}


def profile_verify(dev, reps: int = 8):
    """Kernel-trace workload: config-5 prompt, then `reps` replays of the
    8-row verify graph (the position reset before each)."""
    import torch

    _, t, ids = e2e_model(dev, torch.float16)
    t.capture_verify([8])
    t.reset()
    t.prefill(ids)
    N = t.pos
    for _ in range(reps):
        t.pos_dev.fill_(N)
        t._verify_graphs[8].replay()
    torch.cuda.synchronize()


def e2e_cpu_baseline(dev, budget_s: float):
    """BASELINE config 5 on the host cores through the reference's own CPU
    path: each token's 168 projections by the reference's q4_gemv_sym
    (oracle/_ref, compiled from its q4_gemv.cpp; the scalar loop on x86,
    q4_gemv.cpp:240-247) over the model's packed int4 codes and scales, as
    Q4Linear calls it for one row (q4_linear.py:49-68); RMSNorm, RoPE, the
    int8 cache, attention and the tied lm_head in numpy (oracle/model.py).
    The 512-token prompt runs untimed through the dense numpy restatement;
    the timed part is greedy decode steps after it, first on one thread
    (numpy's BLAS pinned to 1: the reference's execution model), then on
    every core of the process's affinity (each projection's rows dealt to one
    thread per core, the BLAS pinned to the same count). Without oracle/_ref
    both legs use the dense numpy restatement (kind "port")."""
    import copy

    import torch
    from threadpoolctl import threadpool_limits

    from oracle import cpu
    from oracle import model as OM
    from siliconfer_amd.model.config import rope_tables

    ref = cpu.ref_available()
    cfg, m, ids = e2e_model(dev, torch.float32)
    W = m.export_weights(packed=ref)
    cos, sin = rope_tables(cfg, m.max_seq)
    del m
    torch.cuda.empty_cache()
    cache0 = OM.KVCache(cfg.num_hidden_layers)
    t0 = time.perf_counter()
    tok0 = OM.greedy(OM.forward(W, cfg, ids, cache0, cos, sin)[-1])
    t_prefill = time.perf_counter() - t0

    def leg(threads, budget):
        cache = copy.deepcopy(cache0)
        if ref:
            def lin(L, name, x):
                pk, s32, g = L[name + "_q4"]
                return cpu.gemv_sym_ref_rows(pk, s32, x, g, threads)[None, :]
        else:
            lin = OM.dense
        with threadpool_limits(limits=threads):
            tok, n, t1 = tok0, 0, time.perf_counter()
            while time.perf_counter() - t1 < budget and n < E2E_TOKENS - 1:
                tok = OM.greedy(OM.forward(W, cfg, [tok], cache, cos, sin, linear=lin)[-1])
                n += 1
            dt = time.perf_counter() - t1
        return n, dt

    n1, dt1 = leg(1, budget_s)
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    nn, dtn = leg(cores, budget_s / 3)
    kind = "reference" if ref else "port"
    what = ("the reference's q4_gemv_sym per projection (168 per token) + numpy norms, RoPE, "
            "int8-cache attention and tied lm_head" if ref else
            "numpy fp32 over the dequantized int4 weights and the int8 cache")
    return {"value": round(n1 / dt1, 3), "unit": "tok/s", "cores": 1, "blas_threads": 1, "kind": kind,
            "sample": f"{n1} greedy decode steps in {dt1:.1f} s after the 512-token prompt "
                      f"(prompt untimed, {t_prefill:.1f} s dense numpy); {what}",
            "all_cores": {"value": round(nn / dtn, 3), "unit": "tok/s", "cores": cores,
                          "blas_threads": cores, "kind": kind,
                          "sample": f"{nn} decode steps in {dtn:.1f} s, each projection's rows dealt to "
                                    f"{cores} OpenMP threads"}}


def cpu_baseline(budget_s: float):
    """Reference CPU kernel on a bounded sample of the same sweep."""
    from oracle import cpu

    kind = "reference" if cpu.ref_available() else "port"
    rng = np.random.default_rng(7)
    data = []
    for i, (N, K) in enumerate(SHAPES):
        pk, s = quantize_shape(N, K, 2 + i)
        s32 = s.astype(np.float16).astype(np.float32)
        X = rng.normal(0, 1, (8, K)).astype(np.float16).astype(np.float32)
        data.append((N, K, pk, s32, X))

    def sweep(nthreads, impl):
        nbytes = 0
        for N, K, pk, s32, X in data:
            for B in BATCHES:
                if impl == "reference":
                    cpu.gemm_sym(pk, s32, X[:B], GROUP, impl="reference")
                else:
                    cpu.gemm_sym(pk, s32, X[:B], GROUP, nthreads=nthreads, impl="port")
                nbytes += alg_bytes(N, K, B)
        return nbytes

    def timed(nthreads, impl, budget):
        sweep(nthreads, impl)  # warm
        t0 = time.perf_counter()
        n, nbytes = 0, 0
        while True:
            nbytes += sweep(nthreads, impl)
            n += 1
            if time.perf_counter() - t0 >= budget:
                break
        dt = time.perf_counter() - t0
        return nbytes / dt / 1e9, n, dt

    gbs1, n1, dt1 = timed(1, kind, budget_s)
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    gbsn, nn, dtn = timed(cores, "port", budget_s / 3)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(gbs1, 3), "unit": "GB/s", "cores": 1, "kind": kind,
        "sample": f"{n1} full config-3 sweeps (3 shapes x batch 1,2,4,8; batch>1 as the "
                  f"reference's GEMM loop of GEMVs) in {dt1:.1f} s, fp32 scales/x as the "
                  f"reference takes them",
        "all_cores": {"value": round(gbsn, 3), "cores": cores, "kind": "port",
                      "sample": f"{nn} sweeps in {dtn:.1f} s, OpenMP row split over every core "
                                "in the process's affinity"},
        "cpu_model": cpu_model, "nproc": os.cpu_count(),
    }


PROFILE_WARM, PROFILE_STEPS = 8, 64


def profile_kernels(dev) -> None:
    """The timed region's own launches for rocprofv3 (trace or counters):
    PROFILE_WARM + PROFILE_STEPS replays of the captured sweep graphs (the
    summary drops the warm ones), a 256 MiB device copy (read 256 MiB + write
    256 MiB) that calibrates FETCH_SIZE / WRITE_SIZE, the per-launch floor
    (graph replays of the empty launch and of the plain reads, as bench.py
    times them), then the secondary kernels' cases (config 1, 2, 4 and the KV
    append), launched once per cold copy."""
    import torch

    sweep = GpuSweep(dev)
    sweep.capture()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(sweep.stream):
        sweep.run(0, PROFILE_WARM)
        e0.record(sweep.stream)  # events are markers, not dispatches: the trace's order is unchanged
        sweep.run(PROFILE_WARM, PROFILE_STEPS)
        e1.record(sweep.stream)
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
    torch.cuda.synchronize()
    sweep_us = e0.elapsed_time(e1) * 1e3 / PROFILE_STEPS
    empty, reads = floor_us(dev, sweep.stream, sorted({alg_bytes(N, K, 1) for N, K in SHAPES}))
    secondary(dev, sweep.stream, eager=True)
    print(json.dumps({"profile_kernels": f"{PROFILE_WARM} + {PROFILE_STEPS} graph replays of the "
                                         "12-case sweep", "calibration_copy_bytes": 256 << 20,
                      "sweep_us_events_under_this_run": round(sweep_us, 3),
                      "floor_us_events_under_this_run": {"empty": round(empty, 3),
                                                         **{str(k): round(v, 3) for k, v in reads.items()}}}))


CALIB_BYTES = 256 << 20
MI355X_SIMDS = 256 * 4
MI355X_CLOCK_HZ = 2.4e9  # peak engine clock


def calibration_copy(dev) -> None:
    """Three device copies of CALIB_BYTES (read + write CALIB_BYTES each): what
    FETCH_SIZE / WRITE_SIZE read for them scales every other dispatch's count."""
    import torch

    src = torch.empty(CALIB_BYTES, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def summarize_kernels(trace_csv: str, *pmc_csvs: str) -> dict:
    """Per-kernel summary of a `bench.py --profile-case` run under rocprofv3:
    durations from the --kernel-trace CSV; from --pmc counter CSVs, the median
    per dispatch of every counter, HBM bytes (FETCH_SIZE + WRITE_SIZE, each
    scaled by what it reads for the calibration copy) with the GB/s they give
    over the mean duration, and the MFMA busy fraction: SQ_VALU_MFMA_BUSY_CYCLES
    over the cycles of 1024 SIMDs at 2.4 GHz for the mean duration (the CSV
    sums GRBM_GUI_ACTIVE over its instances, so it is reported, not divided by)."""
    import csv
    import statistics

    per = {}
    for r in csv.DictReader(open(trace_csv)):
        k = _short_kernel(r["Kernel_Name"])
        if "copyBuffer" in r["Kernel_Name"]:
            continue
        per.setdefault(k, {"dur": [], "ctr": {}})["dur"].append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    scale = {}
    for path in pmc_csvs:
        rows = list(csv.DictReader(open(path)))
        for r in rows:
            name, v = r["Counter_Name"], float(r["Counter_Value"])
            if "copyBuffer" in r["Kernel_Name"]:
                if name in ("FETCH_SIZE", "WRITE_SIZE"):
                    scale[name] = max(scale.get(name, 0.0), v)
                continue
            k = _short_kernel(r["Kernel_Name"])
            per.setdefault(k, {"dur": [], "ctr": {}})["ctr"].setdefault(name, []).append(v)
    out = {}
    for k, d in per.items():
        e = {}
        if d["dur"]:
            e.update(n=len(d["dur"]), mean_us=round(statistics.fmean(d["dur"]), 3),
                     median_us=round(statistics.median(d["dur"]), 3), min_us=round(min(d["dur"]), 3))
        ctr = {n: statistics.median(v) for n, v in d["ctr"].items()}
        if ctr:
            e["counters_median_per_dispatch"] = {n: round(v, 1) for n, v in ctr.items()}
        if "FETCH_SIZE" in ctr and "WRITE_SIZE" in ctr and scale:
            ff = CALIB_BYTES / 1024 / scale["FETCH_SIZE"]
            wf = CALIB_BYTES / 1024 / scale["WRITE_SIZE"]
            e["fetch_bytes"] = int(ctr["FETCH_SIZE"] * ff * 1024)
            e["write_bytes"] = int(ctr["WRITE_SIZE"] * wf * 1024)
            e["calibration"] = {"fetch_scale": round(ff, 4), "write_scale": round(wf, 4)}
            if "mean_us" in e:
                e["hbm_GBps"] = round((e["fetch_bytes"] + e["write_bytes"]) / e["mean_us"] / 1e3, 1)
                e["hbm_frac_of_8TBps"] = round(e["hbm_GBps"] / 8000, 4)
        if "SQ_VALU_MFMA_BUSY_CYCLES" in ctr and "mean_us" in e:
            e["mfma_busy_frac"] = round(ctr["SQ_VALU_MFMA_BUSY_CYCLES"] /
                                        (MI355X_SIMDS * e["mean_us"] * 1e-6 * MI355X_CLOCK_HZ), 4)
        if "SQ_WAIT_INST_ANY" in ctr and "SQ_WAVE_CYCLES" in ctr:
            e["wave_cycles_waiting_frac"] = round(ctr["SQ_WAIT_INST_ANY"] / ctr["SQ_WAVE_CYCLES"], 4)
        if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in ctr:
            e["mfma_bf16_flop"] = int(ctr["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512)
        if "SQ_VALU_MFMA_COEXEC_CYCLES" in ctr and ctr.get("SQ_VALU_MFMA_BUSY_CYCLES"):
            e["mfma_cycles_with_valu_frac"] = round(
                ctr["SQ_VALU_MFMA_COEXEC_CYCLES"] / ctr["SQ_VALU_MFMA_BUSY_CYCLES"], 4)
        if ctr.get("SQ_WAVES"):
            mix = {n[len("SQ_INSTS_"):].lower(): round(ctr[n] / ctr["SQ_WAVES"], 1)
                   for n in ("SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_INSTS_SALU") if n in ctr}
            if mix:
                e["instructions_per_wave"] = mix
        out[k] = e
    meds = [e["median_us"] for k, e in out.items() if k.startswith("k_") and "median_us" in e]
    if meds:
        out["sum_of_kernel_medians_us"] = round(sum(meds), 3)
    return out


def _short_kernel(name: str) -> str:
    import re

    m = (re.search(r"k_q4_gemv_blkILi(\d)ELb(\d)ELi(\d)ELi(\d)ELi(\d+)ELb(\d)ELi(\d)ELb(\d)E", name) or
         re.search(r"k_q4_gemv_blk<(\d), (\w+), (\d), (\d), (\d+), (\w+), (\d), (\w+)(?:, \w+)?>",
                   name.replace("true", "1").replace("false", "0")))
    if m:
        x = {"0": "f32", "1": "f16", "2": "bf16"}[m.group(1)]
        pre = {"0": "", "1": ",pre=rmsnorm", "2": ",pre=silu", "3": ",pre=attn-merge"}[m.group(7)]
        rope = ",rope+append" if m.group(8) == "1" else ""
        src = "lds" if m.group(6) == "1" else "direct"
        return (f"k_q4_gemv_blk<x={x},asym={m.group(2)},gk={m.group(3)},T={m.group(4)},"
                f"BPW={m.group(5)},{src}{pre}{rope}>")
    m = re.search(r"(k_[a-z0-9_]+|__amd_rocclr_[A-Za-z]+|at::native::[a-z_]+)", name)
    return m.group(1) if m else name[:40]


def sweep_cases():
    return [(N, K, B) for N, K in SHAPES for B in BATCHES]


def summarize_profile(trace_csv=None, fetch_csv=None, write_csv=None) -> dict:
    """Summaries of rocprofv3 CSV outputs of `bench.py --profile-kernels`: the
    sweep's GEMV dispatches (the first ones of either GEMV kernel, in launch
    order, after the warm replays) labelled with their case by position in the
    12-launch replay; per-case duration
    stats from a --kernel-trace run, and per-case HBM bytes from FETCH_SIZE /
    WRITE_SIZE runs, scaled by what the counters read for the 256 MiB
    calibration copy (the largest copy dispatch)."""
    import csv
    import statistics

    cs = sweep_cases()
    skip = PROFILE_WARM * len(cs)
    labels = [cs[i % len(cs)] for i in range(PROFILE_STEPS * len(cs))]

    def sweep_rows(rows, id_key):
        gemv = sorted((r for r in rows if "k_q4_gemv" in r["Kernel_Name"]), key=lambda r: int(r[id_key]))
        return list(zip(labels, gemv[skip:skip + len(labels)]))

    out = {"cases": [{"N": N, "K": K, "B": B, "launches": PROFILE_STEPS} for N, K, B in cs]}
    if trace_csv:
        rows = list(csv.DictReader(open(trace_csv)))
        per = {}
        for lab, r in sweep_rows(rows, "Dispatch_Id"):
            per.setdefault(lab, (_short_kernel(r["Kernel_Name"]), []))[1].append(
                (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        for c in out["cases"]:
            k, v = per.get((c["N"], c["K"], c["B"]), ("", []))
            if v:
                c.update(kernel=k, n=len(v), mean_us=round(statistics.fmean(v), 3),
                         median_us=round(statistics.median(v), 3), min_us=round(min(v), 3))
        means = [c["mean_us"] for c in out["cases"] if "mean_us" in c]
        if len(means) == len(cs):
            out["sweep_kernel_sum_mean_us"] = round(sum(means), 3)
            out["sweep_kernel_sum_median_us"] = round(sum(c["median_us"] for c in out["cases"]), 3)
        # the floor kernels of the same run: the empty launch, and the plain
        # reads by grid size (one per byte count)
        fl = {}
        for r in rows:
            if "k_empty" in r["Kernel_Name"] or "k_read" in r["Kernel_Name"]:
                key = "empty" if "k_empty" in r["Kernel_Name"] else f"read_grid{r['Grid_Size_X']}"
                fl.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        if fl:
            out["floor_traced_us"] = {k: {"n": len(v), "median": round(statistics.median(v), 3),
                                          "mean": round(statistics.fmean(v), 3)} for k, v in fl.items()}
        copies = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rows
                  if "copyBuffer" in r["Kernel_Name"]]
        if copies:
            out["copy_us"] = {"n": len(copies), "median": round(statistics.median(copies), 3),
                              "max": round(max(copies), 3)}
    if fetch_csv and write_csv:
        def load(p):
            rows = list(csv.DictReader(open(p)))
            val = {int(r["Dispatch_Id"]): float(r["Counter_Value"]) for r in rows}
            copy_kib = max(float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"])
            per = {}
            for lab, r in sweep_rows(rows, "Dispatch_Id"):
                per.setdefault(lab, []).append(val[int(r["Dispatch_Id"])])
            return per, copy_kib
        (f, fk), (w, wk) = load(fetch_csv), load(write_csv)
        ff, wf = (256 << 20) / 1024 / fk, (256 << 20) / 1024 / wk
        for c in out["cases"]:
            lab = (c["N"], c["K"], c["B"])
            if lab in f and lab in w:
                c["fetch_bytes"] = int(statistics.median(f[lab]) * ff * 1024)
                c["write_bytes"] = int(statistics.median(w[lab]) * wf * 1024)
                c["hbm_bytes"] = c["fetch_bytes"] + c["write_bytes"]
                c["alg_bytes"] = alg_bytes(*lab)
                c["hbm_over_alg"] = round(c["hbm_bytes"] / c["alg_bytes"], 4)
        hb = [c["hbm_bytes"] for c in out["cases"] if "hbm_bytes" in c]
        out["fetch_scale"], out["write_scale"] = round(ff, 4), round(wf, 4)
        if hb:
            out["hbm_bytes_per_launch_avg"] = int(statistics.fmean(hb))
    return out


def summarize_e2e(trace_csv: str, steps: int = 16) -> dict:
    """Per-kernel time per decoded token from a rocprofv3 --kernel-trace run of
    `bench.py --profile-e2e` (or --profile-verify): the dispatches from the
    k_embed of the first of the last `steps` steps on, grouped by kernel; per
    kernel its dispatches per step, median and mean duration, and median x
    dispatches per step. `kernel_us_per_token_median` sums the last column:
    the statistic set against the untraced step time."""
    import csv
    import re
    import statistics

    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    starts = [i for i, r in enumerate(rows) if "k_embed" in r["Kernel_Name"]]
    steps = min(steps, len(starts) - 1)  # the first k_embed is the prompt's
    dec = rows[starts[-steps]:]
    per = {}
    for r in dec:
        name = r["Kernel_Name"]
        m = re.search(r"(k_[a-z0-9_]+)(?:<([^>]*)>|I(\S+?)EEEv)?", name.replace("(anonymous namespace)::", ""))
        key = _short_kernel(name) if "k_q4_gemv" in name else (m.group(1) + (f"<{m.group(2)}>" if m and m.group(2) else "") if m else name[:40])
        per.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    out = [{"kernel": k, "per_token": len(v) / steps, "median_us": round(statistics.median(v), 3),
            "mean_us": round(statistics.fmean(v), 3), "min_us": round(min(v), 3),
            "median_us_per_token": round(statistics.median(v) * len(v) / steps, 1)}
           for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1]))]
    return {"steps": steps, "kernels": out,
            "kernel_us_per_token_median": round(sum(statistics.median(v) * len(v) for v in per.values())
                                                / steps, 1),
            "kernel_us_per_token_mean": round(sum(sum(v) for v in per.values()) / steps, 1)}


def load_traffic():
    try:
        with open(PMC_FILE) as f:
            d = json.load(f)
        return d.get("hbm_bytes_per_launch_avg"), d
    except (OSError, ValueError):
        return None, None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true", help="skip the other kernels' timings")
    ap.add_argument("--no-e2e", action="store_true", help="skip the config-5 end-to-end decode")
    ap.add_argument("--profile-e2e", action="store_true",
                    help="only run eager config-5 decode steps (for rocprofv3)")
    ap.add_argument("--profile-verify", action="store_true",
                    help="only run config-5 8-row verify graph replays (for rocprofv3)")
    ap.add_argument("--no-spec", action="store_true", help="skip the speculative-decoding leg")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of reference CPU work")
    ap.add_argument("--eager", action="store_true", help="launch from Python instead of HIP graphs")
    ap.add_argument("--profile-case", choices=SECONDARY_CASES,
                    help="only time one secondary case (its graph replays, for rocprofv3)")
    ap.add_argument("--profile-kernels", action="store_true",
                    help="only run the sweep's graph replays and the secondary kernels (for rocprofv3)")
    ap.add_argument("--summarize-e2e", metavar="CSV",
                    help="per-kernel time per token from a kernel trace of --profile-e2e")
    ap.add_argument("--sweep-attn-splits", type=int, metavar="HEAD_DIM",
                    help="time config-4-shaped attention over T x split count and exit")
    ap.add_argument("--summarize-kernels", nargs="+", metavar="CSV",
                    help="TRACE_CSV [PMC_CSV ...]: per-kernel summary of a --profile-case run")
    ap.add_argument("--summarize-profile", nargs="+", metavar="CSV",
                    help="TRACE_CSV [FETCH_CSV WRITE_CSV]: summarize rocprofv3 output and exit")
    args = ap.parse_args()

    if args.summarize_e2e:
        print(json.dumps(summarize_e2e(args.summarize_e2e), indent=1))
        return 0
    if args.summarize_kernels:
        print(json.dumps(summarize_kernels(*args.summarize_kernels), indent=1))
        return 0
    if args.summarize_profile:
        paths = args.summarize_profile + [None] * 3
        print(json.dumps(summarize_profile(*paths[:3]), indent=1))
        return 0

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only; --gpus must be 1 "
              "(the hot path's multi-GPU sharding is a design, not a built path)", file=sys.stderr)
        return 2

    import torch

    from siliconfer_amd import _lib

    if not _lib.hip_available():
        raise SystemExit("bench.py needs a gfx950 GPU and the built libsiliconfer_hip.so")
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.sweep_attn_splits:
        d = args.sweep_attn_splits
        Ts = (128, 512, 1024, 2048, 4096, 8192, 16384) if d <= 64 else (256, 512, 2048, 4096, 8192, 16384)
        print(json.dumps(sweep_attn_splits(dev, d, Ts, splits=(1, 8, 16, 32, 64, 128))))
        return 0
    if args.profile_case:
        st = torch.cuda.Stream(dev)
        print(json.dumps(secondary(dev, st, only={args.profile_case})))
        calibration_copy(dev)
        return 0
    if args.profile_kernels:
        profile_kernels(dev)
        return 0
    if args.profile_verify:
        profile_verify(dev)
        print(json.dumps({"profile_verify": "prefill 512 + 8 replays of the 8-row verify graph"}))
        return 0
    if args.profile_e2e:
        print(json.dumps(profile_e2e(dev)))
        return 0

    sweep = GpuSweep(dev)
    if not args.eager:
        sweep.capture()

    with torch.cuda.stream(sweep.stream):
        sweep.run(0, args.warmup)
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(sweep.stream)
        sweep.run(args.warmup, args.steps)
        t1.record(sweep.stream)
        torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / args.steps
    value = sweep.step_bytes / (ms_per_step * 1e-3) / 1e9

    us = sweep.per_case_us()
    case_bytes = [alg_bytes(N, K, B) for N, K, B, *_ in sweep.cases]
    # the roofline's kernel figure from the timed region itself: average
    # algorithmic bytes per launch over the average launch duration (the step
    # is the 12 launches back to back), so it equals `value`
    step_us = ms_per_step * 1e3
    achieved = sum(case_bytes) / (step_us * 1e-6) / 1e9
    empty_us, read_us = floor_us(dev, sweep.stream, case_bytes)
    floor_sum = sum(read_us[b] for b in case_bytes)
    cases = [{"N": N, "K": K, "B": B, "us": round(t, 3),
              "GBps": round(b / (t * 1e-6) / 1e9, 1), "floor_us": round(read_us[b], 3),
              "frac_of_floor": round(read_us[b] / t, 4)}
             for (N, K, B, *_), t, b in zip(sweep.cases, us, case_bytes)]
    traffic, _ = load_traffic()
    sec = None if args.no_secondary else secondary(dev, sweep.stream)
    e2e = None if args.no_e2e else e2e_decode(dev)
    if e2e is not None and not args.no_cpu:
        e2e["cpu_baseline"] = e2e_cpu_baseline(dev, args.cpu_budget)
    spec = None if (args.no_e2e or args.no_spec) else e2e_speculative(dev)
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_budget)

    line = {
        "metric": "int4 GEMV achieved HBM GB/s (% of peak) at 7B shapes; decode tok/s at 0.5B",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 x fp16 -> fp32",
        "data": "synthetic (seeded N(0,0.02) weights RTN int4, N(0,1) fp16 activations)",
        "config": {
            "workload": "BASELINE config 3: 7B-shape int4 decode GEMV sweep, sym g=128, "
                        "W [4096,4096] [11008,4096] [4096,11008] x batch 1,2,4,8, cold HBM",
            "launch": "eager" if args.eager else "hipgraph",
            "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "frac_of_floor": round(floor_sum / step_us, 4),
            "avg_launch_us": round(step_us / len(case_bytes), 4),
            "floor": {"empty_launch_us": round(empty_us, 3),
                      "read_GBps": round(sum(case_bytes) / (floor_sum * 1e-6) / 1e9, 1),
                      "read_frac_of_peak": round(sum(case_bytes) / (floor_sum * 1e-6) / 1e9
                                                 / HBM_PEAK_GBS, 4),
                      "what": "sf_floor_read of each case's algorithmic bytes (one 16-byte load "
                              "per lane, cold), timed like the cases in the same run; "
                              "frac_of_floor = sum of floor times / the timed step"},
            "traffic": traffic,
            "kernel": "sf_q4_gemv (k_q4_gemv_blk: MFMA over the unit-order blob, every batch); "
                      "achieved = average algorithmic bytes per launch / average launch duration of "
                      "the timed region (HIP events around the K graph replays of the 12-case "
                      "sweep, on the stream the launches run on); cases[].us time each case alone",
            "alg_bytes_per_launch_avg": int(sum(case_bytes) / len(case_bytes)),
        },
        "cases": cases,
        "decode_tok_s": None if e2e is None else e2e["fp16"]["decode_tok_s"],
        "e2e_config5": e2e,
        "speculative_config5": spec,
        "secondary": sec,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
