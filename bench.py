"""Benchmark: int4 decode GEMV achieved HBM GB/s at 7B shapes.

One step = one pass over config 3's sweep on one GPU: symmetric int4 RTN, group
128, W in {[4096,4096], [11008,4096], [4096,11008]} x batch {1, 2, 4, 8}, fp16
activations, fp32 accumulation — 12 GEMV launches. Every launch reads a
different copy of its weight blob (>= 512 MB of copies per shape, twice the
256 MB last-level cache), so the weights come from HBM. The step's launches are
replayed from HIP graphs.

Printed JSON (one line):
  value         whole-job algorithmic GB/s: sum of per-launch algorithmic bytes
                over the timed steps / wall time between HIP events bracketing
                the K timed steps (inputs resident in HBM);
  roofline      the GEMV kernel: achieved = algorithmic bytes per launch /
                average launch duration (HIP events around each launch on the
                launch stream), against the 8 TB/s MI355X HBM peak;
  cpu_baseline  the reference's own CPU kernel (q4_gemv.cpp / q4_gemm.cpp,
                compiled from /root/reference into oracle/_ref) or, when that
                library is absent, the C restatement oracle/q4_cpu.c, on a
                bounded sample of the same sweep, single-threaded as the
                reference runs; `all_cores` adds the restatement on every core.

Algorithmic bytes per launch (B = batch): N*K/2 (int4) + 2*N*K/128 (fp16
scales) + 2*B*K (fp16 x) + 2*B*N (fp16 y).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008)]
BATCHES = [1, 2, 4, 8]
GROUP = 128
COLD_BYTES = 512 << 20


def alg_bytes(N: int, K: int, B: int, g: int = GROUP) -> int:
    return N * K // 2 + 2 * N * (K // g) + 2 * B * K + 2 * B * N


def quantize_shape(N, K, seed):
    """Config-3 synthetic weights: W ~ N(0, 0.02) RTN-quantized, symmetric, g=128."""
    from siliconfer_amd.kernels import pack_weights_sym

    rng = np.random.default_rng(seed)
    W = rng.normal(0, 0.02, (N, K)).astype(np.float32)
    return pack_weights_sym(W, GROUP)


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
            copies = max(2, -(-COLD_BYTES // w.nbytes))
            blobs = [w.blob] + [w.blob.clone() for _ in range(copies - 1)]
            self.keep += blobs
            self.n_rot = max(self.n_rot, copies)
            x = torch.as_tensor(rng.normal(0, 1, (8, K)).astype(np.float16)).to(dev)
            self.keep.append(x)
            for B in BATCHES:
                y = torch.empty((B, N), dtype=torch.float16, device=dev)
                self.keep.append(y)
                self.cases.append((N, K, B, [b.data_ptr() for b in blobs], x.data_ptr(), y.data_ptr()))
        self.step_bytes = sum(alg_bytes(N, K, B) for N, K, B, *_ in self.cases)
        self.graphs = None

    def launch(self, ci: int, rot: int) -> None:
        N, K, B, blobs, xp, yp = self.cases[ci]
        rc = self.lib.sf_q4_gemv(blobs[rot % len(blobs)], xp, 1, yp, 1, None, None, 0, B, N, K,
                                 GROUP, 0, self.stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(self.lib.sf_last_error().decode())

    def eager_step(self, rot: int) -> None:
        for ci in range(len(self.cases)):
            self.launch(ci, rot)

    def capture(self) -> None:
        torch = self.torch
        self.graphs = []
        for rot in range(self.n_rot):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=self.stream):
                self.eager_step(rot)
            self.graphs.append(g)
        self.torch.cuda.synchronize()

    def step(self, i: int) -> None:
        if self.graphs is not None:
            self.graphs[i % self.n_rot].replay()
        else:
            self.eager_step(i)

    def per_launch_us(self, reps: int):
        """Average duration of each case's launch, from HIP event pairs around it."""
        torch = self.torch
        out = []
        with torch.cuda.stream(self.stream):
            for ci in range(len(self.cases)):
                ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                      for _ in range(reps)]
                for r in range(reps):
                    ev[r][0].record(self.stream)
                    self.launch(ci, r + 1)
                    ev[r][1].record(self.stream)
                self.stream.synchronize()
                ts = sorted(a.elapsed_time(b) * 1e3 for a, b in ev)
                out.append(float(np.mean(ts)))
        return out


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
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    cores = max(1, min(avail, int(os.environ.get("OMP_NUM_THREADS", "16") or 16), 16))
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
                      "sample": f"{nn} sweeps in {dtn:.1f} s, OpenMP row split"},
        "cpu_model": cpu_model,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of reference CPU work")
    ap.add_argument("--eager", action="store_true", help="launch from Python instead of HIP graphs")
    ap.add_argument("--event-reps", type=int, default=50)
    args = ap.parse_args()

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
    sweep = GpuSweep(dev)
    if not args.eager:
        sweep.capture()

    with torch.cuda.stream(sweep.stream):
        for i in range(args.warmup):
            sweep.step(i)
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(sweep.stream)
        for i in range(args.steps):
            sweep.step(args.warmup + i)
        t1.record(sweep.stream)
        torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / args.steps
    value = sweep.step_bytes / (ms_per_step * 1e-3) / 1e9

    us = sweep.per_launch_us(args.event_reps)
    case_bytes = [alg_bytes(N, K, B) for N, K, B, *_ in sweep.cases]
    achieved = sum(case_bytes) / (sum(us) * 1e-6) / 1e9
    cases = [{"N": N, "K": K, "B": B, "us": round(t, 3),
              "GBps": round(b / (t * 1e-6) / 1e9, 1)}
             for (N, K, B, *_), t, b in zip(sweep.cases, us, case_bytes)]

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
            "traffic": None,
            "kernel": "sf_q4_gemv (k_q4_gemv), per-launch HIP events, cold HBM",
        },
        "cases": cases,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
