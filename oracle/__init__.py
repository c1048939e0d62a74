"""CPU oracle for the quantized-inference hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference (`ALI-AL-MARJANI/siliconfer`)
computes on its int4 `Q4Linear` GEMV/GEMM path and its int8-KV decode attention
path. It is the checker the HIP kernels are compared against:

* `oracle.primitives` — quantize / pack / unpack / dequant formulas
  (reference `siliconfer/quant/primitives.py`, `siliconfer/kernels/neon/__init__.py`).
* `oracle.linear`     — float64 textbook GEMV / GEMM over dequantized weights
  (reference `siliconfer/kernels/neon/q4_gemv.cpp`, `q4_gemm.cpp`, and the
  reference tests' own oracle `tests/test_kernel.py:28-31,161-164`).
* `oracle.attention`  — int8 KV quantization and textbook softmax attention plus
  the split-T flash combine (reference `siliconfer/model/kv_cache.py`,
  `siliconfer/kernels/metal/q4_attention.py`).
* `oracle.cpu`        — ctypes bindings to `q4_cpu.c` (C restatement of the
  reference's scalar CPU kernels, used as the timed CPU baseline) and to
  `_ref/libref_q4.so` (the reference's own `q4_gemv.cpp`/`q4_gemm.cpp`
  compiled from `/root/reference` by `oracle/Makefile`, when present).

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may
import anything here. The product package `siliconfer_amd` never does.

Pinning status of each function is recorded in its docstring. Every function
here is pinned by at least one of: the reference's literal vectors, golden
vectors produced by the compiled reference C++ (`tests/golden/`), exhaustive
enumeration, or closed-form / invariant checks in `tests/test_oracle_*.py`.
"""
