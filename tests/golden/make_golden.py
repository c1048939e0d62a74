"""Write tests/golden/*.npz: golden vectors from the reference's own compiled kernels.

The outputs come from /root/reference/siliconfer/kernels/neon/q4_gemv.cpp and
q4_gemm.cpp (q4_gemv_sym_scalar, q4_gemv_sym_neon -> scalar on x86,
q4_gemm_sym_neon), compiled by oracle/Makefile into oracle/_ref/libref_q4.so.
Inputs are seeded and quantized with the oracle's restatement of
pack_weights_sym (pinned separately by tests/test_oracle_primitives.py).

Each case stores: packed uint8 [N, K/2]; scales float32 [N, K/g] (the
reference's fp32 scales); scales16 (those scales rounded to fp16, as the device
blob stores them); x / X float32 (values exactly representable in fp16);
y_ref from the reference kernel with the fp32 scales and y_ref16 with the
fp16-rounded scales. Run from the repo root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import cpu, primitives  # noqa: E402

CASES = [
    # name, N, K, g, T (0 = GEMV), seed   — shapes of the reference's tests
    ("gemv_128x256_g64", 128, 256, 64, 0, 42),      # tests/test_kernel.py:68-80
    ("gemv_128x256_g128", 128, 256, 128, 0, 42),
    ("gemv_64x128_g128", 64, 128, 128, 0, 7),       # :83-94
    ("gemv_1x128_g128", 1, 128, 128, 0, 5),         # :121-129
    ("gemv_96x896_g64", 96, 896, 64, 0, 11),        # config-1 row width
    ("gemv_40x4096_g128", 40, 4096, 128, 0, 12),    # config-3 row width
    ("gemm_64x128_g128_T4", 64, 128, 128, 4, 99),   # :136-151
    ("gemm_64x128_g128_T32", 64, 128, 128, 32, 99),
]


def make_case(N, K, g, T, seed):
    rng = np.random.default_rng(seed)
    W = rng.normal(0, 1, (N, K)).astype(np.float32)
    xs = (T, K) if T else (K,)
    x = rng.normal(0, 1, xs).astype(np.float16).astype(np.float32)
    packed, scales = primitives.pack_weights_sym(W, g)
    scales16 = scales.astype(np.float16)
    s16_as32 = scales16.astype(np.float32)
    if T:
        y = cpu.gemm_sym(packed, scales, x, g, impl="reference")
        y16 = cpu.gemm_sym(packed, s16_as32, x, g, impl="reference")
    else:
        y = cpu.gemv_sym(packed, scales, x, g, impl="reference")
        y16 = cpu.gemv_sym(packed, s16_as32, x, g, impl="reference")
        ys = cpu.gemv_sym(packed, scales, x, g, impl="reference_scalar")
        assert np.array_equal(y, ys), "reference NEON-entry and scalar kernels disagree"
    return dict(packed=packed, scales=scales, scales16=scales16, x=x, y_ref=y, y_ref16=y16,
                N=N, K=K, g=g, T=T, seed=seed)


def main() -> None:
    if not cpu.ref_available():
        cpu.build()
    if not cpu.ref_available():
        raise SystemExit("oracle/_ref/libref_q4.so missing: needs /root/reference")
    for name, N, K, g, T, seed in CASES:
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **make_case(N, K, g, T, seed))
        print("wrote", name)


if __name__ == "__main__":
    main()
