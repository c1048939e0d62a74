// ref_glue.cpp — C-linkage entry points onto the reference's own C++ kernels.
// TEST INFRASTRUCTURE ONLY. Compiled by oracle/Makefile together with the
// reference sources where they lie (/root/reference/siliconfer/kernels/neon/
// q4_gemv.cpp, q4_gemm.cpp), so ctypes can call the reference implementation
// itself: q4_gemv_sym_scalar (q4_gemv.cpp:262-297), q4_gemv_sym_neon (on x86
// this routes to the scalar kernel, q4_gemv.cpp:240-247) and q4_gemm_sym_neon
// (q4_gemm.cpp:12-27).  The reference's asymmetric entry points are not
// exposed: on a non-ARM host they compute the symmetric kernel
// (q4_gemv.cpp:249-255), so they cannot serve as an asym oracle here.
#include <omp.h>

#include "q4_gemv.h"

extern "C" {
void ref_q4_gemv_sym_scalar(const uint8_t* W, const float* s, const float* x, float* y,
                            int out_f, int in_f, int g) {
  q4_gemv_sym_scalar(W, s, x, y, out_f, in_f, g);
}
void ref_q4_gemv_sym(const uint8_t* W, const float* s, const float* x, float* y,
                     int out_f, int in_f, int g) {
  q4_gemv_sym_neon(W, s, x, y, out_f, in_f, g);
}
void ref_q4_gemm_sym(const uint8_t* W, const float* s, const float* X, float* Y,
                     int out_f, int in_f, int T, int g) {
  q4_gemm_sym_neon(W, s, X, Y, out_f, in_f, T, g);
}
// The reference's q4_gemv_sym over `parts` row slices on an OpenMP team of
// `parts` threads: each row's sum is the reference's own, only the rows are
// dealt out (the CPU baseline's all-cores leg).
void ref_q4_gemv_sym_rows(const uint8_t* W, const float* s, const float* x, float* y,
                          int out_f, int in_f, int g, int parts) {
  const int n_groups = in_f / g;
#pragma omp parallel for num_threads(parts) schedule(static, 1)
  for (int i = 0; i < parts; ++i) {
    const int r0 = (int)((long long)out_f * i / parts), r1 = (int)((long long)out_f * (i + 1) / parts);
    if (r1 > r0)
      q4_gemv_sym_neon(W + (size_t)r0 * (in_f / 2), s + (size_t)r0 * n_groups, x, y + r0, r1 - r0, in_f, g);
  }
}
}
