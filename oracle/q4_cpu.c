/* q4_cpu.c — C restatement of the reference's CPU hot path. TEST INFRASTRUCTURE
 * ONLY: used as the checker's C twin and as the timed CPU baseline in bench.py.
 *
 * Reference anchors (/root/reference):
 *   oc_gemv_sym    siliconfer/kernels/neon/q4_gemv.cpp:262-297 (q4_gemv_sym_scalar;
 *                  on x86 this is what q4_gemv_sym_neon runs, :240-247)
 *   oc_gemv_asym   siliconfer/kernels/neon/q4_gemv.cpp:145-238 (math of
 *                  q4_gemv_asym_neon, done correctly; the reference's own x86
 *                  fallback routes asym to the symmetric kernel, :249-255)
 *   oc_gemm_*      siliconfer/kernels/neon/q4_gemm.cpp:12-51 (loop of GEMVs)
 *   oc_attn_decode dequantize the int8 cache then softmax attention, the
 *                  reference tests' oracle (tests/test_metal_attention.py:21-32)
 *
 * Every entry point takes `nthreads`: 1 reproduces the reference's execution
 * model (single thread, q4_gemv.cpp:49 plain row loop); >1 splits rows over
 * OpenMP threads.  Scales/zeros/activations are fp32 as in the reference
 * (bindings.cpp:18-19); callers upcast fp16 data exactly.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline int nib_signed(unsigned v) { return v < 8 ? (int)v : (int)v - 16; }

static void gemv_sym_rows(const uint8_t *W, const float *s, const float *x, float *y,
                          int r0, int r1, int K, int g) {
  const int ng = K / g, hg = g / 2;
  for (int i = r0; i < r1; ++i) {
    const uint8_t *wr = W + (size_t)i * (K / 2);
    float yi = 0.f;
    for (int gi = 0; gi < ng; ++gi) {
      const uint8_t *wg = wr + gi * hg;
      const float *xg = x + gi * g;
      float part = 0.f;
      for (int c = 0; c < hg; ++c) {
        unsigned b = wg[c];
        part += (float)nib_signed(b & 15u) * xg[2 * c];
        part += (float)nib_signed(b >> 4) * xg[2 * c + 1];
      }
      yi += part * s[(size_t)i * ng + gi];
    }
    y[i] = yi;
  }
}

static void gemv_asym_rows(const uint8_t *W, const float *s, const float *z, const float *x,
                           float *y, int r0, int r1, int K, int g) {
  const int ng = K / g, hg = g / 2;
  for (int i = r0; i < r1; ++i) {
    const uint8_t *wr = W + (size_t)i * (K / 2);
    float yi = 0.f;
    for (int gi = 0; gi < ng; ++gi) {
      const uint8_t *wg = wr + gi * hg;
      const float *xg = x + gi * g;
      float dot = 0.f, xs = 0.f;
      for (int c = 0; c < hg; ++c) {
        unsigned b = wg[c];
        dot += (float)(b & 15u) * xg[2 * c] + (float)(b >> 4) * xg[2 * c + 1];
        xs += xg[2 * c] + xg[2 * c + 1];
      }
      yi += (dot - z[(size_t)i * ng + gi] * xs) * s[(size_t)i * ng + gi];
    }
    y[i] = yi;
  }
}

static int clamp_threads(int n) { return n < 1 ? 1 : n; }

void oc_gemv_sym(const uint8_t *W, const float *s, const float *x, float *y,
                 int N, int K, int g, int nthreads) {
  nthreads = clamp_threads(nthreads);
  if (nthreads == 1) { gemv_sym_rows(W, s, x, y, 0, N, K, g); return; }
#pragma omp parallel num_threads(nthreads)
  {
#ifdef _OPENMP
    int t = omp_get_thread_num(), nt = omp_get_num_threads();
#else
    int t = 0, nt = 1;
#endif
    int r0 = (int)((long long)N * t / nt), r1 = (int)((long long)N * (t + 1) / nt);
    gemv_sym_rows(W, s, x, y, r0, r1, K, g);
  }
}

void oc_gemv_asym(const uint8_t *W, const float *s, const float *z, const float *x, float *y,
                  int N, int K, int g, int nthreads) {
  nthreads = clamp_threads(nthreads);
  if (nthreads == 1) { gemv_asym_rows(W, s, z, x, y, 0, N, K, g); return; }
#pragma omp parallel num_threads(nthreads)
  {
#ifdef _OPENMP
    int t = omp_get_thread_num(), nt = omp_get_num_threads();
#else
    int t = 0, nt = 1;
#endif
    int r0 = (int)((long long)N * t / nt), r1 = (int)((long long)N * (t + 1) / nt);
    gemv_asym_rows(W, s, z, x, y, r0, r1, K, g);
  }
}

void oc_gemm_sym(const uint8_t *W, const float *s, const float *X, float *Y,
                 int T, int N, int K, int g, int nthreads) {
  for (int t = 0; t < T; ++t)
    oc_gemv_sym(W, s, X + (size_t)t * K, Y + (size_t)t * N, N, K, g, nthreads);
}

void oc_gemm_asym(const uint8_t *W, const float *s, const float *z, const float *X, float *Y,
                  int T, int N, int K, int g, int nthreads) {
  for (int t = 0; t < T; ++t)
    oc_gemv_asym(W, s, z, X + (size_t)t * K, Y + (size_t)t * N, N, K, g, nthreads);
}

/* One (b, h) decode attention row over the dequantized cache, fp32 math.
 * q [D]; codes [T, D] int8 (row pitch D); scales [T]. */
static void attn_row(const float *q, const int8_t *kc, const float *ks, const int8_t *vc,
                     const float *vs, float *out, int T, int D, float scale, float *sc) {
  /* No infinities: this file is built with -ffast-math like the reference. */
  for (int d = 0; d < D; ++d) out[d] = 0.f;
  if (T <= 0) return;
  float m = 0.f;
  for (int t = 0; t < T; ++t) {
    const int8_t *kr = kc + (size_t)t * D;
    float dot = 0.f;
    for (int d = 0; d < D; ++d) dot += q[d] * (float)kr[d];
    sc[t] = dot * ks[t] * scale;
    if (t == 0 || sc[t] > m) m = sc[t];
  }
  float l = 0.f;
  for (int t = 0; t < T; ++t) {
    float p = expf(sc[t] - m);
    l += p;
    const int8_t *vr = vc + (size_t)t * D;
    float pv = p * vs[t];
    for (int d = 0; d < D; ++d) out[d] += pv * (float)vr[d];
  }
  float inv = 1.f / (l > 1e-20f ? l : 1e-20f);
  for (int d = 0; d < D; ++d) out[d] *= inv;
}

/* q [B,H,D] f32; codes [B,KVH,Tcap,D] i8; scales [B,KVH,Tcap] f32; out [B,H,D]. */
int oc_attn_decode(const float *q, const int8_t *kc, const float *ks, const int8_t *vc,
                   const float *vs, float *out, int B, int H, int KVH, int T, int Tcap,
                   int D, float scale, int nthreads) {
  if (KVH <= 0 || H % KVH) return -1;
  const int grp = H / KVH;
  nthreads = clamp_threads(nthreads);
#pragma omp parallel for num_threads(nthreads) collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      float *sc = (float *)malloc(sizeof(float) * (size_t)(T > 0 ? T : 1));
      int kh = h / grp;
      size_t base = ((size_t)b * KVH + kh) * (size_t)Tcap;
      attn_row(q + ((size_t)b * H + h) * D, kc + base * D, ks + base, vc + base * D, vs + base,
               out + ((size_t)b * H + h) * D, T, D, scale, sc);
      free(sc);
    }
  return 0;
}

int oc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
