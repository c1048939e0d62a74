// q4_anyg.hip — int4 GEMV / GEMM for any group size, over the block-layout blob.
//
// y[m, n] = sum_k s[n, k / g] * (q[n, k] - z[n, k / g]) * x[m, k], fp32 sums: the
// reference's q4_gemv_* / q4_gemm_* (/root/reference/siliconfer/kernels/neon/
// q4_gemv.cpp:37-297, q4_gemm.cpp:12-51) for the group sizes the MFMA kernels do
// not take: those that are not a multiple of 32 (a group boundary inside one
// MFMA's 32 k; the reference runs them through its scalar tail, q4_gemv.cpp:124-134),
// and fp32 activations whose LDS staging does not fit at long K.
//
// A workgroup owns one weight tile (16 rows) and up to 8 rows of x. Thread t
// takes row r = t % 16 and the units u = t / 16, t / 16 + 16, ... of K; in each
// unit it reads its row's 64 code bytes (four 16-byte pieces, one per k-piece)
// and walks k in increasing order, so the group's scale and zero-point are
// looked up only when k crosses into the next group. Each weight is
// dequantized once as (q - z) * s (exact in fp32: at most 5 + 11 significant
// bits) and multiplied into every x row. The 16 unit streams of a row are
// summed through LDS in stream order (bitwise repeatable).
#include "q4_gemv_blk.h"

using sf_gemv::kUnitK;

namespace {

constexpr int kStreams = 16, kRowsM = 8;

template <int XDT, bool ASYM>
__global__ void __launch_bounds__(256) k_q4_anyg(const uint8_t *__restrict__ w, const f16 *__restrict__ st,
                                                 const uint8_t *__restrict__ zt, const void *__restrict__ x,
                                                 void *y, int ydt, float *y32, const void *bias, int bdt,
                                                 int M, int N, int K, int G, uint32_t gmul, int nblk) {
  __shared__ float red[kStreams][kRowsM][16];
  const int tid = threadIdx.x, r = tid & 15, stream = tid >> 4;
  const int tile = blockIdx.x, m0 = blockIdx.y * kRowsM;
  const int mrows = min(kRowsM, M - m0);
  const int n = min(tile * 16 + r, N - 1);  // rows past N: a valid row, never stored
  float acc[kRowsM];
#pragma unroll
  for (int m = 0; m < kRowsM; ++m) acc[m] = 0.f;
  const size_t srow = (size_t)(n >> 3) * G;
  int gcur = -1;
  float s = 0.f, z = 8.f;
  for (int u = stream; u < nblk; u += kStreams) {
    const uint8_t *unit = w + ((size_t)tile * nblk + u) * 1024;
    u32x4 pc[4];
#pragma unroll
    for (int kg = 0; kg < 4; ++kg) pc[kg] = *(const u32x4 *)(unit + (r + 16 * kg) * 16);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int kg = 0; kg < 4; ++kg) {
        const uint32_t d = pc[kg][j];
        const int kb = u * kUnitK + 32 * j + 8 * kg;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int k = kb + e;
          if (k >= K) break;
          const int gi = (int)(((uint64_t)(uint32_t)k * gmul) >> 30);
          if (gi != gcur) {
            gcur = gi;
            s = (float)st[(srow + gi) * 8 + (n & 7)];
            if constexpr (ASYM) z = (float)((zt[(srow + gi) * 4 + ((n & 7) >> 1)] >> (4 * (n & 1))) & 15u);
          }
          const float code = (float)((d >> (4 * (e >> 1) + 16 * (e & 1))) & 15u);
          const float wq = (code - z) * s;
#pragma unroll
          for (int m = 0; m < kRowsM; ++m)
            if (m < mrows) acc[m] = fmaf(wq, sf_load_as_f32<XDT>(x, (size_t)(m0 + m) * K + k), acc[m]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kRowsM; ++m) red[stream][m][r] = acc[m];
  __syncthreads();
  if (tid < kRowsM * 16) {
    const int m = tid >> 4, c = tid & 15, row = tile * 16 + c;
    if (m < mrows && row < N) {
      float v = red[0][m][c];
      for (int q = 1; q < kStreams; ++q) v += red[q][m][c];
      sf_gemv::store_out(y, ydt, y32, bias, bdt, (size_t)(m0 + m) * N + row, row, v);
    }
  }
}

template <int XDT>
void launch_x(bool asym, dim3 grid, hipStream_t s, const uint8_t *w, const f16 *st, const uint8_t *zt,
              const void *x, void *y, int ydt, float *y32, const void *bias, int bdt, int M, int N,
              int K, int G, uint32_t gmul, int nblk) {
  if (asym)
    k_q4_anyg<XDT, true><<<grid, 256, 0, s>>>(w, st, zt, x, y, ydt, y32, bias, bdt, M, N, K, G, gmul, nblk);
  else
    k_q4_anyg<XDT, false><<<grid, 256, 0, s>>>(w, st, zt, x, y, ydt, y32, bias, bdt, M, N, K, G, gmul, nblk);
}

}  // namespace

// Shared by sf_q4_gemv and sf_q4_gemm (shapes already validated by the caller).
int sf_q4_anyg(const void *blob, const void *x, int x_dtype, void *y, int y_dtype, float *y_f32,
               const void *bias, int bias_dtype, int M, int N, int K, int g, int has_zeros,
               void *stream) {
  BlobLayout L;
  sf_blob_layout(N, K, g, has_zeros, &L);
  const uint8_t *w = (const uint8_t *)blob;
  const int nblk = (K + kUnitK - 1) / kUnitK;
  const uint32_t gmul = (uint32_t)(((1ull << 30) + g - 1) / g);
  SF_REQUIRE((uint64_t)K * g < (1ull << 30), SF_EUNSUPPORTED,
             "in_features=%d with group_size=%d is beyond this kernel's group arithmetic", K, g);
  const dim3 grid((N + 15) / 16, (M + kRowsM - 1) / kRowsM);
  const f16 *st = (const f16 *)(w + L.s_off);
  const uint8_t *zt = has_zeros ? w + L.z_off : nullptr;
  hipStream_t s = (hipStream_t)stream;
  if (x_dtype == SF_F16)
    launch_x<SF_F16>(has_zeros, grid, s, w, st, zt, x, y, y_dtype, y_f32, bias, bias_dtype, M, N, K, L.G, gmul, nblk);
  else if (x_dtype == SF_BF16)
    launch_x<SF_BF16>(has_zeros, grid, s, w, st, zt, x, y, y_dtype, y_f32, bias, bias_dtype, M, N, K, L.G, gmul, nblk);
  else
    launch_x<SF_F32>(has_zeros, grid, s, w, st, zt, x, y, y_dtype, y_f32, bias, bias_dtype, M, N, K, L.G, gmul, nblk);
  return sf_check_launch("sf_q4 (any group size)");
}
