// q4_gemm.hip — int4 prefill GEMM on CDNA4 MFMA (gfx950).
//
// Y[m, n] = sum_k X[m, k] * (q[n,k] - z[n,g(k)]) * s[n,g(k)], fp32 accumulation:
// the reference's q4_gemm_sym / q4_gemm_asym
// (/root/reference/siliconfer/kernels/neon/q4_gemm.cpp:12-51), which loop the
// GEMV over the T rows and re-stream W for each; here W is read once per
// 128-row block of X.
//
// Exactness without a per-group epilogue: with an fp16 scale, the dequantized
// weight w = (q - z) * s has at most 15 significant bits, so it is exactly
// w_hi + w_lo with w_hi = w truncated to bf16 (8 bits) and w_lo = w - w_hi (at
// most 7 bits, also exact in bf16). The workgroup dequantizes its W tile once
// into LDS as these two bf16 tiles, and every wave runs
// v_mfma_f32_32x32x16_bf16 on X*W_hi + X*W_lo. bf16 activations are exact
// operands; fp16 / fp32 activations are split the same way into bf16 hi + lo
// (fp16 exactly, fp32 to ~16 bits) and all four products are accumulated, so
// fp16 activations give exact products like the bf16 ones.
//
// Tiling: 128 x 128 output tile per 256-thread workgroup (2 x 2 waves, each
// 64 x 64 = 2 x 2 MFMA 32x32 tiles), K steps of 64 staged through padded LDS
// rows, next step's global loads issued before the current step's MFMAs. When
// the tile grid is too small to fill the GPU, K is split across workgroups
// into an fp32 workspace and summed by a second kernel in a fixed order.
#include "sf_common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDS_PITCH = BK + 8;  // bf16 elements per LDS row (+16 B breaks bank conflicts)
constexpr int NTHREADS = 256;

__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) {
  // top 16 bits of a (low half) and of b (high half)
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// One thread's share of the X tile: row tid/2, 32 consecutive k starting at
// 32*(tid%2). Loaded into registers as raw bits.
template <int XDT>
struct XRegs {
  static constexpr int NQ = XDT == SF_F32 ? 8 : 4;  // 16-byte loads
  u32x4 v[NQ];
};

template <int XDT>
__device__ __forceinline__ void load_x(XRegs<XDT> &r, const void *X, int M, int K, int m, int k) {
  const bool ok = m < M && k < K;
  const size_t esz = XDT == SF_F32 ? 4 : 2;
  const u32x4 *p = (const u32x4 *)((const char *)X + ((size_t)m * K + k) * esz);
#pragma unroll
  for (int i = 0; i < XRegs<XDT>::NQ; ++i) r.v[i] = ok ? p[i] : u32x4{0u, 0u, 0u, 0u};
}

// Split 2 fp32 values into (hi pair, lo pair) of bf16: hi = truncation, lo = rest.
__device__ __forceinline__ void split2(float a, float b, uint32_t &hi, uint32_t &lo) {
  const uint32_t ua = sf_bitcast<uint32_t>(a) & 0xFFFF0000u;
  const uint32_t ub = sf_bitcast<uint32_t>(b) & 0xFFFF0000u;
  const float ra = a - sf_bitcast<float>(ua);
  const float rb = b - sf_bitcast<float>(ub);
  hi = hi_pair(ua, ub);
  lo = hi_pair(sf_bitcast<uint32_t>(ra), sf_bitcast<uint32_t>(rb));
}

// Write the thread's 32 activations to the LDS tiles (hi only for bf16).
template <int XDT>
__device__ __forceinline__ void store_x(const XRegs<XDT> &r, uint16_t *xs_hi, uint16_t *xs_lo,
                                        int lrow, int lk) {
  u32x4 *dh = (u32x4 *)(xs_hi + lrow * LDS_PITCH + lk);
  if constexpr (XDT == SF_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) dh[i] = r.v[i];
  } else {
    u32x4 *dl = (u32x4 *)(xs_lo + lrow * LDS_PITCH + lk);
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // 8 activations per 16-byte LDS store
      float f[8];
      if constexpr (XDT == SF_F16) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const half2_t h = sf_bitcast<half2_t>(r.v[i][j]);
          f[2 * j] = (float)h.x;
          f[2 * j + 1] = (float)h.y;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = sf_bitcast<float>(r.v[2 * i + j / 4][j % 4]);
      }
      u32x4 h4, l4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t hp, lp;
        split2(f[2 * j], f[2 * j + 1], hp, lp);
        h4[j] = hp;
        l4[j] = lp;
      }
      dh[i] = h4;
      dl[i] = l4;
    }
  }
}

// One thread's share of the W tile: 16 bytes (32 nibbles) of row n at k.
struct WRegs {
  u32x4 w;
  float s, zs;  // scale and z*scale
};

__device__ __forceinline__ void load_w(WRegs &r, const uint8_t *__restrict__ wq,
                                       const f16 *__restrict__ st, const uint8_t *__restrict__ zt,
                                       int N, int K, int G, int g, int n, int k) {
  if (n < N && k < K) {
    r.w = *(const u32x4 *)(wq + (size_t)n * (K >> 1) + (k >> 1));
    const int grp = k / g;
    const size_t cell = (size_t)(n >> 3) * G + grp;
    const float s = (float)st[cell * 8 + (n & 7)];
    uint32_t z = 8u;  // offset-binary symmetric codes
    if (zt) z = (zt[cell * 4 + ((n & 7) >> 1)] >> (4 * (n & 1))) & 15u;
    r.s = s;
    r.zs = (float)z * s;
  } else {
    r.w = u32x4{0u, 0u, 0u, 0u};
    r.s = 0.f;
    r.zs = 0.f;
  }
}

// Dequantize 32 weights exactly and store them as bf16 hi / lo LDS rows.
__device__ __forceinline__ void store_w(const WRegs &r, uint16_t *ws_hi, uint16_t *ws_lo, int lrow,
                                        int lk) {
  u32x4 *dh = (u32x4 *)(ws_hi + lrow * LDS_PITCH + lk);
  u32x4 *dl = (u32x4 *)(ws_lo + lrow * LDS_PITCH + lk);
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // dword i holds k = 8i .. 8i+7
    const uint32_t d = r.w[i];
    const uint32_t lo4 = d & 0x0F0F0F0Fu, hi4 = (d >> 4) & 0x0F0F0F0Fu;
    float v[8];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      v[2 * b] = fmaf((float)((lo4 >> (8 * b)) & 0xFFu), r.s, -r.zs);      // k = 8i + 2b
      v[2 * b + 1] = fmaf((float)((hi4 >> (8 * b)) & 0xFFu), r.s, -r.zs);  // k = 8i + 2b + 1
    }
    u32x4 h4, l4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t hp, lp;
      split2(v[2 * j], v[2 * j + 1], hp, lp);
      h4[j] = hp;
      l4[j] = lp;
    }
    dh[i] = h4;
    dl[i] = l4;
  }
}

template <int XDT>
__global__ void __launch_bounds__(NTHREADS, 2)
k_q4_gemm(const uint8_t *__restrict__ wq, const f16 *__restrict__ st,
          const uint8_t *__restrict__ zt, const void *__restrict__ X, void *__restrict__ Y,
          int ydt, float *__restrict__ y32, const void *__restrict__ bias, int bdt,
          float *__restrict__ part, int M, int N, int K, int G, int g, int ksplit,
          int steps_per_split) {
  constexpr bool XSPLIT = XDT != SF_BF16;
  __shared__ __attribute__((aligned(16))) uint16_t xs_hi[BM * LDS_PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t xs_lo[XSPLIT ? BM * LDS_PITCH : 8];
  __shared__ __attribute__((aligned(16))) uint16_t ws_hi[BN * LDS_PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t ws_lo[BN * LDS_PITCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;  // wave tile origin in the block tile
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int split = blockIdx.z;
  const int nsteps_total = (K + BK - 1) / BK;
  const int s0 = split * steps_per_split;
  const int s1 = min(s0 + steps_per_split, nsteps_total);

  // staging assignment: row tid/2, 32-element half tid%2
  const int lrow = tid >> 1, lk = (tid & 1) * 32;

  float16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  XRegs<XDT> xr;
  WRegs wr;
  if (s0 < s1) {
    load_x<XDT>(xr, X, M, K, m0 + lrow, s0 * BK + lk);
    load_w(wr, wq, st, zt, N, K, G, g, n0 + lrow, s0 * BK + lk);
  }
  for (int step = s0; step < s1; ++step) {
    __syncthreads();
    store_x<XDT>(xr, xs_hi, xs_lo, lrow, lk);
    store_w(wr, ws_hi, ws_lo, lrow, lk);
    __syncthreads();
    if (step + 1 < s1) {
      load_x<XDT>(xr, X, M, K, m0 + lrow, (step + 1) * BK + lk);
      load_w(wr, wq, st, zt, N, K, G, g, n0 + lrow, (step + 1) * BK + lk);
    }
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      const int kofs = kk + (lane >> 5) * 8;
      bf16x8_t ah[2], al[2], bh[2], bl[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = wm + i * 32 + (lane & 31);
        ah[i] = *(const bf16x8_t *)(xs_hi + r * LDS_PITCH + kofs);
        if constexpr (XSPLIT) al[i] = *(const bf16x8_t *)(xs_lo + r * LDS_PITCH + kofs);
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int c = wn + j * 32 + (lane & 31);
        bh[j] = *(const bf16x8_t *)(ws_hi + c * LDS_PITCH + kofs);
        bl[j] = *(const bf16x8_t *)(ws_lo + c * LDS_PITCH + kofs);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);
          if constexpr (XSPLIT) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bl[j], acc[i][j], 0, 0, 0);
          }
        }
    }
  }

  // Output: acc[i][j][r] is C[row][col], row = 8*(r/4) + 4*(lane/32) + r%4,
  // col = lane % 32, within MFMA tile (i, j).
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn + j * 32 + (lane & 31);
      if (col >= N) continue;
      float bv = 0.f;
      if (bias && ksplit == 1) {
        if (bdt == SF_F32) bv = ((const float *)bias)[col];
        else if (bdt == SF_F16) bv = (float)((const f16 *)bias)[col];
        else bv = sf_bf16_to_f32(((const uint16_t *)bias)[col]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row >= M) continue;
        const size_t idx = (size_t)row * N + col;
        const float v = acc[i][j][r];
        if (ksplit > 1) {
          part[(size_t)split * M * N + idx] = v;
        } else {
          const float o = v + bv;
          if (y32) y32[idx] = o;
          if (Y) {
            if (ydt == SF_BF16) ((uint16_t *)Y)[idx] = sf_f32_to_bf16(o);
            else if (ydt == SF_F16) ((f16 *)Y)[idx] = (f16)o;
            else ((float *)Y)[idx] = o;
          }
        }
      }
    }
}

__global__ void __launch_bounds__(256)
k_splitk_reduce(const float *__restrict__ part, void *__restrict__ Y, int ydt, float *__restrict__ y32,
                const void *__restrict__ bias, int bdt, int M, int N, int ksplit) {
  const size_t MN = (size_t)M * N;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < MN;
       idx += (size_t)gridDim.x * blockDim.x) {
    float v = 0.f;
    for (int s = 0; s < ksplit; ++s) v += part[(size_t)s * MN + idx];
    if (bias) {
      const int col = (int)(idx % N);
      if (bdt == SF_F32) v += ((const float *)bias)[col];
      else if (bdt == SF_F16) v += (float)((const f16 *)bias)[col];
      else v += sf_bf16_to_f32(((const uint16_t *)bias)[col]);
    }
    if (y32) y32[idx] = v;
    if (Y) {
      if (ydt == SF_BF16) ((uint16_t *)Y)[idx] = sf_f32_to_bf16(v);
      else if (ydt == SF_F16) ((f16 *)Y)[idx] = (f16)v;
      else ((float *)Y)[idx] = v;
    }
  }
}

// K split count: enough (tile, split) workgroups to give every CU one, each
// split keeping at least 4 K steps.
int choose_ksplit(int M, int N, int K) {
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  const int steps = (K + BK - 1) / BK;
  int s = 1;
  while (tiles * s * 2 <= 256 && steps / (s * 2) >= 4 && s < 8) s *= 2;
  return s;
}

}  // namespace

extern "C" size_t sf_q4_gemm_workspace_bytes(int M, int N, int K, int group_size) {
  (void)group_size;
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int s = choose_ksplit(M, N, K);
  return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

extern "C" int sf_q4_gemm(const void *blob, const void *x, int x_dtype, void *y, int y_dtype,
                          float *y_f32, const void *bias, int bias_dtype, int M, int N, int K,
                          int group_size, int has_zeros, void *workspace, size_t workspace_bytes,
                          void *stream) {
  SF_REQUIRE(M > 0 && N > 0 && K > 0 && group_size > 0, SF_EINVAL,
             "invalid shape M=%d N=%d K=%d group_size=%d", M, N, K, group_size);
  SF_REQUIRE(K % group_size == 0, SF_EINVAL, "in_features must be divisible by group_size");
  SF_REQUIRE(group_size % 32 == 0, SF_EUNSUPPORTED,
             "group_size=%d: this build's kernels need a multiple of 32", group_size);
  SF_REQUIRE(blob && x && (y || y_f32), SF_EINVAL, "null pointer argument");
  SF_REQUIRE(x_dtype == SF_F16 || x_dtype == SF_BF16 || x_dtype == SF_F32, SF_EINVAL,
             "bad activation dtype %d", x_dtype);
  SF_REQUIRE(y_dtype == SF_F16 || y_dtype == SF_BF16 || y_dtype == SF_F32, SF_EINVAL,
             "bad output dtype %d", y_dtype);
  SF_REQUIRE(!bias || bias_dtype == SF_F16 || bias_dtype == SF_BF16 || bias_dtype == SF_F32,
             SF_EINVAL, "bad bias dtype %d", bias_dtype);
  SF_REQUIRE(((uintptr_t)blob & 255) == 0 && ((uintptr_t)x & 15) == 0, SF_EINVAL,
             "blob must be 256-byte aligned and X 16-byte aligned");
  BlobLayout L;
  sf_blob_layout(N, K, group_size, has_zeros, &L);
  const int ksplit = choose_ksplit(M, N, K);
  if (ksplit > 1) {
    const size_t need = (size_t)ksplit * M * N * sizeof(float);
    SF_REQUIRE(workspace && workspace_bytes >= need, SF_EINVAL,
               "GEMM workspace too small: %zu < %zu", workspace_bytes, need);
  }
  const int nsteps = (K + BK - 1) / BK;
  const int steps_per_split = (nsteps + ksplit - 1) / ksplit;
  const uint8_t *w = (const uint8_t *)blob;
  const f16 *st = (const f16 *)(w + L.s_off);
  const uint8_t *zt = has_zeros ? w + L.z_off : nullptr;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM, ksplit);
  float *part = (float *)workspace;
#define SF_GEMM_LAUNCH(XD)                                                                       \
  k_q4_gemm<XD><<<grid, NTHREADS, 0, s>>>(w, st, zt, x, y, y_dtype, y_f32, bias, bias_dtype, part, \
                                          M, N, K, L.G, group_size, ksplit, steps_per_split)
  if (x_dtype == SF_BF16) SF_GEMM_LAUNCH(SF_BF16);
  else if (x_dtype == SF_F16) SF_GEMM_LAUNCH(SF_F16);
  else SF_GEMM_LAUNCH(SF_F32);
#undef SF_GEMM_LAUNCH
  int rc = sf_check_launch("sf_q4_gemm");
  if (rc || ksplit == 1) return rc;
  const size_t MN = (size_t)M * N;
  unsigned rg = (unsigned)((MN + 255) / 256);
  if (rg > 65535u * 16u) rg = 65535u * 16u;
  k_splitk_reduce<<<rg, 256, 0, s>>>(part, y, y_dtype, y_f32, bias, bias_dtype, M, N, ksplit);
  return sf_check_launch("sf_q4_gemm(reduce)");
}
