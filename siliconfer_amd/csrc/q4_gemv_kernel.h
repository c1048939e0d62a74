// q4_gemv_kernel.h — int4 decode GEMV for batch 1..8 on gfx950 (no MFMA).
//
// Computes y[b, n] = sum_g s[n,g] * sum_{k in g} (q[n,k] - z[n,g]) * x[b,k] with
// fp32 accumulation: the reference's q4_gemv_sym / q4_gemv_asym
// (/root/reference/siliconfer/kernels/neon/q4_gemv.cpp:37-238), which apply the
// scale once per group partial (:136, :234).
//
// Work mapping (HBM-bound; the design goal is every load instruction of a wave
// reading 1 KB of contiguous weight bytes, with the whole matrix in flight):
//  * A "chunk" is 16 bytes of a row = 32 consecutive K elements. C = K/32
//    chunks per row. A "rowset" is P >= C lanes (P = 32, or C rounded up to a
//    multiple of 64) that own chunk c = lane index for R consecutive rows.
//    Lane c of a rowset loads chunk c of each of its R rows with one 16-byte
//    nontemporal load per row; consecutive lanes read consecutive chunks, so
//    each wave instruction covers 1 KB (or a whole row when K < 2048).
//  * The 32 activations of chunk c (per batch row) are loaded once per lane,
//    reordered into the pairs the dequantized nibbles come out in, and reused
//    for all R rows.
//  * Dequant is exact: a nibble n is OR-ed into the mantissa of fp16 1024
//    (0x6400|n = 1024+n, or 1024+16n for the upper nibble of a byte pair, then
//    scaled by 1/16), and 1024+z (or 64+z) is subtracted with one packed fp16
//    op, giving the integer q - z exactly. Offset-binary storage makes the
//    symmetric case z = 8. v_dot2_f32_f16 then accumulates two products per
//    instruction in fp32. Each row's 32-element partial is multiplied by its
//    fp32-converted group scale.
//  * bf16 / fp32 activations use v_dot2_f32_bf16 instead: the nibble is OR-ed
//    into bf16 128 (0x4300|n = 128+n, exact), the dot product runs on 128+n,
//    and the offset is removed once per row with the lane's precomputed
//    sum(x): sum((128+n)x) - (128+z) sum(x) = sum((n-z)x). fp32 activations
//    are split into bf16 hi + lo parts (two dot2 chains, ~16 mantissa bits).
//  * The R row partials of the P lanes are summed by a butterfly
//    reduce-scatter inside the wave (each step halves the values a lane holds),
//    then across the rowset's waves through LDS when P > 64.
#pragma once
#include "sf_common.h"

namespace sf_gemv {

template <int R>
struct ScaleLoad;

template <>
struct ScaleLoad<4> {
  __device__ __forceinline__ static void load(const f16 *tile_base, int row0, int N, float (&s)[4]) {
    u32x2 v = {0u, 0u};
    if (row0 < N) v = *(const u32x2 *)(tile_base + (row0 & 7));
    half2_t a = __builtin_bit_cast(half2_t, v.x), b = __builtin_bit_cast(half2_t, v.y);
    s[0] = (float)a.x; s[1] = (float)a.y; s[2] = (float)b.x; s[3] = (float)b.y;
  }
};

template <>
struct ScaleLoad<8> {
  __device__ __forceinline__ static void load(const f16 *tile_base, int row0, int N, float (&s)[8]) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row0 < N) v = *(const u32x4 *)tile_base;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      half2_t h = __builtin_bit_cast(half2_t, v[i]);
      s[2 * i] = (float)h.x;
      s[2 * i + 1] = (float)h.y;
    }
  }
};

// Zero-points of R rows (R = 4 or 8) of one group as nibbles in a u32.
template <int R>
__device__ __forceinline__ uint32_t load_zeros(const uint8_t *cell, int row0, int N) {
  if (row0 >= N) return 0u;
  if constexpr (R == 8) return *(const uint32_t *)cell;
  else return (uint32_t)(*(const uint16_t *)(cell + ((row0 & 7) >> 1)));
}

// Butterfly reduce-scatter of v[b][0..R) across a Q-lane group (Q = 32 or 64).
// Afterwards lane p holds, in v[b][0..R>>S), the rowset sums of rows
// (p >> (LQ-S)) * (R>>S) + j, where S = min(log2 R, log2 Q).
template <int B, int R, int Q>
__device__ __forceinline__ void rowset_reduce(float (&v)[B][R], int p) {
  constexpr int LQ = Q == 64 ? 6 : 5;
  constexpr int LR = R == 8 ? 3 : 2;
  constexpr int S = LR < LQ ? LR : LQ;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int off = Q >> (s + 1);
    const bool up = (p & off) != 0;
    const int H = R >> (s + 1);
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
      for (int j = 0; j < H; ++j) {
        const float lo = v[b][j], hi = v[b][j + H];
        const float send = up ? lo : hi;
        const float keep = up ? hi : lo;
        v[b][j] = keep + sf_shfl_xor(send, off);
      }
  }
#pragma unroll
  for (int off = Q >> (S + 1); off >= 1; off >>= 1)
#pragma unroll
    for (int b = 0; b < B; ++b)
#pragma unroll
      for (int j = 0; j < (R >> S); ++j) v[b][j] += sf_shfl_xor(v[b][j], off);
}

__device__ __forceinline__ void store_out(void *y, int ydt, float *y32, const void *bias, int bdt,
                                          size_t idx, int row, float v) {
  if (bias) {
    if (bdt == SF_F32) v += ((const float *)bias)[row];
    else if (bdt == SF_F16) v += (float)((const f16 *)bias)[row];
    else v += sf_bf16_to_f32(((const uint16_t *)bias)[row]);
  }
  if (y32) y32[idx] = v;
  if (y) {
    if (ydt == SF_F16) ((f16 *)y)[idx] = (f16)v;
    else if (ydt == SF_BF16) ((uint16_t *)y)[idx] = sf_f32_to_bf16(v);
    else ((float *)y)[idx] = v;
  }
}

// Activations of chunk c for one batch row, regrouped into the pair order the
// dequantized nibbles come out in: pair j of dword q4 = (x[8q4+j], x[8q4+j+4]).
template <int XDT>
struct Act;

template <>
struct Act<SF_F16> {
  half2_t p[16];
  __device__ __forceinline__ void load(const void *x, size_t off) {
    const u32x4 *xq = (const u32x4 *)((const f16 *)x + off);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const u32x4 v = xq[q4];
      const half2_t a = __builtin_bit_cast(half2_t, v.x), b = __builtin_bit_cast(half2_t, v.y);
      const half2_t c = __builtin_bit_cast(half2_t, v.z), d = __builtin_bit_cast(half2_t, v.w);
      p[4 * q4 + 0] = half2_t{a.x, c.x};
      p[4 * q4 + 1] = half2_t{a.y, c.y};
      p[4 * q4 + 2] = half2_t{b.x, d.x};
      p[4 * q4 + 3] = half2_t{b.y, d.y};
    }
  }
};

__device__ __forceinline__ uint32_t pair_lo_lo(uint32_t a, uint32_t b) { return (a & 0xFFFFu) | (b << 16); }
__device__ __forceinline__ uint32_t pair_hi_hi(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xFFFF0000u); }

template <>
struct Act<SF_BF16> {
  bf16x2_t p[16];
  float sum;  // sum of the 32 activations (exact bf16 values, fp32 adds)
  __device__ __forceinline__ void load(const void *x, size_t off) {
    const u32x4 *xq = (const u32x4 *)((const uint16_t *)x + off);
    sum = 0.f;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const u32x4 v = xq[q4];
      p[4 * q4 + 0] = __builtin_bit_cast(bf16x2_t, pair_lo_lo(v.x, v.z));
      p[4 * q4 + 1] = __builtin_bit_cast(bf16x2_t, pair_hi_hi(v.x, v.z));
      p[4 * q4 + 2] = __builtin_bit_cast(bf16x2_t, pair_lo_lo(v.y, v.w));
      p[4 * q4 + 3] = __builtin_bit_cast(bf16x2_t, pair_hi_hi(v.y, v.w));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sum += __builtin_bit_cast(float, v[i] << 16) + __builtin_bit_cast(float, v[i] & 0xFFFF0000u);
    }
  }
};

template <>
struct Act<SF_F32> {
  bf16x2_t hi[16], lo[16];
  float sum;  // sum of (hi + lo) over the 32 activations
  __device__ __forceinline__ void load(const void *x, size_t off) {
    const float4_t *xq = (const float4_t *)((const float *)x + off);
    sum = 0.f;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const float4_t a = xq[2 * q4], b = xq[2 * q4 + 1];  // x[8q4 .. 8q4+8)
      float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      uint16_t h[8], l[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        h[i] = sf_f32_to_bf16(v[i]);
        const float hf = sf_bf16_to_f32(h[i]);
        l[i] = sf_f32_to_bf16(v[i] - hf);
        sum += hf + sf_bf16_to_f32(l[i]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hi[4 * q4 + j] = __builtin_bit_cast(bf16x2_t, (uint32_t)h[j] | ((uint32_t)h[j + 4] << 16));
        lo[4 * q4 + j] = __builtin_bit_cast(bf16x2_t, (uint32_t)l[j] | ((uint32_t)l[j + 4] << 16));
      }
    }
  }
};

// Dot product of one 16-byte weight chunk (offset-binary nibbles, zero z) with
// the lane's 32 activations, without the group scale.
template <int XDT>
__device__ __forceinline__ float chunk_dot(const u32x4 &wq, uint32_t z, const Act<XDT> &a) {
  if constexpr (XDT == SF_F16) {
    const half2_t c1 = __builtin_bit_cast(half2_t, (0xE400u | z) * 0x10001u);        // -(1024+z)
    const half2_t c2 = __builtin_bit_cast(half2_t, (0xD400u + 16u * z) * 0x10001u);  // -(64+z)
    const half2_t sixteenth = {(f16)0.0625f, (f16)0.0625f};
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t d = wq[j], d8 = d >> 8;
      const half2_t v0 = __builtin_bit_cast(half2_t, (d & 0x000F000Fu) | 0x64006400u) + c1;
      const half2_t v1 = __builtin_bit_cast(half2_t, (d & 0x00F000F0u) | 0x64006400u) * sixteenth + c2;
      const half2_t v2 = __builtin_bit_cast(half2_t, (d8 & 0x000F000Fu) | 0x64006400u) + c1;
      const half2_t v3 = __builtin_bit_cast(half2_t, (d8 & 0x00F000F0u) | 0x64006400u) * sixteenth + c2;
      t = __builtin_amdgcn_fdot2(v0, a.p[4 * j + 0], t, false);
      t = __builtin_amdgcn_fdot2(v1, a.p[4 * j + 1], t, false);
      t = __builtin_amdgcn_fdot2(v2, a.p[4 * j + 2], t, false);
      t = __builtin_amdgcn_fdot2(v3, a.p[4 * j + 3], t, false);
    }
    return t;
  } else {
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t d = wq[j];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bf16x2_t v = __builtin_bit_cast(bf16x2_t, ((d >> (4 * i)) & 0x000F000Fu) | 0x43004300u);
        if constexpr (XDT == SF_BF16) {
          t = __builtin_amdgcn_fdot2_f32_bf16(v, a.p[4 * j + i], t, false);
        } else {
          t = __builtin_amdgcn_fdot2_f32_bf16(v, a.hi[4 * j + i], t, false);
          t = __builtin_amdgcn_fdot2_f32_bf16(v, a.lo[4 * j + i], t, false);
        }
      }
    }
    return t - (float)(128u + z) * a.sum;
  }
}

template <int B, int R, int Q, bool ASYM, int XDT>
__global__ void __launch_bounds__(512)
k_q4_gemv(const uint8_t *__restrict__ w, const f16 *__restrict__ stile,
          const uint8_t *__restrict__ ztile, const void *__restrict__ x, void *__restrict__ y,
          int ydt, float *__restrict__ y32, const void *__restrict__ bias, int bdt, int N, int K,
          int G, int cpg_shift, int C, int P, int RS) {
  __shared__ float red[8][B * R];
  const int tid = threadIdx.x;
  const int rs = tid / P;
  const int c = tid - rs * P;
  const int row0 = (blockIdx.x * RS + rs) * R;
  const int Kh = K >> 1;

  float acc[B][R];
#pragma unroll
  for (int b = 0; b < B; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[b][r] = 0.f;

  if (c < C && row0 < N) {
    // weights first: every load of the lane in flight before any math
    u32x4 wv[R];
    const uint8_t *wp = w + (size_t)row0 * Kh + (size_t)c * 16;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (row0 + r < N) wv[r] = __builtin_nontemporal_load((const u32x4 *)(wp + (size_t)r * Kh));
      else wv[r] = u32x4{0u, 0u, 0u, 0u};
    }
    const int grp = c >> cpg_shift;
    const size_t cell = (size_t)(row0 >> 3) * G + grp;
    float sc[R];
    ScaleLoad<R>::load(stile + cell * 8, row0, N, sc);
    uint32_t zn = 0x88888888u;  // offset-binary symmetric codes: z = 8
    if constexpr (ASYM) zn = load_zeros<R>(ztile + cell * 4, row0, N);

    Act<XDT> xa[B];
#pragma unroll
    for (int b = 0; b < B; ++b) xa[b].load(x, (size_t)b * K + (size_t)c * 32);

#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t z = (zn >> (4 * r)) & 15u;
#pragma unroll
      for (int b = 0; b < B; ++b) acc[b][r] = chunk_dot<XDT>(wv[r], z, xa[b]) * sc[r];
    }
  }

  const int p = tid & (Q - 1);
  rowset_reduce<B, R, Q>(acc, p);

  constexpr int LQ = Q == 64 ? 6 : 5;
  constexpr int LR = R == 8 ? 3 : 2;
  constexpr int S = LR < LQ ? LR : LQ;
  constexpr int RF = R >> S;
  const int idx = p >> (LQ - S);
  const bool writer = (p & ((1 << (LQ - S)) - 1)) == 0;

  if (P <= 64) {
    if (writer) {
#pragma unroll
      for (int j = 0; j < RF; ++j) {
        const int row = row0 + idx * RF + j;
        if (row < N)
#pragma unroll
          for (int b = 0; b < B; ++b)
            store_out(y, ydt, y32, bias, bdt, (size_t)b * N + row, row, acc[b][j]);
      }
    }
    return;
  }
  // P > 64: one wave per 64 chunks; combine the rowset's waves through LDS.
  const int wave = tid >> 6;
  if (writer) {
#pragma unroll
    for (int j = 0; j < RF; ++j)
#pragma unroll
      for (int b = 0; b < B; ++b) red[wave][(idx * RF + j) * B + b] = acc[b][j];
  }
  __syncthreads();
  const int nwr = P >> 6;
  if (tid < RS * R * B) {
    const int rs2 = tid / (R * B);
    const int rem = tid - rs2 * (R * B);
    const int r = rem / B, b = rem - r * B;
    float s = 0.f;
    for (int wi = 0; wi < nwr; ++wi) s += red[rs2 * nwr + wi][rem];
    const int row = (blockIdx.x * RS + rs2) * R + r;
    if (row < N) store_out(y, ydt, y32, bias, bdt, (size_t)b * N + row, row, s);
  }
}

struct GemvPlan {
  int C, P, Q, WG, RS, R, grid, cpg_shift;
};

inline int ilog2(int v) {
  int l = 0;
  while ((1 << (l + 1)) <= v) ++l;
  return l;
}

inline int plan_gemv(int B, int N, int K, int g, GemvPlan *pl) {
  pl->C = K / 32;
  pl->P = pl->C <= 32 ? 32 : ((pl->C + 63) / 64) * 64;
  SF_REQUIRE(pl->P <= 512, SF_EUNSUPPORTED, "in_features=%d exceeds this GEMV's limit of 16384", K);
  pl->Q = pl->P == 32 ? 32 : 64;
  pl->WG = pl->P <= 256 ? 256 : pl->P;
  pl->RS = pl->WG / pl->P;
  pl->R = B <= 2 ? 8 : 4;
  const int rows_per_wg = pl->RS * pl->R;
  pl->grid = (N + rows_per_wg - 1) / rows_per_wg;
  pl->cpg_shift = ilog2(g / 32);
  return SF_OK;
}

template <int B, int R, int Q, bool A, int X>
void launch_t(const GemvPlan &pl, const uint8_t *w, const f16 *st, const uint8_t *zt, const void *x,
              void *y, int ydt, float *y32, const void *bias, int bdt, int N, int K, int G,
              hipStream_t s) {
  k_q4_gemv<B, R, Q, A, X><<<pl.grid, pl.WG, 0, s>>>(w, st, zt, x, y, ydt, y32, bias, bdt, N, K,
                                                     G, pl.cpg_shift, pl.C, pl.P, pl.RS);
}

template <int B, int R, int X>
void launch_bqx(const GemvPlan &pl, bool asym, const uint8_t *w, const f16 *st, const uint8_t *zt,
                const void *x, void *y, int ydt, float *y32, const void *bias, int bdt, int N,
                int K, int G, hipStream_t s) {
  if (pl.Q == 64) {
    if (asym) launch_t<B, R, 64, true, X>(pl, w, st, zt, x, y, ydt, y32, bias, bdt, N, K, G, s);
    else launch_t<B, R, 64, false, X>(pl, w, st, zt, x, y, ydt, y32, bias, bdt, N, K, G, s);
  } else {
    if (asym) launch_t<B, R, 32, true, X>(pl, w, st, zt, x, y, ydt, y32, bias, bdt, N, K, G, s);
    else launch_t<B, R, 32, false, X>(pl, w, st, zt, x, y, ydt, y32, bias, bdt, N, K, G, s);
  }
}

struct GemvArgs {
  const uint8_t *w; const f16 *st; const uint8_t *zt; const void *x; void *y; int ydt; float *y32;
  const void *bias; int bdt; int B, N, K, G; bool asym; hipStream_t s;
};

template <int X>
void launch_x(const GemvPlan &pl, const GemvArgs &a) {
#define SF_GEMV_CASE(BB, RR) \
  case BB: launch_bqx<BB, RR, X>(pl, a.asym, a.w, a.st, a.zt, a.x, a.y, a.ydt, a.y32, a.bias, a.bdt, a.N, a.K, a.G, a.s); break;
  if constexpr (X == SF_F32) {  // fp32 activations: at most 2 rows per launch (registers)
    switch (a.B) {
      SF_GEMV_CASE(1, 8)
      SF_GEMV_CASE(2, 8)
    }
    return;
  }
  switch (a.B) {
    SF_GEMV_CASE(1, 8)
    SF_GEMV_CASE(2, 8)
    SF_GEMV_CASE(3, 4)
    SF_GEMV_CASE(4, 4)
    SF_GEMV_CASE(5, 4)
    SF_GEMV_CASE(6, 4)
    SF_GEMV_CASE(7, 4)
    SF_GEMV_CASE(8, 4)
  }
#undef SF_GEMV_CASE
}

}  // namespace sf_gemv
