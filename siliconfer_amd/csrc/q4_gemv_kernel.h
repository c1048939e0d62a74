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
#include <stdlib.h>

#include "sf_common.h"

namespace sf_gemv {

// Scales of R consecutive rows (row0 % R == 0) of one group from the tiled
// [octet][group][8] fp16 array; cell points at the (row0 / 8, group) octet.
template <int R>
__device__ __forceinline__ void load_scales(const f16 *cell, size_t octet_stride, int row0, int N,
                                            float (&s)[R]) {
  if constexpr (R >= 8) {
#pragma unroll
    for (int o = 0; o < R / 8; ++o) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (row0 + 8 * o < N) v = *(const u32x4 *)(cell + (size_t)o * octet_stride);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half2_t h = sf_bitcast<half2_t>(v[i]);
        s[8 * o + 2 * i] = (float)h.x;
        s[8 * o + 2 * i + 1] = (float)h.y;
      }
    }
  } else if constexpr (R == 4) {
    u32x2 v = {0u, 0u};
    if (row0 < N) v = *(const u32x2 *)(cell + (row0 & 7));
    const half2_t a = sf_bitcast<half2_t>(v.x), b = sf_bitcast<half2_t>(v.y);
    s[0] = (float)a.x; s[1] = (float)a.y; s[2] = (float)b.x; s[3] = (float)b.y;
  } else {
    uint32_t v = 0u;
    if (row0 < N) v = *(const uint32_t *)(cell + (row0 & 7));
    const half2_t a = sf_bitcast<half2_t>(v);
    s[0] = (float)a.x; s[1] = (float)a.y;
  }
}

// Zero-point nibbles of R consecutive rows of one group (row r at bits 4r).
template <int R>
__device__ __forceinline__ uint64_t load_zeros(const uint8_t *cell, size_t octet_stride, int row0, int N) {
  if (row0 >= N) return 0u;
  if constexpr (R == 16) {
    const uint64_t lo = *(const uint32_t *)cell;
    const uint64_t hi = row0 + 8 < N ? *(const uint32_t *)(cell + octet_stride) : 0u;
    return lo | (hi << 32);
  } else if constexpr (R == 8) {
    return *(const uint32_t *)cell;
  } else if constexpr (R == 4) {
    return *(const uint16_t *)(cell + ((row0 & 7) >> 1));
  } else {
    return *(const uint8_t *)(cell + ((row0 & 7) >> 1));
  }
}

// (a & m) | c in one instruction (the compiler splits it in two when both
// constants would need literal operands).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(c));
  return r;
}

// Value of the butterfly partner at lane distance OFF. OFF <= 8 uses DPP
// (quad permutes and the 8-/16-lane mirrors: the partner always has the
// opposite bit OFF and the same higher bits, which is all a butterfly step
// needs); larger distances go through ds_bpermute.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return sf_bitcast<float>(__builtin_amdgcn_update_dpp(0, sf_bitcast<int>(v), CTRL, 0xF, 0xF, false));
}

template <int OFF>
__device__ __forceinline__ float partner(float v) {
  if constexpr (OFF == 1) return dpp_f<0xB1>(v);        // quad_perm [1,0,3,2]
  else if constexpr (OFF == 2) return dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  else if constexpr (OFF == 4) return dpp_f<0x141>(v);  // row_half_mirror: i <-> 7-i
  else if constexpr (OFF == 8) return dpp_f<0x140>(v);  // row_mirror: i <-> 15-i
  else return __shfl_xor(v, OFF, 64);
}

// Butterfly reduce-scatter of v[b][0..R) across a Q-lane group, starting at
// lane distance OFF = Q/2 with RC values per lane. Each step at distance OFF
// keeps the half of the values selected by the lane's own bit OFF and adds the
// partner's same half; once one value is left the remaining steps are plain
// sums. Afterwards lane p holds, in v[b][0..R>>S), the group sums of rows
// (p >> (log2 Q - S)) * (R >> S) + j, S = min(log2 R, log2 Q).
template <int B, int R, int OFF, int RC>
__device__ __forceinline__ void butterfly(float (&v)[B][R], int p) {
  if constexpr (OFF >= 1) {
    if constexpr (RC > 1) {
      constexpr int H = RC / 2;
      const bool up = (p & OFF) != 0;
#pragma unroll
      for (int b = 0; b < B; ++b)
#pragma unroll
        for (int j = 0; j < H; ++j) {
          const float lo = v[b][j], hi = v[b][j + H];
          const float send = up ? lo : hi;
          const float keep = up ? hi : lo;
          v[b][j] = keep + partner<OFF>(send);
        }
      butterfly<B, R, OFF / 2, H>(v, p);
    } else {
#pragma unroll
      for (int b = 0; b < B; ++b) v[b][0] += partner<OFF>(v[b][0]);
      butterfly<B, R, OFF / 2, 1>(v, p);
    }
  }
}

template <int V>
constexpr int clog2() { return V <= 1 ? 0 : 1 + clog2<V / 2>(); }

// bias: [N] added to every batch row, or y32 itself (fp32): each output then
// adds its own previous value (a residual add, per batch row)
__device__ __forceinline__ void store_out(void *y, int ydt, float *y32, const void *bias, int bdt,
                                          size_t idx, int row, float v) {
  if (bias) {
    if (bias == y32) v += y32[idx];
    else if (bdt == SF_F32) v += ((const float *)bias)[row];
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
  __device__ __forceinline__ void build(const u32x4 (&xq)[4]) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const u32x4 v = xq[q4];
      const half2_t a = sf_bitcast<half2_t>(v.x), b = sf_bitcast<half2_t>(v.y);
      const half2_t c = sf_bitcast<half2_t>(v.z), d = sf_bitcast<half2_t>(v.w);
      p[4 * q4 + 0] = half2_t{a.x, c.x};
      p[4 * q4 + 1] = half2_t{a.y, c.y};
      p[4 * q4 + 2] = half2_t{b.x, d.x};
      p[4 * q4 + 3] = half2_t{b.y, d.y};
    }
  }
  __device__ __forceinline__ void load(const void *x, size_t off) {
    const u32x4 *xq = (const u32x4 *)((const f16 *)x + off);
    const u32x4 v[4] = {xq[0], xq[1], xq[2], xq[3]};
    build(v);
  }
  // from fp32 values, rounded as an fp16 activation buffer would hold them
  __device__ __forceinline__ void from_f32(const float (&f)[32]) {
    u32x4 v[4];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      v[i / 4][i % 4] = sf_bitcast<uint32_t>(half2_t{(f16)f[2 * i], (f16)f[2 * i + 1]});
    build(v);
  }
};

__device__ __forceinline__ uint32_t pair_lo_lo(uint32_t a, uint32_t b) { return (a & 0xFFFFu) | (b << 16); }
__device__ __forceinline__ uint32_t pair_hi_hi(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xFFFF0000u); }

template <>
struct Act<SF_BF16> {
  bf16x2_t p[16];
  float sum;  // sum of the 32 activations (exact bf16 values, fp32 adds)
  __device__ __forceinline__ void build(const u32x4 (&xq)[4]) {
    sum = 0.f;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const u32x4 v = xq[q4];
      p[4 * q4 + 0] = sf_bitcast<bf16x2_t>(pair_lo_lo(v.x, v.z));
      p[4 * q4 + 1] = sf_bitcast<bf16x2_t>(pair_hi_hi(v.x, v.z));
      p[4 * q4 + 2] = sf_bitcast<bf16x2_t>(pair_lo_lo(v.y, v.w));
      p[4 * q4 + 3] = sf_bitcast<bf16x2_t>(pair_hi_hi(v.y, v.w));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sum += sf_bitcast<float>(v[i] << 16) + sf_bitcast<float>(v[i] & 0xFFFF0000u);
    }
  }
  __device__ __forceinline__ void load(const void *x, size_t off) {
    const u32x4 *xq = (const u32x4 *)((const uint16_t *)x + off);
    const u32x4 v[4] = {xq[0], xq[1], xq[2], xq[3]};
    build(v);
  }
  __device__ __forceinline__ void from_f32(const float (&f)[32]) {
    u32x4 v[4];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      v[i / 4][i % 4] = (uint32_t)sf_f32_to_bf16(f[2 * i]) | ((uint32_t)sf_f32_to_bf16(f[2 * i + 1]) << 16);
    build(v);
  }
};

template <>
struct Act<SF_F32> {
  bf16x2_t hi[16], lo[16];
  float sum;  // sum of (hi + lo) over the 32 activations
  __device__ __forceinline__ void from_f32(const float (&f)[32]) {
    sum = 0.f;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      uint16_t h[8], l[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = f[8 * q4 + i];
        h[i] = sf_f32_to_bf16(v);
        const float hf = sf_bf16_to_f32(h[i]);
        l[i] = sf_f32_to_bf16(v - hf);
        sum += hf + sf_bf16_to_f32(l[i]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hi[4 * q4 + j] = sf_bitcast<bf16x2_t>((uint32_t)h[j] | ((uint32_t)h[j + 4] << 16));
        lo[4 * q4 + j] = sf_bitcast<bf16x2_t>((uint32_t)l[j] | ((uint32_t)l[j + 4] << 16));
      }
    }
  }
  __device__ __forceinline__ void load(const void *x, size_t off) {
    const float4_t *xq = (const float4_t *)((const float *)x + off);
    float f[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4_t v = xq[i];
      f[4 * i] = v.x; f[4 * i + 1] = v.y; f[4 * i + 2] = v.z; f[4 * i + 3] = v.w;
    }
    from_f32(f);
  }
};

// Dot product of one 16-byte weight chunk (offset-binary nibbles, zero z) with
// the lane's 32 activations, without the group scale.
template <int XDT>
__device__ __forceinline__ float chunk_dot(const u32x4 &wq, uint32_t z, const Act<XDT> &a) {
  if constexpr (XDT == SF_F16) {
    const half2_t c1 = sf_bitcast<half2_t>((0xE400u | z) * 0x10001u);        // -(1024+z)
    const half2_t c2 = sf_bitcast<half2_t>((0xD400u + 16u * z) * 0x10001u);  // -(64+z)
    const half2_t sixteenth = {(f16)0.0625f, (f16)0.0625f};
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t d = wq[j], d8 = d >> 8;
      const half2_t v0 = sf_bitcast<half2_t>(and_or(d, 0x000F000Fu, 0x64006400u)) + c1;
      const half2_t v1 = sf_bitcast<half2_t>(and_or(d, 0x00F000F0u, 0x64006400u)) * sixteenth + c2;
      const half2_t v2 = sf_bitcast<half2_t>(and_or(d8, 0x000F000Fu, 0x64006400u)) + c1;
      const half2_t v3 = sf_bitcast<half2_t>(and_or(d8, 0x00F000F0u, 0x64006400u)) * sixteenth + c2;
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
        const bf16x2_t v = sf_bitcast<bf16x2_t>(and_or(d >> (4 * i), 0x000F000Fu, 0x43004300u));
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

// PRE (batch 1 only) folds the producer of x into the activation load: x is
// then the fp32 source row and each lane builds its 32 activations itself,
// rounded to XDT exactly as sf_rmsnorm / sf_silu_mul would store them
// (PRE_RMSNORM: src * inv_rms(src) * pre_w, the norm from sf_row_inv_rms;
// PRE_SILU: silu(src[k]) * src[K + k]). Every lane then issues its loads at
// clamped positions, so the norm's wave reduction runs with all lanes active.
constexpr int PRE_NONE = 0, PRE_RMSNORM = 1, PRE_SILU = 2;

// ROPE (batch 1): the workgroup's R * RS output rows are one head of the fused q|k|v projection, and instead
// of storing them it applies RoPE and the KV-cache append to them
// (sf_rope_append_head) at the device position *pos_dev.
template <int B, int R, int Q, bool ASYM, int XDT, int PRE = PRE_NONE, bool ROPE = false>
__global__ void __launch_bounds__(512)
k_q4_gemv(const uint8_t *__restrict__ w, const f16 *__restrict__ stile,
          const uint8_t *__restrict__ ztile, const void *__restrict__ x, void *__restrict__ y,
          int ydt, float *__restrict__ y32, const void *__restrict__ bias, int bdt, int N, int K,
          int G, int cpg_shift, int C, int P, int RS, const float *__restrict__ pre_w, float eps,
          SfRopeAppend rope, const int *__restrict__ pos_dev) {
  static_assert(PRE == PRE_NONE || B == 1, "folded producers are batch-1 only");
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

  if constexpr (PRE != PRE_NONE) {
    const bool valid = c < C && row0 < N;
    const int cc = min(c, C - 1);
    const int grp = cc >> cpg_shift;
    const size_t cell = (size_t)(min(row0, N - 1) >> 3) * G + grp;
    float sc[R];
    load_scales<R>(stile + cell * 8, (size_t)G * 8, row0, N, sc);
    uint64_t zn = 0x8888888888888888ull;
    if constexpr (ASYM) zn = load_zeros<R>(ztile + cell * 4, (size_t)G * 4, row0, N);
    const float *src = (const float *)x;
    // the norm's row loads first: its sum then needs none of the weights
    // (the host checks K % 32 == 0 and a 16-byte aligned row)
    SfRowNorm norm;
    if constexpr (PRE == PRE_RMSNORM) norm.issue<true>(src, nullptr, K);
    float f[32], g2[32];
    {
      // PRE_SILU: gate and up; PRE_RMSNORM: the row chunk and its norm weights
      const float4_t *a = (const float4_t *)(src + (size_t)cc * 32);
      const float4_t *b = PRE == PRE_SILU ? (const float4_t *)(src + K + (size_t)cc * 32)
                                          : (const float4_t *)(pre_w + (size_t)cc * 32);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float4_t u = a[i], v = b[i];
        f[4 * i] = u.x; f[4 * i + 1] = u.y; f[4 * i + 2] = u.z; f[4 * i + 3] = u.w;
        g2[4 * i] = v.x; g2[4 * i + 1] = v.y; g2[4 * i + 2] = v.z; g2[4 * i + 3] = v.w;
      }
    }
    u32x4 wv[R];
    const uint8_t *wp = w + (size_t)cc * 16;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, N - 1);
      wv[r] = __builtin_nontemporal_load((const u32x4 *)(wp + (size_t)row * Kh));
    }
    // the weight stream goes out before the activation math (the scheduler
    // would otherwise move the loads below it to save registers)
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PRE == PRE_RMSNORM) {
      const float inv = norm.finish(src, nullptr, K, eps);
#pragma unroll
      for (int i = 0; i < 32; ++i) f[i] = sf_opaque(f[i] * inv * g2[i]);  // as k_rmsnorm
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) f[i] = sf_silu_mul(f[i], g2[i]);
    }
    Act<XDT> xa;
    xa.from_f32(f);
    // no branch on `valid` (the compiler would sink the weight loads into it)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t z = (uint32_t)(zn >> (4 * r)) & 15u;
      const float d = chunk_dot<XDT>(wv[r], z, xa) * sc[r];
      acc[0][r] = valid ? d : 0.f;
    }
  } else if (c < C && row0 < N) {
    // small, cache-resident operands first, then the weight stream, so each
    // row's math can start as soon as its own 16 bytes arrive
    const int grp = c >> cpg_shift;
    const size_t cell = (size_t)(row0 >> 3) * G + grp;
    float sc[R];
    load_scales<R>(stile + cell * 8, (size_t)G * 8, row0, N, sc);
    uint64_t zn = 0x8888888888888888ull;  // offset-binary symmetric codes: z = 8
    if constexpr (ASYM) zn = load_zeros<R>(ztile + cell * 4, (size_t)G * 4, row0, N);
    Act<XDT> xa[B];
#pragma unroll
    for (int b = 0; b < B; ++b) xa[b].load(x, (size_t)b * K + (size_t)c * 32);

    // Rows past N re-read row N-1 (no branch splits the load batch); their
    // scales are the zero padding of the tiled scale array.
    u32x4 wv[R];
    const uint8_t *wp = w + (size_t)c * 16;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = min(row0 + r, N - 1);
      wv[r] = __builtin_nontemporal_load((const u32x4 *)(wp + (size_t)row * Kh));
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t z = (uint32_t)(zn >> (4 * r)) & 15u;
#pragma unroll
      for (int b = 0; b < B; ++b) acc[b][r] = chunk_dot<XDT>(wv[r], z, xa[b]) * sc[r];
    }
  }

  const int p = tid & (Q - 1);
  butterfly<B, R, Q / 2, R>(acc, p);

  constexpr int LQ = clog2<Q>();
  constexpr int LR = clog2<R>();
  constexpr int S = LR < LQ ? LR : LQ;
  constexpr int RF = R >> S;
  const int idx = p >> (LQ - S);
  const bool writer = (p & ((1 << (LQ - S)) - 1)) == 0;

  if constexpr (ROPE) {
    static_assert(B == 1 && Q <= 64, "the folded RoPE runs at batch 1, one wave per rowset");
    __shared__ float hv[256];  // the head: the workgroup's R * RS rows, bias added
    if (writer) {
#pragma unroll
      for (int j = 0; j < RF; ++j) {
        const int lr = rs * R + idx * RF + j;
        float v = acc[0][j];
        if (bias) {
          const int row = row0 + idx * RF + j;
          if (bdt == SF_F32) v += ((const float *)bias)[row];
          else if (bdt == SF_F16) v += (float)((const f16 *)bias)[row];
          else v += sf_bf16_to_f32(((const uint16_t *)bias)[row]);
        }
        hv[lr] = v;
      }
    }
    __syncthreads();
    if (tid < 64) {
      const int pos = *pos_dev;
      if (pos >= 0 && pos < rope.T_cap && pos < rope.max_pos)
        sf_rope_append_head(rope, hv, blockIdx.x, pos, 0);
    }
    return;
  }
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

// Rows per rowset. Defaults: 8 for batch <= 2, else 4 (register budget);
// SF_GEMV_R in the environment overrides it within the instantiated set.
inline int pick_rows(int B, int xdt) {
  int r = B <= 2 ? 8 : 4;
  if (const char *e = getenv("SF_GEMV_R")) {
    const int v = atoi(e);
    const bool ok = B <= 2 ? (v == 4 || v == 8 || (v == 16 && xdt != SF_F32)) : (v == 2 || v == 4);
    if (ok) r = v;
  }
  return r;
}

inline int plan_gemv(int B, int N, int K, int g, int xdt, GemvPlan *pl, int rows = 0) {
  pl->C = K / 32;
  pl->P = pl->C <= 32 ? 32 : ((pl->C + 63) / 64) * 64;
  SF_REQUIRE(pl->P <= 512, SF_EUNSUPPORTED, "in_features=%d exceeds this GEMV's limit of 16384", K);
  pl->Q = pl->P == 32 ? 32 : 64;
  // rowsets of P lanes fill a 256-thread group when P divides 256; otherwise
  // one rowset per group (no idle waves)
  pl->WG = 256 % pl->P == 0 ? 256 : pl->P;
  pl->RS = pl->WG / pl->P;
  pl->R = rows ? rows : pick_rows(B, xdt);
  const int rows_per_wg = pl->RS * pl->R;
  pl->grid = (N + rows_per_wg - 1) / rows_per_wg;
  pl->cpg_shift = ilog2(g / 32);
  return SF_OK;
}

template <int B, int R, int Q, bool A, int X, int PRE = PRE_NONE, bool ROPE = false>
void launch_t(const GemvPlan &pl, const uint8_t *w, const f16 *st, const uint8_t *zt, const void *x,
              void *y, int ydt, float *y32, const void *bias, int bdt, int N, int K, int G,
              hipStream_t s, const float *pre_w = nullptr, float eps = 0.f,
              const SfRopeAppend *rope = nullptr, const int *pos_dev = nullptr) {
  const SfRopeAppend ra = rope ? *rope : SfRopeAppend{};
  k_q4_gemv<B, R, Q, A, X, PRE, ROPE><<<pl.grid, pl.WG, 0, s>>>(
      w, st, zt, x, y, ydt, y32, bias, bdt, N, K, G, pl.cpg_shift, pl.C, pl.P, pl.RS, pre_w, eps, ra,
      pos_dev);
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

template <int B, int X>
void launch_b(const GemvPlan &pl, const GemvArgs &a) {
#define SF_GEMV_R(RR) \
  launch_bqx<B, RR, X>(pl, a.asym, a.w, a.st, a.zt, a.x, a.y, a.ydt, a.y32, a.bias, a.bdt, a.N, a.K, a.G, a.s)
  if constexpr (B <= 2) {
    if (pl.R == 4) SF_GEMV_R(4);
    else if (pl.R == 16 && X != SF_F32) { if constexpr (X != SF_F32) SF_GEMV_R(16); }
    else SF_GEMV_R(8);
  } else {
    if (pl.R == 2) SF_GEMV_R(2);
    else SF_GEMV_R(4);
  }
#undef SF_GEMV_R
}

template <int X>
void launch_x(const GemvPlan &pl, const GemvArgs &a) {
  if constexpr (X == SF_F32) {  // fp32 activations: at most 2 rows per launch (registers)
    if (a.B == 1) launch_b<1, X>(pl, a);
    else launch_b<2, X>(pl, a);
  } else {
    switch (a.B) {
      case 1: launch_b<1, X>(pl, a); break;
      case 2: launch_b<2, X>(pl, a); break;
      case 3: launch_b<3, X>(pl, a); break;
      case 4: launch_b<4, X>(pl, a); break;
      case 5: launch_b<5, X>(pl, a); break;
      case 6: launch_b<6, X>(pl, a); break;
      case 7: launch_b<7, X>(pl, a); break;
      default: launch_b<8, X>(pl, a); break;
    }
  }
}

// Batch-1 GEMV with a folded producer (PRE_RMSNORM / PRE_SILU); the plan has R = 8.
template <int X>
void launch_pre(const GemvPlan &pl, const GemvArgs &a, int pre, const float *pre_w, float eps) {
#define SF_PRE_T(Q, A, P)                                                                       \
  launch_t<1, 8, Q, A, X, P>(pl, a.w, a.st, a.zt, a.x, a.y, a.ydt, a.y32, a.bias, a.bdt, a.N, a.K, \
                             a.G, a.s, pre_w, eps)
#define SF_PRE_QA(P)                          \
  do {                                        \
    if (pl.Q == 64) {                         \
      if (a.asym) SF_PRE_T(64, true, P);      \
      else SF_PRE_T(64, false, P);            \
    } else {                                  \
      if (a.asym) SF_PRE_T(32, true, P);      \
      else SF_PRE_T(32, false, P);            \
    }                                         \
  } while (0)
  if (pre == PRE_RMSNORM) SF_PRE_QA(PRE_RMSNORM);
  else SF_PRE_QA(PRE_SILU);
#undef SF_PRE_QA
#undef SF_PRE_T
}

// The batch-1 qkv projection with the input RMSNorm folded in and RoPE + the
// KV-cache append folded into its epilogue; the plan has Q = 32 and R * RS
// rows = one head per workgroup (the host checks).
template <int X>
void launch_pre_rope(const GemvPlan &pl, const GemvArgs &a, const float *pre_w, float eps,
                     const SfRopeAppend &rope, const int *pos_dev) {
  if (a.asym)
    launch_t<1, 8, 32, true, X, PRE_RMSNORM, true>(pl, a.w, a.st, a.zt, a.x, nullptr, 0, nullptr,
                                                   a.bias, a.bdt, a.N, a.K, a.G, a.s, pre_w, eps,
                                                   &rope, pos_dev);
  else
    launch_t<1, 8, 32, false, X, PRE_RMSNORM, true>(pl, a.w, a.st, a.zt, a.x, nullptr, 0, nullptr,
                                                    a.bias, a.bdt, a.N, a.K, a.G, a.s, pre_w, eps,
                                                    &rope, pos_dev);
}

}  // namespace sf_gemv
