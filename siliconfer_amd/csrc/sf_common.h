// sf_common.h — shared internals of libsiliconfer_hip.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/siliconfer_hip.h"

typedef _Float16 f16;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// errors (host)
// ---------------------------------------------------------------------------
int sf_fail(int code, const char *fmt, ...);  // records message, returns code
int sf_check_launch(const char *what);        // hipGetLastError -> SF_EHIP

#define SF_REQUIRE(cond, code, ...)          \
  do {                                       \
    if (!(cond)) return sf_fail(code, __VA_ARGS__); \
  } while (0)

static inline size_t sf_align256(size_t v) { return (v + 255) & ~(size_t)255; }

// ---------------------------------------------------------------------------
// int4 weight blob layout
//
//   [0, w_bytes)        the codes, OFFSET-BINARY (code + 8 for symmetric
//                       weights, the unsigned code for asymmetric ones; both
//                       kinds dequantize as (code - z) * s, z = 8 when
//                       symmetric), in 1 KB units of 16 rows x 128 k ordered
//                       [row tile][k unit] (NTI = ceil(N/16) tiles, NB =
//                       ceil(K/128) units per tile). Byte 16 l + 4 j + i of a
//                       unit belongs to row 16 tile + l % 16; its dword j holds
//                       the 8 codes of k = 128 unit + 32 j + 8 (l / 16) + e,
//                       code e at bits 4 (e / 2) + 16 (e % 2): even codes in
//                       the low half, odd ones in the high half, so one mask
//                       lifts the pair (e, e + 1) into the two 16-bit lanes.
//                       Rows past N and k past K hold code 8 (symmetric) / 0.
//                       A wave's 64 lanes loading 16 bytes each read one unit
//                       (1 KB contiguous) and hold the B operand of four
//                       16x16x32 MFMAs.
//   [s_off, ...)        fp16 scales, tiled [ceil(N/8)][G][8]: the 8 rows of a
//                       row-octet are contiguous for each group. Pad rows hold 0.
//   [z_off, ...)        asymmetric only: zero-points, tiled [ceil(N/8)][G][4]
//                       bytes; byte j of a (octet, group) cell holds row 2j in
//                       bits 0-3 and row 2j+1 in bits 4-7.
// ---------------------------------------------------------------------------
struct BlobLayout {
  int N, K, g, G, NT, NTI, NB;  // NT = row octets, NTI = 16-row tiles, NB = 128-k units
  size_t w_bytes, s_off, s_bytes, z_off, z_bytes, total;
};

static inline bool sf_blob_layout(int N, int K, int g, int has_zeros, BlobLayout *L) {
  if (N <= 0 || K <= 0 || g <= 0 || (K % 2) || (K % g)) return false;
  L->N = N;
  L->K = K;
  L->g = g;
  L->G = K / g;
  L->NT = (N + 7) / 8;
  L->NTI = (N + 15) / 16;
  L->NB = (K + 127) / 128;
  L->w_bytes = (size_t)L->NTI * L->NB * 1024;
  L->s_off = sf_align256(L->w_bytes);
  L->s_bytes = (size_t)L->NT * L->G * 8 * 2;
  L->z_off = sf_align256(L->s_off + L->s_bytes);
  L->z_bytes = has_zeros ? (size_t)L->NT * L->G * 4 : 0;
  L->total = has_zeros ? L->z_off + L->z_bytes : L->s_off + L->s_bytes;
  return true;
}

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
// Bit reinterpretation by value. Applied directly to an ext_vector element
// (`v.z`, `v[i]`), this compiler's __builtin_bit_cast reads element 0 instead;
// taking the argument by value first makes every use safe, so kernel code
// only uses sf_bitcast.
template <class To, class From>
__host__ __device__ __forceinline__ To sf_bitcast(From v) {
  static_assert(sizeof(To) == sizeof(From), "sf_bitcast size mismatch");
  return __builtin_bit_cast(To, v);
}

__device__ __forceinline__ float sf_bf16_to_f32(uint16_t b) {
  return sf_bitcast<float>((uint32_t)b << 16);
}

// fp32 -> bf16, round to nearest even (gfx950's v_cvt_pk_bf16_f32; NaN stays NaN)
__device__ __forceinline__ uint16_t sf_f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

template <int DT>
__device__ __forceinline__ float sf_load_as_f32(const void *p, size_t i) {
  if constexpr (DT == SF_F32) return ((const float *)p)[i];
  else if constexpr (DT == SF_F16) return (float)((const f16 *)p)[i];
  else return sf_bf16_to_f32(((const uint16_t *)p)[i]);
}

// 8 contiguous elements starting at element i (i a multiple of 8, p 16-byte
// aligned) with 16-byte loads
template <int DT>
__device__ __forceinline__ void sf_load8_as_f32(const void *p, size_t i, float (&f)[8]) {
  if constexpr (DT == SF_F32) {
    const float4_t a = ((const float4_t *)p)[i / 4], b = ((const float4_t *)p)[i / 4 + 1];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[j] = a[j];
      f[4 + j] = b[j];
    }
  } else {
    const u32x4 w = ((const u32x4 *)p)[i / 8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t x = w[j];
      if constexpr (DT == SF_F16) {
        f[2 * j] = (float)sf_bitcast<f16>((uint16_t)(x & 0xffffu));
        f[2 * j + 1] = (float)sf_bitcast<f16>((uint16_t)(x >> 16));
      } else {
        f[2 * j] = sf_bitcast<float>(x << 16);
        f[2 * j + 1] = sf_bitcast<float>(x & 0xffff0000u);
      }
    }
  }
}

template <int DT>
__device__ __forceinline__ void sf_store_from_f32(void *p, size_t i, float v) {
  if constexpr (DT == SF_F32) ((float *)p)[i] = v;
  else if constexpr (DT == SF_F16) ((f16 *)p)[i] = (f16)v;
  else ((uint16_t *)p)[i] = sf_f32_to_bf16(v);
}

// v as an fp32 value in a register. A product converted to fp16 right away
// can otherwise become one v_fma_mixlo_f16 (a single rounding instead of fp32
// then fp16), whatever the contraction setting; every kernel that rounds a
// product to an activation dtype goes through this, so the folded and unfolded
// decoder paths agree bit for bit.
__device__ __forceinline__ float sf_opaque(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// v rounded to DT and back: the value a DT buffer would hand the next kernel.
template <int DT>
__device__ __forceinline__ float sf_round_as(float v) {
  v = sf_opaque(v);
  if constexpr (DT == SF_F32) return v;
  else if constexpr (DT == SF_F16) return (float)(f16)v;
  else return sf_bf16_to_f32(sf_f32_to_bf16(v));
}

__device__ __forceinline__ float sf_shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

template <int CTRL>
__device__ __forceinline__ float sf_dpp(float v) {
  return sf_bitcast<float>(__builtin_amdgcn_update_dpp(0, sf_bitcast<int>(v), CTRL, 0xF, 0xF, false));
}

// A value and its partner 16 (32) lanes away, lane xor 16 (xor 32), with
// gfx950's row-swapping permutes: the pair comes back in some order, both
// register-only (a shuffle is an LDS round trip). max and + of the same two
// operands give the shuffle-based step's bits. All 64 lanes must be active.
__device__ __forceinline__ float2_t sf_swap16_pair(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(sf_bitcast<uint32_t>(v), sf_bitcast<uint32_t>(v), false, false);
  return float2_t{sf_bitcast<float>((uint32_t)r[0]), sf_bitcast<float>((uint32_t)r[1])};
}
__device__ __forceinline__ float2_t sf_swap32_pair(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(sf_bitcast<uint32_t>(v), sf_bitcast<uint32_t>(v), false, false);
  return float2_t{sf_bitcast<float>((uint32_t)r[0]), sf_bitcast<float>((uint32_t)r[1])};
}

// A pairwise tree across aligned groups of GS lanes (GS = 1, 2, 4, ..., 64;
// uniform): every lane of a group gets the group's tree sum, the levels those
// of sf_wave_sum (once a block of lanes holds one value, the mirrors pair it
// with the next block; each level adds a value and its partner, so both get
// the same bits). Branch-free: every level is computed, those at or past GS
// are dropped by a select. All 64 lanes must be active. sf_group_tree_max:
// the same groups' max.
__device__ __forceinline__ float sf_group_tree_max(float v, int GS) {
  float t = fmaxf(v, sf_dpp<0xB1>(v));
  v = GS > 1 ? t : v;
  t = fmaxf(v, sf_dpp<0x4E>(v));
  v = GS > 2 ? t : v;
  t = fmaxf(v, sf_dpp<0x141>(v));
  v = GS > 4 ? t : v;
  t = fmaxf(v, sf_dpp<0x140>(v));
  v = GS > 8 ? t : v;
  float2_t p = sf_swap16_pair(v);
  v = GS > 16 ? fmaxf(p.x, p.y) : v;
  p = sf_swap32_pair(v);
  return GS > 32 ? fmaxf(p.x, p.y) : v;
}
__device__ __forceinline__ float sf_group_tree_sum(float v, int GS) {
  float t = v + sf_dpp<0xB1>(v);  // quad_perm [1,0,3,2]
  v = GS > 1 ? t : v;
  t = v + sf_dpp<0x4E>(v);        // quad_perm [2,3,0,1]
  v = GS > 2 ? t : v;
  t = v + sf_dpp<0x141>(v);       // row_half_mirror
  v = GS > 4 ? t : v;
  t = v + sf_dpp<0x140>(v);       // row_mirror
  v = GS > 8 ? t : v;
  float2_t p = sf_swap16_pair(v);
  v = GS > 16 ? p.x + p.y : v;
  p = sf_swap32_pair(v);
  return GS > 32 ? p.x + p.y : v;
}

// Sum over the 64 lanes of a wave; every lane gets the same bits (each step
// adds a value and its butterfly partner, and fp addition commutes).
__device__ __forceinline__ float sf_wave_sum(float v) {
  v += sf_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += sf_dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += sf_dpp<0x141>(v);  // row_half_mirror
  v += sf_dpp<0x140>(v);  // row_mirror
  float2_t p = sf_swap16_pair(v);
  v = p.x + p.y;
  p = sf_swap32_pair(v);
  return p.x + p.y;
}

// 1 / sqrt(mean((x + delta)^2) + eps) over one row of H fp32 values, computed
// by one whole wave in a fixed order. Every kernel that normalises a row uses
// this, so the RMSNorm kernel and the projections that fold the norm into
// their activation load produce the same bits. All 64 lanes must be active.
// With H % 4 == 0 and 16-byte aligned rows (VEC), lane l takes the float4s
// l + 64 u (u = 0..7) of each pass of 512, all of a pass's loads before its
// fmas (clamped indices, out-of-range values zeroed by a select); otherwise a
// scalar loop. Then sf_wave_sum. issue() loads u = 0..3 of the first pass
// early (a caller can put them ahead of its other loads); finish() continues
// the same fma chain.
struct SfRowNorm {
  float4_t v[4];
  bool vec;

  template <bool ASSUME_VEC = false>
  __device__ __forceinline__ void issue(const float *__restrict__ x, const float *__restrict__ delta,
                                        int H) {
    vec = ASSUME_VEC || ((H & 3) == 0 && ((uintptr_t)x & 15) == 0 &&
                         (!delta || ((uintptr_t)delta & 15) == 0));
    if (!vec) return;
    const int lane = threadIdx.x & 63, n4 = H >> 2;
    const float4_t *x4 = (const float4_t *)x, *d4 = (const float4_t *)delta;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(lane + 64 * u, n4 - 1);
      v[u] = x4[i];
      if (delta) v[u] += d4[i];
    }
  }

  __device__ __forceinline__ float finish(const float *__restrict__ x,
                                          const float *__restrict__ delta, int H, float eps) {
    const int lane = threadIdx.x & 63;
    float ss = 0.f;
    if (vec) {
      const int n4 = H >> 2;
      const float4_t *x4 = (const float4_t *)x, *d4 = (const float4_t *)delta;
      auto acc = [&](const float4_t &t0, bool in) {
        const float4_t t = in ? t0 : float4_t{0.f, 0.f, 0.f, 0.f};
        ss = fmaf(t.x, t.x, ss);
        ss = fmaf(t.y, t.y, ss);
        ss = fmaf(t.z, t.z, ss);
        ss = fmaf(t.w, t.w, ss);
      };
#pragma unroll
      for (int u = 0; u < 4; ++u) acc(v[u], lane + 64 * u < n4);
      // the rest in batches of 4 float4 per lane, in the same order as one
      // batch of 8 (so the sum is the same bits; fewer registers held)
      for (int base = 0; base < n4; base += 512) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (base == 0 && h == 0) continue;  // the first pass's u < 4 came from issue()
          if (base + 256 * h >= n4) break;    // nothing left in range (adds only zeros)
          float4_t w[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int i = min(base + 256 * h + lane + 64 * u, n4 - 1);
            w[u] = x4[i];
            if (delta) w[u] += d4[i];
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) acc(w[u], base + 256 * h + lane + 64 * u < n4);
        }
      }
    } else {
      for (int h = lane; h < H; h += 64) {
        float t = x[h];
        if (delta) t += delta[h];
        ss = fmaf(t, t, ss);
      }
    }
    ss = sf_wave_sum(ss);
    return 1.f / sqrtf(ss / (float)H + eps);
  }
};

__device__ __forceinline__ float sf_row_inv_rms(const float *__restrict__ x,
                                                const float *__restrict__ delta, int H, float eps) {
  SfRowNorm n;
  n.issue(x, delta, H);
  return n.finish(x, delta, H, eps);
}

// RoPE + KV-cache append of one head of one row of the fused q|k|v projection
// (rotate-half RoPE, /root/reference/siliconfer/model/layers.py:58-66, then
// quantize_kv of kv_cache.py:49-63 into the cache), done by one whole wave:
// x holds the head's D fp32 values (bias included), pos its position. q heads
// go rotated to q_out row `row`; k heads rotated, v heads as they are, are
// quantized per (head, token) — s = max|x| / 127 (1 if 0), code =
// clip(rint(x / s)) — into the cache at pos (batch 1). Lane l owns the pairs
// (d, d + D/2) for d = l, l + 64 (D <= 256). Shared by the RoPE/append kernel
// and the qkv projection that folds it into its epilogue, so both store the
// same bits.
struct SfRopeAppend {
  const float *cos_t, *sin_t;
  int max_pos;
  void *q_out;
  int q_dtype;
  int8_t *k_codes;
  void *k_scales;
  int8_t *v_codes;
  void *v_scales;
  int scale_dtype, H, KVH, D, T_cap;
};

// Max over the 64 lanes of a wave (every lane gets it): the within-row steps
// as DPP moves, the cross-row ones as permlane swaps. All lanes active.
__device__ __forceinline__ float sf_wave_max(float v) {
  v = fmaxf(v, sf_dpp<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, sf_dpp<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, sf_dpp<0x141>(v));  // row_half_mirror
  v = fmaxf(v, sf_dpp<0x140>(v));  // row_mirror
  float2_t p = sf_swap16_pair(v);
  v = fmaxf(p.x, p.y);
  p = sf_swap32_pair(v);
  return fmaxf(p.x, p.y);
}

__device__ __forceinline__ void sf_store_dt(void *p, int dt, size_t i, float v) {
  if (dt == SF_F32) ((float *)p)[i] = v;
  else if (dt == SF_F16) ((f16 *)p)[i] = (f16)v;
  else ((uint16_t *)p)[i] = sf_f32_to_bf16(v);
}

// The cos / sin table entries of the lane's dims at `pos` (lane + 64 j < D / 2),
// for a caller that issues them ahead of the rotation.
struct SfRopeCS {
  static constexpr int MAXP = 2;  // D <= 256
  float c[MAXP], s[MAXP];
};

__device__ __forceinline__ SfRopeCS sf_rope_load_cs(const SfRopeAppend &a, int pos) {
  const int lane = threadIdx.x & 63, half = a.D >> 1;
  SfRopeCS r;
#pragma unroll
  for (int j = 0; j < SfRopeCS::MAXP; ++j) {
    const int d = lane + 64 * j;
    r.c[j] = r.s[j] = 0.f;
    if (d < half) {
      r.c[j] = a.cos_t[(size_t)pos * half + d];
      r.s[j] = a.sin_t[(size_t)pos * half + d];
    }
  }
  return r;
}

// One head's rotate-half RoPE at `pos` (q and k heads; v passes through) from
// its D fp32 values x, then q to q_out row `row`, or k / v quantized into the
// cache row `pos` (abs-max / 127 per vector, round half to even, clip).
__device__ __forceinline__ void sf_rope_append_head(const SfRopeAppend &a, const float *x, int head,
                                                    int pos, int row, const SfRopeCS &cs) {
  const int lane = threadIdx.x & 63;
  const int D = a.D, half = D >> 1;
  const bool is_q = head < a.H, is_k = !is_q && head < a.H + a.KVH;
  constexpr int MAXP = SfRopeCS::MAXP;
  float lo[MAXP], hi[MAXP];
#pragma unroll
  for (int j = 0; j < MAXP; ++j) {
    const int d = lane + 64 * j;
    lo[j] = hi[j] = 0.f;
    if (d < half) {
      const float u = x[d], w = x[d + half];
      if (is_q || is_k) {
        // separately rounded products, as x * cos + rotate(x) * sin in fp32
#pragma clang fp contract(off)
        const float c = cs.c[j], s = cs.s[j];
        lo[j] = u * c - w * s;
        hi[j] = w * c + u * s;
      } else {
        lo[j] = u;
        hi[j] = w;
      }
    }
  }
  if (is_q) {
#pragma unroll
    for (int j = 0; j < MAXP; ++j) {
      const int d = lane + 64 * j;
      if (d < half) {
        const size_t o = ((size_t)row * a.H + head) * D + d;
        sf_store_dt(a.q_out, a.q_dtype, o, lo[j]);
        sf_store_dt(a.q_out, a.q_dtype, o + half, hi[j]);
      }
    }
    return;
  }
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < MAXP; ++j) amax = fmaxf(amax, fmaxf(fabsf(lo[j]), fabsf(hi[j])));
  amax = sf_wave_max(amax);
  const float s = amax == 0.f ? 1.f : amax / 127.f;
  const int kvh = is_k ? head - a.H : head - a.H - a.KVH;
  const size_t crow = (size_t)kvh * a.T_cap + pos;
  int8_t *codes = (is_k ? a.k_codes : a.v_codes) + crow * D;
#pragma unroll
  for (int j = 0; j < MAXP; ++j) {
    const int d = lane + 64 * j;
    if (d < half) {
      codes[d] = (int8_t)(int)fminf(fmaxf(__builtin_rintf(lo[j] / s), -128.f), 127.f);
      codes[d + half] = (int8_t)(int)fminf(fmaxf(__builtin_rintf(hi[j] / s), -128.f), 127.f);
    }
  }
  if (lane == 0) sf_store_dt(is_k ? a.k_scales : a.v_scales, a.scale_dtype, crow, s);
}

__device__ __forceinline__ void sf_rope_append_head(const SfRopeAppend &a, const float *x, int head,
                                                    int pos, int row) {
  sf_rope_append_head(a, x, head, pos, row, sf_rope_load_cs(a, pos));
}

// silu(g) * u as the decoder computes it (one formula for every kernel):
// g * (1 / (1 + exp(-g))) * u with the hardware reciprocal (1 ulp) instead of
// an IEEE division, which takes about ten instructions.
__device__ __forceinline__ float sf_silu_mul(float g, float u) {
  return sf_opaque(g * __builtin_amdgcn_rcpf(1.f + expf(-g)) * u);
}
