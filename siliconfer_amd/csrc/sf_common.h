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
//   [0, N*K/2)          packed nibbles in the canonical row-major order
//                       (byte (n, j) holds k = 2j in bits 0-3 and k = 2j+1 in
//                       bits 4-7) but OFFSET-BINARY: code + 8 for symmetric
//                       weights (canonical byte ^ 0x88), the unsigned code for
//                       asymmetric weights. Both kinds then dequantize as
//                       (nibble - z) * s with z = 8 for symmetric.
//   [s_off, ...)        fp16 scales, tiled [ceil(N/8)][G][8]: the 8 rows of a
//                       row-octet are contiguous for each group, so a thread
//                       that owns 8 rows of one group loads them with one
//                       16-byte load. Pad rows hold 0.
//   [z_off, ...)        asymmetric only: zero-points, tiled [ceil(N/8)][G][4]
//                       bytes; byte j of a (octet, group) cell holds row 2j in
//                       bits 0-3 and row 2j+1 in bits 4-7.
// ---------------------------------------------------------------------------
struct BlobLayout {
  int N, K, g, G, NT;  // NT = row octets
  size_t w_bytes, s_off, s_bytes, z_off, z_bytes, total;
};

static inline bool sf_blob_layout(int N, int K, int g, int has_zeros, BlobLayout *L) {
  if (N <= 0 || K <= 0 || g <= 0 || (K % 2) || (K % g)) return false;
  L->N = N;
  L->K = K;
  L->g = g;
  L->G = K / g;
  L->NT = (N + 7) / 8;
  L->w_bytes = (size_t)N * (size_t)(K / 2);
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

// round-to-nearest-even float -> bf16 bits (NaN kept quiet)
__device__ __forceinline__ uint16_t sf_f32_to_bf16(float f) {
  uint32_t u = sf_bitcast<uint32_t>(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
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

__device__ __forceinline__ float sf_shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }
