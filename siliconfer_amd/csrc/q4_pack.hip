// q4_pack.hip — canonical int4 weights <-> device blob (layout in sf_common.h).
//
// The canonical form is the reference's (siliconfer/kernels/neon/__init__.py:
// 42-81): nibble-packed rows, two's-complement (sym) or unsigned (asym) codes.
// The blob changes four things: codes become offset-binary so one dequant path
// serves both kinds; they are regrouped into 1 KB units of 16 rows x 128 k in
// the order a wave's MFMA operands take them (each GEMV load instruction reads
// one contiguous unit); scales are tiled by row octets; zero-points are packed
// 2 per byte.
#include "sf_common.h"

namespace {

// Eight canonical codes (code e at bits 4e) <-> the blob's pairing (code e at
// bits 4 (e / 2) + 16 (e % 2)).
__device__ __forceinline__ uint32_t pair_codes(uint32_t p) {
  auto pack = [](uint32_t v) {  // the low nibbles of v's four bytes -> 16 bits
    v = (v | (v >> 4)) & 0x00FF00FFu;
    return (v | (v >> 8)) & 0x0000FFFFu;
  };
  return pack(p & 0x0F0F0F0Fu) | (pack((p >> 4) & 0x0F0F0F0Fu) << 16);
}

__device__ __forceinline__ uint32_t unpair_codes(uint32_t v) {
  auto spread = [](uint32_t x) {  // 16 bits -> the low nibbles of four bytes
    x = (x | (x << 8)) & 0x00FF00FFu;
    return (x | (x << 4)) & 0x0F0F0F0Fu;
  };
  return spread(v & 0xFFFFu) | (spread(v >> 16) << 4);
}

// One thread per blob dword: unit u = o / 256, lane l = (o % 256) / 4, dword j = o % 4.
__global__ void k_repack_w(const uint8_t *__restrict__ in, uint32_t *__restrict__ out, int N, int K,
                           int NB, size_t ndw, uint32_t xor_mask) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < ndw; o += stride) {
    const size_t u = o >> 8;
    const int l = (int)((o >> 2) & 63), j = (int)(o & 3);
    const int tile = (int)(u / NB), blk = (int)(u % NB);
    const int row = 16 * tile + (l & 15), k0 = 128 * blk + 32 * j + 8 * (l >> 4);
    uint32_t v = 0u;  // pad: code 8 (symmetric) / 0 after the mask
    if (row < N && k0 < K) {
      const uint8_t *src = in + (size_t)row * (K / 2) + k0 / 2;
      if (K % 8 == 0) {
        v = *(const uint32_t *)src;
      } else {  // rows are not dword-aligned: whole bytes up to K
        for (int b = 0; b < 4 && k0 + 2 * b < K; ++b) v |= (uint32_t)src[b] << (8 * b);
      }
      v = pair_codes(v);
    }
    out[o] = v ^ xor_mask;
  }
}

// One thread per canonical dword (8 codes of one row).
__global__ void k_unpack_w(const uint32_t *__restrict__ blob, uint8_t *__restrict__ out, int N, int K,
                           int NB, uint32_t xor_mask) {
  const int per_row = (K + 7) / 8;  // dwords of 8 codes, the last one partial when K % 8
  const size_t total = (size_t)N * per_row;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += stride) {
    const int row = (int)(o / per_row), k0 = 8 * (int)(o % per_row);
    const int blk = k0 / 128, j = (k0 % 128) / 32, kg = (k0 % 32) / 8;
    const size_t u = (size_t)(row / 16) * NB + blk;
    const uint32_t v = unpair_codes(blob[u * 256 + (size_t)(kg * 16 + row % 16) * 4 + j] ^ xor_mask);
    uint8_t *dst = out + (size_t)row * (K / 2) + k0 / 2;
    if (K % 8 == 0) {
      *(uint32_t *)dst = v;
    } else {
      for (int b = 0; b < 4 && k0 + 2 * b < K; ++b) dst[b] = (uint8_t)(v >> (8 * b));
    }
  }
}

__global__ void k_repack_s(const f16 *__restrict__ s, f16 *__restrict__ out, int N, int G, int NT) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t total = (size_t)NT * G * 8;
  if (i >= total) return;
  int r = (int)(i & 7);
  size_t tg = i >> 3;
  int gi = (int)(tg % G);
  int t = (int)(tg / G);
  int row = t * 8 + r;
  out[i] = row < N ? s[(size_t)row * G + gi] : (f16)0.0f;
}

__global__ void k_repack_z(const uint8_t *__restrict__ z, uint8_t *__restrict__ out, int N, int G,
                           int NT) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t total = (size_t)NT * G * 4;
  if (i >= total) return;
  int j = (int)(i & 3);
  size_t tg = i >> 2;
  int gi = (int)(tg % G);
  int t = (int)(tg / G);
  int r0 = t * 8 + 2 * j;
  uint8_t lo = r0 < N ? (z[(size_t)r0 * G + gi] & 15) : 0;
  uint8_t hi = r0 + 1 < N ? (z[(size_t)(r0 + 1) * G + gi] & 15) : 0;
  out[i] = (uint8_t)(lo | (hi << 4));
}

__global__ void k_unpack_s(const f16 *__restrict__ tiled, f16 *__restrict__ s, int N, int G) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)N * G) return;
  int row = (int)(i / G), gi = (int)(i % G);
  s[i] = tiled[((size_t)(row >> 3) * G + gi) * 8 + (row & 7)];
}

__global__ void k_unpack_z(const uint8_t *__restrict__ tiled, uint8_t *__restrict__ z, int N, int G) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)N * G) return;
  int row = (int)(i / G), gi = (int)(i % G);
  uint8_t b = tiled[((size_t)(row >> 3) * G + gi) * 4 + ((row & 7) >> 1)];
  z[i] = (row & 1) ? (b >> 4) : (b & 15);
}

int check_shape(int N, int K, int g) {
  SF_REQUIRE(N > 0 && K > 0 && g > 0, SF_EINVAL, "invalid shape N=%d K=%d group_size=%d", N, K, g);
  SF_REQUIRE(K % 2 == 0, SF_EINVAL, "W must be 2-D [out, in/2]");
  SF_REQUIRE(K % g == 0, SF_EINVAL, "in_features must be divisible by group_size");
  return SF_OK;
}

unsigned grid_for(size_t n, unsigned block, unsigned cap = 65535u * 4u) {
  size_t b = (n + block - 1) / block;
  if (b == 0) b = 1;
  return (unsigned)(b > cap ? cap : b);
}

}  // namespace

extern "C" size_t sf_q4_blob_bytes(int N, int K, int group_size, int has_zeros) {
  BlobLayout L;
  if (!sf_blob_layout(N, K, group_size, has_zeros, &L)) return 0;
  return L.total;
}

extern "C" int sf_q4_repack(const uint8_t *packed, const void *scales_f16, const uint8_t *zeros_u8,
                            int N, int K, int group_size, void *blob, size_t blob_bytes,
                            void *stream) {
  int rc = check_shape(N, K, group_size);
  if (rc) return rc;
  SF_REQUIRE(packed && scales_f16 && blob, SF_EINVAL, "null pointer argument");
  SF_REQUIRE(((uintptr_t)packed & 15) == 0 && ((uintptr_t)blob & 255) == 0, SF_EINVAL,
             "packed must be 16-byte aligned and blob 256-byte aligned");
  BlobLayout L;
  sf_blob_layout(N, K, group_size, zeros_u8 != nullptr, &L);
  SF_REQUIRE(blob_bytes >= L.total, SF_EINVAL, "blob too small: %zu < %zu", blob_bytes, L.total);
  hipStream_t st = (hipStream_t)stream;
  uint8_t *b = (uint8_t *)blob;
  const size_t ndw = L.w_bytes / 4;
  const uint32_t mask = zeros_u8 ? 0u : 0x88888888u;
  k_repack_w<<<grid_for(ndw, 256), 256, 0, st>>>(packed, (uint32_t *)b, N, K, L.NB, ndw, mask);
  size_t ns = (size_t)L.NT * L.G * 8;
  k_repack_s<<<grid_for(ns, 256, 0x7fffffffu), 256, 0, st>>>((const f16 *)scales_f16,
                                                             (f16 *)(b + L.s_off), N, L.G, L.NT);
  if (zeros_u8) {
    size_t nz = (size_t)L.NT * L.G * 4;
    k_repack_z<<<grid_for(nz, 256, 0x7fffffffu), 256, 0, st>>>(zeros_u8, b + L.z_off, N, L.G,
                                                               L.NT);
  }
  return sf_check_launch("sf_q4_repack");
}

extern "C" int sf_q4_unpack(const void *blob, int N, int K, int group_size, int has_zeros,
                            uint8_t *packed, void *scales_f16, uint8_t *zeros_u8, void *stream) {
  int rc = check_shape(N, K, group_size);
  if (rc) return rc;
  SF_REQUIRE(blob && packed && scales_f16 && (!has_zeros || zeros_u8), SF_EINVAL,
             "null pointer argument");
  SF_REQUIRE(((uintptr_t)packed & 15) == 0 && ((uintptr_t)blob & 255) == 0, SF_EINVAL,
             "packed must be 16-byte aligned and blob 256-byte aligned");
  BlobLayout L;
  sf_blob_layout(N, K, group_size, has_zeros, &L);
  hipStream_t st = (hipStream_t)stream;
  const uint8_t *b = (const uint8_t *)blob;
  const uint32_t mask = has_zeros ? 0u : 0x88888888u;
  k_unpack_w<<<grid_for((size_t)N * ((K + 7) / 8), 256), 256, 0, st>>>((const uint32_t *)b, packed, N, K,
                                                                  L.NB, mask);
  size_t ns = (size_t)N * L.G;
  k_unpack_s<<<grid_for(ns, 256, 0x7fffffffu), 256, 0, st>>>((const f16 *)(b + L.s_off),
                                                             (f16 *)scales_f16, N, L.G);
  if (has_zeros)
    k_unpack_z<<<grid_for(ns, 256, 0x7fffffffu), 256, 0, st>>>(b + L.z_off, zeros_u8, N, L.G);
  return sf_check_launch("sf_q4_unpack");
}
