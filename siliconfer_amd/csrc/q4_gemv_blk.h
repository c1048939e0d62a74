// q4_gemv_blk.h — int4 decode GEMV (batch 1..8) on MFMA, over the block-layout blob.
//
// y[b, n] = sum_g s[n,g] * sum_{k in g} (q[n,k] - z[n,g]) * x[b,k], fp32 sums: the
// reference's q4_gemv_sym / q4_gemv_asym
// (/root/reference/siliconfer/kernels/neon/q4_gemv.cpp:37-238), with each group's
// partial scaled once (:136, :234).
//
// Operands. The blob's weights come in 1 KB units of 16 rows x 128 k (layout in
// sf_common.h): lane l of a wave loads bytes [16 l, 16 l + 16) of a unit, i.e. row
// l % 16 and k-piece kg = l / 16, and dword j of those 16 bytes holds the eight
// codes of k = 128 blk + 32 j + 8 kg + e. One wave load instruction therefore
// reads one whole unit (1 KB contiguous), and its 64 lanes hold the B operand of
// four v_mfma_f32_16x16x32 — MFMA j covers the 32 k of [128 blk + 32 j, +32), 16
// weight rows wide. The A operand is the batch: lane l supplies row m = l % 16,
// the same eight k, as 16 bytes of activations in natural order. Rows m >= B
// feed output rows that are never stored.
//
// Two arithmetic paths, both exact in the weights:
//  * fp16 activations: a code c is OR-ed into the mantissa of fp16 1024
//    (0x6400 | c = 1024 + c; the odd codes of a dword sit in the upper half of
//    each 16-bit lane, the pairs come out as (k, k + 1)), and one packed
//    subtract of 1024 + z leaves the integer q - z; v_mfma_f32_16x16x32_f16
//    sums the exact products in fp32.
//  * bf16 and fp32 activations: the code goes into bf16 128 (0x4300 | c, exact),
//    v_mfma_f32_16x16x32_bf16 sums (128 + c) x, and the offset is removed from
//    each group's partial as -(128 + z) * sum(x), where sum(x) over the same k
//    comes from one more MFMA against a B operand of ones (shared by every row
//    tile of the wave). fp32 activations are split exactly as the GEMM
//    splits them: bf16 high parts in A rows 0..7, the remainders in rows 8..15
//    (batch <= 8); the two halves of the result are added per wave.
// A scale group's partial is folded once with its fp16 scale, in fp32 (g a
// multiple of 128: once per unit; 64: per two MFMAs; any other multiple of 32:
// per MFMA).
//
// Work split. A workgroup owns T row tiles (16 T rows) and all of K; wave w
// takes units [w BPW, (w + 1) BPW) of each tile. Up to 4 units per wave every
// weight load (T x BPW per lane) is issued before the first MFMA; a longer K
// split issues two units up front and each further unit at the top of the
// iteration two units before its use (a wave that asks for 8+ KB at once
// stalls on the memory pipe with its first units already in registers, and
// computes nothing until the last of its loads has gone out). Partials are
// summed across the waves through LDS in wave order (fixed order: bitwise
// repeatable, and independent of T and of where the activations come from).
// Activations come from one of two places:
//  * XL: the workgroup stages x in LDS once (fp16 / bf16 as they are; fp32 as
//    high and low bf16 rows; zero past K), loading it before the weight stream
//    and storing it after; A fragments are LDS reads. A folded producer
//    (PRE_RMSNORM / PRE_SILU / PRE_MERGE) computes the activations while
//    staging them, rounded as sf_rmsnorm / sf_silu_mul / the attention's merge
//    launch would store them, so a fused launch gives the same bits as the
//    producer followed by the plain GEMV. PRE_MERGE combines split-T attention
//    partials (split_merge.h) into the o-projection's input, one 8-dim piece
//    per thread with every split's loads in flight before the weights.
//  * direct: every lane loads its own fragments (buffer loads; rows >= B and k
//    >= K read past the resource and return zero without touching memory),
//    the first XR units ahead of the weights and the rest in a ring. Used for
//    larger batches, where staging the whole x in LDS costs more than it
//    saves.
#pragma once
#include <stdlib.h>
#include <type_traits>

#include "sf_common.h"
#include "split_merge.h"

namespace sf_gemv {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int PRE_NONE = 0, PRE_RMSNORM = 1, PRE_SILU = 2, PRE_MERGE = 3;
constexpr int kMaxWaves = 16;
constexpr int kUnitK = 128;             // k per weight unit (16 rows x 64 bytes)
constexpr int kXlMaxBytes = 80 * 1024;  // LDS budget of the staged activations (two workgroups per CU)

// (a & m) | c. With m and c in registers (see DequantConsts) the compiler makes
// one v_and_or_b32 of it; two literal constants would split it in two. Plain
// code rather than inline assembly: the compiler must see the instruction to
// keep the wait states an MFMA needs after a VALU write of its operands.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) { return (a & m) | c; }

// The dequant masks and magic exponents, held in registers (opaque to the
// compiler, so it cannot fold them back into literal operands).
struct DequantConsts {
  uint32_t lo, hi, f16m, bf16m;
  __device__ __forceinline__ DequantConsts()
      : lo(0x000F000Fu), hi(0x00F000F0u), f16m(0x64006400u), bf16m(0x43004300u) {
    asm volatile("" : "+v"(lo), "+v"(hi), "+v"(f16m), "+v"(bf16m));
  }
};

// bias: [N] added to every batch row, or y32 itself (fp32): each output then
// adds its own previous value (a residual add, per batch row)
// The addend of output idx (row `row`): bias[row], or with bias == y32 the
// output's previous value (the residual add).
__device__ __forceinline__ float bias_value(const void *bias, int bdt, const float *y32, size_t idx,
                                            int row) {
  if (bias == y32) return y32[idx];
  if (bdt == SF_F32) return ((const float *)bias)[row];
  if (bdt == SF_F16) return (float)((const f16 *)bias)[row];
  return sf_bf16_to_f32(((const uint16_t *)bias)[row]);
}

// The addend's raw bits, loaded early without being used: two 16-bit loads at
// an address chosen without a branch (fp32: its low and high halves; 16-bit
// types: the value twice), so that no conversion, and no wait for this load
// or for any load issued before it, sits between here and the epilogue.
struct AddendBits {
  uint32_t lo = 0, hi = 0;
};
__device__ __forceinline__ AddendBits addend_load(const void *bias, int bdt, const float *y32, size_t idx,
                                                  int row) {
  const bool res = bias == y32, wide = res || bdt == SF_F32;
  const char *p = res ? (const char *)(y32 + idx) : (const char *)bias + (size_t)row * (wide ? 4 : 2);
  AddendBits r;
  r.lo = *(const uint16_t *)p;
  r.hi = *(const uint16_t *)(p + (wide ? 2 : 0));
  return r;
}
__device__ __forceinline__ float addend_value(AddendBits r, const void *bias, int bdt, const float *y32) {
  asm volatile("" : "+v"(r.lo), "+v"(r.hi));  // converted here, at the point of use
  if (bias == y32 || bdt == SF_F32) return sf_bitcast<float>(r.lo | (r.hi << 16));
  if (bdt == SF_F16) return (float)sf_bitcast<f16>((uint16_t)r.lo);
  return sf_bf16_to_f32((uint16_t)r.lo);
}

// Stores v (its addend already added) to y32 and / or y.
__device__ __forceinline__ void store_sum(void *y, int ydt, float *y32, size_t idx, float v) {
  if (y32) y32[idx] = v;
  if (y) {
    if (ydt == SF_F16) ((f16 *)y)[idx] = (f16)v;
    else if (ydt == SF_BF16) ((uint16_t *)y)[idx] = sf_f32_to_bf16(v);
    else ((float *)y)[idx] = v;
  }
}

__device__ __forceinline__ void store_out(void *y, int ydt, float *y32, const void *bias, int bdt,
                                          size_t idx, int row, float v) {
  if (bias) v += bias_value(bias, bdt, y32, idx, row);
  if (y32) y32[idx] = v;
  if (y) {
    if (ydt == SF_F16) ((f16 *)y)[idx] = (f16)v;
    else if (ydt == SF_BF16) ((uint16_t *)y)[idx] = sf_f32_to_bf16(v);
    else ((float *)y)[idx] = v;
  }
}

// Scale groups per unit: GK 0 = g a multiple of 128 (one group per unit),
// 1 = g 64 (MFMAs 0-1 and 2-3), 2 = any other multiple of 32 (one group per
// MFMA, looked up per MFMA).
template <int GK>
struct GroupShape {
  static constexpr int SLOTS = GK == 0 ? 1 : GK == 1 ? 2 : 4;  // scale slots per unit
  static constexpr int SPAN = 4 / SLOTS;                        // MFMAs per slot
};

// Kernel arguments (one struct: fewer kernarg bytes to set up per launch).
struct BlkArgs {
  const uint8_t *w;   // weight units
  const f16 *st;      // tiled scales [ceil(N/8)][G][8]
  const uint8_t *zt;  // tiled zero-points [ceil(N/8)][G][4] (asymmetric)
  const void *x;      // [B][K] activations, or the producer's fp32 source
  void *y;
  int ydt;
  float *y32;
  const void *bias;
  int bdt;
  int B, N, K, G, g, nblk, ntiles;
  uint32_t gmul;      // ceil(2^30 / g): k / g = (k * gmul) >> 30
  int uq, ur;         // units per wave: uq, one more for the first ur waves
  int xp;             // LDS row pitch of the staged activations (elements)
  const float *pre_w; // RMSNorm weight (PRE_RMSNORM)
  float eps;
  const float *mml;   // PRE_MERGE: split (m, l) pairs (x is the split acc)
  int ms, md;         // PRE_MERGE: splits, head_dim
  int nt;             // threads per workgroup (the launch's block size)
};

// Activations staged per thread in XL mode, in pieces of 8 consecutive k of one
// batch row: 16 bytes of fp16 / bf16, 32 of fp32, and 64 (source + weight / up
// half) for the folded RMSNorm / SwiGLU; the folded merge holds its split
// partials apart, one piece per thread.
template <int XDT, int PRE>
struct XPiece {
  static constexpr int NQ = PRE == PRE_MERGE ? 1 : PRE != PRE_NONE ? 4 : XDT == SF_F32 ? 2 : 1;  // 16-byte loads
  static constexpr int PER_THREAD = PRE == PRE_MERGE ? 1 : PRE != PRE_NONE ? 2 : XDT == SF_F32 ? 2 : 4;
};

inline int pieces_per_thread(int pre, int xdt) {
  return pre == PRE_MERGE ? 1 : pre != PRE_NONE ? 2 : xdt == SF_F32 ? 2 : 4;
}

// fp32 -> (bf16 high, bf16 remainder) of two values, packed in pairs (the GEMM's split).
__device__ __forceinline__ void split_pair(float a, float b, uint32_t &hi, uint32_t &lo) {
  const uint32_t ua = sf_bitcast<uint32_t>(a) & 0xFFFF0000u;
  const uint32_t ub = sf_bitcast<uint32_t>(b) & 0xFFFF0000u;
  const float ra = a - sf_bitcast<float>(ua);
  const float rb = b - sf_bitcast<float>(ub);
  hi = (ua >> 16) | ub;
  lo = (sf_bitcast<uint32_t>(ra) >> 16) | (sf_bitcast<uint32_t>(rb) & 0xFFFF0000u);
}

// LDS row of the staged activations that A row m reads: fp32 keeps the high
// parts in rows 0..B-1 and the remainders in rows B..2B-1 (A rows 8..8+B-1);
// rows without data read row 0 (their results are never stored).
template <int XDT>
__device__ __forceinline__ int a_row(int m, int B) {
  if constexpr (XDT == SF_F32) return m < B ? m : (m >= 8 && m - 8 < B) ? B + m - 8 : 0;
  else return m < B ? m : 0;
}

// B operand of MFMA j for one weight dword: the exact integers q - z in fp16.
__device__ __forceinline__ u32x4 dequant_f16(uint32_t d, uint32_t z, const DequantConsts &k) {
  const half2_t c1 = sf_bitcast<half2_t>((0xE400u | z) * 0x10001u);        // -(1024 + z)
  const half2_t c2 = sf_bitcast<half2_t>((0xD400u + 16u * z) * 0x10001u);  // -(64 + z)
  const half2_t sixteenth = {(f16)0.0625f, (f16)0.0625f};
  const uint32_t d8 = d >> 8;
  const half2_t v0 = sf_bitcast<half2_t>(and_or(d, k.lo, k.f16m)) + c1;
  const half2_t v1 = sf_bitcast<half2_t>(and_or(d, k.hi, k.f16m)) * sixteenth + c2;
  const half2_t v2 = sf_bitcast<half2_t>(and_or(d8, k.lo, k.f16m)) + c1;
  const half2_t v3 = sf_bitcast<half2_t>(and_or(d8, k.hi, k.f16m)) * sixteenth + c2;
  return u32x4{sf_bitcast<uint32_t>(v0), sf_bitcast<uint32_t>(v1), sf_bitcast<uint32_t>(v2),
               sf_bitcast<uint32_t>(v3)};
}

// B operand for the bf16 path: 128 + code, exact (the offset comes off each
// group's partial).
__device__ __forceinline__ u32x4 dequant_bf16(uint32_t d, const DequantConsts &k) {
  return u32x4{and_or(d, k.lo, k.bf16m), and_or(d >> 4, k.lo, k.bf16m),
               and_or(d >> 8, k.lo, k.bf16m), and_or(d >> 12, k.lo, k.bf16m)};
}

template <int XDT>
__device__ __forceinline__ float4_t mfma(const u32x4 &a, const u32x4 &b, const float4_t &c) {
  if constexpr (XDT == SF_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(sf_bitcast<half8_t>(a), sf_bitcast<half8_t>(b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(sf_bitcast<bf16x8_t>(a), sf_bitcast<bf16x8_t>(b), c,
                                                   0, 0, 0);
}

// Values of one staged piece (8 consecutive k of source row b at k0), as the
// activation buffer of dtype XDT would hold them (XDT fp32: the fp32 values).
template <int XDT, int PRE>
__device__ __forceinline__ void piece_values(const u32x4 (&q)[XPiece<XDT, PRE>::NQ], float inv,
                                             float (&f)[8]) {
  if constexpr (PRE == PRE_NONE) {
    if constexpr (XDT == SF_F16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half2_t h = sf_bitcast<half2_t>(q[0][i]);
        f[2 * i] = (float)h.x;
        f[2 * i + 1] = (float)h.y;
      }
    } else if constexpr (XDT == SF_BF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[2 * i] = sf_bitcast<float>(q[0][i] << 16);
        f[2 * i + 1] = sf_bitcast<float>(q[0][i] & 0xFFFF0000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = sf_bitcast<float>(q[i / 4][i % 4]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float a = sf_bitcast<float>(q[i / 4][i % 4]), c = sf_bitcast<float>(q[2 + i / 4][i % 4]);
      f[i] = PRE == PRE_RMSNORM ? sf_opaque(a * inv * c) : sf_silu_mul(a, c);
    }
  }
}

// Waves per workgroup a variant may run with: 16 (128 registers) for all but
// the folded RMSNorm with more than four weight units per lane, which also
// holds the norm's row loads and gets the budget of 8 waves.
__host__ __device__ constexpr int max_waves(int pre, int t_bpw) {
  return pre == PRE_RMSNORM && t_bpw > 4 ? 8 : kMaxWaves;
}

// KC: the K split loops over chunks of BPW units (K beyond what the waves
// hold at once); the other variants compile with one chunk as straight-line code.
template <int XDT, bool ASYM, int GK, int T, int BPW, bool XL, int PRE, bool ROPE, bool KC>
__global__ void __launch_bounds__(max_waves(PRE, T * BPW) * 64)
k_q4_gemv_blk(BlkArgs a, SfRopeAppend rope, const int *__restrict__ pos_dev) {
  static_assert(XL || (PRE == PRE_NONE && XDT != SF_F32), "folded producers and fp32 activations stage in LDS");
  static_assert(!ROPE || (T == 4 && PRE == PRE_RMSNORM), "the folded RoPE takes one 64-row head per workgroup");
  typedef GroupShape<GK> GS;
  typedef XPiece<XDT, PRE> XP;
  constexpr bool BFP = XDT != SF_F16;                 // bf16 MFMA path (offset via sum(x))
  // direct mode: units of x held in registers (fewer when zero-points, several
  // scale slots or the sums of the bf16 path need the room)
  //
  // A unit's activations take two direct loads, not four. The A operand has 16
  // rows and only rows < B (B <= 8) are ever stored, so lane row nl loads
  // fragment 2 p + nl / 8 of batch row nl % 8 (p = 0, 1), and a DPP row rotate
  // by 8 hands rows 0..7 the fragments rows 8..15 loaded (the same operand
  // values in every stored row: the same bits). A ring slot then holds half
  // the registers, so the ring is twice as deep as the four-load one was
  // (with the four-load depth the rotate's latency sat in front of the MFMAs
  // and measured slower at K = 11008; twice as deep, 4-5% faster there at
  // batch 3-8, and 0.3-0.4 us faster at K = 4096, batch 5-8).
  constexpr int XR4 = BPW <= 2 ? BPW : (ASYM || BFP || GK != 0) ? 2 : 3;  // the four-load depth
  constexpr int XR = XL ? 1 : (2 * XR4 < BPW ? 2 * XR4 : BPW);
  constexpr int XPRE = XL ? 0 : (XR == BPW ? BPW : XR - 1);
  constexpr bool X2 = !XL;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ float inv_s[8];
  // Every argument the prologue reads, fetched in one round at entry: left to
  // itself the compiler splits these scalar loads around the prologue's first
  // branches, and each round is a wait on the kernel-argument memory before
  // any activation or weight load goes out.
  asm volatile("" ::"s"(a.w), "s"(a.st), "s"(a.zt), "s"(a.x), "s"(a.y), "s"(a.y32), "s"(a.bias),
               "s"(a.pre_w), "s"(a.mml), "s"(a.B), "s"(a.N), "s"(a.K), "s"(a.G), "s"(a.nblk),
               "s"(a.ntiles), "s"(a.gmul), "s"(a.uq), "s"(a.ur), "s"(a.xp), "s"(a.bdt), "s"(a.ydt),
               "s"(a.ms), "s"(a.md), "s"(a.eps), "s"(a.nt));
  // the thread count from the arguments (blockDim is a further read of the
  // dispatch's own arguments)
  const int tid = threadIdx.x, lane = tid & 63, NT = a.nt, nw = NT >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * T * 16;
  const int B = a.B, K = a.K, G = a.G;
  const int KP = a.nblk * kUnitK;
  // the RoPE position (device memory) as the first vector load, read only
  // after the weights have gone out: a scalar load would be waited for by
  // the next wait on the kernel's arguments, ahead of every weight load
  int rpos_v = 0;
  if constexpr (ROPE) rpos_v = __hip_atomic_load(pos_dev, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int nt[T], ti[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    nt[t] = min(n0 + t * 16 + nl, a.N - 1);  // rows past N: a valid row's scales, never stored
    ti[t] = min((int)blockIdx.x * T + t, a.ntiles - 1);
  }
  // K split: wave w takes uq units, one more for the first ur waves, and the
  // last wave what is left (cnt >= 1), in chunks of BPW units: one chunk
  // unless K exceeds what the waves' registers hold at once
  const int blk0 = wave * a.uq + min(wave, a.ur);
  const int cnt = min(a.uq + (wave < a.ur ? 1 : 0), a.nblk - blk0);
  const int nch = KC ? (cnt + BPW - 1) / BPW : 1;

  uint16_t *const xl = (uint16_t *)smem;                               // XL: [rows][xp]
  const int xl_rows = XDT == SF_F32 ? 2 * B : B;
  float *const red = (float *)(smem + (XL ? (size_t)xl_rows * a.xp * 2 : 0));  // [nw][8][T*16]

  // ---- activations, first part: XL pieces (8 consecutive k of one row, in the
  // flat [B][K] order) or direct fragments, before the weights
  const int kpr = K / 8;  // pieces per row
  auto piece_row = [&](int p) {  // p / kpr without a division (B <= 8)
    int b = 0;
    for (int i = 1; i < B; ++i) b += p >= i * kpr;
    return b;
  };
  u32x4 xq[XL ? XP::PER_THREAD : 1][XP::NQ];
  SfRowNorm nrm;
  // folded merge: (m, l) and 8 acc values of each split for the thread's piece
  // (threads without a piece and splits past the last load nothing)
  constexpr int MS = PRE == PRE_MERGE ? kMergeFoldMaxSplits : 1;
  float2_t mq[MS];
  u32x4 aq[MS][2];
  if constexpr (PRE == PRE_MERGE) {
    if (tid < B * kpr) {
      const int b = piece_row(tid), k = 8 * (tid - b * kpr);
      const int h = k / a.md;
      const size_t row = (size_t)b * (K / a.md) + h;
      const int d0 = k - h * a.md;
#pragma unroll
      for (int s = 0; s < MS; ++s)
        if (s < a.ms) {
          const size_t ps = row * a.ms + s;
          mq[s] = *(const float2_t *)(a.mml + ps * 2);
          const u32x4 *src = (const u32x4 *)((const float *)a.x + ps * a.md + d0);
          aq[s][0] = src[0];
          aq[s][1] = src[1];
        }
    }
  } else if constexpr (XL) {
#pragma unroll
    for (int q = 0; q < XP::PER_THREAD; ++q) {
      if (q > 0 && tid + q * NT >= B * kpr) break;  // uniform for all but one wave
      const int p = min(tid + q * NT, B * kpr - 1);
      if constexpr (PRE == PRE_NONE) {
        const u32x4 *src = (const u32x4 *)((const char *)a.x + (size_t)p * (XDT == SF_F32 ? 32 : 16));
#pragma unroll
        for (int i = 0; i < XP::NQ; ++i) xq[q][i] = src[i];
      } else {
        const int b = piece_row(p), k = 8 * (p - b * kpr);
        const size_t stride = PRE == PRE_SILU ? 2 * (size_t)K : (size_t)K;
        const float *s0 = (const float *)a.x + (size_t)b * stride + k;
        const float *s1 = PRE == PRE_SILU ? s0 + K : a.pre_w + k;
        xq[q][0] = ((const u32x4 *)s0)[0];
        xq[q][1] = ((const u32x4 *)s0)[1];
        xq[q][2] = ((const u32x4 *)s1)[0];
        xq[q][3] = ((const u32x4 *)s1)[1];
      }
    }
    if constexpr (PRE == PRE_RMSNORM)
      if (wave < B) nrm.issue<true>((const float *)a.x + (size_t)wave * K, nullptr, K);
  }
  // ---- the epilogue's operands of the decoder's folded variants, loaded now
  // so that the epilogue waits on no round trip of its own: the addend of each
  // output (when every output has a thread of its own: thread e stores output
  // e) and the RoPE position (the plain GEMV keeps its loads in the epilogue:
  // the early form costs it about 2% on its own)
  const int n_out = B * T * 16;
  const bool out_pre = (PRE != PRE_NONE || ROPE) && n_out <= NT;
  AddendBits addend;
  if (out_pre && tid < n_out && a.bias) {
    const int b = tid / (T * 16), row = n0 + tid - b * (T * 16);
    if (row < a.N) addend = addend_load(a.bias, a.bdt, a.y32, (size_t)b * a.N + row, row);
  }
  int rpos = 0;
  bool rope_ok = false;
  SfRopeCS rcs{};
  __amdgpu_buffer_rsrc_t xrs;
  int xoff = 0;
  u32x4 xs[XR][4];
  if constexpr (!XL) {
    xrs = __builtin_amdgcn_make_buffer_rsrc((void *)a.x, 0, B * K * 2, 0x00020000);
    const int xrow = X2 ? nl & 7 : nl;
    xoff = xrow < B ? (xrow * K + 8 * kg) * 2 : 0x40000000;
  }
  const float4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0
  const int arow = a_row<XDT>(nl, B);
  const DequantConsts dk;
  float acc[T][4];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[t][r] = 0.f;

  for (int c = 0; c < nch; ++c) {  // wave-uniform
  const int cb = blk0 + c * BPW, ccnt = min(BPW, cnt - c * BPW);
  const int blast = cb + ccnt - 1;  // units past the chunk's own re-read its last one
  auto xload = [&](int i) {
    if constexpr (!XL) {
      const int kb = min(cb + i, blast) * kUnitK;
#pragma unroll
      for (int j = 0; j < (X2 ? 2 : 4); ++j) {
        const int jj = X2 ? 2 * j + (nl >> 3) : j;  // the fragment this lane fetches
        const int o = kb + 32 * jj + 8 * kg < K ? xoff + (kb + 32 * jj) * 2 : 0x40000000;
        xs[i % XR][j] = __builtin_amdgcn_raw_buffer_load_b128(xrs, o, 0, 0);
      }
    }
  };
  if constexpr (!XL) {
#pragma unroll
    for (int i = 0; i < XPRE; ++i) xload(i);
  }

  // ---- the scales and zero-points of every (tile, unit, slot) (small; the
  // folds need them right after each unit's MFMAs), then the weights. The
  // group of a slot is wave-uniform: k / g as a multiply-shift (exact for
  // k * g < 2^30).
  uint32_t sbits[T][BPW][GS::SLOTS], zbits[T][BPW][GS::SLOTS];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int kb = min(cb + i, blast) * kUnitK;
#pragma unroll
    for (int sl = 0; sl < GS::SLOTS; ++sl) {
      const uint32_t k = (uint32_t)(kb + 32 * GS::SPAN * sl);
      const int gi = min((int)(((uint64_t)k * a.gmul) >> 30), G - 1);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const size_t cell = (size_t)(nt[t] >> 3) * G + gi;
        sbits[t][i][sl] = ((const uint16_t *)a.st)[cell * 8 + (nt[t] & 7)];
        if constexpr (ASYM) zbits[t][i][sl] = a.zt[cell * 4 + ((nt[t] & 7) >> 1)];
      }
    }
  }
  // units issued before the first MFMA (the rest go out one per unit, PD ahead)
  constexpr int PD = BPW >= 8 ? 2 : BPW;
  u32x4 wv[T][BPW];
  auto wload = [&](int i) {
#pragma unroll
    for (int t = 0; t < T; ++t)
      wv[t][i] = __builtin_nontemporal_load(
          (const u32x4 *)(a.w + ((size_t)ti[t] * a.nblk + min(cb + i, blast)) * 1024 + lane * 16));
  };
#pragma unroll
  for (int i = 0; i < PD; ++i) wload(i);
  // every load above goes out before any math (the scheduler would otherwise
  // hold some back behind the first waits to save registers)
  __builtin_amdgcn_sched_barrier(0);
  // the RoPE table rows at the position (after the weights: they need the
  // position's value, and arrive long before the epilogue)
  if constexpr (ROPE) {
    asm volatile("" : "+v"(rpos_v));  // read here, not right behind its load
    rpos = rpos_v;
    rope_ok = rpos >= 0 && rpos < rope.T_cap && rpos < rope.max_pos;
    if (c == 0 && tid < 64 && rope_ok) rcs = sf_rope_load_cs(rope, rpos);
  }

  // ---- XL (first chunk): finish the producer, stage the activations, sync
  if constexpr (XL) if (c == 0) {
    if constexpr (PRE == PRE_RMSNORM) {
      const float *src = (const float *)a.x;
      for (int b = wave; b < B; b += nw) {  // uniform per wave; all lanes active
        if (b != wave) nrm.issue<true>(src + (size_t)b * K, nullptr, K);
        const float r = nrm.finish(src + (size_t)b * K, nullptr, K, a.eps);
        if (lane == 0) inv_s[b] = r;
      }
      __syncthreads();
    }
#pragma unroll
    for (int q = 0; q < XP::PER_THREAD; ++q) {
      const int p = tid + q * NT;
      if (p < B * kpr) {
        const int b = piece_row(p), k = 8 * (p - b * kpr);
        float f[8];
        if constexpr (PRE == PRE_MERGE) {
          float M = -INFINITY;
#pragma unroll
          for (int s = 0; s < MS; ++s)
            if (s < a.ms) M = fmaxf(M, mq[s].x);
          const float mref = sf_merge_mref(M);
          const int P = sf_merge_span(a.ms);
          float w[MS], tl[MS];
#pragma unroll
          for (int s = 0; s < MS; ++s) {
            w[s] = s < a.ms ? sf_merge_weight(mq[s].x, mref) : 0.f;
            tl[s] = s < a.ms ? sf_merge_term(mq[s].y, w[s]) : 0.f;
          }
          const float L = sf_tree_sum(tl, P);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float tv[MS];
#pragma unroll
            for (int s = 0; s < MS; ++s)
              tv[s] = s < a.ms ? sf_merge_term(sf_bitcast<float>(aq[s][e / 4][e % 4]), w[s]) : 0.f;
            f[e] = sf_merge_finish(L, sf_tree_sum(tv, P));
          }
        } else {
          piece_values<XDT, PRE>(xq[q], PRE == PRE_RMSNORM ? inv_s[b] : 1.f, f);
        }
        u32x4 hv, lv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float f0 = f[2 * e], f1 = f[2 * e + 1];
          if constexpr (XDT == SF_F16) {
            hv[e] = sf_bitcast<uint32_t>(half2_t{(f16)f0, (f16)f1});
          } else if constexpr (XDT == SF_BF16) {
            hv[e] = (uint32_t)sf_f32_to_bf16(f0) | ((uint32_t)sf_f32_to_bf16(f1) << 16);
          } else {
            uint32_t h2, l2;
            split_pair(f0, f1, h2, l2);
            hv[e] = h2;
            lv[e] = l2;
          }
        }
        *(u32x4 *)(xl + (size_t)b * a.xp + k) = hv;
        if constexpr (XDT == SF_F32) *(u32x4 *)(xl + (size_t)(B + b) * a.xp + k) = lv;
      }
    }
    // zeros past K up to the last unit's end (K is a multiple of 32)
    const int ppr = (KP - K) / 8;
    for (int p = tid; p < xl_rows * ppr; p += NT) {
      const int r = p / ppr;
      *(u32x4 *)(xl + (size_t)r * a.xp + K + 8 * (p - r * ppr)) = u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
  }

  // ---- the MFMAs, unit by unit
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    if (i + PD < BPW) {
      wload(i + PD);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (!XL)
      if (i + XPRE < BPW) xload(i + XPRE);
    const int kb = min(cb + i, blast) * kUnitK;
    u32x4 av[4];
    if constexpr (X2) {
      auto from_row8 = [](const u32x4 &v) {  // each lane takes the value of lane + 8 of its row
        u32x4 r;
#pragma unroll
        for (int d = 0; d < 4; ++d) r[d] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v[d], 0x128, 0xF, 0xF, false);
        return r;
      };
      av[0] = xs[i % XR][0];
      av[1] = from_row8(xs[i % XR][0]);
      av[2] = xs[i % XR][1];
      av[3] = from_row8(xs[i % XR][1]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (XL) av[j] = *(const u32x4 *)(xl + (size_t)arow * a.xp + kb + 32 * j + 8 * kg);
        else av[j] = xs[i % XR][j];
      }
    }
    // bf16 path: sum(x) of each slot's k (rows m = 4 kg + r of the lane)
    float4_t xsum[GS::SLOTS];
    if constexpr (BFP) {
#pragma unroll
      for (int sl = 0; sl < GS::SLOTS; ++sl) {
        xsum[sl] = zero4;
#pragma unroll
        for (int u = 0; u < GS::SPAN; ++u) xsum[sl] = mfma<XDT>(av[sl * GS::SPAN + u], ones, xsum[sl]);
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
      for (int sl = 0; sl < GS::SLOTS; ++sl) {
        uint32_t z = 8u;  // offset-binary symmetric codes
        if constexpr (ASYM) {
          uint32_t zb = zbits[t][i][sl];
          asm volatile("" : "+v"(zb));  // use the loaded bits here, not right after the load
          z = (zb >> (4 * (nt[t] & 1))) & 15u;
        }
        // each chain starts from zero and accumulates in place (an accumulator
        // start taken from other registers lets the register allocator reuse
        // them while the MFMA still reads them)
        float4_t part = zero4;
#pragma unroll
        for (int u = 0; u < GS::SPAN; ++u) {
          const int j = sl * GS::SPAN + u;
          const uint32_t d = wv[t][i][j];
          const u32x4 bw = BFP ? dequant_bf16(d, dk) : dequant_f16(d, z, dk);
          part = mfma<XDT>(av[j], bw, part);
        }
        if constexpr (BFP) {  // remove the offset: sum((128 + c) x) - (128 + z) sum(x)
          const float zc = -(float)(128u + z);
#pragma unroll
          for (int r = 0; r < 4; ++r) part[r] = fmaf(zc, xsum[sl][r], part[r]);
        }
        uint32_t sb = sbits[t][i][sl];
        asm volatile("" : "+v"(sb));  // convert at the point of use (keeps the load in flight)
        const float s = (float)sf_bitcast<f16>((uint16_t)sb);
        // units past the wave's own (last wave only) are computed on re-read
        // data and dropped here: a branch around them would cut the unrolled
        // units into blocks the scheduler cannot interleave (and, without the
        // staging barrier, let the compiler sink their loads into it)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = i < ccnt ? fmaf(part[r], s, acc[t][r]) : acc[t][r];
      }
    }
  }
  }  // K chunks

  // ---- fold the waves (wave order) and store
  if constexpr (XDT == SF_F32) {  // high + remainder rows: lane l (rows 4kg+r) + lane l^32 (rows 8+4kg+r)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float2_t pr = sf_swap32_pair(acc[t][r]);  // the lane and lane ^ 32
        acc[t][r] = pr.x + pr.y;
      }
  }
  if (kg < 2) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[(wave * 8 + 4 * kg + r) * (T * 16) + t * 16 + nl] = acc[t][r];
  }
  __syncthreads();
  // one output's partials, summed in wave order: for the wave counts the
  // plans use, all the reads go out before the first add (a loop over the
  // runtime count leaves the compiler's remainder iterations each waiting on
  // its read; reading a fixed maximum of slots instead measured slower)
  auto wave_sum = [&](int idx) {
    float v = 0.f;
    auto sum_n = [&](auto n) {
      constexpr int N = decltype(n)::value;
      float pv[N];
#pragma unroll
      for (int wi = 0; wi < N; ++wi) pv[wi] = red[wi * 8 * (T * 16) + idx];
#pragma unroll
      for (int wi = 0; wi < N; ++wi) v += pv[wi];
    };
    switch (nw) {  // wave-uniform
      case 7: sum_n(std::integral_constant<int, 7>{}); break;
      case 8: sum_n(std::integral_constant<int, 8>{}); break;
      case 10: sum_n(std::integral_constant<int, 10>{}); break;
      case 11: sum_n(std::integral_constant<int, 11>{}); break;
      case 14: sum_n(std::integral_constant<int, 14>{}); break;
      case 16: sum_n(std::integral_constant<int, 16>{}); break;
      default:
        for (int wi = 0; wi < nw; ++wi) v += red[wi * 8 * (T * 16) + idx];
    }
    return v;
  };
  if constexpr (ROPE) {
    float *hv = red + nw * 8 * (T * 16);  // the head's 64 outputs, bias added
    if (tid < 64) {  // B = 1, 64 outputs: out_pre holds
      float v = wave_sum(tid);
      if (a.bias) v += addend_value(addend, a.bias, a.bdt, a.y32);
      hv[tid] = v;
    }
    __syncthreads();
    if (tid < 64 && rope_ok) sf_rope_append_head(rope, hv, blockIdx.x, rpos, 0, rcs);
    return;
  }
  for (int e = tid; e < n_out; e += NT) {
    const int b = e / (T * 16), c = e - b * (T * 16);
    const int row = n0 + c;
    if (row >= a.N) continue;
    float v = wave_sum(b * (T * 16) + c);
    if (out_pre) {
      if (a.bias) v += addend_value(addend, a.bias, a.bdt, a.y32);
      store_sum(a.y, a.ydt, a.y32, (size_t)b * a.N + row, v);
    } else {
      store_out(a.y, a.ydt, a.y32, a.bias, a.bdt, (size_t)b * a.N + row, row, v);
    }
  }
}

// ---------------------------------------------------------------------------
// host side: plans and launches
// ---------------------------------------------------------------------------
// Units per wave come from a compiled set so that every register array has a
// compile-time size and every load can be issued before the first MFMA.
constexpr int kBpwSet[6] = {1, 2, 4, 8, 11, 12};  // 11: K = 11008 (86 units) over 8 waves
constexpr int kMergeMaxBpw = 4;  // the folded merge: K = H * head_dim up to 64 units

struct BlkPlan {
  int T, BPW, nw, grid, nblk, ntiles, xl, xp, uq, ur, kc;
  size_t lds;
};

inline int group_kind(int g) { return g % 128 == 0 ? 0 : g == 64 ? 1 : 2; }

// The most units per wave a group kind's registers allow (scale and zero bits
// per unit grow with the slots; the bf16 path holds the slots' sums as well).
// With 16 waves this covers K up to 16384 for groups of 64 and 128 (8192 for
// other multiples of 32). The bf16 path at groups of 64 keeps to 4 units where
// 16 waves suffice: its 8-unit variants spill registers (correct, slower).
__host__ __device__ constexpr int max_bpw(int gk, bool bf) {
  return gk == 0 ? (bf ? 8 : 12) : gk == 1 ? 8 : 4;
}
inline int soft_max_bpw(int gk, bool bf) { return gk == 1 && bf ? 4 : max_bpw(gk, bf); }

inline size_t xl_bytes(int B, int xdt, int nblk) {
  const int rows = xdt == SF_F32 ? 2 * B : B;
  return (size_t)rows * (nblk * kUnitK + 8) * 2;
}

// The split of K over waves (and so the summation order) depends on (B, N, K,
// g) only; where the activations come from (`xl`) does not change the bits.
// pre != PRE_NONE and fp32 activations need XL; returns false when that does
// not fit (LDS, or pieces per thread).
inline bool plan_blk(int B, int N, int K, int g, int xdt, int pre, bool rope, BlkPlan *p) {
  p->nblk = (K + kUnitK - 1) / kUnitK;
  p->ntiles = (N + 15) / 16;
  const int gk = group_kind(g);
  const bool wide = B > 4 && p->ntiles >= 512 && p->nblk <= 32 && gk != 2 && pre != PRE_MERGE;
  p->T = rope ? 4 : wide ? 4 : 1;
  const int maxb = max_bpw(gk, xdt != SF_F16);
  const size_t xb = xl_bytes(B, xdt, p->nblk);
  auto bucket = [](int need) {
    for (int i = 0; i < 6; ++i)
      if (kBpwSet[i] >= need) return kBpwSet[i];
    return kBpwSet[5];
  };
  int bpw, nw;
  if (wide) {
    bpw = p->nblk <= 16 ? 1 : 2;
  } else {
    // waves per workgroup: 16 for larger batches, for matrices with fewer row
    // tiles than CUs and a K of at least 32 units, and for K of at least 64
    // units (K is then spread over more waves; measured on 4096 x 11008 and
    // 896 x 4864; 4096 x 4096, one tile per CU, runs faster at batch <= 4 on
    // 8 waves of 4 units than on 16 of 2)
    const int target =
        B > 4 || (p->ntiles < 256 && p->nblk >= 32) || (p->ntiles <= 256 && p->nblk >= 64) ? 16 : 8;
    bpw = bucket((p->nblk + target - 1) / target);
  }
  const int soft = soft_max_bpw(gk, xdt != SF_F16);
  if (bpw > soft) bpw = (p->nblk + soft - 1) / soft <= kMaxWaves ? soft : maxb;
  nw = (p->nblk + bpw - 1) / bpw;
  p->BPW = bpw;
  p->nw = nw;
  p->uq = bpw;  // units per wave; the last wave takes what is left
  p->ur = 0;
  p->kc = 0;
  if (nw > max_waves(pre, p->T * bpw)) {
    // K beyond what the waves hold at once: the plain GEMV's waves loop over
    // chunks of BPW units, the units split as evenly as 16 waves allow (a
    // folded producer or the RoPE epilogue is not built for it)
    if (pre != PRE_NONE || rope || p->T != 1) return false;
    p->nw = nw = kMaxWaves;
    p->uq = p->nblk / nw;
    p->ur = p->nblk % nw;
    p->kc = 1;
  }
  // the folded RMSNorm's variants hold about 16 waves per CU: two row tiles
  // per workgroup when one would leave workgroups for a second round (T does
  // not change any row's summation order)
  if (pre == PRE_RMSNORM && p->T == 1 && p->BPW <= 2 && p->ntiles > 256 * (16 / p->nw)) p->T = 2;
  if (p->nw > max_waves(pre, p->T * p->BPW)) return false;
  if (pre == PRE_MERGE && p->BPW > kMergeMaxBpw) return false;  // variants compiled up to 4 units
  p->grid = (p->ntiles + p->T - 1) / p->T;
  const int per_thread = pieces_per_thread(pre, xdt);
  const bool xl_fit = xb <= (size_t)kXlMaxBytes &&
                      (size_t)B * (K / 8) <= (size_t)per_thread * p->nw * 64;
  const bool need_xl = pre != PRE_NONE || xdt == SF_F32;
  if (need_xl && !xl_fit) return false;
  p->xl = need_xl || (xl_fit && B <= 4);
  p->xp = p->nblk * kUnitK + 8;
  const size_t red = (size_t)p->nw * 8 * p->T * 16 * 4 + (rope ? 64 * 4 : 0);
  p->lds = (p->xl ? xb : 0) + red;
  return true;
}

struct GemvArgs {
  const uint8_t *w; const f16 *st; const uint8_t *zt; const void *x; void *y; int ydt; float *y32;
  const void *bias; int bdt; int B, N, K, G, g; bool asym; hipStream_t s;
  const float *mml = nullptr; int ms = 0, md = 0;  // the folded merge's (m, l), splits, head_dim
};

template <int X, bool A, int GK, int T, int BPW, bool XL, int PRE, bool ROPE, bool KC = false>
void launch_cfg(const BlkPlan &p, const GemvArgs &g, const float *pre_w, float eps,
                const SfRopeAppend *rope, const int *pos_dev) {
  if (p.lds > 64 * 1024) {
    static bool attr = false;  // raise the dynamic LDS limit once per variant
    if (!attr) {
      (void)hipFuncSetAttribute((const void *)k_q4_gemv_blk<X, A, GK, T, BPW, XL, PRE, ROPE, KC>,
                          hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
      attr = true;
    }
  }
  const uint32_t gmul = (uint32_t)(((1ull << 30) + g.g - 1) / g.g);
  const BlkArgs ba{g.w, g.st, g.zt, g.x, g.y, g.ydt, g.y32, g.bias, g.bdt, g.B, g.N, g.K, g.G, g.g,
                   p.nblk, p.ntiles, gmul, p.uq, p.ur, p.xp, pre_w, eps, g.mml, g.ms, g.md,
                   p.nw * 64};
  const SfRopeAppend ra = rope ? *rope : SfRopeAppend{};
  k_q4_gemv_blk<X, A, GK, T, BPW, XL, PRE, ROPE, KC><<<p.grid, p.nw * 64, p.lds, g.s>>>(ba, ra, pos_dev);
}

// Runtime units-per-wave -> compiled variant. Compiled: T = 1 with every count
// of the set the group kind allows; T = 2 (the folded RMSNorm on many row
// tiles) up to 4; T = 4 (wide matrices at batch > 4, and the folded RoPE) with
// 1, 2 and, for the RoPE, 4.
template <int X, bool A, int GK, int T, bool XL, int PRE, bool ROPE>
void by_bpw(const BlkPlan &p, const GemvArgs &g, const float *pre_w, float eps,
            const SfRopeAppend *rope, const int *pos_dev) {
  constexpr int MB = T == 4            ? (GK == 2 ? (ROPE ? 2 : 0) : ROPE ? 4 : 2)
                     : T == 2          ? (GK == 2 ? 2 : 4)
                     : PRE == PRE_MERGE ? (max_bpw(GK, X != SF_F16) < kMergeMaxBpw ? max_bpw(GK, X != SF_F16) : kMergeMaxBpw)
                                       : max_bpw(GK, X != SF_F16);
#define SF_BPW(N)                                                                 \
  case N:                                                                         \
    if constexpr (N <= MB) launch_cfg<X, A, GK, T, N, XL, PRE, ROPE>(p, g, pre_w, eps, rope, pos_dev); \
    break;
  switch (p.BPW) {
    SF_BPW(1) SF_BPW(2) SF_BPW(4) SF_BPW(8) SF_BPW(11) SF_BPW(12)
    default: break;
  }
#undef SF_BPW
}

// The chunked plain GEMV (plan kc): T = 1 at the group kind's largest unit
// count (a plan that needs chunks always takes it).
template <int X, bool A, int GK>
void launch_kc(const BlkPlan &p, const GemvArgs &g) {
  constexpr int MB = max_bpw(GK, X != SF_F16);
  if (p.BPW != MB) return;
  if (p.xl) launch_cfg<X, A, GK, 1, MB, true, PRE_NONE, false, true>(p, g, nullptr, 0.f, nullptr, nullptr);
  else if constexpr (X != SF_F32) launch_cfg<X, A, GK, 1, MB, false, PRE_NONE, false, true>(p, g, nullptr, 0.f, nullptr, nullptr);
}

template <int X, bool A, int GK>
void by_mode(const BlkPlan &p, const GemvArgs &g, int pre, const float *pre_w, float eps,
             const SfRopeAppend *rope, const int *pos_dev) {
  if (p.kc) {
    launch_kc<X, A, GK>(p, g);
    return;
  }
  if (rope) {
    by_bpw<X, A, GK, 4, true, PRE_RMSNORM, true>(p, g, pre_w, eps, rope, pos_dev);
    return;
  }
#define SF_T(XL, PRE)                                                              \
  do {                                                                             \
    if (p.T == 4) by_bpw<X, A, GK, 4, XL, PRE, false>(p, g, pre_w, eps, rope, pos_dev); \
    else by_bpw<X, A, GK, 1, XL, PRE, false>(p, g, pre_w, eps, rope, pos_dev);         \
  } while (0)
  if (pre == PRE_RMSNORM && p.T == 2) by_bpw<X, A, GK, 2, true, PRE_RMSNORM, false>(p, g, pre_w, eps, rope, pos_dev);
  else if (pre == PRE_RMSNORM) SF_T(true, PRE_RMSNORM);
  else if (pre == PRE_SILU) SF_T(true, PRE_SILU);
  else if (pre == PRE_MERGE) by_bpw<X, A, GK, 1, true, PRE_MERGE, false>(p, g, nullptr, 0.f, nullptr, nullptr);
  else if (p.xl) SF_T(true, PRE_NONE);
  else if constexpr (X != SF_F32) SF_T(false, PRE_NONE);
#undef SF_T
}

// One (activation dtype, symmetry)'s launches; each pair is instantiated in a
// file of its own (compile time).
template <int X, bool A>
void launch_blk(const BlkPlan &p, const GemvArgs &g, int pre, const float *pre_w, float eps,
                const SfRopeAppend *rope, const int *pos_dev) {
  switch (group_kind(g.g)) {
    case 0: by_mode<X, A, 0>(p, g, pre, pre_w, eps, rope, pos_dev); break;
    case 1: by_mode<X, A, 1>(p, g, pre, pre_w, eps, rope, pos_dev); break;
    default: by_mode<X, A, 2>(p, g, pre, pre_w, eps, rope, pos_dev); break;
  }
}

#define SF_GEMV_BLK_EXTERN(X, A)                                                             \
  extern template void launch_blk<X, A>(const BlkPlan &, const GemvArgs &, int, const float *, \
                                        float, const SfRopeAppend *, const int *);
SF_GEMV_BLK_EXTERN(SF_F16, false)
SF_GEMV_BLK_EXTERN(SF_F16, true)
SF_GEMV_BLK_EXTERN(SF_BF16, false)
SF_GEMV_BLK_EXTERN(SF_BF16, true)
SF_GEMV_BLK_EXTERN(SF_F32, false)
SF_GEMV_BLK_EXTERN(SF_F32, true)
#undef SF_GEMV_BLK_EXTERN

}  // namespace sf_gemv
