// q4_gemm.hip — int4 prefill GEMM on CDNA4 MFMA (gfx950).
//
// Y[m, n] = sum_k X[m, k] * (q[n,k] - z[n,g(k)]) * s[n,g(k)], fp32 accumulation:
// the reference's q4_gemm_sym / q4_gemm_asym
// (/root/reference/siliconfer/kernels/neon/q4_gemm.cpp:12-51), which loop the
// GEMV over the T rows and re-stream W for each; here W is read once per
// 128-row block of X. Both kernels fold each scale group's fp32 partial into
// the result once, with the group's fp16 scale: y = sum_g s_g * sum_{k in g}
// x_k (q_k - z), the reference's own grouping (q4_gemv.cpp:136).
//
// Two kernels, one 128 x 128 output tile per workgroup (the same tiling, so
// the same split-K choice and workspace):
//  * k_q4_gemm_ws (fp16 / bf16 activations; groups of 32, 64 or a multiple
//    of 128): every operand byte (X fragments, the blob's W units, scales,
//    zero-points) goes straight into LDS with buffer / global loads ... lds,
//    four stages deep; four convert waves turn the next step's codes into
//    the exact integers q - z as MFMA B operands in LDS while eight math
//    waves run the MFMAs and the per-group folds (described above the
//    kernel).
//  * k_q4_gemm (fp32 activations and the other multiples of 32): staging
//    threads dequantize the W tile once into LDS as the integers q - z (exact
//    in fp16 and bf16); fp32 activations are split into bf16 high and low
//    parts (two MFMAs); 128 x 128 per 512 threads (2 x 4 waves of 64 x 32),
//    K steps of 64 through two padded LDS buffers with each step's global
//    loads three steps ahead in registers; the output goes back through LDS
//    as whole row segments.
// When the tile grid is too small to fill the GPU, K is split across
// workgroups into an fp32 workspace and summed by a second kernel in a fixed
// order.
#include <stdlib.h>

#include "q4_gemv_blk.h"
#include "sf_common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kGemmGemvRows = 16;  // sf_q4_gemm runs up to this many rows as 8-row batch GEMVs
constexpr int LDS_PITCH = BK + 8;  // bf16 elements per LDS row (+16 B breaks bank conflicts)
constexpr int NTHREADS = 512;      // 8 waves: two per SIMD, so one's VALU overlaps another's MFMA
constexpr int KPT = BM * BK / NTHREADS;  // 16 elements of X (and of W) staged per thread per step
constexpr int WAVE_M = 64, WAVE_N = 32;  // wave tile: 2 x 1 MFMA 32x32 tiles
constexpr int OUT_PITCH = WAVE_N + 4;    // fp32 pitch of a wave's output tile staged in LDS
static_assert(BN * BK / NTHREADS == KPT, "X and W staging shares must match");
static_assert((BM / WAVE_M) * (BN / WAVE_N) * 64 == NTHREADS, "wave grid must cover the tile");

__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) {
  // top 16 bits of a (low half) and of b (high half)
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// One thread's share of the X tile: row tid/4, KPT consecutive k starting at
// KPT*(tid%4). Loaded into registers as raw bits; loads are unconditional
// (clamped in-bounds address; K is a multiple of 32) so they stay in flight,
// and rows or k past the end are zeroed when the registers are staged.
template <int XDT>
struct XRegs {
  static constexpr int NQ = KPT * (XDT == SF_F32 ? 4 : 2) / 16;  // 16-byte loads
  u32x4 v[NQ];
  bool ok;
};

template <int XDT>
__device__ __forceinline__ void load_x(XRegs<XDT> &r, const void *X, int M, int K, int m, int k) {
  r.ok = m < M && k < K;
  const size_t esz = XDT == SF_F32 ? 4 : 2;
  const u32x4 *p =
      (const u32x4 *)((const char *)X + ((size_t)min(m, M - 1) * K + min(k, K - KPT)) * esz);
#pragma unroll
  for (int i = 0; i < XRegs<XDT>::NQ; ++i) r.v[i] = p[i];
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

// Write the thread's KPT activations to the LDS tiles: fp16 / bf16 as they
// are, fp32 as bf16 high and low parts.
template <int XDT>
__device__ __forceinline__ void store_x(const XRegs<XDT> &r, uint16_t *xs_hi, uint16_t *xs_lo,
                                        int lrow, int lk) {
  u32x4 *dh = (u32x4 *)(xs_hi + lrow * LDS_PITCH + lk);
  const uint32_t keep = r.ok ? 0xFFFFFFFFu : 0u;
  if constexpr (XDT != SF_F32) {
#pragma unroll
    for (int i = 0; i < KPT / 8; ++i) dh[i] = r.v[i] & keep;
  } else {
    u32x4 *dl = (u32x4 *)(xs_lo + lrow * LDS_PITCH + lk);
#pragma unroll
    for (int i = 0; i < KPT / 8; ++i) {  // 8 activations per 16-byte LDS store
      float f[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = sf_bitcast<float>(r.v[2 * i + j / 4][j % 4] & keep);
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

// One thread's share of the W tile: KPT = 16 codes of row n from k (two
// dwords of the blob's unit: k-pieces k and k + 8 of the same MFMA slice sit in
// lanes 16 apart), and the raw scale / zero-point bits of that (row, group);
// converted at staging (a step never straddles a group: g is a multiple of 32
// and KPT divides 32).
struct WRegs {
  u32x2 w;
  uint32_t sbits, zbyte;
  bool ok;
};

template <bool ASYM>
__device__ __forceinline__ void load_w(WRegs &r, const uint8_t *__restrict__ wq,
                                       const f16 *__restrict__ st, const uint8_t *__restrict__ zt,
                                       int N, int K, int G, int g, int n, int k) {
  r.ok = n < N && k < K;
  const int nc = min(n, N - 1), kc = min(k, K - KPT);
  const int nb = (K + 127) >> 7, kb = kc & 127;
  const uint8_t *unit = wq + ((size_t)(nc >> 4) * nb + (kc >> 7)) * 1024;
  const int lane = ((kb & 31) >> 3) * 16 + (nc & 15);
  r.w.x = *(const uint32_t *)(unit + lane * 16 + (kb >> 5) * 4);
  r.w.y = *(const uint32_t *)(unit + (lane + 16) * 16 + (kb >> 5) * 4);
  const size_t cell = (size_t)(nc >> 3) * G + kc / g;
  r.sbits = ((const uint16_t *)st)[cell * 8 + (nc & 7)];
  if constexpr (ASYM) r.zbyte = zt[cell * 4 + ((nc & 7) >> 1)];
}

// Store the thread's KPT weights as the integers q - z (fp16 when MT is
// SF_F16, else bf16; zero past the matrix) and, from the threads at the start
// of a 32-k half, the row's scale for that half into the scale table.
template <bool ASYM, int MT>
__device__ __forceinline__ void store_w(const WRegs &r, uint16_t *ws, uint16_t *ss, int lrow,
                                        int lk) {
  u32x4 *d = (u32x4 *)(ws + lrow * LDS_PITCH + lk);
  // row n's zero-point nibble: the low one for even n, the high one for odd n
  // (offset-binary symmetric codes have z = 8)
  uint32_t z = 8u;
  if constexpr (ASYM) z = (r.zbyte >> (4 * (lrow & 1))) & 15u;
  const uint32_t keep = r.ok ? 0xFFFFFFFFu : 0u;
#pragma unroll
  for (int i = 0; i < KPT / 8; ++i) {  // dword i holds k = 8i .. 8i+7, code e at 4(e/2) + 16(e%2)
    const uint32_t dw = i == 0 ? r.w.x : r.w.y;
    u32x4 o;
#pragma unroll
    for (int b = 0; b < 4; ++b) {  // pair (k = 8i + 2b, 8i + 2b + 1) in the two 16-bit halves
      const uint32_t pq = (dw >> (4 * b)) & 0x000F000Fu;
      if constexpr (MT == SF_F16) {
        // 1024 + q as fp16, minus (1024 + z): exact
        const half2_t v = sf_bitcast<half2_t>(pq | 0x64006400u) +
                          sf_bitcast<half2_t>((0xE400u | z) * 0x10001u);
        o[b] = sf_bitcast<uint32_t>(v);
      } else {
        const float f0 = (float)(int)((pq & 0xFu) - z), f1 = (float)(int)((pq >> 16) - z);
        o[b] = hi_pair(sf_bitcast<uint32_t>(f0), sf_bitcast<uint32_t>(f1));
      }
    }
    d[i] = o & keep;
  }
  if ((lk & 31) == 0) ss[lrow * 2 + (lk >> 5)] = (uint16_t)r.sbits;
}

// Write 8 consecutive outputs (nv of them in range) to the fp32 copy and / or
// the output in its dtype; 16-byte stores when `vec` (row pitch and bases
// allow it) and all 8 are in range.
__device__ __forceinline__ void store_row8(const float (&v)[8], int nv, bool vec, float *y32,
                                           void *Y, int ydt, size_t idx) {
  if (y32) {
    if (vec && nv == 8) {
      ((float4_t *)(y32 + idx))[0] = float4_t{v[0], v[1], v[2], v[3]};
      ((float4_t *)(y32 + idx))[1] = float4_t{v[4], v[5], v[6], v[7]};
    } else {
      for (int e = 0; e < nv; ++e) y32[idx + e] = v[e];
    }
  }
  if (!Y) return;
  if (ydt == SF_F32) {
    float *d = (float *)Y + idx;
    if (vec && nv == 8) {
      ((float4_t *)d)[0] = float4_t{v[0], v[1], v[2], v[3]};
      ((float4_t *)d)[1] = float4_t{v[4], v[5], v[6], v[7]};
    } else {
      for (int e = 0; e < nv; ++e) d[e] = v[e];
    }
    return;
  }
  uint16_t b[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    b[e] = ydt == SF_BF16 ? sf_f32_to_bf16(v[e]) : sf_bitcast<uint16_t>((f16)v[e]);
  uint16_t *d = (uint16_t *)Y + idx;
  if (vec && nv == 8) {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = (uint32_t)b[2 * e] | ((uint32_t)b[2 * e + 1] << 16);
    *(u32x4 *)d = w;
  } else {
    for (int e = 0; e < nv; ++e) d[e] = b[e];
  }
}

// GK: the group size's shape, fixed at compile time so the per-group folds
// are straight-line code: 0 = 32 (two groups per K step), 1 = 64 (one per
// step), 2 = a multiple of 128 (a group spans several steps; a test per
// step), 3 = any other multiple of 32 (a test per 16-k slice).
template <int XDT, bool ASYM, int GK>
__global__ void __launch_bounds__(NTHREADS, 2)
k_q4_gemm(const uint8_t *__restrict__ wq, const f16 *__restrict__ st,
          const uint8_t *__restrict__ zt, const void *__restrict__ X, void *__restrict__ Y,
          int ydt, float *__restrict__ y32, const void *__restrict__ bias, int bdt,
          float *__restrict__ part, int M, int N, int K, int G, int g, int ksplit,
          int steps_per_split, bool vec) {
  constexpr bool XSPLIT = XDT == SF_F32;             // fp32 activations: bf16 hi + lo
  constexpr int MT = XDT == SF_F16 ? SF_F16 : SF_BF16;  // MFMA operand type
  constexpr int XB = BM * LDS_PITCH, WB = BN * LDS_PITCH;  // one LDS buffer of each tile
  constexpr int SB = BN * 2;                               // scales: 2 halves of the step per row
  constexpr int SMEM_U16 = 2 * XB * (XSPLIT ? 2 : 1) + 2 * WB + 2 * SB;
  constexpr int NWAVES = NTHREADS / 64;
  constexpr int OUT_U16 = NWAVES * WAVE_M * OUT_PITCH * 2;
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM_U16 > OUT_U16 ? SMEM_U16 : OUT_U16];
  uint16_t *const xs_hi = smem;
  uint16_t *const xs_lo = smem + 2 * XB;  // used only when XSPLIT
  uint16_t *const ws = smem + 2 * XB * (XSPLIT ? 2 : 1);
  uint16_t *const ss = ws + 2 * WB;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  constexpr int WGN = BN / WAVE_N;  // waves across the tile's columns
  const int wm = (wave / WGN) * WAVE_M, wn = (wave % WGN) * WAVE_N;  // wave tile origin
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int split = blockIdx.z;
  const int nsteps_total = (K + BK - 1) / BK;
  const int s0 = split * steps_per_split;
  const int s1 = min(s0 + steps_per_split, nsteps_total);

  // staging assignment: row tid / (BK / KPT), KPT consecutive k
  const int lrow = tid / (BK / KPT), lk = (tid % (BK / KPT)) * KPT;

  float16_t acc[2], gp[2];  // the result, and the current scale group's partial
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = gp[i][r] = 0.f;

  // Loads past the split's last step re-read that step (in bounds, unused), so
  // every load is unconditional and stays in flight.
  auto load = [&](int step, XRegs<XDT> &xr, WRegs &wr) {
    const int k = min(step, s1 - 1) * BK + lk;
    load_x<XDT>(xr, X, M, K, m0 + lrow, k);
    load_w<ASYM>(wr, wq, st, zt, N, K, G, g, n0 + lrow, k);
  };
  auto store = [&](int step, const XRegs<XDT> &xr, const WRegs &wr) {
    const int b = step & 1;
    store_x<XDT>(xr, xs_hi + b * XB, xs_lo + (XSPLIT ? b * XB : 0), lrow, lk);
    store_w<ASYM, MT>(wr, ws + b * WB, ss + b * SB, lrow, lk);
  };
  // a lane's accumulators all belong to output column c: one scale per group
  auto fold = [&](float sc) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][r] = fmaf(gp[i][r], sc, acc[i][r]);
  };
  const float16_t zero16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f,
                            0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // one K step; `fresh`: the step starts a scale group (its first MFMAs take
  // a zero accumulator), `last`: the step ends one (fold after it)
  auto compute_step = [&](int step, bool fresh, bool last) {
    const int b = step & 1;
    const uint16_t *xh = xs_hi + b * XB, *xl = xs_lo + (XSPLIT ? b * XB : 0);
    const uint16_t *wt = ws + b * WB;
    const int c = wn + (lane & 31);
    const int kb = step * BK;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      // a group starts here: the slice's MFMAs take a zero accumulator
      const bool zc = GK == 3 ? (kk % 32 == 0 && ((kb + kk) % g == 0 || (kk == 0 && step == s0)))
                              : (kk == 0 && fresh) || (GK == 0 && kk == 32);
      const int kofs = kk + (lane >> 5) * 8;
      u32x4 ah[2], al[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int r = wm + i * 32 + (lane & 31);
        ah[i] = *(const u32x4 *)(xh + r * LDS_PITCH + kofs);
        if constexpr (XSPLIT) al[i] = *(const u32x4 *)(xl + r * LDS_PITCH + kofs);
      }
      const u32x4 bw = *(const u32x4 *)(wt + c * LDS_PITCH + kofs);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float16_t cin = zc ? zero16 : gp[i];
        if constexpr (MT == SF_F16) {
          gp[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sf_bitcast<half8_t>(ah[i]),
                                                         sf_bitcast<half8_t>(bw), cin, 0, 0, 0);
        } else {
          gp[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(sf_bitcast<bf16x8_t>(ah[i]),
                                                          sf_bitcast<bf16x8_t>(bw), cin, 0, 0, 0);
          if constexpr (XSPLIT)
            gp[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(sf_bitcast<bf16x8_t>(al[i]),
                                                            sf_bitcast<bf16x8_t>(bw), gp[i], 0, 0, 0);
        }
      }
      // a group ends after this 16-k slice: scale the partial once
      const bool end = GK == 3 ? (kk % 32 == 16 && ((kb + kk + 16) % g == 0 ||
                                                    (kk == BK - 16 && step == s1 - 1)))
                               : (GK == 0 && kk == 16) || (kk == BK - 16 && last);
      if (end) fold((float)sf_bitcast<f16>(ss[b * SB + c * 2 + (kk >> 5)]));
    }
  };
  // g = 32 / 64: every step starts and ends its groups; g >= 128: a group
  // spans g / 64 steps (and a split's last step closes its open group)
  auto compute = [&](int step) {
    if constexpr (GK < 2 || GK == 3) {
      compute_step(step, true, true);  // (GK 3 decides per slice)
    } else {
      const int spg = g / BK;
      const bool fresh = step % spg == 0 || step == s0;
      const bool last = (step + 1) % spg == 0 || step == s1 - 1;
      if (fresh && last) compute_step(step, true, true);
      else if (fresh) compute_step(step, true, false);
      else if (last) compute_step(step, false, true);
      else compute_step(step, false, false);
    }
  };

  // Pipeline: three register stages of global loads (a step's loads are issued
  // three steps before it is staged) and two LDS buffers, one barrier per step.
  // At the top of the loop for step s: LDS buffer s&1 holds step s, xb/wb hold
  // step s+1, xc/wc step s+2, xa/wa step s+3. Staging is unconditional (past
  // the end it re-stages the last step into the buffer no one reads again), so
  // it shares a basic block with the MFMAs and the two can interleave.
  if (s0 < s1) {
    XRegs<XDT> xa, xb, xc;
    WRegs wa, wb, wc;
    load(s0, xa, wa);
    load(s0 + 1, xb, wb);
    load(s0 + 2, xc, wc);
    store(s0, xa, wa);
    __syncthreads();
    load(s0 + 3, xa, wa);
    for (int s = s0; s < s1; s += 3) {
      store(s + 1, xb, wb);
      compute(s);
      __syncthreads();
      if (s + 1 >= s1) break;
      load(s + 4, xb, wb);
      store(s + 2, xc, wc);
      compute(s + 1);
      __syncthreads();
      if (s + 2 >= s1) break;
      load(s + 5, xc, wc);
      store(s + 3, xa, wa);
      compute(s + 2);
      __syncthreads();
      if (s + 3 >= s1) break;
      load(s + 6, xa, wa);
    }
  }

  // Output. acc[i][r] is C[row][col] with row = 8*(r/4) + 4*(lane/32) + r%4,
  // col = lane % 32 within MFMA tile i: a lane holds one column, so each wave
  // stages its WAVE_M x WAVE_N tile in LDS and writes it back as row segments
  // of 8 values per lane (16-byte stores, whole cache lines per instruction).
  __syncthreads();  // every wave is done with the operand buffers
  float *ot = (float *)smem + wave * WAVE_M * OUT_PITCH;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      ot[(i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * OUT_PITCH + (lane & 31)] = acc[i][r];
  __syncthreads();
  constexpr int SEGS = WAVE_N / 8;  // 8-column segments per row
#pragma unroll 2
  for (int it = 0; it < WAVE_M * SEGS / 64; ++it) {
    const int seg = it * 64 + lane;
    const int rl = seg / SEGS, cl = (seg % SEGS) * 8;
    const int row = m0 + wm + rl, col = n0 + wn + cl;
    if (row >= M || col >= N) continue;
    float v[8];
    {
      const float4_t a = *(const float4_t *)(ot + rl * OUT_PITCH + cl);
      const float4_t c = *(const float4_t *)(ot + rl * OUT_PITCH + cl + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[4 + e] = c[e];
      }
    }
    const int nv = min(8, N - col);
    const size_t idx = (size_t)row * N + col;
    if (ksplit > 1) {
      float *dst = part + (size_t)split * M * N + idx;
      if (vec && nv == 8) {
        ((float4_t *)dst)[0] = float4_t{v[0], v[1], v[2], v[3]};
        ((float4_t *)dst)[1] = float4_t{v[4], v[5], v[6], v[7]};
      } else {
        for (int e = 0; e < nv; ++e) dst[e] = v[e];
      }
      continue;
    }
    if (bias) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int cc = min(col + e, N - 1);
        if (bdt == SF_F32) v[e] += ((const float *)bias)[cc];
        else if (bdt == SF_F16) v[e] += (float)((const f16 *)bias)[cc];
        else v[e] += sf_bf16_to_f32(((const uint16_t *)bias)[cc]);
      }
    }
    store_row8(v, nv, vec, y32, Y, ydt, idx);
  }
}

// Sum of the K-split partials in split order (deterministic), plus bias, to
// the outputs; 8 consecutive elements per thread.
__global__ void __launch_bounds__(256)
k_splitk_reduce(const float *__restrict__ part, void *__restrict__ Y, int ydt, float *__restrict__ y32,
                const void *__restrict__ bias, int bdt, int M, int N, int ksplit, bool vec) {
  const size_t MN = (size_t)M * N;
  const size_t n8 = (MN + 7) / 8;
  for (size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x; t < n8;
       t += (size_t)gridDim.x * blockDim.x) {
    const size_t idx = t * 8;
    const int row = (int)(idx / N), col = (int)(idx - (size_t)row * N);
    float v[8];
    int nv = 8;
    if (vec) {  // N % 8 == 0: the 8 elements are in one row
      float4_t a = {0.f, 0.f, 0.f, 0.f}, c = a;
      for (int s = 0; s < ksplit; ++s) {
        a += ((const float4_t *)(part + (size_t)s * MN + idx))[0];
        c += ((const float4_t *)(part + (size_t)s * MN + idx))[1];
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[4 + e] = c[e];
      }
    } else {
      nv = (int)min((size_t)8, MN - idx);
      for (int e = 0; e < 8; ++e) {
        v[e] = 0.f;
        if (e < nv)
          for (int s = 0; s < ksplit; ++s) v[e] += part[(size_t)s * MN + idx + e];
      }
    }
    if (vec) {
      if (bias)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int cc = col + e;
          if (bdt == SF_F32) v[e] += ((const float *)bias)[cc];
          else if (bdt == SF_F16) v[e] += (float)((const f16 *)bias)[cc];
          else v[e] += sf_bf16_to_f32(((const uint16_t *)bias)[cc]);
        }
      store_row8(v, 8, true, y32, Y, ydt, idx);
    } else {
      for (int e = 0; e < nv; ++e) {
        float o = v[e];
        const size_t id = idx + e;
        if (bias) {
          const int cc = (int)(id % N);
          if (bdt == SF_F32) o += ((const float *)bias)[cc];
          else if (bdt == SF_F16) o += (float)((const f16 *)bias)[cc];
          else o += sf_bf16_to_f32(((const uint16_t *)bias)[cc]);
        }
        if (y32) y32[id] = o;
        if (Y) {
          if (ydt == SF_BF16) ((uint16_t *)Y)[id] = sf_f32_to_bf16(o);
          else if (ydt == SF_F16) ((f16 *)Y)[id] = (f16)o;
          else ((float *)Y)[id] = o;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// LDS-streamed, wave-specialised GEMM: fp16 / bf16 activations, group sizes
// 32, 64 and multiples of 128
// ---------------------------------------------------------------------------
// The same 128 x 128 output tile on 512 threads, K steps of 64. Every operand
// byte is fetched once per workgroup, straight into LDS by buffer / global
// loads ... lds, one of four stages per step, three steps ahead:
//  * X: 16 fragments of 1 KB, each one MFMA's A operand in lane order (lane
//    l: row l % 32, k 8 (l / 32) .. + 7 of a 16-k slice); rows past M and k
//    past K read as zero.
//  * W: the tile's 8 units (16 columns x 128 k, 1 KB each, the blob's own
//    layout); the 8 codes of slice kk of a lane's column are one dword of the
//    column's unit lane (piece 2 (kk % 2) + l / 32, 32-k slice 2 (s % 2) +
//    kk / 2).
//  * the scale rows (16 cells of 8 fp16) and zero-point rows (16 cells of 8
//    nibbles) of the step's groups.
// The waves split by kind of work, two math waves and one convert wave per
// SIMD (waves w, w + 4 and w + 8 share one), so that MFMAs run beside the
// VALU work (with every wave doing both, the per-step barrier keeps the waves
// of a SIMD in the same phase and the two kinds of work take turns), and one
// math wave's MFMAs fill the other's waits on LDS and on its fold:
//  * waves 0..7 (math): rows 32 (w / 2) .. + 31 and columns 64 (w % 2) ..
//    + 63 as 1 x 2 v_mfma_f32_32x32x16 tiles; each group's fp32 partial is
//    folded into the result with its fp16 scale once per group (the
//    reference's grouping, q4_gemv.cpp:136);
//  * waves 8..11 (convert): during step s, wave 8 + c turns the codes of
//    column block c (32 columns) of step s + 1 into the exact integers q - z
//    as bf16 or fp16 MFMA B operands (lane order) in one of two LDS operand
//    buffers, which the math waves read in step s + 1.
// The math waves issue every load, in a fixed order per step: math wave w
// loads W unit w, then, for w < groups per step, that group's scale row or,
// with zero-points and groups per step <= w < 2 groups per step, zero-point
// row w - groups per step, then X fragments 4 (w / 2) + 2 (w % 2), + 1. At the
// top of step s a math wave waits (s_waitcnt vmcnt) until at most its X loads
// of step s + 1 and its loads of step s + 2 are outstanding: its X of step s
// and its W and scale / zero-point rows of step s + 1, which the convert
// waves read during step s, have landed. The convert waves issue nothing and
// only convert: with the W loads in the convert waves, each of them spent
// about a third of its step waiting to issue its loads behind the math
// waves' X loads (shader-clock stamps), and that wave set the step time;
// moving them measured 8% faster at config 2.
constexpr int G_BM = 128, G_BN = 128, G_BK = 64, G_STAGES = 4;
constexpr int G_MATH = 8, G_THREADS = (G_MATH + 4) * 64;  // math waves, then 4 convert waves
constexpr int G_XL = 16 / G_MATH;               // X fragments a math wave loads per step
constexpr int G_MR = 4 * 4 / G_MATH / 2;        // 32-row blocks per math wave (2 column blocks each)
constexpr int G_FRAG = 1024;                    // one A fragment (32 rows x 16 k)
constexpr int G_X_BYTES = 16 * G_FRAG;          // a step's X
constexpr int G_W_OFF = G_X_BYTES, G_W_BYTES = 8 * 1024;  // the tile's 8 units
constexpr int G_S_OFF = G_W_OFF + G_W_BYTES;    // scales: 1 KB per group of the step
template <int NG>
constexpr int g_z_off() { return G_S_OFF + NG * 1024; }   // zero-points: 256 B per group
template <int NG>
constexpr int g_stage_bytes() { return g_z_off<NG>() + NG * 256; }
// one step's B operands: 4 column blocks x 4 slices x 64 lanes x 16 B
constexpr int G_B_BYTES = 4 * 4 * 64 * 16;
template <int NG>
constexpr int g_lds_bytes() { return G_STAGES * g_stage_bytes<NG>() + 2 * G_B_BYTES; }

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void gbl_void;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Wait until at most n vector-memory operations of this wave are outstanding
// (gfx9 s_waitcnt: vmcnt in bits 3:0 and 15:14; exp and lgkm left at their maxima).
#define SF_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
// The workgroup barrier without __syncthreads' release fence, which would wait
// for every outstanding load (the loads into LDS count as writes); the asm
// clobber keeps the compiler from moving memory accesses across it. Ordering
// is explicit: SF_WAIT_VM before it for this wave's loads, and every LDS
// access of the previous step has completed (its result feeding an MFMA, a
// fold or a store) before the wave gets here.
#define SF_BARRIER()                   \
  do {                                 \
    asm volatile("" ::: "memory");     \
    __builtin_amdgcn_s_barrier();      \
    asm volatile("" ::: "memory");     \
  } while (0)

// One byte of v, sign-extended, to fp32 (an SDWA source select: the byte's
// extraction, sign extension and conversion in one instruction).
#define SF_SBYTE_F32(out, v, B)                                                                   \
  asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_" #B \
      : "=v"(out)                                                                              \
      : "v"(v))

// The bf16 B operand of 8 codes (one dword of a unit lane) as the exact
// integers code - z: the dword's nibble i is k element 2 i (i < 4) or
// 2 (i - 4) + 1, the pairs the GEMV's dequantization forms
// ((d >> 4 i) & 0x000F000F). The nibbles of each half go one per byte, and
// ((b ^ 0x80) - z) ^ 0x80 turns byte b into the two's complement int8 of
// b - z with no borrow between bytes (0x80 + b - z stays in 0x71..0x8F), so
// each byte converts to fp32 exactly in one instruction; code - z
// (|.| <= 15) is exact in bf16. 19 VALU instructions per 8 codes, against 28
// for the same values through per-nibble extracts, integer subtracts and
// conversions.
__device__ __forceinline__ u32x4 dequant_bf16_exact(uint32_t d, uint32_t z) {
  const uint32_t zz = z * 0x01010101u;
  const uint32_t e = (((d & 0x0F0F0F0Fu) ^ 0x80808080u) - zz) ^ 0x80808080u;         // nibbles 0,2,4,6
  const uint32_t o = ((((d >> 4) & 0x0F0F0F0Fu) ^ 0x80808080u) - zz) ^ 0x80808080u;  // nibbles 1,3,5,7
  float e0, e1, e2, e3, o0, o1, o2, o3;
  SF_SBYTE_F32(e0, e, 0);
  SF_SBYTE_F32(e1, e, 1);
  SF_SBYTE_F32(e2, e, 2);
  SF_SBYTE_F32(e3, e, 3);
  SF_SBYTE_F32(o0, o, 0);
  SF_SBYTE_F32(o1, o, 1);
  SF_SBYTE_F32(o2, o, 2);
  SF_SBYTE_F32(o3, o, 3);
  auto pk = [](float a, float b) {
    const float2_t f = {a, b};
    return sf_bitcast<uint32_t>(__builtin_convertvector(f, bf16x2_t));
  };
  return u32x4{pk(e0, e2), pk(o0, o2), pk(e1, e3), pk(o1, o3)};
}

template <int XDT, bool ASYM, int GK>
__global__ void __launch_bounds__(G_THREADS)
k_q4_gemm_ws(const uint8_t *__restrict__ wq, const f16 *__restrict__ st,
             const uint8_t *__restrict__ zt, const void *__restrict__ X, void *__restrict__ Y,
             int ydt, float *__restrict__ y32, const void *__restrict__ bias, int bdt,
             float *__restrict__ part, int M, int N, int K, int G, int g, int ksplit,
             int steps_per_split, bool vec) {
  static_assert(XDT == SF_F16 || XDT == SF_BF16, "fp16 / bf16 activations");
  constexpr bool BF = XDT == SF_BF16;
  constexpr int NG = GK == 0 ? 2 : 1;  // groups per step (g = 32: two)
  constexpr int SB = g_stage_bytes<NG>(), ZO = g_z_off<NG>();
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // stages, then 2 operand buffers
  uint8_t *const bops = smem + G_STAGES * SB;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool math = wave < G_MATH;
  const int cw = math ? wave : wave - G_MATH;       // index among the waves of its kind
  const int l32 = lane & 31, h = lane >> 5;
  const int m0 = blockIdx.y * G_BM, n0 = blockIdx.x * G_BN;
  const int split = blockIdx.z;
  const int nsteps_total = (K + G_BK - 1) / G_BK;
  const int s0 = split * steps_per_split;
  const int s1 = min(s0 + steps_per_split, nsteps_total);
  const int nblk = (K + 127) >> 7;
  const int ntiles = (N + 15) >> 4, ncells = (N + 7) >> 3;
  const int spg = GK == 2 ? g / G_BK : 1;  // steps per group

  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc((void *)X, 0, M * K * 2, 0x00020000);
  // math wave cw loads row block cw / 2's fragments G_XL (cw % 2) ..
  const int mrow = m0 + (cw >> 1) * 32 + l32;
  const bool mrow_ok = mrow < M;
  // a scale row (math waves 0 .. NG - 1) or a zero-point row (NG .. 2 NG - 1)
  const bool extra = math && (cw < NG || (ASYM && cw < 2 * NG));
  const int cell = min((n0 >> 3) + (lane & 15), ncells - 1);  // lanes 16.. repeat lane 15's row
  auto issue = [&](int step) {
    const int sc = min(step, s1 - 1);
    uint8_t *stage = smem + (step & 3) * SB;
    if (!math) return;
    {
      const int wtile = min((n0 >> 4) + cw, ntiles - 1);
      const uint8_t *unit = wq + ((size_t)wtile * nblk + (sc >> 1)) * 1024 + lane * 16;
      __builtin_amdgcn_global_load_lds((gbl_void *)unit, (lds_void *)(stage + G_W_OFF + cw * 1024), 16, 0, 0);
    }
    if (extra) {
      const int q = cw < NG ? cw : cw - NG;  // the group of the step whose row this wave loads
      const int gi = min(GK == 0 ? 2 * sc + q : GK == 1 ? sc : sc / spg, G - 1);
      const size_t c = (size_t)cell * G + gi;
      if (cw < NG)
        __builtin_amdgcn_global_load_lds((gbl_void *)(st + c * 8), (lds_void *)(stage + G_S_OFF + q * 1024),
                                         16, 0, 0);
      else
        __builtin_amdgcn_global_load_lds((gbl_void *)(zt + c * 4), (lds_void *)(stage + ZO + q * 256), 4, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < G_XL; ++i) {
      const int f = G_XL * (cw & 1) + i;
      const int k = sc * G_BK + f * 16 + 8 * h;
      // past the resource (reads zero) unless in range; a select, not a branch
      const uint32_t in = ((uint32_t)mrow * (uint32_t)K + (uint32_t)k) * 2u;
      const uint32_t keep = 0u - (uint32_t)(mrow_ok && k < K);
      const uint32_t off = (in & keep) | (0x80000000u & ~keep);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (lds_void *)(stage + (4 * (cw >> 1) + f) * G_FRAG), 16,
                                               off, 0, 0, 0);
    }
  };

  // ---- convert waves: step t's codes of column block cw into operand buffer t % 2
  const sf_gemv::DequantConsts dk;
  auto convert = [&](int t) {
    const uint8_t *stage = smem + (t & 3) * SB;
    uint8_t *bo = bops + (t & 1) * G_B_BYTES;
    const int n = min(n0 + 32 * cw + l32, N - 1);  // past N: column N - 1 (never stored)
    const int wl = G_W_OFF + ((n >> 4) - (n0 >> 4)) * 1024 + (h * 16 + (n & 15)) * 16 + (t & 1) * 8;
    const u32x2 lo = *(const u32x2 *)(stage + wl), hi = *(const u32x2 *)(stage + wl + 512);
    const uint32_t d[4] = {lo.x, hi.x, lo.y, hi.y};  // slices 0..3
    uint32_t z[NG];
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      if constexpr (ASYM)
        z[q] = (stage[ZO + q * 256 + ((n >> 3) - (n0 >> 3)) * 4 + ((n & 7) >> 1)] >> (4 * (n & 1))) & 15u;
      else
        z[q] = 8u;  // offset-binary symmetric codes
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint32_t zq = z[GK == 0 ? kk >> 1 : 0];
      const u32x4 b = BF ? dequant_bf16_exact(d[kk], zq) : sf_gemv::dequant_f16(d[kk], zq, dk);
      *(u32x4 *)(bo + (cw * 4 + kk) * 1024 + lane * 16) = b;
    }
  };

  // ---- math waves: row blocks G_MR (cw / 2) + r, column blocks 2 (cw % 2) + j
  const int rb0 = G_MR * (cw >> 1), cb0 = 2 * (cw & 1);
  const int wn = 32 * cb0;
  int s_lds[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = min(n0 + wn + 32 * j + l32, N - 1);
    s_lds[j] = G_S_OFF + ((n >> 3) - (n0 >> 3)) * 16 + (n & 7) * 2;
  }
  const float16_t zero16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f,
                            0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float16_t acc[G_MR][2], gp[G_MR][2];
#pragma unroll
  for (int r = 0; r < G_MR; ++r)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[r][j] = gp[r][j] = zero16;
  // the group's scale of the lane's columns
  auto scales = [&](const uint8_t *stage, int q, float (&sc)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) sc[j] = (float)*(const f16 *)(stage + s_lds[j] + q * 1024);
  };
  // acc += s * partial
  auto fold = [&](const float (&sc)[2]) {
#pragma unroll
    for (int r = 0; r < G_MR; ++r)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[r][j][e] = fmaf(gp[r][j][e], sc[j], acc[r][j][e]);
  };
  // a 16-k slice's operands, read one slice ahead of its MFMAs so that each
  // wait on LDS covers reads issued a slice earlier
  struct Ops {
    u32x4 a[G_MR], b[2];
  };
  auto ld = [&](const uint8_t *stage, const uint8_t *bo, int kk, Ops &o) {
#pragma unroll
    for (int r = 0; r < G_MR; ++r) o.a[r] = *(const u32x4 *)(stage + ((rb0 + r) * 4 + kk) * G_FRAG + lane * 16);
#pragma unroll
    for (int j = 0; j < 2; ++j) o.b[j] = *(const u32x4 *)(bo + ((cb0 + j) * 4 + kk) * 1024 + lane * 16);
  };
  // one 16-k slice's MFMAs (open: the slice starts its group)
  auto mm = [&](const Ops &o, bool open) {
#pragma unroll
    for (int r = 0; r < G_MR; ++r)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float16_t cin = open ? zero16 : gp[r][j];
        if constexpr (BF)
          gp[r][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(sf_bitcast<bf16x8_t>(o.a[r]),
                                                             sf_bitcast<bf16x8_t>(o.b[j]), cin, 0, 0, 0);
        else
          gp[r][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sf_bitcast<half8_t>(o.a[r]),
                                                            sf_bitcast<half8_t>(o.b[j]), cin, 0, 0, 0);
      }
  };
  // `iss` (the loads of a later step) runs after the second slice. A group
  // that ends with a step is folded at the top of the next one, while that
  // step's first operand reads are in flight (its partials are not written
  // again before the next step's first MFMAs; its scales are read at once,
  // before the stage can be refilled).
  float pend_s[2] = {0.f, 0.f};
  bool pending = false;
  auto math_step = [&](int step, auto &&iss) {
    const uint8_t *stage = smem + (step & 3) * SB;
    const uint8_t *bo = bops + (step & 1) * G_B_BYTES;
    Ops o0, o1;
    ld(stage, bo, 0, o0);
    ld(stage, bo, 1, o1);
    if (pending) fold(pend_s);
    pending = false;
    if constexpr (GK == 1) {
      mm(o0, true);
      ld(stage, bo, 2, o0);
      mm(o1, false);
      iss();
      ld(stage, bo, 3, o1);
      mm(o0, false);
      mm(o1, false);
      scales(stage, 0, pend_s);
      pending = true;
    } else if constexpr (GK == 0) {
      mm(o0, true);
      ld(stage, bo, 2, o0);
      mm(o1, false);
      iss();
      ld(stage, bo, 3, o1);
      float sa[2];
      scales(stage, 0, sa);
      fold(sa);
      mm(o0, true);
      mm(o1, false);
      scales(stage, 1, pend_s);
      pending = true;
    } else {
      const bool fresh = step % spg == 0 || step == s0;
      const bool last = (step + 1) % spg == 0 || step == s1 - 1;
      if (fresh) mm(o0, true);
      else mm(o0, false);
      ld(stage, bo, 2, o0);
      mm(o1, false);
      iss();
      ld(stage, bo, 3, o1);
      mm(o0, false);
      mm(o1, false);
      if (last) {
        scales(stage, 0, pend_s);
        pending = true;
      }
    }
  };

  // Pipeline. Loads of step s go out during step s - 3 (the first three in
  // the prologue) into the stage step s - 4 used; after the barrier at the top
  // of step s every wave is done with step s - 1's stage and operand buffer
  // (s + 1) % 2, the X of step s and the W, scale and zero-point rows of step
  // s + 1 have landed, and operand buffer s % 2 holds step s's operands.
  // Nothing the compiler loads into registers goes to global memory inside
  // the loop, so these loads are the only vector-memory counts. A math wave
  // issues L = 1 + extra + G_XL loads per step.
  if (s0 < s1) {
    issue(s0);
    issue(s0 + 1);
    issue(s0 + 2);
    if (math) {  // W and the scale / zero-point row of step s0 (its X and two later steps' may remain)
      if (extra) SF_WAIT_VM(G_XL + 2 * (G_XL + 2));
      else SF_WAIT_VM(G_XL + 2 * (G_XL + 1));
    }
    SF_BARRIER();
    if (!math) convert(s0);
    for (int s = s0; s < s1; s += 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int step = s + u;
        if (step >= s1) break;
        if (math) {  // X of step s, W and rows of step s + 1 (X of s + 1 and step s + 2's may remain)
          if (extra) SF_WAIT_VM(G_XL + G_XL + 2);
          else SF_WAIT_VM(G_XL + G_XL + 1);
        }
        SF_BARRIER();
        if (math) {
          math_step(step, [&] { issue(step + 3); });
        } else {
          if (step + 1 < s1) convert(step + 1);
        }
      }
    }
  }

  // Output: every wave done with the stages and every load landed, then each
  // math wave stages its tile one 32-row block at a time in its own LDS region
  // and writes it back as 8-column row segments (16-byte stores). 16-bit
  // outputs without split or fp32 copy round in registers (bias added first)
  // and stage 16-bit values; the rest stage fp32 values, one 32-column block
  // at a time.
  if (math && pending) fold(pend_s);  // the last group's fold
  SF_WAIT_VM(0);
  __syncthreads();
  if (!math) return;
#pragma unroll
  for (int r = 0; r < G_MR; ++r) {
    const int wm = 32 * (rb0 + r);
    if (ksplit == 1 && !y32 && Y && vec && (ydt == SF_BF16 || ydt == SF_F16)) {
      constexpr int P16 = 64 + 8;  // halfword pitch of a staged row
      uint16_t *ot16 = (uint16_t *)smem + cw * 32 * P16;
      float bc[2] = {0.f, 0.f};
      if (bias) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int cc = min(n0 + wn + 32 * j + l32, N - 1);
          bc[j] = bdt == SF_F32 ? ((const float *)bias)[cc]
                  : bdt == SF_F16 ? (float)((const f16 *)bias)[cc]
                                  : sf_bf16_to_f32(((const uint16_t *)bias)[cc]);
        }
      }
      const bool obf = ydt == SF_BF16;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float v = acc[r][j][e] + bc[j];
          ot16[(8 * (e >> 2) + 4 * h + (e & 3)) * P16 + 32 * j + l32] =
              obf ? sf_f32_to_bf16(v) : sf_bitcast<uint16_t>((f16)v);
        }
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int seg = it * 64 + lane;
        const int rl = seg >> 3, cl = (seg & 7) * 8;
        const int row = m0 + wm + rl, col = n0 + wn + cl;
        const u32x4 w8 = *(const u32x4 *)(ot16 + rl * P16 + cl);
        if (row >= M || col >= N) continue;
        uint16_t *d = (uint16_t *)Y + (size_t)row * N + col;
        if (col + 8 <= N) {
          *(u32x4 *)d = w8;
        } else {
          for (int e = 0; e < N - col; ++e) d[e] = (uint16_t)(w8[e >> 1] >> (16 * (e & 1)));
        }
      }
      continue;
    }
    constexpr int P32 = 32 + 4;  // fp32 pitch of a staged 32-column block
    float *ot = (float *)smem + cw * 32 * P32;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int e = 0; e < 16; ++e) ot[(8 * (e >> 2) + 4 * h + (e & 3)) * P32 + l32] = acc[r][j][e];
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int seg = it * 64 + lane;
        const int rl = seg >> 2, cl = (seg & 3) * 8;
        const int row = m0 + wm + rl, col = n0 + wn + 32 * j + cl;
        float v[8];
        {
          const float4_t x0 = *(const float4_t *)(ot + rl * P32 + cl);
          const float4_t x1 = *(const float4_t *)(ot + rl * P32 + cl + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = x0[e];
            v[4 + e] = x1[e];
          }
        }
        if (row >= M || col >= N) continue;
        const int nv = min(8, N - col);
        const size_t idx = (size_t)row * N + col;
        if (ksplit > 1) {
          float *dst = part + (size_t)split * M * N + idx;
          if (vec && nv == 8) {
            ((float4_t *)dst)[0] = float4_t{v[0], v[1], v[2], v[3]};
            ((float4_t *)dst)[1] = float4_t{v[4], v[5], v[6], v[7]};
          } else {
            for (int e = 0; e < nv; ++e) dst[e] = v[e];
          }
          continue;
        }
        if (bias) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int cc = min(col + e, N - 1);
            if (bdt == SF_F32) v[e] += ((const float *)bias)[cc];
            else if (bdt == SF_F16) v[e] += (float)((const f16 *)bias)[cc];
            else v[e] += sf_bf16_to_f32(((const uint16_t *)bias)[cc]);
          }
        }
        store_row8(v, nv, vec, y32, Y, ydt, idx);
      }
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

int sf_q4_anyg(const void *blob, const void *x, int x_dtype, void *y, int y_dtype, float *y_f32,
               const void *bias, int bias_dtype, int M, int N, int K, int g, int has_zeros, void *stream);

extern "C" size_t sf_q4_gemm_workspace_bytes(int M, int N, int K, int group_size) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0 || group_size % 32) return 0;
  const int s = choose_ksplit(M, N, K);
  return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

// The GEMM launch; `partials` leaves a split shape's K-split partials in the
// workspace (no reduce launch, no output) for a consumer that sums them in
// split order itself.
static int q4_gemm_impl(const void *blob, const void *x, int x_dtype, void *y, int y_dtype,
                        float *y_f32, const void *bias, int bias_dtype, int M, int N, int K,
                        int group_size, int has_zeros, void *workspace, size_t workspace_bytes,
                        void *stream, bool partials) {
  SF_REQUIRE(M > 0 && N > 0 && K > 0 && group_size > 0, SF_EINVAL,
             "invalid shape M=%d N=%d K=%d group_size=%d", M, N, K, group_size);
  SF_REQUIRE(K % group_size == 0, SF_EINVAL, "in_features must be divisible by group_size");
  SF_REQUIRE(blob && x && (partials || y || y_f32), SF_EINVAL, "null pointer argument");
  SF_REQUIRE(x_dtype == SF_F16 || x_dtype == SF_BF16 || x_dtype == SF_F32, SF_EINVAL,
             "bad activation dtype %d", x_dtype);
  SF_REQUIRE(y_dtype == SF_F16 || y_dtype == SF_BF16 || y_dtype == SF_F32, SF_EINVAL,
             "bad output dtype %d", y_dtype);
  SF_REQUIRE(!bias || bias_dtype == SF_F16 || bias_dtype == SF_BF16 || bias_dtype == SF_F32,
             SF_EINVAL, "bad bias dtype %d", bias_dtype);
  SF_REQUIRE(((uintptr_t)blob & 255) == 0 && ((uintptr_t)x & 15) == 0, SF_EINVAL,
             "blob must be 256-byte aligned and X 16-byte aligned");
  if (group_size % 32)  // a group boundary inside an MFMA's k: the any-group-size kernel
    return sf_q4_anyg(blob, x, x_dtype, y, y_dtype, y_f32, bias, bias_dtype, M, N, K, group_size,
                      has_zeros, stream);
  // Up to 16 rows: batch GEMVs of 8 rows (the reference's GEMM is a loop of
  // GEMVs too). A tile kernel's K loop costs the same per step for 9 rows as
  // for 128, and two GEMV launches measured 30-40% faster at 9-16 rows on
  // 4864 x 896, 896 x 4864, 4096 x 4096 and 11008 x 4096 (even at 24 rows,
  // the tile kernel ahead from 32). y_f32 passed as the bias too is the
  // GEMV's per-row residual form, not a per-column bias: such a call stays here.
  if (!partials && M <= kGemmGemvRows && !(bias && bias == (const void *)y_f32)) {
    sf_gemv::BlkPlan p;
    if (sf_gemv::plan_blk(M < 8 ? M : 8, N, K, group_size, x_dtype, sf_gemv::PRE_NONE, false, &p)) {
      const size_t xsz = x_dtype == SF_F32 ? 4 : 2, ysz = y_dtype == SF_F32 ? 4 : 2;
      for (int m0 = 0; m0 < M; m0 += 8) {
        const int mb = M - m0 < 8 ? M - m0 : 8;
        const int rc = sf_q4_gemv(blob, (const char *)x + (size_t)m0 * K * xsz, x_dtype,
                                  y ? (char *)y + (size_t)m0 * N * ysz : nullptr, y_dtype,
                                  y_f32 ? y_f32 + (size_t)m0 * N : nullptr, bias, bias_dtype, mb, N,
                                  K, group_size, has_zeros, stream);
        if (rc) return rc;
      }
      return SF_OK;
    }
  }
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
  // 16-byte output stores need rows of whole 16-byte multiples and aligned bases
  const bool vec = N % 8 == 0 && ((uintptr_t)y & 15) == 0 && ((uintptr_t)y_f32 & 15) == 0 &&
                   ((uintptr_t)part & 15) == 0;
  // W-direct kernel: fp16 / bf16 activations, groups of 32, 64 or a multiple of
  // 128, X within a buffer resource's 2 GB range
  const char *wd_env = getenv("SF_GEMM_WDIRECT");
  const bool wdirect = !(wd_env && wd_env[0] == '0') && x_dtype != SF_F32 &&
                       (group_size == 32 || group_size == 64 || group_size % 128 == 0) &&
                       (size_t)M * K * 2 <= 0x7FFFFFFFu;
  if (wdirect) {
    static_assert(G_BM == BM && G_BN == BN && G_BK == BK, "one tiling: one split choice");
#define SF_GW_LAUNCH(XD, AS, GKV)                                                              \
  do {                                                                                       \
    constexpr size_t lds = (size_t)g_lds_bytes<GKV == 0 ? 2 : 1>();                         \
    static bool attr = false; /* raise the dynamic LDS limit once per variant */             \
    if (!attr) {                                                                             \
      (void)hipFuncSetAttribute((const void *)k_q4_gemm_ws<XD, AS, GKV>,                     \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);       \
      attr = true;                                                                           \
    }                                                                                        \
    k_q4_gemm_ws<XD, AS, GKV><<<grid, G_THREADS, lds, s>>>(w, st, zt, x, y, y_dtype, y_f32,  \
                                                          bias, bias_dtype, part, M, N, K,   \
                                                          L.G, group_size, ksplit,            \
                                                          steps_per_split, vec);              \
  } while (0)
#define SF_GW_G(XD, AS)                                  \
  do {                                                   \
    if (group_size == 32) SF_GW_LAUNCH(XD, AS, 0);       \
    else if (group_size == 64) SF_GW_LAUNCH(XD, AS, 1);  \
    else SF_GW_LAUNCH(XD, AS, 2);                        \
  } while (0)
    if (x_dtype == SF_BF16) {
      if (has_zeros) SF_GW_G(SF_BF16, true);
      else SF_GW_G(SF_BF16, false);
    } else {
      if (has_zeros) SF_GW_G(SF_F16, true);
      else SF_GW_G(SF_F16, false);
    }
#undef SF_GW_G
#undef SF_GW_LAUNCH
  } else {
#define SF_GEMM_LAUNCH(XD, AS)                                                               \
  do {                                                                                       \
    if (group_size == 32)                                                                    \
      k_q4_gemm<XD, AS, 0><<<grid, NTHREADS, 0, s>>>(w, st, zt, x, y, y_dtype, y_f32, bias,  \
                                                     bias_dtype, part, M, N, K, L.G,         \
                                                     group_size, ksplit, steps_per_split, vec); \
    else if (group_size == 64)                                                               \
      k_q4_gemm<XD, AS, 1><<<grid, NTHREADS, 0, s>>>(w, st, zt, x, y, y_dtype, y_f32, bias,  \
                                                     bias_dtype, part, M, N, K, L.G,         \
                                                     group_size, ksplit, steps_per_split, vec); \
    else if (group_size % 64)                                                                \
      k_q4_gemm<XD, AS, 3><<<grid, NTHREADS, 0, s>>>(w, st, zt, x, y, y_dtype, y_f32, bias,  \
                                                     bias_dtype, part, M, N, K, L.G,         \
                                                     group_size, ksplit, steps_per_split, vec); \
    else                                                                                     \
      k_q4_gemm<XD, AS, 2><<<grid, NTHREADS, 0, s>>>(w, st, zt, x, y, y_dtype, y_f32, bias,  \
                                                     bias_dtype, part, M, N, K, L.G,         \
                                                     group_size, ksplit, steps_per_split, vec); \
  } while (0)
#define SF_GEMM_X(AS)                                  \
  do {                                                 \
    if (x_dtype == SF_BF16) SF_GEMM_LAUNCH(SF_BF16, AS); \
    else if (x_dtype == SF_F16) SF_GEMM_LAUNCH(SF_F16, AS); \
    else SF_GEMM_LAUNCH(SF_F32, AS);                   \
  } while (0)
  if (has_zeros) SF_GEMM_X(true);
  else SF_GEMM_X(false);
#undef SF_GEMM_X
#undef SF_GEMM_LAUNCH
  }
  int rc = sf_check_launch(partials ? "sf_q4_gemm_partials" : "sf_q4_gemm");
  if (rc || ksplit == 1 || partials) return rc;
  const size_t n8 = ((size_t)M * N + 7) / 8;
  unsigned rg = (unsigned)((n8 + 255) / 256);
  if (rg > 65535u * 16u) rg = 65535u * 16u;
  k_splitk_reduce<<<rg, 256, 0, s>>>(part, y, y_dtype, y_f32, bias, bias_dtype, M, N, ksplit, vec);
  return sf_check_launch("sf_q4_gemm(reduce)");
}

extern "C" int sf_q4_gemm(const void *blob, const void *x, int x_dtype, void *y, int y_dtype,
                          float *y_f32, const void *bias, int bias_dtype, int M, int N, int K,
                          int group_size, int has_zeros, void *workspace, size_t workspace_bytes,
                          void *stream) {
  return q4_gemm_impl(blob, x, x_dtype, y, y_dtype, y_f32, bias, bias_dtype, M, N, K, group_size,
                      has_zeros, workspace, workspace_bytes, stream, false);
}

extern "C" int sf_q4_gemm_splits(int M, int N, int K, int group_size) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0 || K % group_size || group_size % 32) return 0;
  return choose_ksplit(M, N, K);
}

extern "C" int sf_q4_gemm_partials(const void *blob, const void *x, int x_dtype, int M, int N,
                                   int K, int group_size, int has_zeros, void *workspace,
                                   size_t workspace_bytes, void *stream) {
  const int s = sf_q4_gemm_splits(M, N, K, group_size);
  SF_REQUIRE(s > 1, SF_EINVAL,
             "sf_q4_gemm_partials: M=%d N=%d K=%d group_size=%d runs unsplit (use sf_q4_gemm)", M,
             N, K, group_size);
  return q4_gemm_impl(blob, x, x_dtype, nullptr, SF_F32, nullptr, nullptr, SF_F32, M, N, K,
                      group_size, has_zeros, workspace, workspace_bytes, stream, true);
}
