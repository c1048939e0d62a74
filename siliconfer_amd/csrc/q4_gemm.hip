// q4_gemm.hip — int4 prefill GEMM on CDNA4 MFMA (gfx950).
//
// Y[m, n] = sum_k X[m, k] * (q[n,k] - z[n,g(k)]) * s[n,g(k)], fp32 accumulation:
// the reference's q4_gemm_sym / q4_gemm_asym
// (/root/reference/siliconfer/kernels/neon/q4_gemm.cpp:12-51), which loop the
// GEMV over the T rows and re-stream W for each; here W is read once per
// 128-row block of X.
//
// Exact products, scale per group: the workgroup dequantizes its W tile once
// into LDS as the integers q - z (|q - z| <= 15, exact in fp16 and in bf16)
// and every wave runs one MFMA per product on them — v_mfma_f32_32x32x16_f16
// for fp16 activations, _bf16 for bf16 ones (fp32 activations are split into
// bf16 high and low parts, two MFMAs) — accumulating each scale group's
// partial in fp32 and folding it into the result with the group's fp16 scale,
// once per group: y = sum_g s_g * sum_{k in g} x_k (q_k - z), the reference's
// own grouping (q4_gemv.cpp:136). Each staging thread writes its row's scale
// into a small LDS table beside the W tile; a lane reads its column's.
//
// Tiling: 128 x 128 output tile per 512-thread workgroup (2 x 4 waves, each
// 64 x 32 = 2 MFMA 32x32 tiles; two waves per SIMD), K steps of 64 staged
// through two padded LDS buffers (74 KB); each
// step's global loads are issued three steps ahead (a ring of three register
// stages) so HBM latency hides behind the MFMAs. The output tile goes back
// through LDS so that stores are whole row segments. When the tile grid is
// too small to fill the GPU, K is split across workgroups into an fp32
// workspace and summed by a second kernel in a fixed order.
#include "sf_common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
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

extern "C" int sf_q4_gemm(const void *blob, const void *x, int x_dtype, void *y, int y_dtype,
                          float *y_f32, const void *bias, int bias_dtype, int M, int N, int K,
                          int group_size, int has_zeros, void *workspace, size_t workspace_bytes,
                          void *stream) {
  SF_REQUIRE(M > 0 && N > 0 && K > 0 && group_size > 0, SF_EINVAL,
             "invalid shape M=%d N=%d K=%d group_size=%d", M, N, K, group_size);
  SF_REQUIRE(K % group_size == 0, SF_EINVAL, "in_features must be divisible by group_size");
  SF_REQUIRE(blob && x && (y || y_f32), SF_EINVAL, "null pointer argument");
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
  int rc = sf_check_launch("sf_q4_gemm");
  if (rc || ksplit == 1) return rc;
  const size_t n8 = ((size_t)M * N + 7) / 8;
  unsigned rg = (unsigned)((n8 + 255) / 256);
  if (rg > 65535u * 16u) rg = 65535u * 16u;
  k_splitk_reduce<<<rg, 256, 0, s>>>(part, y, y_dtype, y_f32, bias, bias_dtype, M, N, ksplit, vec);
  return sf_check_launch("sf_q4_gemm(reduce)");
}
