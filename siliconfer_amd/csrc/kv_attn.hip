// kv_attn.hip — int8 KV cache append and split-T decode attention (gfx950).
//
// sf_kv_quant_append: per (b, head, t) vector of D values,
//   s = max|x| / 127 (1 if max|x| == 0), code = clip(rint(x / s), -128, 127),
// in fp32 with correctly rounded division — the reference's quantize_kv
// (/root/reference/siliconfer/model/kv_cache.py:49-63) — written straight into
// a preallocated cache at its current length instead of the reference's
// per-step concatenation (kv_cache.py:99-102).
//
// sf_attn_decode_i8kv: one query token per (b, h) against T cached tokens,
// the reference's fused_quantized_attention_decode
// (/root/reference/siliconfer/kernels/metal/q4_attention.py:80-261):
//  * split-T: tile = ceil(T / n_splits) tokens per split, the reference's
//    tiling (q4_attention.py:231-234), so n_splits plays the role of n_tiles;
//  * one workgroup per (split, kv head, head block, b) serves ALL the query
//    heads that share the kv head (GQA) from one read of the K/V codes — the
//    reference's kernel re-reads each kv head once per query head (:103);
//  * inside a split, lanes are (token, 8-dim octet) with all query heads of
//    the block in registers; each lane keeps its own online softmax (in base
//    2, scores pre-scaled by log2 e) over its tokens, loading K and V codes
//    with 8-byte loads a batch ahead; the lane states are merged through LDS;
//  * the split partials (m, l, acc[D]) go to a workspace and a second,
//    small launch merges them with the reference's combine rule
//    (q4_attention.py:63-70, 256-261; split_merge.h), one lane per output
//    element; the decoder instead folds that merge into its o-projection
//    GEMV (sf_q4_gemv_attn_merge). A single split writes the output directly.
#include <math.h>
#include <stdlib.h>

#include <mutex>

#include "sf_common.h"
#include "split_merge.h"

namespace {

constexpr int kAttnThreads = 256;

// ---------------------------------------------------------------------------
// KV quantize + append
// ---------------------------------------------------------------------------
template <int IDT, int SDT>
__global__ void __launch_bounds__(256)
k_kv_quant_append(const void *__restrict__ k_new, const void *__restrict__ v_new,
                  int8_t *__restrict__ k_codes, void *__restrict__ k_scales,
                  int8_t *__restrict__ v_codes, void *__restrict__ v_scales, int KVH, int T_new,
                  int T_off, int T_cap, int D, int tpv_log2, long long n_vec) {
  // tpv = threads per vector (power of two), each thread handles 8 values
  const int tpv = 1 << tpv_log2;
  const long long gid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long vec = gid >> tpv_log2;  // over 2 * B * KVH * T_new (K then V)
  const int sl = (int)(gid & (tpv - 1));
  const bool live = vec < n_vec;
  const long long half = n_vec >> 1;
  const bool is_v = live && vec >= half;
  const long long vi = is_v ? vec - half : vec;
  const void *src = is_v ? v_new : k_new;
  const int t = live ? (int)(vi % T_new) : 0;
  const long long bh = live ? vi / T_new : 0;  // b * KVH + h
  const int d0 = sl * 8;
  float xv[8];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    xv[i] = 0.f;
    if (live && d0 + i < D) xv[i] = sf_load_as_f32<IDT>(src, (size_t)vi * D + d0 + i);
    amax = fmaxf(amax, fabsf(xv[i]));
  }
  for (int off = tpv >> 1; off >= 1; off >>= 1) amax = fmaxf(amax, sf_shfl_xor(amax, off));
  if (!live) return;
  const float s = amax == 0.f ? 1.f : amax / 127.f;
  const size_t row = (size_t)bh * T_cap + (size_t)(T_off + t);
  int8_t *dst = (is_v ? v_codes : k_codes) + row * D;
  union {
    int8_t c[8];
    uint64_t u;
  } pk;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float qv = __builtin_rintf(xv[i] / s);
    qv = fminf(fmaxf(qv, -128.f), 127.f);
    pk.c[i] = (int8_t)(int)qv;
  }
  if (d0 + 8 <= D) {
    *(uint64_t *)(dst + d0) = pk.u;
  } else {
    for (int i = 0; d0 + i < D; ++i) dst[d0 + i] = pk.c[i];
  }
  if (sl == 0) sf_store_from_f32<SDT>(is_v ? v_scales : k_scales, row, s);
}

// ---------------------------------------------------------------------------
// split-T decode attention
// ---------------------------------------------------------------------------
constexpr int kMaxD = 256;
constexpr int kMaxSplits = 512;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr int kAttnBatch = 4;  // rows per lane per load batch

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return sf_bitcast<float>(__builtin_amdgcn_update_dpp(0, sf_bitcast<int>(v), CTRL, 0xF, 0xF, false));
}

// v + value of the lane at distance `off` in an aligned group of 2*off lanes
// (DPP for off <= 8; the mirror patterns pair a lane with one of the other
// half, and by symmetry every lane of the group ends with the full sum).
__device__ __forceinline__ float add_partner(float v, int off) {
  switch (off) {
    case 1: return v + dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
    case 2: return v + dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
    case 4: return v + dpp_f<0x141>(v);   // row_half_mirror
    case 8: return v + dpp_f<0x140>(v);   // row_mirror
    default: return v + __shfl_xor(v, off, 64);
  }
}

__device__ __forceinline__ float max_partner(float v, int off) {
  switch (off) {
    case 1: return fmaxf(v, dpp_f<0xB1>(v));
    case 2: return fmaxf(v, dpp_f<0x4E>(v));
    case 4: return fmaxf(v, dpp_f<0x141>(v));
    case 8: return fmaxf(v, dpp_f<0x140>(v));
    default: return fmaxf(v, __shfl_xor(v, off, 64));
  }
}

// max / sum over aligned groups of 32 lanes; every lane gets the result
__device__ __forceinline__ float group32_max(float v) {
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) v = max_partner(v, off);
  return v;
}
__device__ __forceinline__ float group32_sum(float v) {
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) v = add_partner(v, off);
  return v;
}

__device__ __forceinline__ void i8x8_to_f32(u32x2 c, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = (float)(int8_t)(c.x >> (8 * i));
    f[4 + i] = (float)(int8_t)(c.y >> (8 * i));
  }
}

template <int HB>
constexpr int attn_smem_floats() {
  // acc [NS][HB][D] (NS * D <= 2048 per head), m and l [NS][HB] (NS <= 256),
  // M and L [HB]
  return 2048 * HB + 2 * 256 * HB + 2 * HB;
}

// One workgroup per (split, kv head, block of HB query heads, batch row); the
// split covers `tile` tokens. Lanes are (token, 8-dim octet): OCT lanes hold
// one token's K and V codes (an 8-byte load each), so each code is converted
// once for all HB heads of the block, whose q octets (pre-scaled by
// scale * log2 e) sit in registers. A row is the 64 / OCT tokens one load
// instruction covers; wave w walks rows w, w + 4, ... in batches of
// kAttnBatch rows with the next batch's loads in flight, and each lane keeps
// its own online-softmax state per head (m, l, acc[8]) with no block-level
// synchronisation. At the end the NS = 4 * 64 / OCT lane states of each head
// are merged through LDS into the split's partial; with one split it is the
// output, otherwise the partial of the split (merged by a later launch).
template <int QDT, int SDT, int HB>
__global__ void __launch_bounds__(kAttnThreads)
k_attn_decode(const void *__restrict__ q, const int8_t *__restrict__ kc,
              const void *__restrict__ ks, const int8_t *__restrict__ vc,
              const void *__restrict__ vs, float *part_acc, float *part_ml,
              void *__restrict__ out, int odt, int H, int KVH, int T, const int *__restrict__ T_dev,
              int causal, int T_cap, int D, float qscale, int n_splits, int oct_log2) {
  constexpr int NT = kAttnThreads, NW = kAttnWaves, U = kAttnBatch;
  __shared__ __attribute__((aligned(16))) float smem[attn_smem_floats<HB>()];

  const int OCT = 1 << oct_log2;  // lanes per token
  const int R = 64 >> oct_log2;   // tokens per row
  const int NS = NW * R;          // lane states per head in the workgroup

  const int split = blockIdx.x;
  const int G = H / KVH;
  const int n_hblk = (G + HB - 1) / HB;
  const int kvh = blockIdx.y / n_hblk;
  const int hblk = blockIdx.y - kvh * n_hblk;
  const int nh = min(HB, G - hblk * HB);
  const int b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int oct = lane & (OCT - 1);
  const int grp = lane >> oct_log2;
  const int slot = wave * R + grp;
  const int d0 = oct * 8;
  const bool dact = d0 < D;
  const int dq = dact ? d0 : 0;
  // Length: the host's T, or a device length plus T (decode steps replayed
  // from a graph), or for a causal prefill T0 tokens before query row b plus
  // the row itself (T0 = the host's T, or the device length); the cache then
  // has batch 1.
  int Tv = T_dev ? *T_dev + T : T;
  if (causal) Tv = (T_dev ? *T_dev : T) + b + 1;
  Tv = max(0, min(Tv, T_cap));
  const int tile = (Tv + n_splits - 1) / n_splits;
  const int t0 = split * tile, t1 = min(t0 + tile, Tv);
  const size_t base = ((size_t)(causal ? 0 : b) * KVH + kvh) * (size_t)T_cap;
  const size_t bh0 = (size_t)b * H + (size_t)kvh * G + (size_t)hblk * HB;

  float qr[HB][8];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    sf_load8_as_f32<QDT>(q, (bh0 + min(h, nh - 1)) * D + dq, qr[h]);
#pragma unroll
    for (int i = 0; i < 8; ++i) qr[h][i] = (h < nh && dact) ? qr[h][i] * qscale : 0.f;
  }

  float m[HB], l[HB], acc[HB][8];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.f;
  }

  struct Batch {
    u32x2 k[U], v[U];
    float ks[U], vs[U];
  };
  // row step k of this wave covers tokens t0 + (wave + NW k) R + [0, R)
  const int nrows = (t1 - t0 + R - 1) / R;
  const int nsteps = (nrows + NW - 1) / NW;
  auto token = [&](int k) { return t0 + (wave + NW * k) * R + grp; };
  auto load = [&](int k0, Batch &bt) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = min(token(k0 + u), t1 - 1);  // past the end: re-read, masked
      const size_t row = base + t;
      bt.k[u] = *(const u32x2 *)(kc + row * D + dq);
      bt.v[u] = *(const u32x2 *)(vc + row * D + dq);
      bt.ks[u] = sf_load_as_f32<SDT>(ks, row);
      bt.vs[u] = sf_load_as_f32<SDT>(vs, row);
    }
  };
  auto compute = [&](int k0, const Batch &bt) {
    float s[U][HB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float kf[8];
      i8x8_to_f32(bt.k[u], kf);
#pragma unroll
      for (int h = 0; h < HB; ++h) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) a = fmaf(qr[h][i], kf[i], a);
        s[u][h] = a;
      }
    }
    // sum over the OCT lanes of the token (uniform branches on OCT)
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1)
      if (OCT > off)
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int h = 0; h < HB; ++h) s[u][h] = add_partner(s[u][h], off);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool valid = token(k0 + u) < t1;
#pragma unroll
      for (int h = 0; h < HB; ++h) s[u][h] = valid ? s[u][h] * bt.ks[u] : -INFINITY;
    }
    float m_ref[HB];
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      float mx = s[0][h];
#pragma unroll
      for (int u = 1; u < U; ++u) mx = fmaxf(mx, s[u][h]);
      const float m_new = fmaxf(m[h], mx);
      m_ref[h] = m_new == -INFINITY ? 0.f : m_new;
      const float c = __builtin_amdgcn_exp2f(m[h] - m_ref[h]);  // exp2(-inf) = 0
      l[h] *= c;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] *= c;
      m[h] = m_new;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float vf[8];
      i8x8_to_f32(bt.v[u], vf);
#pragma unroll
      for (int h = 0; h < HB; ++h) {
        const float p = __builtin_amdgcn_exp2f(s[u][h] - m_ref[h]);
        l[h] += p;
        const float pv = p * bt.vs[u];  // the V scale folded into P
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(pv, vf[i], acc[h][i]);
      }
    }
  };

  if (nsteps > 0) {
    // loads are unconditional (past the end they re-read the last token) so
    // the next batch stays in flight while the current one is computed
    Batch b0, b1;
    load(0, b0);
    for (int k0 = 0; k0 < nsteps; k0 += 2 * U) {
      load(k0 + U, b1);
      compute(k0, b0);
      if (k0 + U >= nsteps) break;
      load(k0 + 2 * U, b0);
      compute(k0 + U, b1);
    }
  }

  // ---- merge the NS lane states of each head (LDS)
  float *accs = smem;               // [NS][HB][D]
  float *ms = accs + NS * HB * D;   // [NS][HB]: m, then the state weights
  float *ls = ms + NS * HB;         // [NS][HB]
  float *Ms = ls + NS * HB, *Ls = Ms + HB;
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    if (h < nh && dact) {
      float4_t *dst = (float4_t *)(accs + ((size_t)slot * HB + h) * D + d0);
      dst[0] = float4_t{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
      dst[1] = float4_t{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
    }
    if (h < nh && oct == 0) {
      ms[slot * HB + h] = m[h];
      ls[slot * HB + h] = l[h];
    }
  }
  __syncthreads();
  // state weights: 32 lanes per head, lane j covering states j, j + 32, ...
  {
    const int h = tid >> 5, j = tid & 31;
    const bool on = h < nh;
    float mx = -INFINITY;
    if (on)
      for (int s = j; s < NS; s += 32) mx = fmaxf(mx, ms[s * HB + h]);
    const float M = group32_max(mx);
    const float M_ref = M == -INFINITY ? 0.f : M;
    float lsum = 0.f;
    if (on)
      for (int s = j; s < NS; s += 32) {
        const float w = __builtin_amdgcn_exp2f(ms[s * HB + h] - M_ref);
        ms[s * HB + h] = w;
        lsum = fmaf(w, ls[s * HB + h], lsum);
      }
    lsum = group32_sum(lsum);
    if (on && j == 0) {
      Ms[h] = M;
      Ls[h] = lsum;
    }
  }
  __syncthreads();
  const bool single = n_splits == 1;
  const int nq = D >> 2;
  for (int it = tid; it < nh * nq; it += NT) {
    const int h = it / nq, dq4 = (it - h * nq) * 4;
    float4_t a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0;
#pragma unroll 4
    for (int s = 0; s < NS; s += 2) {  // NS is a multiple of 4
      a0 += *(const float4_t *)(accs + ((size_t)s * HB + h) * D + dq4) * ms[s * HB + h];
      a1 += *(const float4_t *)(accs + ((size_t)(s + 1) * HB + h) * D + dq4) * ms[(s + 1) * HB + h];
    }
    const float4_t a = a0 + a1;
    if (single) {
      const float L = Ls[h];
      const float inv = L > 0.f ? 1.f / L : 0.f;
      const size_t o = (bh0 + h) * D + dq4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = a[i] * inv;
        if (odt == SF_F32) ((float *)out)[o + i] = v;
        else if (odt == SF_F16) ((f16 *)out)[o + i] = (f16)v;
        else ((uint16_t *)out)[o + i] = sf_f32_to_bf16(v);
      }
    } else {
      *(float4_t *)(part_acc + ((bh0 + h) * n_splits + split) * D + dq4) = a;
    }
  }
  if (!single && tid < nh)
    *(float2_t *)(part_ml + ((bh0 + tid) * n_splits + split) * 2) = float2_t{Ms[tid], Ls[tid]};
}

// ---------------------------------------------------------------------------
// MFMA decode attention: G <= 16 query heads per kv head, D = 64 or 128
// ---------------------------------------------------------------------------
// Per wave, 32-token tiles of one split (tile j of the split goes to wave
// j % 4). q . K^T and P V run as v_mfma_f32_16x16x32_f16 with the heads on the
// 16-wide N side (rows >= G are zero queries whose outputs are dropped):
//  * S^T = K q^T: A = the K codes of 16 tokens (lane l: token l % 16, dims
//    D/4 (l / 16) + 8 ks .. + 7 of k-step ks; int8 -> fp16 is exact), B = q
//    (fp16; fp32 / bf16 queries as an fp16 hi + lo pair, two MFMAs). C holds
//    tokens 4 (l / 16) + i, head l % 16 — for the two 16-token halves of the
//    tile, the 8 tokens T_g = {4g .. 4g+3, 16+4g .. 16+4g+3}, g = l / 16.
//  * Scores are scaled (k scale x softmax scale x log2 e) and masked, and each
//    head keeps a base-2 online softmax; a head's max is taken over its 4
//    lanes (shuffles) so that m is the same in all of them.
//  * O^T = V^T P^T: B = P^T needs exactly the 8 tokens T_g in lane l, which
//    the QK output already holds (the V scale folded into P, fp16 hi + lo);
//    A = V^T: the wave stages the tile's V codes in LDS (row pitch D + 8
//    bytes, which keeps the reads below free of bank conflicts) and reads 8
//    tokens of one dim per lane with ds_read_b64_tr_b8: within each 16-lane
//    group, lane i < 8 receives byte i of the rows that the even lanes
//    address and lane 8 + i byte i of the odd lanes' rows, so lane 2s + h of
//    group g addresses token T_g[s], dims 16 db + 8 h .. + 7.
// The next tile's loads are issued before the current tile's math. At the
// end the wave states are merged through LDS into the split's partial (or
// the output).
constexpr int kMfmaMaxSplits = 128;

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

// 8 int8 codes (two dwords, byte order kept) -> 8 exact fp16 values: the
// offset-binary byte b + 128 in the low mantissa byte of fp16 1024, minus 1152.
__device__ __forceinline__ half8_t i8x8_to_h8(uint32_t lo, uint32_t hi) {
  const uint32_t a = lo ^ 0x80808080u, b = hi ^ 0x80808080u;
  const half2_t off = {(f16)-1152.f, (f16)-1152.f};
  const half2_t p0 = sf_bitcast<half2_t>(__builtin_amdgcn_perm(0x64646464u, a, 0x04010400u)) + off;
  const half2_t p1 = sf_bitcast<half2_t>(__builtin_amdgcn_perm(0x64646464u, a, 0x04030402u)) + off;
  const half2_t p2 = sf_bitcast<half2_t>(__builtin_amdgcn_perm(0x64646464u, b, 0x04010400u)) + off;
  const half2_t p3 = sf_bitcast<half2_t>(__builtin_amdgcn_perm(0x64646464u, b, 0x04030402u)) + off;
  return half8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

template <int D, int NW>
constexpr int attn_mfma_smem_floats() {
  // V tiles [NW][32][D + 8] bytes, then wave states m, l [NW][16] and O [NW][16][D]
  return NW * 32 * (D + 8) / 4 + 2 * NW * 16 + NW * 16 * D;
}

// NW waves per workgroup, NB of a wave's tiles in flight. NW = 4 serves
// split-T launches; one split per
// (b, kv head) runs 16 waves with one tile each in flight at head_dim 64 (more
// tiles per wave spill at 128 VGPRs) and 8 waves with 2 at head_dim 128, so a
// 512-token cache is one round of loads and needs no cross-workgroup merge.
// The cache's 32-token tiles go round robin: split s takes tiles s, s + S,
// s + 2 S, ..., and its wave w every NW-th of those (tile j = s + S (w + NW i)).
// Which tiles a wave owns does not depend on the cache length, so a wave's
// first NB tiles are loaded before the length (device memory on the decode
// path) has arrived; rows are clamped into the cache and tokens at or past the
// length are masked. Tiles start on 32-token boundaries, so when T_cap % 4 ==
// 0 (vscale) a lane's 8 scales are two aligned 4-token loads.
// max / sum of a value and its partners 16 and 32 lanes away (see sf_swap16_pair)
__device__ __forceinline__ float max_x16_x32(float v) {
  float2_t p = sf_swap16_pair(v);
  v = fmaxf(p.x, p.y);
  p = sf_swap32_pair(v);
  return fmaxf(p.x, p.y);
}
__device__ __forceinline__ float sum_x16_x32(float v) {
  float2_t p = sf_swap16_pair(v);
  v = p.x + p.y;
  p = sf_swap32_pair(v);
  return p.x + p.y;
}

template <int QDT, int SDT, int D, int NW, int NB>
__global__ void __launch_bounds__(NW * 64)
k_attn_mfma(const void *__restrict__ q, const int8_t *__restrict__ kc, const void *__restrict__ ks,
            const int8_t *__restrict__ vc, const void *__restrict__ vs, float *part_acc,
            float *part_ml, void *__restrict__ out, int odt, int H, int KVH,
            int T, const int *__restrict__ T_dev, int causal, int T_cap, float qscale,
            int n_splits, int vscale) {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static_assert(NW == kAttnWaves || NW == 8 || NW == 16, "4 waves (split-T), 8 or 16 (one split)");
  constexpr int NT = NW * 64;
  constexpr int KS = D / 32;       // q.k k-steps per token
  constexpr int DB = D / 16;       // P V dim blocks
  constexpr int KW = D / 16;       // K dwords per lane per token (D/4 bytes)
  constexpr int VC = D / 32;       // 16-byte V chunks per lane per tile
  constexpr int PITCH = D + 8;     // V tile row pitch in LDS, bytes
  constexpr bool QSPLIT = QDT != SF_F16;
  __shared__ __attribute__((aligned(16))) float smem[attn_mfma_smem_floats<D, NW>()];
  // every argument fetched in one round at entry (left to itself the compiler
  // splits the scalar loads around the first branches, one wait per round)
  asm volatile("" ::"s"(q), "s"(kc), "s"(ks), "s"(vc), "s"(vs), "s"(part_acc), "s"(part_ml), "s"(out),
               "s"(odt), "s"(H), "s"(KVH), "s"(T), "s"(T_dev), "s"(causal), "s"(T_cap), "s"(qscale),
               "s"(n_splits), "s"(vscale));

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = H / KVH;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane & 15, g = lane >> 4;
  const size_t base = ((size_t)(causal ? 0 : b) * KVH + kvh) * (size_t)T_cap;
  const int jstep = n_splits * NW, j0 = split + n_splits * wave;  // this wave's tiles j0 + jstep i
  const size_t bh0 = (size_t)b * H + (size_t)kvh * G;

  // q as the B operand of S^T = K q^T: lane (head hl, group g), k-step ks:
  // q[hl][D/4 g + 8 ks .. + 7]
  half8_t qh[KS], ql[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    float f[8];
    sf_load8_as_f32<QDT>(q, (bh0 + min(hl, G - 1)) * D + g * (D / 4) + 8 * k, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float v = hl < G ? f[i] : 0.f;
      qh[k][i] = (f16)v;
      ql[k][i] = (f16)(v - (float)qh[k][i]);
    }
  }

  struct Tile {
    u32x4 k[2][KW / 4];  // K dwords of tokens hl and 16 + hl
    u32x4 v[VC];         // V chunks for the LDS stage
    // scale bits of the lane's tokens T_g as loaded (converted in compute, so
    // that no use of a load waits on the tile's other loads and holds back
    // the next tile's): token r's word is [r / 4][r % 4] (fp32 bits, or fp16 /
    // bf16 in the low half), but with vscale fp16 pairs, tokens 4 h2 + 2 i and
    // + 1 in the halves of word [h2][i]
    u32x4 kw[2], vw[2];
  };
  auto tok_of = [&](int r) { return (r < 4 ? 4 * g + r : 16 + 4 * g + (r - 4)); };
  // tile j's rows (clamped into the cache: a tile is loaded before the length
  // is known, and its tokens past the length are masked in compute)
  auto load = [&](int j, Tile &tl) {
    const int tb = 32 * j;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int t = min(tb + 16 * h2 + hl, T_cap - 1);
      const u32x4 *kp = (const u32x4 *)(kc + (base + t) * D + g * (D / 4));
#pragma unroll
      for (int c = 0; c < KW / 4; ++c) tl.k[h2][c] = kp[c];
    }
#pragma unroll
    for (int c = 0; c < VC; ++c) {
      const int ch = lane + 64 * c, tok = ch / (D / 16), piece = ch % (D / 16);
      const int t = min(tb + tok, T_cap - 1);
      tl.v[c] = *(const u32x4 *)(vc + (base + t) * D + piece * 16);
    }
    if (vscale) {
      // tokens tb + 4g .. + 3 and tb + 16 + 4g .. + 3: aligned 4-token groups;
      // a group past T_cap is moved back inside (its tokens are masked anyway)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const size_t row = base + min(tb + 16 * h2 + 4 * g, T_cap - 4);
        if constexpr (SDT == SF_F16) {
          const u32x2 a = *(const u32x2 *)((const f16 *)ks + row);
          const u32x2 c = *(const u32x2 *)((const f16 *)vs + row);
          tl.kw[h2].x = a.x, tl.kw[h2].y = a.y;
          tl.vw[h2].x = c.x, tl.vw[h2].y = c.y;
        } else {
          tl.kw[h2] = *(const u32x4 *)((const float *)ks + row);
          tl.vw[h2] = *(const u32x4 *)((const float *)vs + row);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const size_t row = base + min(tb + tok_of(r), T_cap - 1);
        if constexpr (SDT == SF_F32) {
          tl.kw[r >> 2][r & 3] = ((const uint32_t *)ks)[row];
          tl.vw[r >> 2][r & 3] = ((const uint32_t *)vs)[row];
        } else {
          tl.kw[r >> 2][r & 3] = ((const uint16_t *)ks)[row];
          tl.vw[r >> 2][r & 3] = ((const uint16_t *)vs)[row];
        }
      }
    }
  };
  // scale r of a tile from its loaded bits
  auto scale_of = [&](const u32x4 (&w4)[2], int r) {
    if constexpr (SDT == SF_F32) {
      return sf_bitcast<float>(w4[r >> 2][r & 3]);
    } else {
      // both candidates at constant indices, then a select
      const uint32_t wp = w4[r >> 2][(r >> 1) & 1] >> (16 * (r & 1));
      const uint32_t w1 = w4[r >> 2][r & 3];
      const uint32_t w = SDT == SF_F16 && vscale ? wp : w1;
      if constexpr (SDT == SF_F16) return (float)sf_bitcast<f16>((uint16_t)w);
      else return sf_bf16_to_f32((uint16_t)w);
    }
  };

  // the wave's first tiles (those that start inside the cache), then the length
  // The device-side length goes out as a vector load right behind the first
  // tile's (a scalar load would be waited for by the next kernel-argument
  // wait, before any tile goes out), so waiting for it leaves the later tiles
  // in flight.
  Tile tl[NB];
  int tdev = 0;
#pragma unroll
  for (int u = 0; u < NB; ++u) {
    if (32 * (j0 + jstep * u) < T_cap) load(j0 + jstep * u, tl[u]);
    if (u == 0 && T_dev) tdev = __hip_atomic_load(T_dev, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  asm volatile("" : "+v"(tdev));  // read here, not right behind its load
  int Tv = T_dev ? tdev + T : T;
  if (causal) Tv = (T_dev ? tdev : T) + b + 1;
  Tv = max(0, min(Tv, T_cap));
  const int ntot = (Tv + 31) / 32;  // tiles holding tokens
  const int mine = j0 < ntot ? (ntot - j0 + jstep - 1) / jstep : 0;

  uint8_t *vt = (uint8_t *)smem + wave * 32 * PITCH;
  float m = -INFINITY, lsum = 0.f;
  float4_t O[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) O[d] = float4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int j, const Tile &tl) {
    const int tb = 32 * j;
    float tks[8], tvs[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      tks[r] = scale_of(tl.kw, r);
      tvs[r] = scale_of(tl.vw, r);
    }
    // S^T for the two 16-token halves
    float4_t S[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      S[h2] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const u32x4 w = tl.k[h2][k / 2];
        const half8_t a = (k & 1) ? i8x8_to_h8(w.z, w.w) : i8x8_to_h8(w.x, w.y);
        S[h2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[k], S[h2], 0, 0, 0);
        if constexpr (QSPLIT) S[h2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[k], S[h2], 0, 0, 0);
      }
    }
    float sc[8];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const bool valid = tb + tok_of(r) < Tv;
      sc[r] = valid ? S[r >> 2][r & 3] * (tks[r] * qscale) : -INFINITY;
      mx = fmaxf(mx, sc[r]);
    }
    mx = max_x16_x32(mx);
    const float m_new = fmaxf(m, mx);
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    const float c = __builtin_amdgcn_exp2f(m - m_ref);  // exp2(-inf) = 0
    m = m_new;
    half8_t ph, pl;
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const float p = __builtin_amdgcn_exp2f(sc[r] - m_ref);
      ps += p;
      // masked tokens weigh exactly 0 (their scale may be any stale value)
      const float pv = tb + tok_of(r) < Tv ? p * tvs[r] : 0.f;
      ph[r] = (f16)pv;
      pl[r] = (f16)(pv - (float)ph[r]);
    }
    lsum = fmaf(lsum, c, ps);
    // V tile -> LDS (this wave's region; LDS accesses of a wave stay in order)
#pragma unroll
    for (int cc = 0; cc < VC; ++cc) {
      const int ch = lane + 64 * cc, tok = ch / (D / 16), piece = ch % (D / 16);
      uint2 *dst = (uint2 *)(vt + tok * PITCH + piece * 16);
      dst[0] = uint2{tl.v[cc].x, tl.v[cc].y};
      dst[1] = uint2{tl.v[cc].z, tl.v[cc].w};
    }
    const int vtok = tok_of(hl >> 1);
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      typedef int v2i __attribute__((ext_vector_type(2)));
      const v2i r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (__attribute__((address_space(3))) v2i *)(vt + vtok * PITCH + 16 * d + 8 * (hl & 1)));
      const half8_t a = i8x8_to_h8((uint32_t)r.x, (uint32_t)r.y);
      O[d] *= c;
      O[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ph, O[d], 0, 0, 0);
      O[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pl, O[d], 0, 0, 0);
    }
  };

  // this wave's tiles j0 + jstep i, i < mine; NB of them in flight (slot
  // i % NB, compile-time after unrolling)
  for (int i0 = 0; i0 < mine; i0 += NB) {
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int i = i0 + u;
      if (i < mine) {
        compute(j0 + jstep * i, tl[u]);
        if (i + NB < mine) load(j0 + jstep * (i + NB), tl[u]);
      }
    }
  }
  lsum = sum_x16_x32(lsum);

  // ---- merge the 4 wave states (LDS)
  float *ms = smem + NW * 32 * PITCH / 4;  // [NW][16]
  float *ls = ms + NW * 16;                // [NW][16]
  float *os = ls + NW * 16;                // [NW][16][D]
  if (g == 0) {
    ms[wave * 16 + hl] = m;
    ls[wave * 16 + hl] = lsum;
  }
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int i = 0; i < 4; ++i) os[(wave * 16 + hl) * D + 16 * d + 4 * g + i] = O[d][i];
  __syncthreads();
  const bool single = n_splits == 1;
  constexpr int NQ = D / 4;
  for (int it = tid; it < G * NQ; it += NT) {
    const int h = it / NQ, d4 = (it - h * NQ) * 4;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, ms[w * 16 + h]);
    const float M_ref = M == -INFINITY ? 0.f : M;
    float L = 0.f;
    float4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = __builtin_amdgcn_exp2f(ms[w * 16 + h] - M_ref);
      L = fmaf(wt, ls[w * 16 + h], L);
      a += *(const float4_t *)(os + (w * 16 + h) * D + d4) * wt;
    }
    if (single) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      const size_t o = (bh0 + h) * D + d4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = a[i] * inv;
        if (odt == SF_F32) ((float *)out)[o + i] = v;
        else if (odt == SF_F16) ((f16 *)out)[o + i] = (f16)v;
        else ((uint16_t *)out)[o + i] = sf_f32_to_bf16(v);
      }
    } else {
      *(float4_t *)(part_acc + ((bh0 + h) * n_splits + split) * D + d4) = a;
      if (d4 == 0) *(float2_t *)(part_ml + ((bh0 + h) * n_splits + split) * 2) = float2_t{M, L};
    }
  }
}

int pow2_log2_at_least(int v) {
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
}

// ---------------------------------------------------------------------------
// causal prefill attention, flash style on MFMA
// ---------------------------------------------------------------------------
// The prompt's query rows of one kv head are the (token, head) pairs
// c = t * G + h; a workgroup owns 16 consecutive ones as the 16 MFMA columns,
// and its waves share the key tiles 0, 32, 64, ... up to the causal limit of
// the last row round robin (wave w takes tiles w, w + NW, ...), each keeping
// every row's online softmax (base 2) as the decode kernel keeps each head's:
// S^T = K Q^T (K codes -> exact fp16 as the A operand, the rows' q as the B
// operand, fp16 hi + lo for fp32 / bf16 q), a key past a row's own limit
// T0 + t + 1 weighs exactly 0, and O^T = V^T P^T takes P^T from the S^T
// registers (V scale folded, hi + lo) and V^T from the wave's LDS stage
// through ds_read_b64_tr_b8. The wave states (m, l, O per row) merge through
// LDS at the end with the decode kernel's rule. Workgroups go out longest
// rows first, the kv heads interleaved, so the short early rows fill in
// behind them. Every K / V tile is read once per workgroup (16 query rows),
// not once per query row.
constexpr int kPfWaves = 4;

template <int QDT, int SDT, int D>
__global__ void __launch_bounds__(kPfWaves * 64)
k_attn_prefill_mfma(const void *__restrict__ q, const int8_t *__restrict__ kc,
                    const void *__restrict__ ks, const int8_t *__restrict__ vc,
                    const void *__restrict__ vs, void *__restrict__ out, int odt, int H, int KVH,
                    int T_q, int T0, const int *__restrict__ T0_dev, int T_cap, float qscale,
                    int vscale) {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  constexpr int NW = kPfWaves, NB = 2;
  constexpr int KS = D / 32, DB = D / 16, KW = D / 16, VC = D / 32, PITCH = D + 8;
  constexpr bool QSPLIT = QDT != SF_F16;
  __shared__ __attribute__((aligned(16))) float smem[NW * 32 * PITCH / 4];
  __shared__ __attribute__((aligned(16))) float os[NW * 16 * D];  // wave states: O
  __shared__ float ms[NW * 16], ls[NW * 16];                     // and m, l per row

  const int kvh = (int)(blockIdx.x % (unsigned)KVH);
  const int G = H / KVH;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hl = lane & 15, g = lane >> 4;
  const int ncol = T_q * G;
  const int nblk = (ncol + 15) >> 4;
  const int c0 = (nblk - 1 - (int)(blockIdx.x / (unsigned)KVH)) * 16;  // longest rows first
  if (c0 < 0) return;  // workgroup-uniform (the host's grid has none past the rows)
  const int start = T0_dev ? *T0_dev : T0;
  const int c = min(c0 + hl, ncol - 1);  // columns past the rows repeat the last one (not stored)
  const int tq = c / G, hh = c - tq * G;
  const int lim = max(0, min(start + tq + 1, T_cap));             // keys this row sees
  const int t1 = max(0, min(start + (min(c0 + 15, ncol - 1) / G) + 1, T_cap));  // the wave's last row's
  const size_t base = (size_t)kvh * T_cap;
  const size_t qrow = (size_t)tq * H + (size_t)kvh * G + hh;

  half8_t qh[KS], ql[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    float f[8];
    sf_load8_as_f32<QDT>(q, qrow * D + g * (D / 4) + 8 * k, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qh[k][i] = (f16)f[i];
      ql[k][i] = (f16)(f[i] - (float)qh[k][i]);
    }
  }

  struct Tile {
    u32x4 k[2][KW / 4];
    u32x4 v[VC];
    float ks[8], vs[8];
  };
  const int ntiles = (t1 + 31) / 32;
  const int mine = wave < ntiles ? (ntiles - wave + NW - 1) / NW : 0;  // tiles wave + NW i
  auto tok_of = [&](int r) { return (r < 4 ? 4 * g + r : 16 + 4 * g + (r - 4)); };
  auto load = [&](int j, Tile &tl) {
    const int tb = 32 * j;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int t = min(tb + 16 * h2 + hl, t1 - 1);
      const u32x4 *kp = (const u32x4 *)(kc + (base + t) * D + g * (D / 4));
#pragma unroll
      for (int cc = 0; cc < KW / 4; ++cc) tl.k[h2][cc] = kp[cc];
    }
#pragma unroll
    for (int cc = 0; cc < VC; ++cc) {
      const int ch = lane + 64 * cc, tok = ch / (D / 16), piece = ch % (D / 16);
      const int t = min(tb + tok, t1 - 1);
      tl.v[cc] = *(const u32x4 *)(vc + (base + t) * D + piece * 16);
    }
    if (vscale) {
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const size_t row = base + min(tb + 16 * h2 + 4 * g, T_cap - 4);
        if constexpr (SDT == SF_F16) {
          const u32x2 a = *(const u32x2 *)((const f16 *)ks + row);
          const u32x2 b2 = *(const u32x2 *)((const f16 *)vs + row);
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const half2_t ka = sf_bitcast<half2_t>(a[i]), va = sf_bitcast<half2_t>(b2[i]);
            tl.ks[4 * h2 + 2 * i] = (float)ka.x;
            tl.ks[4 * h2 + 2 * i + 1] = (float)ka.y;
            tl.vs[4 * h2 + 2 * i] = (float)va.x;
            tl.vs[4 * h2 + 2 * i + 1] = (float)va.y;
          }
        } else {
          const float4_t a = *(const float4_t *)((const float *)ks + row);
          const float4_t b2 = *(const float4_t *)((const float *)vs + row);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            tl.ks[4 * h2 + i] = a[i];
            tl.vs[4 * h2 + i] = b2[i];
          }
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const size_t row = base + min(tb + tok_of(r), t1 - 1);
        tl.ks[r] = sf_load_as_f32<SDT>(ks, row);
        tl.vs[r] = sf_load_as_f32<SDT>(vs, row);
      }
    }
  };

  uint8_t *vt = (uint8_t *)smem + wave * 32 * PITCH;
  float m = -INFINITY, lsum = 0.f;
  float4_t O[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) O[d] = float4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int j, const Tile &tl) {
    const int tb = 32 * j;
    float4_t S[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      S[h2] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < KS; ++k) {
        const u32x4 w = tl.k[h2][k / 2];
        const half8_t a = (k & 1) ? i8x8_to_h8(w.z, w.w) : i8x8_to_h8(w.x, w.y);
        S[h2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qh[k], S[h2], 0, 0, 0);
        if constexpr (QSPLIT) S[h2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[k], S[h2], 0, 0, 0);
      }
    }
    float sc[8];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const bool valid = tb + tok_of(r) < lim;
      sc[r] = valid ? S[r >> 2][r & 3] * (tl.ks[r] * qscale) : -INFINITY;
      mx = fmaxf(mx, sc[r]);
    }
    mx = max_x16_x32(mx);
    const float m_new = fmaxf(m, mx);
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    const float cf = __builtin_amdgcn_exp2f(m - m_ref);
    m = m_new;
    half8_t ph, pl;
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const bool valid = tb + tok_of(r) < lim;
      const float p = valid ? __builtin_amdgcn_exp2f(sc[r] - m_ref) : 0.f;
      ps += p;
      // masked keys weigh exactly 0 (a scale past the cached length may be any value)
      const float pv = valid ? p * tl.vs[r] : 0.f;
      ph[r] = (f16)pv;
      pl[r] = (f16)(pv - (float)ph[r]);
    }
    lsum = fmaf(lsum, cf, ps);
#pragma unroll
    for (int cc = 0; cc < VC; ++cc) {
      const int ch = lane + 64 * cc, tok = ch / (D / 16), piece = ch % (D / 16);
      uint2 *dst = (uint2 *)(vt + tok * PITCH + piece * 16);
      dst[0] = uint2{tl.v[cc].x, tl.v[cc].y};
      dst[1] = uint2{tl.v[cc].z, tl.v[cc].w};
    }
    const int vtok = tok_of(hl >> 1);
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      typedef int v2i __attribute__((ext_vector_type(2)));
      const v2i r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (__attribute__((address_space(3))) v2i *)(vt + vtok * PITCH + 16 * d + 8 * (hl & 1)));
      const half8_t a = i8x8_to_h8((uint32_t)r.x, (uint32_t)r.y);
      O[d] *= cf;
      O[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ph, O[d], 0, 0, 0);
      O[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pl, O[d], 0, 0, 0);
    }
  };

  Tile tl[NB];
#pragma unroll
  for (int u = 0; u < NB; ++u)
    if (u < mine) load(wave + NW * u, tl[u]);
  for (int i0 = 0; i0 < mine; i0 += NB) {
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int i = i0 + u;
      if (i < mine) {
        compute(wave + NW * i, tl[u]);
        if (i + NB < mine) load(wave + NW * (i + NB), tl[u]);
      }
    }
  }
  lsum = sum_x16_x32(lsum);

  // ---- merge the wave states (a wave without tiles holds m = -inf, l = 0, O = 0)
  if (g == 0) {
    ms[wave * 16 + hl] = m;
    ls[wave * 16 + hl] = lsum;
  }
#pragma unroll
  for (int d = 0; d < DB; ++d)
    *(float4_t *)(os + (wave * 16 + hl) * D + 16 * d + 4 * g) = O[d];
  __syncthreads();
  for (int e = threadIdx.x; e < 16 * (D / 4); e += NW * 64) {
    const int h = e / (D / 4), d4 = (e - h * (D / 4)) * 4;
    const int col = c0 + h;
    if (col >= ncol) continue;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, ms[w * 16 + h]);
    const float M_ref = M == -INFINITY ? 0.f : M;
    float L = 0.f;
    float4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = __builtin_amdgcn_exp2f(ms[w * 16 + h] - M_ref);
      L = fmaf(wt, ls[w * 16 + h], L);
      a += *(const float4_t *)(os + (w * 16 + h) * D + d4) * wt;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const int tq = col / G, hh = col - tq * G;
    const size_t o = ((size_t)tq * H + (size_t)kvh * G + hh) * D + d4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = a[i] * inv;
      if (odt == SF_F32) ((float *)out)[o + i] = v;
      else if (odt == SF_F16) ((f16 *)out)[o + i] = (f16)v;
      else ((uint16_t *)out)[o + i] = sf_f32_to_bf16(v);
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" int sf_kv_quant_append(const void *k_new, const void *v_new, int in_dtype,
                                  int8_t *k_codes, void *k_scales, int8_t *v_codes,
                                  void *v_scales, int scale_dtype, int B, int KVH, int T_new,
                                  int T_off, int T_cap, int D, void *stream) {
  SF_REQUIRE(B > 0 && KVH > 0 && T_new >= 0 && T_off >= 0 && D > 0, SF_EINVAL,
             "invalid KV shape B=%d KVH=%d T_new=%d T_off=%d D=%d", B, KVH, T_new, T_off, D);
  SF_REQUIRE(T_off + T_new <= T_cap, SF_EINVAL, "KV cache overflow: %d + %d > capacity %d", T_off,
             T_new, T_cap);
  SF_REQUIRE(D % 8 == 0 && D <= 256, SF_EUNSUPPORTED, "head_dim=%d: need D %% 8 == 0 and D <= 256",
             D);
  SF_REQUIRE(k_new && v_new && k_codes && k_scales && v_codes && v_scales, SF_EINVAL,
             "null pointer argument");
  SF_REQUIRE((((uintptr_t)k_codes | (uintptr_t)v_codes) & 7) == 0, SF_EINVAL,
             "KV code buffers must be 8-byte aligned");
  SF_REQUIRE(in_dtype >= SF_F32 && in_dtype <= SF_BF16, SF_EINVAL, "bad input dtype %d", in_dtype);
  SF_REQUIRE(scale_dtype == SF_F16 || scale_dtype == SF_F32, SF_EINVAL, "bad scale dtype %d",
             scale_dtype);
  if (T_new == 0) return SF_OK;
  const int tpv_log2 = pow2_log2_at_least(D / 8);
  const long long n_vec = 2LL * B * KVH * T_new;
  const long long threads = n_vec << tpv_log2;
  const unsigned grid = (unsigned)((threads + 255) / 256);
  hipStream_t st = (hipStream_t)stream;
#define SF_KV_LAUNCH(I, S)                                                                     \
  k_kv_quant_append<I, S><<<grid, 256, 0, st>>>(k_new, v_new, k_codes, k_scales, v_codes,      \
                                                v_scales, KVH, T_new, T_off, T_cap, D, tpv_log2, \
                                                n_vec)
  if (scale_dtype == SF_F16) {
    if (in_dtype == SF_F32) SF_KV_LAUNCH(SF_F32, SF_F16);
    else if (in_dtype == SF_F16) SF_KV_LAUNCH(SF_F16, SF_F16);
    else SF_KV_LAUNCH(SF_BF16, SF_F16);
  } else {
    if (in_dtype == SF_F32) SF_KV_LAUNCH(SF_F32, SF_F32);
    else if (in_dtype == SF_F16) SF_KV_LAUNCH(SF_F16, SF_F32);
    else SF_KV_LAUNCH(SF_BF16, SF_F32);
  }
#undef SF_KV_LAUNCH
  return sf_check_launch("sf_kv_quant_append");
}

namespace {

// Merge launch of a split-T call, with the rule of split_merge.h: GS lanes
// per output element (row bh, dim d), GS = the tree's span P up to 64; lane g
// loads the (m, l, acc) of splits [g SPL, (g + 1) SPL), SPL = P / GS, and
// sums that block's subtree in registers; the max and the tree's upper
// levels run across the lanes (every load of a lane in flight at once, no
// lane walking the splits one by one).
constexpr int kMergeThreads = 256;

template <int SPL>
__global__ void __launch_bounds__(kMergeThreads)
k_attn_merge(const float *__restrict__ acc, const float *__restrict__ ml, void *__restrict__ out,
             int odt, int rows, int D, int S) {
  // every argument fetched in one round at entry (the compiler would split them)
  asm volatile("" ::"s"(acc), "s"(ml), "s"(out), "s"(odt), "s"(rows), "s"(D), "s"(S));
  const int P = sf_merge_span(S), GS = P / SPL;
  // workgroup i runs on XCD i % 8: the blocks of outputs are dealt so that
  // each XCD takes one contiguous eighth of them (its L2 then fetches only the
  // partials of those heads, not every head's)
  const int nb = gridDim.x, per_x = (nb + 7) >> 3, xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
  const int full = nb - 8 * (per_x - 1);  // XCDs that take per_x blocks (the rest per_x - 1)
  const int blk = xcd < full ? xcd * per_x + j : full * per_x + (xcd - full) * (per_x - 1) + j;
  const int e = blk * (kMergeThreads / GS) + threadIdx.x / GS, g = threadIdx.x % GS;
  const int n = rows * D, ec = min(e, n - 1);  // lanes past the last output compute, then drop
  const int bh = ec / D, d = ec - bh * D;
  const float2_t *mlr = (const float2_t *)ml + (size_t)bh * S;
  const float *ar = acc + (size_t)bh * S * D + d;
  float mv[SPL], lv[SPL], av[SPL];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < SPL; ++k) {
    const int sp = g * SPL + k, sc = min(sp, S - 1);
    const float2_t m = mlr[sc];
    mv[k] = sp < S ? m.x : -INFINITY;
    lv[k] = m.y;
    av[k] = ar[(size_t)sc * D];
    mx = fmaxf(mx, mv[k]);
  }
  const float mref = sf_merge_mref(sf_group_tree_max(mx, GS));
#pragma unroll
  for (int k = 0; k < SPL; ++k) {
    const bool in = g * SPL + k < S;
    const float w = in ? sf_merge_weight(mv[k], mref) : 0.f;
    av[k] = in ? sf_merge_term(av[k], w) : 0.f;
    lv[k] = in ? sf_merge_term(lv[k], w) : 0.f;
  }
  const float v = sf_group_tree_sum(sf_tree_sum(av, SPL), GS);
  const float L = sf_group_tree_sum(sf_tree_sum(lv, SPL), GS);
  if (g == 0 && e < n) {
    const float r = sf_merge_finish(L, v);
    if (odt == SF_F32) ((float *)out)[e] = r;
    else if (odt == SF_F16) ((f16 *)out)[e] = (f16)r;
    else ((uint16_t *)out)[e] = sf_f32_to_bf16(r);
  }
}

}  // namespace

// Workspace: the split partials of split_merge.h, acc [B*H][S][D] fp32 then
// (m, l) [B*H][S][2]. Nothing in it needs clearing: every split writes its
// partial before the merge reads it.
extern "C" size_t sf_attn_workspace_bytes(int B, int H, int D, int n_splits) {
  if (B <= 0 || H <= 0 || D <= 0 || n_splits <= 0) return 0;
  if (n_splits > kMaxSplits) n_splits = kMaxSplits;
  size_t acc_off, ml_off;
  return sf_split_ws_parts(B * H, D, n_splits, &acc_off, &ml_off);
}

extern "C" int sf_attn_default_splits_d(int B, int KVH, int T, int D) {
  // One split (one workgroup per (b, kv head), no merge launch) up to 160
  // tokens; beyond, 32 tokens per split up to 2048 cached tokens and 64 above,
  // 8 to 128 splits. Measured on MI355X at 14 / 2 heads, graph-timed over cold
  // caches (us at the rule's count, other counts in parentheses):
  //   head_dim 64:  T = 128: 4.8 (1);  512: 5.6 (16; 1: 6.4);  1024: 5.7 (32; 64:
  //                 5.8);  2048: 5.8 (64; 32: 5.9);  4096: 6.2 (64; 128: 6.2, 32:
  //                 6.5);  8192: 6.7 (128; 64: 6.8);  16384: 7.4 (128; 64: 7.6);
  //   head_dim 128: T = 512: 6.4 (16; 1: 9.2);  2048: 6.8 (64; 32: 6.9);  4096:
  //                 7.4 (64; 128: 7.5);  8192: 8.2 (128; 64: 8.3);  16384: 9.3
  //                 (128; 64: 10.1).
  // Eight waves per split workgroup (one tile each) instead of four measured
  // no faster at 4096-16384 tokens.
  (void)B;
  (void)KVH;
  (void)D;
  if (T <= 160) return 1;
  const int tps = T <= 2048 ? 32 : 64;
  int s = (T + tps - 1) / tps;
  if (s < 8) s = 8;
  if (s > 128) s = 128;
  return s;
}

extern "C" int sf_attn_default_splits(int B, int KVH, int T) {
  return sf_attn_default_splits_d(B, KVH, T, 64);
}

static int attn_heads_per_block(int G) {
  return G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : G <= 6 ? 6 : G <= 7 ? 7 : 8;
}

// Shared checks and launch. T_dev: device length (plus T); causal: prefill
// rows, query row b sees T + b + 1 tokens of a batch-1 cache.
// The merge launch after a split attention launch (none for one split, or
// when the caller merges the partials itself).
static int attn_merge_launch(const char *what, const float *part_acc, const float *part_ml,
                             void *out, int odt, int rows, int D, int n_splits, hipStream_t st,
                             int merge) {
  if (n_splits > 1 && merge) {
    const int n = rows * D;
    const int P = sf_merge_span(n_splits), spl = P > 64 ? P / 64 : 1, per_block = kMergeThreads / (P / spl);
    const unsigned grid = (unsigned)((n + per_block - 1) / per_block);
    if (spl == 1) k_attn_merge<1><<<grid, kMergeThreads, 0, st>>>(part_acc, part_ml, out, odt, rows, D, n_splits);
    else if (spl == 2) k_attn_merge<2><<<grid, kMergeThreads, 0, st>>>(part_acc, part_ml, out, odt, rows, D, n_splits);
    else if (spl == 4) k_attn_merge<4><<<grid, kMergeThreads, 0, st>>>(part_acc, part_ml, out, odt, rows, D, n_splits);
    else k_attn_merge<8><<<grid, kMergeThreads, 0, st>>>(part_acc, part_ml, out, odt, rows, D, n_splits);
  }
  return sf_check_launch(what);
}

// merge = 0 leaves a split launch's partials in the workspace for a consumer
// that merges them itself (sf_q4_gemv_attn_merge).
static int attn_launch(const char *what, const void *q, int q_dtype, const int8_t *k_codes,
                       const void *k_scales, const int8_t *v_codes, const void *v_scales,
                       int scale_dtype, void *out, int out_dtype, void *workspace,
                       size_t workspace_bytes, int B, int H, int KVH, int T, const int *T_dev,
                       int causal, int T_cap, int D, float scale, int n_splits, void *stream,
                       int merge = 1) {
  SF_REQUIRE(H % KVH == 0, SF_EINVAL, "n_heads=%d not a multiple of n_kv_heads=%d", H, KVH);
  SF_REQUIRE(D <= kMaxD, SF_EINVAL, "head_dim=%d exceeds kernel's compile-time max 256", D);
  SF_REQUIRE(D % 8 == 0, SF_EUNSUPPORTED, "head_dim=%d: need a multiple of 8", D);
  SF_REQUIRE(q && k_codes && k_scales && v_codes && v_scales && out, SF_EINVAL,
             "null pointer argument");
  SF_REQUIRE(q_dtype >= SF_F32 && q_dtype <= SF_BF16 && out_dtype >= SF_F32 && out_dtype <= SF_BF16,
             SF_EINVAL, "bad q/out dtype");
  SF_REQUIRE(scale_dtype == SF_F16 || scale_dtype == SF_F32, SF_EINVAL, "bad scale dtype %d",
             scale_dtype);
  SF_REQUIRE((((uintptr_t)k_codes | (uintptr_t)v_codes) & 7) == 0, SF_EINVAL,
             "KV code buffers must be 8-byte aligned");
  SF_REQUIRE(((uintptr_t)q & 15) == 0, SF_EINVAL, "q must be 16-byte aligned");
  if (n_splits > kMaxSplits) n_splits = kMaxSplits;
  if (n_splits < 1) n_splits = 1;
  size_t acc_off = 0, ml_off = 0;
  float *part_acc = nullptr, *part_ml = nullptr;
  if (n_splits > 1) {
    SF_REQUIRE(workspace, SF_EINVAL, "null workspace");
    SF_REQUIRE(((uintptr_t)workspace & 255) == 0, SF_EINVAL, "workspace must be 256-byte aligned");
    const size_t need = sf_attn_workspace_bytes(B, H, D, n_splits);
    SF_REQUIRE(workspace_bytes >= need, SF_EINVAL, "attention workspace too small: %zu < %zu",
               workspace_bytes, need);
    sf_split_ws_parts(B * H, D, n_splits, &acc_off, &ml_off);
    part_acc = (float *)((char *)workspace + acc_off);
    part_ml = (float *)((char *)workspace + ml_off);
  }
  const int G = H / KVH;
  const float qscale = scale * 1.4426950408889634f;  // softmax in base 2
  hipStream_t st = (hipStream_t)stream;
  // MFMA kernel: up to 16 query heads per kv head, head_dim 64 or 128,
  // 16-byte aligned codes (SF_ATTN_MFMA=0 keeps the VALU kernel)
  const char *mfma_env = getenv("SF_ATTN_MFMA");
  const bool mfma_ok = !(mfma_env && mfma_env[0] == '0');
  if (mfma_ok && G <= 16 && (D == 64 || D == 128) && n_splits <= kMfmaMaxSplits &&
      (((uintptr_t)k_codes | (uintptr_t)v_codes) & 15) == 0) {
    dim3 grid(n_splits, KVH, B);
    // scale loads in aligned groups of 4 tokens when every row start allows it
    const size_t sal = scale_dtype == SF_F16 ? 8 : 16;
    const int vscale = T_cap % 4 == 0 && (uintptr_t)k_scales % sal == 0 &&
                       (uintptr_t)v_scales % sal == 0;
#define SF_MFMA_LAUNCH(QD, SD, DD, NWV, NBV)                                                     \
  k_attn_mfma<QD, SD, DD, NWV, NBV><<<grid, NWV * 64, 0, st>>>(                                  \
      q, k_codes, k_scales, v_codes, v_scales, part_acc, part_ml, out, out_dtype, H,   \
      KVH, T, T_dev, causal, T_cap, qscale, n_splits, vscale)
#define SF_MFMA_D(QD, SD)                                   \
  do {                                                      \
    if (n_splits == 1) {                                    \
      if (D == 64) SF_MFMA_LAUNCH(QD, SD, 64, 16, 1);       \
      else SF_MFMA_LAUNCH(QD, SD, 128, 8, 2);               \
    } else {                                                \
      if (D == 64) SF_MFMA_LAUNCH(QD, SD, 64, kAttnWaves, 2); \
      else SF_MFMA_LAUNCH(QD, SD, 128, kAttnWaves, 2);      \
    }                                                       \
  } while (0)
    if (scale_dtype == SF_F16) {
      if (q_dtype == SF_F32) SF_MFMA_D(SF_F32, SF_F16);
      else if (q_dtype == SF_F16) SF_MFMA_D(SF_F16, SF_F16);
      else SF_MFMA_D(SF_BF16, SF_F16);
    } else {
      if (q_dtype == SF_F32) SF_MFMA_D(SF_F32, SF_F32);
      else if (q_dtype == SF_F16) SF_MFMA_D(SF_F16, SF_F32);
      else SF_MFMA_D(SF_BF16, SF_F32);
    }
#undef SF_MFMA_D
#undef SF_MFMA_LAUNCH
    return attn_merge_launch(what, part_acc, part_ml, out, out_dtype, B * H, D, n_splits, st, merge);
  }
  const int HB = attn_heads_per_block(G);
  const int n_hblk = (G + HB - 1) / HB;
  const int oct_log2 = pow2_log2_at_least(D / 8);
  dim3 grid(n_splits, KVH * n_hblk, B);
#define SF_ATTN_LAUNCH(QD, SD, HBV)                                                            \
  k_attn_decode<QD, SD, HBV><<<grid, kAttnThreads, 0, st>>>(                                   \
      q, k_codes, k_scales, v_codes, v_scales, part_acc, part_ml, out, out_dtype, H, \
      KVH, T, T_dev, causal, T_cap, D, qscale, n_splits, oct_log2)
#define SF_ATTN_HB(QD, SD)                       \
  do {                                           \
    if (HB == 1) SF_ATTN_LAUNCH(QD, SD, 1);      \
    else if (HB == 2) SF_ATTN_LAUNCH(QD, SD, 2); \
    else if (HB == 4) SF_ATTN_LAUNCH(QD, SD, 4); \
    else if (HB == 6) SF_ATTN_LAUNCH(QD, SD, 6); \
    else if (HB == 7) SF_ATTN_LAUNCH(QD, SD, 7); \
    else SF_ATTN_LAUNCH(QD, SD, 8);              \
  } while (0)
  if (scale_dtype == SF_F16) {
    if (q_dtype == SF_F32) SF_ATTN_HB(SF_F32, SF_F16);
    else if (q_dtype == SF_F16) SF_ATTN_HB(SF_F16, SF_F16);
    else SF_ATTN_HB(SF_BF16, SF_F16);
  } else {
    if (q_dtype == SF_F32) SF_ATTN_HB(SF_F32, SF_F32);
    else if (q_dtype == SF_F16) SF_ATTN_HB(SF_F16, SF_F32);
    else SF_ATTN_HB(SF_BF16, SF_F32);
  }
#undef SF_ATTN_HB
#undef SF_ATTN_LAUNCH
  return attn_merge_launch(what, part_acc, part_ml, out, out_dtype, B * H, D, n_splits, st, merge);
}

extern "C" int sf_attn_decode_i8kv(const void *q, int q_dtype, const int8_t *k_codes,
                                   const void *k_scales, const int8_t *v_codes,
                                   const void *v_scales, int scale_dtype, void *out, int out_dtype,
                                   void *workspace, size_t workspace_bytes, int B, int H, int KVH,
                                   int T, int T_cap, int D, float scale, int n_splits,
                                   void *stream) {
  SF_REQUIRE(B > 0 && H > 0 && KVH > 0 && D > 0 && T >= 0 && T <= T_cap, SF_EINVAL,
             "invalid attention shape B=%d H=%d KVH=%d T=%d T_cap=%d D=%d", B, H, KVH, T, T_cap, D);
  if (n_splits <= 0) n_splits = sf_attn_default_splits_d(B, KVH, T, D);
  // the reference's tiling: n_tiles = max(1, min(n_tiles, T)); tile = ceil(T / n_tiles)
  n_splits = n_splits < (T > 0 ? T : 1) ? n_splits : (T > 0 ? T : 1);
  if (n_splits > kMaxSplits) n_splits = kMaxSplits;
  return attn_launch("sf_attn_decode_i8kv", q, q_dtype, k_codes, k_scales, v_codes, v_scales,
                     scale_dtype, out, out_dtype, workspace, workspace_bytes, B, H, KVH, T,
                     nullptr, 0, T_cap, D, scale, n_splits, stream);
}

extern "C" int sf_attn_decode_i8kv_dev(const void *q, int q_dtype, const int8_t *k_codes,
                                       const void *k_scales, const int8_t *v_codes,
                                       const void *v_scales, int scale_dtype, void *out,
                                       int out_dtype, void *workspace, size_t workspace_bytes, int B,
                                       int H, int KVH, const int *T_dev, int T_add, int T_max,
                                       int T_cap, int D, float scale, int n_splits, void *stream) {
  SF_REQUIRE(B > 0 && H > 0 && KVH > 0 && D > 0 && T_max >= 0 && T_max <= T_cap, SF_EINVAL,
             "invalid attention shape B=%d H=%d KVH=%d T_max=%d T_cap=%d D=%d", B, H, KVH, T_max,
             T_cap, D);
  SF_REQUIRE(T_dev, SF_EINVAL, "null pointer argument");
  if (n_splits <= 0) n_splits = sf_attn_default_splits_d(B, KVH, T_max, D);
  return attn_launch("sf_attn_decode_i8kv_dev", q, q_dtype, k_codes, k_scales, v_codes, v_scales,
                     scale_dtype, out, out_dtype, workspace, workspace_bytes, B, H, KVH, T_add,
                     T_dev, 0, T_cap, D, scale, n_splits, stream);
}

extern "C" int sf_attn_decode_i8kv_partials_dev(const void *q, int q_dtype, const int8_t *k_codes,
                                                const void *k_scales, const int8_t *v_codes,
                                                const void *v_scales, int scale_dtype,
                                                void *workspace, size_t workspace_bytes, int B,
                                                int H, int KVH, const int *T_dev, int T_add,
                                                int T_max, int T_cap, int D, float scale,
                                                int n_splits, void *stream) {
  SF_REQUIRE(B > 0 && H > 0 && KVH > 0 && D > 0 && T_max >= 0 && T_max <= T_cap, SF_EINVAL,
             "invalid attention shape B=%d H=%d KVH=%d T_max=%d T_cap=%d D=%d", B, H, KVH, T_max,
             T_cap, D);
  SF_REQUIRE(T_dev, SF_EINVAL, "null pointer argument");
  SF_REQUIRE(n_splits >= 2 && n_splits <= kMaxSplits, SF_EINVAL,
             "partials need 2..%d splits (got %d)", kMaxSplits, n_splits);
  // `out` is never written by a split launch: the workspace stands in for it
  return attn_launch("sf_attn_decode_i8kv_partials_dev", q, q_dtype, k_codes, k_scales, v_codes,
                     v_scales, scale_dtype, workspace, SF_F32, workspace, workspace_bytes, B, H,
                     KVH, T_add, T_dev, 0, T_cap, D, scale, n_splits, stream, 0);
}

// Flash-style prefill (k_attn_prefill_mfma) for prompt chunks of kPfMinRows
// rows or more at head_dim 64 / 128; shorter chunks (speculative verify rows)
// keep the split-T decode kernel, which spreads a long cache over workgroups.
constexpr int kPfMinRows = 16;

static bool prefill_mfma_ok(int T_q, int H, int KVH, int D, const int8_t *k_codes,
                            const int8_t *v_codes) {
  const char *mfma_env = getenv("SF_ATTN_MFMA");
  const bool mfma_ok = !(mfma_env && mfma_env[0] == '0');
  return mfma_ok && T_q >= kPfMinRows && H % KVH == 0 && (D == 64 || D == 128) &&
         (((uintptr_t)k_codes | (uintptr_t)v_codes) & 15) == 0;
}

static int prefill_mfma_launch(const char *what, const void *q, int q_dtype, const int8_t *k_codes,
                               const void *k_scales, const int8_t *v_codes, const void *v_scales,
                               int scale_dtype, void *out, int out_dtype, int T_q, int H, int KVH,
                               int T0, const int *T0_dev, int T_cap, int D, float scale,
                               void *stream) {
  SF_REQUIRE(q && k_codes && k_scales && v_codes && v_scales && out, SF_EINVAL,
             "null pointer argument");
  SF_REQUIRE(q_dtype >= SF_F32 && q_dtype <= SF_BF16 && out_dtype >= SF_F32 && out_dtype <= SF_BF16,
             SF_EINVAL, "bad q/out dtype");
  SF_REQUIRE(scale_dtype == SF_F16 || scale_dtype == SF_F32, SF_EINVAL, "bad scale dtype %d",
             scale_dtype);
  SF_REQUIRE(((uintptr_t)q & 15) == 0, SF_EINVAL, "q must be 16-byte aligned");
  const int G = H / KVH;
  const float qscale = scale * 1.4426950408889634f;
  const size_t sal = scale_dtype == SF_F16 ? 8 : 16;
  const int vscale = T_cap % 4 == 0 && T_cap >= 4 && (uintptr_t)k_scales % sal == 0 &&
                     (uintptr_t)v_scales % sal == 0;
  const long long ncol = (long long)T_q * G;
  const long long nblk = (ncol + 15) / 16;  // 16-row blocks; one workgroup per block and kv head
  SF_REQUIRE(ncol <= 0x7fffffff && nblk * KVH <= 0x7fffffff, SF_EINVAL,
             "prefill of %d rows is too long", T_q);
  dim3 grid((unsigned)(nblk * KVH), 1, 1);
  hipStream_t st = (hipStream_t)stream;
#define SF_PF_LAUNCH(QD, SD, DD)                                                               \
  k_attn_prefill_mfma<QD, SD, DD><<<grid, kPfWaves * 64, 0, st>>>(                            \
      q, k_codes, k_scales, v_codes, v_scales, out, out_dtype, H, KVH, T_q, T0, T0_dev, T_cap, \
      qscale, vscale)
#define SF_PF_D(QD, SD)                  \
  do {                                   \
    if (D == 64) SF_PF_LAUNCH(QD, SD, 64); \
    else SF_PF_LAUNCH(QD, SD, 128);      \
  } while (0)
  if (scale_dtype == SF_F16) {
    if (q_dtype == SF_F32) SF_PF_D(SF_F32, SF_F16);
    else if (q_dtype == SF_F16) SF_PF_D(SF_F16, SF_F16);
    else SF_PF_D(SF_BF16, SF_F16);
  } else {
    if (q_dtype == SF_F32) SF_PF_D(SF_F32, SF_F32);
    else if (q_dtype == SF_F16) SF_PF_D(SF_F16, SF_F32);
    else SF_PF_D(SF_BF16, SF_F32);
  }
#undef SF_PF_D
#undef SF_PF_LAUNCH
  return sf_check_launch(what);
}

extern "C" int sf_attn_prefill_i8kv(const void *q, int q_dtype, const int8_t *k_codes,
                                    const void *k_scales, const int8_t *v_codes,
                                    const void *v_scales, int scale_dtype, void *out,
                                    int out_dtype, int T_q, int H, int KVH, int T0, int T_cap,
                                    int D, float scale, void *stream) {
  SF_REQUIRE(T_q > 0 && H > 0 && KVH > 0 && D > 0 && T0 >= 0 && T0 + T_q <= T_cap, SF_EINVAL,
             "invalid prefill attention shape T_q=%d H=%d KVH=%d T0=%d T_cap=%d D=%d", T_q, H, KVH,
             T0, T_cap, D);
  if (prefill_mfma_ok(T_q, H, KVH, D, k_codes, v_codes))
    return prefill_mfma_launch("sf_attn_prefill_i8kv", q, q_dtype, k_codes, k_scales, v_codes,
                               v_scales, scale_dtype, out, out_dtype, T_q, H, KVH, T0, nullptr,
                               T_cap, D, scale, stream);
  return attn_launch("sf_attn_prefill_i8kv", q, q_dtype, k_codes, k_scales, v_codes, v_scales,
                     scale_dtype, out, out_dtype, nullptr, 0, T_q, H, KVH, T0, nullptr, 1, T_cap, D,
                     scale, 1, stream);
}

extern "C" int sf_attn_prefill_i8kv_dev(const void *q, int q_dtype, const int8_t *k_codes,
                                        const void *k_scales, const int8_t *v_codes,
                                        const void *v_scales, int scale_dtype, void *out,
                                        int out_dtype, void *workspace, size_t workspace_bytes,
                                        int T_q, int H, int KVH, const int *T0_dev, int T_max,
                                        int T_cap, int D, float scale, int n_splits,
                                        void *stream) {
  SF_REQUIRE(T_q > 0 && H > 0 && KVH > 0 && D > 0 && T_max >= T_q && T_max <= T_cap, SF_EINVAL,
             "invalid prefill attention shape T_q=%d H=%d KVH=%d T_max=%d T_cap=%d D=%d", T_q, H,
             KVH, T_max, T_cap, D);
  SF_REQUIRE(T0_dev, SF_EINVAL, "null pointer argument");
  if (prefill_mfma_ok(T_q, H, KVH, D, k_codes, v_codes))
    return prefill_mfma_launch("sf_attn_prefill_i8kv_dev", q, q_dtype, k_codes, k_scales, v_codes,
                               v_scales, scale_dtype, out, out_dtype, T_q, H, KVH, 0, T0_dev, T_cap,
                               D, scale, stream);
  if (n_splits <= 0) n_splits = sf_attn_default_splits_d(T_q, KVH, T_max, D);
  return attn_launch("sf_attn_prefill_i8kv_dev", q, q_dtype, k_codes, k_scales, v_codes, v_scales,
                     scale_dtype, out, out_dtype, workspace, workspace_bytes, T_q, H, KVH, 0,
                     T0_dev, 1, T_cap, D, scale, n_splits, stream);
}

// ---------------------------------------------------------------------------
// Decode attention that allocates nothing: sf_attn_decode_i8kv with its
// workspace (the split partials) in a file-scope device array. Each GPU the
// library runs on holds its own copy until the process ends; host code
// reaches a device's copy only through the address hipGetSymbolAddress gives
// for it (taken once per device, on the first call, with that device
// current), never through the array's name. Nothing in it needs clearing
// (every split writes its partial before the merge launch reads it). All
// calls on one GPU share the array: calls that overlap on one GPU (two
// streams at once) race.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = 4u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// the current device's copy of `scratch`, set up on its first use
int scratch_for_current_device(void **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  SF_REQUIRE(e == hipSuccess, SF_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
  SF_REQUIRE(dev >= 0 && dev < kMaxDevices, SF_EUNSUPPORTED, "device %d: beyond %d devices", dev,
             kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    SF_REQUIRE(e == hipSuccess && p, SF_EHIP, "hipGetSymbolAddress(scratch): %s",
               hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SF_OK;
}

}  // namespace

extern "C" size_t sf_attn_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int sf_attn_decode_i8kv_noalloc(const void *q, int q_dtype, const int8_t *k_codes,
                                           const void *k_scales, const int8_t *v_codes,
                                           const void *v_scales, int scale_dtype, void *out,
                                           int out_dtype, int B, int H, int KVH, int T, int T_cap,
                                           int D, float scale, int n_splits, void *stream) {
  SF_REQUIRE(B > 0 && H > 0 && KVH > 0 && D > 0 && T >= 0 && T <= T_cap, SF_EINVAL,
             "invalid attention shape B=%d H=%d KVH=%d T=%d T_cap=%d D=%d", B, H, KVH, T, T_cap, D);
  int s = n_splits > 0 ? n_splits : sf_attn_default_splits_d(B, KVH, T, D);
  s = s < (T > 0 ? T : 1) ? s : (T > 0 ? T : 1);
  const size_t need = sf_attn_workspace_bytes(B, H, D, s);
  SF_REQUIRE(need <= kNoAllocScratchBytes, SF_EINVAL,
             "sf_attn_decode_i8kv_noalloc: B=%d H=%d D=%d with %d splits needs %zu bytes of "
             "scratch, more than its fixed %zu; use sf_attn_decode_i8kv with a workspace",
             B, H, D, s, need, kNoAllocScratchBytes);
  void *ws = nullptr;
  int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  return sf_attn_decode_i8kv(q, q_dtype, k_codes, k_scales, v_codes, v_scales, scale_dtype, out,
                             out_dtype, ws, kNoAllocScratchBytes, B, H, KVH, T, T_cap, D, scale, s,
                             stream);
}
