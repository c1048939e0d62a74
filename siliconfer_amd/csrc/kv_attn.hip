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
//  * inside a split, 64-token sub-tiles: scores with lanes along D (8 codes
//    per lane, one 8-byte load), a per-head running max / sum in base 2
//    (scores pre-scaled by log2 e), then P.V with lanes along D again;
//  * the split partials (m, l, acc[D]) are merged by a second kernel with the
//    reference's combine rule (q4_attention.py:63-70, 256-261).
#include <math.h>

#include "sf_common.h"

namespace {

constexpr int kAttnThreads = 256;
constexpr int kSubTile = 64;
constexpr int kHeadsPerBlock = 8;

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
template <int QDT, int SDT>
__global__ void __launch_bounds__(kAttnThreads)
k_attn_split(const void *__restrict__ q, const int8_t *__restrict__ kc,
             const void *__restrict__ ks, const int8_t *__restrict__ vc,
             const void *__restrict__ vs, float *__restrict__ part_acc,
             float *__restrict__ part_ml, int H, int KVH, int T, int T_cap, int D,
             float qscale, int n_splits, int tile, int tpt_log2) {
  constexpr int HB = kHeadsPerBlock;
  extern __shared__ float red[];  // [4 waves][HB][D]
  __shared__ float sc[HB][kSubTile];
  __shared__ float m_s[HB], l_s[HB], c_s[HB];

  const int split = blockIdx.x;
  const int G = H / KVH;
  const int n_hblk = (G + HB - 1) / HB;
  const int kvh = blockIdx.y / n_hblk;
  const int h0 = (blockIdx.y - kvh * n_hblk) * HB;  // first query head (within the group)
  const int nh = min(HB, G - h0);
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int tpt = 1 << tpt_log2;  // lanes per token (8 codes each)
  const int ds = tid & (tpt - 1);
  const int tsub = tid >> tpt_log2;
  const int nsub = kAttnThreads >> tpt_log2;
  const int d0 = ds * 8;
  const bool dact = d0 < D;

  const int t0 = split * tile;
  const int t1 = min(t0 + tile, T);

  // query slice for this lane's 8 dims, pre-scaled by softmax scale * log2(e)
  float qr[HB][8];
#pragma unroll
  for (int h = 0; h < HB; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = 0.f;
      if (h < nh && dact && d0 + i < D)
        v = sf_load_as_f32<QDT>(q, ((size_t)b * H + (size_t)kvh * G + h0 + h) * D + d0 + i) * qscale;
      qr[h][i] = v;
    }
  float acc[HB][8];
#pragma unroll
  for (int h = 0; h < HB; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.f;
  if (tid < HB) {
    m_s[tid] = -INFINITY;
    l_s[tid] = 0.f;
  }
  __syncthreads();

  const size_t base = ((size_t)b * KVH + kvh) * (size_t)T_cap;
  const int wave = tid >> 6, lane = tid & 63;

  for (int tt = t0; tt < t1; tt += kSubTile) {
    const int n = min(kSubTile, t1 - tt);
    // ---- scores
    for (int j = tsub; j < kSubTile; j += nsub) {
      float part[HB];
#pragma unroll
      for (int h = 0; h < HB; ++h) part[h] = 0.f;
      if (j < n && dact) {
        const int8_t *kp = kc + (base + tt + j) * (size_t)D + d0;
        float kf[8];
        if (d0 + 8 <= D) {
          const uint64_t kv = *(const uint64_t *)kp;
#pragma unroll
          for (int i = 0; i < 8; ++i) kf[i] = (float)(int8_t)(kv >> (8 * i));
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) kf[i] = d0 + i < D ? (float)kp[i] : 0.f;
        }
#pragma unroll
        for (int h = 0; h < HB; ++h)
#pragma unroll
          for (int i = 0; i < 8; ++i) part[h] = fmaf(qr[h][i], kf[i], part[h]);
      }
      for (int off = tpt >> 1; off >= 1; off >>= 1)
#pragma unroll
        for (int h = 0; h < HB; ++h) part[h] += sf_shfl_xor(part[h], off);
      if (ds == 0 && j < n) {
        const float ksc = sf_load_as_f32<SDT>(ks, base + tt + j);
#pragma unroll
        for (int h = 0; h < HB; ++h)
          if (h < nh) sc[h][j] = part[h] * ksc;
      }
    }
    __syncthreads();
    // ---- running softmax statistics, one wave per head
    for (int h = wave; h < nh; h += kAttnThreads / 64) {
      float mx = -INFINITY;
      for (int j = lane; j < n; j += 64) mx = fmaxf(mx, sc[h][j]);
      for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, sf_shfl_xor(mx, off));
      const float m_old = m_s[h];
      const float m_new = fmaxf(m_old, mx);
      float sum = 0.f;
      for (int j = lane; j < n; j += 64) {
        const float p = __builtin_amdgcn_exp2f(sc[h][j] - m_new);
        sc[h][j] = p;
        sum += p;
      }
      for (int off = 32; off >= 1; off >>= 1) sum += sf_shfl_xor(sum, off);
      if (lane == 0) {
        const float c = __builtin_amdgcn_exp2f(m_old - m_new);  // exp2(-inf) = 0
        c_s[h] = c;
        l_s[h] = l_s[h] * c + sum;
        m_s[h] = m_new;
      }
    }
    __syncthreads();
    // ---- P.V
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      const float c = h < nh ? c_s[h] : 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] *= c;
    }
    if (dact) {
      for (int j = tsub; j < n; j += nsub) {
        const int8_t *vp = vc + (base + tt + j) * (size_t)D + d0;
        const float vsc = sf_load_as_f32<SDT>(vs, base + tt + j);
        float vf[8];
        if (d0 + 8 <= D) {
          const uint64_t vv = *(const uint64_t *)vp;
#pragma unroll
          for (int i = 0; i < 8; ++i) vf[i] = (float)(int8_t)(vv >> (8 * i)) * vsc;
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) vf[i] = d0 + i < D ? (float)vp[i] * vsc : 0.f;
        }
#pragma unroll
        for (int h = 0; h < HB; ++h) {
          if (h < nh) {
            const float p = sc[h][j];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(p, vf[i], acc[h][i]);
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- reduce acc over the token sub-lanes: in-wave, then across waves
  for (int off = 32; off >= tpt; off >>= 1)
#pragma unroll
    for (int h = 0; h < HB; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] += sf_shfl_xor(acc[h][i], off);
  if (lane < tpt && dact) {
#pragma unroll
    for (int h = 0; h < HB; ++h)
      if (h < nh)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (d0 + i < D) red[((size_t)wave * HB + h) * D + d0 + i] = acc[h][i];
  }
  __syncthreads();
  const int nw = kAttnThreads / 64;
  for (int idx = tid; idx < nh * D; idx += kAttnThreads) {
    const int h = idx / D, d = idx - h * D;
    float s = 0.f;
    for (int w = 0; w < nw; ++w) s += red[((size_t)w * HB + h) * D + d];
    const size_t bh = (size_t)b * H + (size_t)kvh * G + h0 + h;
    part_acc[(bh * n_splits + split) * D + d] = s;
  }
  if (tid < nh) {
    const size_t bh = (size_t)b * H + (size_t)kvh * G + h0 + tid;
    part_ml[(bh * n_splits + split) * 2 + 0] = m_s[tid];
    part_ml[(bh * n_splits + split) * 2 + 1] = l_s[tid];
  }
}

// Merge the split partials of one (b, h): M = max m_s, c_s = 2^(m_s - M),
// out = sum_s c_s acc_s / max(sum_s c_s l_s, 1e-20) (q4_attention.py:256-261).
// The block first reduces M and L over the splits in parallel, keeps c_s in
// LDS, then (dim, split-slice) threads sum their slice and fold through LDS.
constexpr int kCombineThreads = 256;
constexpr int kMaxSplits = 2048;

__device__ __forceinline__ float block_reduce(float v, bool is_max, float *scratch) {
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = sf_shfl_xor(v, off);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  v = scratch[0];
  for (int w = 1; w < kCombineThreads / 64; ++w) v = is_max ? fmaxf(v, scratch[w]) : v + scratch[w];
  return v;
}

__global__ void __launch_bounds__(kCombineThreads)
k_attn_combine(const float *__restrict__ part_acc, const float *__restrict__ part_ml,
               void *__restrict__ out, int odt, int D, int n_splits) {
  __shared__ float c_s[kMaxSplits];
  __shared__ float scratch[kCombineThreads / 64];
  __shared__ float fold[kCombineThreads];
  const size_t bh = blockIdx.x;
  const int tid = threadIdx.x;
  const float *ml = part_ml + bh * n_splits * 2;
  float mx = -INFINITY;
  for (int s = tid; s < n_splits; s += kCombineThreads) mx = fmaxf(mx, ml[2 * s]);
  const float M = block_reduce(mx, true, scratch);
  float lsum = 0.f;
  for (int s = tid; s < n_splits; s += kCombineThreads) {
    const float c = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[2 * s] - M);
    c_s[s] = c;
    lsum = fmaf(ml[2 * s + 1], c, lsum);
  }
  const float L = block_reduce(lsum, false, scratch);  // also orders the c_s writes
  const float inv = 1.f / fmaxf(L, 1e-20f);
  // dims over lanes, splits over slices
  const int nslice = kCombineThreads / D > 0 ? kCombineThreads / D : 1;
  const int d = tid % D, slice = tid / D;
  float a = 0.f;
  if (slice < nslice && d < D) {
    const float *pa = part_acc + bh * n_splits * D + d;
#pragma unroll 4
    for (int s = slice; s < n_splits; s += nslice) a = fmaf(pa[(size_t)s * D], c_s[s], a);
  }
  fold[tid] = a;
  __syncthreads();
  for (int dd = tid; dd < D; dd += kCombineThreads) {
    float v = 0.f;
    for (int sl = 0; sl < nslice; ++sl) v += fold[sl * D + dd];
    v *= inv;
    if (odt == SF_F32) ((float *)out)[bh * D + dd] = v;
    else if (odt == SF_F16) ((f16 *)out)[bh * D + dd] = (f16)v;
    else ((uint16_t *)out)[bh * D + dd] = sf_f32_to_bf16(v);
  }
}

int pow2_log2_at_least(int v) {
  int l = 0;
  while ((1 << l) < v) ++l;
  return l;
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

extern "C" size_t sf_attn_workspace_bytes(int B, int H, int D, int n_splits) {
  if (B <= 0 || H <= 0 || D <= 0 || n_splits <= 0) return 0;
  const size_t rows = (size_t)B * H * n_splits;
  return sf_align256(rows * D * sizeof(float)) + rows * 2 * sizeof(float);
}

extern "C" int sf_attn_default_splits(int B, int KVH, int T) {
  // Enough (split, kv head, b) workgroups to cover the 256 CUs about twice,
  // without tiles shorter than one 64-token sub-tile.
  if (B <= 0 || KVH <= 0 || T <= 0) return 1;
  const int want = (512 + B * KVH - 1) / (B * KVH);
  const int cap = (T + kSubTile - 1) / kSubTile;
  int s = want < cap ? want : cap;
  return s < 1 ? 1 : s;
}

extern "C" int sf_attn_decode_i8kv(const void *q, int q_dtype, const int8_t *k_codes,
                                   const void *k_scales, const int8_t *v_codes,
                                   const void *v_scales, int scale_dtype, void *out, int out_dtype,
                                   void *workspace, size_t workspace_bytes, int B, int H, int KVH,
                                   int T, int T_cap, int D, float scale, int n_splits,
                                   void *stream) {
  SF_REQUIRE(B > 0 && H > 0 && KVH > 0 && D > 0 && T >= 0 && T <= T_cap, SF_EINVAL,
             "invalid attention shape B=%d H=%d KVH=%d T=%d T_cap=%d D=%d", B, H, KVH, T, T_cap, D);
  SF_REQUIRE(H % KVH == 0, SF_EINVAL, "n_heads=%d not a multiple of n_kv_heads=%d", H, KVH);
  SF_REQUIRE(D <= 256, SF_EINVAL, "head_dim=%d exceeds kernel's compile-time max 256", D);
  SF_REQUIRE(D % 8 == 0, SF_EUNSUPPORTED, "head_dim=%d: need a multiple of 8", D);
  SF_REQUIRE(q && k_codes && k_scales && v_codes && v_scales && out && workspace, SF_EINVAL,
             "null pointer argument");
  SF_REQUIRE(q_dtype >= SF_F32 && q_dtype <= SF_BF16 && out_dtype >= SF_F32 && out_dtype <= SF_BF16,
             SF_EINVAL, "bad q/out dtype");
  SF_REQUIRE(scale_dtype == SF_F16 || scale_dtype == SF_F32, SF_EINVAL, "bad scale dtype %d",
             scale_dtype);
  if (n_splits <= 0) n_splits = sf_attn_default_splits(B, KVH, T);
  // the reference's tiling: n_tiles = max(1, min(n_tiles, T)); tile = ceil(T / n_tiles)
  n_splits = n_splits < (T > 0 ? T : 1) ? n_splits : (T > 0 ? T : 1);
  if (n_splits > kMaxSplits) n_splits = kMaxSplits;
  if (n_splits < 1) n_splits = 1;
  const int tile = T > 0 ? (T + n_splits - 1) / n_splits : 0;
  const size_t need = sf_attn_workspace_bytes(B, H, D, n_splits);
  SF_REQUIRE(workspace_bytes >= need, SF_EINVAL, "attention workspace too small: %zu < %zu",
             workspace_bytes, need);
  float *part_acc = (float *)workspace;
  float *part_ml =
      (float *)((char *)workspace + sf_align256((size_t)B * H * n_splits * D * sizeof(float)));
  const int G = H / KVH;
  const int n_hblk = (G + kHeadsPerBlock - 1) / kHeadsPerBlock;
  const int tpt_log2 = pow2_log2_at_least(D / 8);
  const float qscale = scale * 1.4426950408889634f;  // softmax in base 2
  dim3 grid(n_splits, KVH * n_hblk, B);
  const size_t shm = (size_t)(kAttnThreads / 64) * kHeadsPerBlock * D * sizeof(float);
  hipStream_t st = (hipStream_t)stream;
#define SF_ATTN_LAUNCH(QD, SD)                                                                  \
  k_attn_split<QD, SD><<<grid, kAttnThreads, shm, st>>>(q, k_codes, k_scales, v_codes, v_scales, \
                                                         part_acc, part_ml, H, KVH, T, T_cap, D, \
                                                         qscale, n_splits, tile, tpt_log2)
  if (scale_dtype == SF_F16) {
    if (q_dtype == SF_F32) SF_ATTN_LAUNCH(SF_F32, SF_F16);
    else if (q_dtype == SF_F16) SF_ATTN_LAUNCH(SF_F16, SF_F16);
    else SF_ATTN_LAUNCH(SF_BF16, SF_F16);
  } else {
    if (q_dtype == SF_F32) SF_ATTN_LAUNCH(SF_F32, SF_F32);
    else if (q_dtype == SF_F16) SF_ATTN_LAUNCH(SF_F16, SF_F32);
    else SF_ATTN_LAUNCH(SF_BF16, SF_F32);
  }
#undef SF_ATTN_LAUNCH
  int rc = sf_check_launch("sf_attn_decode_i8kv(split)");
  if (rc) return rc;
  k_attn_combine<<<B * H, kCombineThreads, 0, st>>>(part_acc, part_ml, out, out_dtype, D, n_splits);
  return sf_check_launch("sf_attn_decode_i8kv(combine)");
}
