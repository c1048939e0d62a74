// model_ops.hip — the small per-token operations of the decoder around the
// int4 projections and the int8-KV attention (gfx950), for the model runner
// that restates the reference's LlamaModel / generate
// (/root/reference/siliconfer/model/layers.py:14-163, model/llama.py:38-83,
// engine/generate.py:117-180):
//
//   sf_embed            token ids -> fp32 residual rows (embedding gather)
//   sf_rmsnorm          optional residual add, then x * rsqrt(mean(x^2) + eps) * w
//   sf_rope_kv_append   rotate-half RoPE of q and k (host-computed fp32 cos /
//                       sin tables) and the int8 quantize-append of k and v
//   sf_silu_mul         silu(gate) * up
//   sf_lm_head_argmax   dense bf16 logits (the tied embedding) and the greedy
//                       token, with an optional device position increment
//
// Positions and the greedy token can live in device memory, so one decode
// step is a fixed sequence of launches that a HIP graph replays token after
// token with no host round trip.
#include <type_traits>
#include <math.h>

#include "sf_common.h"

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ void store_as(void *p, int dt, size_t i, float v) {
  if (dt == SF_F32) ((float *)p)[i] = v;
  else if (dt == SF_F16) ((f16 *)p)[i] = (f16)v;
  else ((uint16_t *)p)[i] = sf_f32_to_bf16(v);
}

__device__ __forceinline__ float load_as(const void *p, int dt, size_t i) {
  if (dt == SF_F32) return ((const float *)p)[i];
  if (dt == SF_F16) return (float)((const f16 *)p)[i];
  return sf_bf16_to_f32(((const uint16_t *)p)[i]);
}

// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads)
k_embed(const int32_t *__restrict__ ids, const void *__restrict__ table, int tdt,
        float *__restrict__ out, int H, int V) {
  const int r = blockIdx.x;
  int id = ids[r];
  id = id < 0 ? 0 : (id >= V ? V - 1 : id);  // ids are validated on the host
  for (int h = threadIdx.x; h < H; h += blockDim.x)
    out[(size_t)r * H + h] = load_as(table, tdt, (size_t)id * H + h);
}

// ---------------------------------------------------------------------------
// One block per row. mx.fast.rms_norm semantics: fp32 mean of squares,
// x * rsqrt(mean + eps) * w. Every wave computes the row's norm itself with
// sf_row_inv_rms (the order the projections that fold the norm in use too).
__global__ void __launch_bounds__(kThreads)
k_rmsnorm(float *__restrict__ x, const float *__restrict__ delta, const void *__restrict__ w,
          int wdt, void *__restrict__ out, int odt, int H, float eps) {
  const size_t r0 = (size_t)blockIdx.x * H;
  const float inv = sf_row_inv_rms(x + r0, delta ? delta + r0 : nullptr, H, eps);
  if (delta) __syncthreads();  // every wave has read x before it is overwritten
  for (int h = threadIdx.x; h < H; h += blockDim.x) {
    float v = x[r0 + h];
    if (delta) {
      v += delta[r0 + h];
      x[r0 + h] = v;
    }
    store_as(out, odt, r0 + h, sf_opaque(v * inv * load_as(w, wdt, h)));
  }
}

// k_rmsnorm with the residual delta as K-split partials (S of them, MN apart):
// each element's delta summed in split order from 0 (the GEMM reduce's sum)
// goes into x first; after the barrier the row's norm reads x as k_rmsnorm
// reads x + delta, so x and out get k_rmsnorm's bits.
__global__ void __launch_bounds__(kThreads)
k_rmsnorm_parts(float *__restrict__ x, const float *__restrict__ part, int S, size_t MN,
                const void *__restrict__ w, int wdt, void *__restrict__ out, int odt, int H,
                float eps) {
  const size_t r0 = (size_t)blockIdx.x * H;
  constexpr int C = 8;  // partials whose loads go out together (a split GEMM has at most 8)
  if ((H & 3) == 0 && (((uintptr_t)x | (uintptr_t)part) & 15) == 0 && MN % 4 == 0) {
    // 4 consecutive elements per thread, every load in flight before the sums
    float4_t *x4 = (float4_t *)(x + r0);
    for (int i = threadIdx.x; i < (H >> 2); i += blockDim.x) {
      const float4_t xv = x4[i];
      float4_t d = {0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < S; s0 += C) {
        float4_t pv[C];
#pragma unroll
        for (int j = 0; j < C; ++j)
          if (s0 + j < S) pv[j] = ((const float4_t *)(part + (size_t)(s0 + j) * MN + r0))[i];
#pragma unroll
        for (int j = 0; j < C; ++j)
          if (s0 + j < S) d += pv[j];
      }
      x4[i] = xv + d;
    }
  } else {
    for (int h = threadIdx.x; h < H; h += blockDim.x) {
      float d = 0.f;
      for (int s = 0; s < S; ++s) d += part[(size_t)s * MN + r0 + h];
      x[r0 + h] = x[r0 + h] + d;
    }
  }
  __syncthreads();  // the block's x stores are seen by every wave's norm
  const float inv = sf_row_inv_rms(x + r0, nullptr, H, eps);
  for (int h = threadIdx.x; h < H; h += blockDim.x)
    store_as(out, odt, r0 + h, sf_opaque(x[r0 + h] * inv * load_as(w, wdt, h)));
}

// ---------------------------------------------------------------------------
// One wave per (row, head) of the fused q|k|v projection output
// qkv [rows][(H + 2 KVH) * D]: sf_rope_append_head (rotate-half RoPE with the
// host-made fp32 cos / sin tables, q to q_out, k and v quantized per (head,
// token) into the cache at position pos0 + row, batch 1).
__global__ void __launch_bounds__(64)
k_rope_kv_append(const float *__restrict__ qkv, SfRopeAppend a, const int *__restrict__ pos_dev,
                 int pos_host) {
  const int row = blockIdx.x, head = blockIdx.y;
  const int pos = (pos_dev ? *pos_dev : pos_host) + row;
  if (pos < 0 || pos >= a.T_cap || pos >= a.max_pos) return;  // the host keeps positions in range
  const int width = (a.H + 2 * a.KVH) * a.D;
  sf_rope_append_head(a, qkv + (size_t)row * width + (size_t)head * a.D, head, pos, row);
}

// k_rope_kv_append with the q|k|v rows as S K-split partials (MN apart) of the
// projection plus its bias: each value summed in split order from 0, then the
// bias added (the GEMM reduce's arithmetic, so the head sees the values the
// reduce would have stored), staged in LDS for the head.
__global__ void __launch_bounds__(64)
k_rope_kv_append_parts(const float *__restrict__ part, int S, size_t MN,
                       const void *__restrict__ bias, int bdt, SfRopeAppend a,
                       const int *__restrict__ pos_dev, int pos_host) {
  __shared__ float xs[256];
  const int row = blockIdx.x, head = blockIdx.y;
  const int pos = (pos_dev ? *pos_dev : pos_host) + row;
  if (pos < 0 || pos >= a.T_cap || pos >= a.max_pos) return;  // the host keeps positions in range
  const int width = (a.H + 2 * a.KVH) * a.D;
  const size_t base = (size_t)row * width + (size_t)head * a.D;
  constexpr int C = 8;  // partials whose loads go out together
  for (int d = threadIdx.x; d < a.D; d += 64) {
    float v = 0.f;
    for (int s0 = 0; s0 < S; s0 += C) {
      float pv[C];
#pragma unroll
      for (int j = 0; j < C; ++j)
        if (s0 + j < S) pv[j] = part[(size_t)(s0 + j) * MN + base + d];
#pragma unroll
      for (int j = 0; j < C; ++j)
        if (s0 + j < S) v += pv[j];
    }
    if (bias) v += load_as(bias, bdt, (size_t)head * a.D + d);
    xs[d] = v;
  }
  __syncthreads();
  sf_rope_append_head(a, xs, head, pos, row);
}

// ---------------------------------------------------------------------------
// out[r][i] = silu(gu[r][i]) * gu[r][I + i], silu(g) = g / (1 + exp(-g)).
__global__ void __launch_bounds__(kThreads)
k_silu_mul(const float *__restrict__ gu, void *__restrict__ out, int odt, int I, long long n) {
  for (long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x; t < n;
       t += (long long)gridDim.x * blockDim.x) {
    const long long r = t / I, i = t - r * I;
    const float g = gu[r * 2 * I + i], u = gu[r * 2 * I + I + i];
    store_as(out, odt, (size_t)t, sf_silu_mul(g, u));
  }
}

// ---------------------------------------------------------------------------
// logits[v] = sum_k W[v][k] x[k], W bf16 [V][H] (the tied embedding table), x
// staged in LDS as fp32. A wave takes rows w, w + n_waves, ...: its lanes load
// the row in 16-byte chunks (8 bf16), four rows in flight, and a DPP tree
// sums each row. Every wave keeps its best (value, index) — greedy argmax,
// lowest index on ties like mx.argmax — the block folds them, writes its
// partial with agent-scope atomic stores, and the last block to finish
// (counter) folds all partials, writes the token, resets the counter and
// increments the device position if asked.
constexpr int kHeadBlocks = 1024;
constexpr int kHeadMaxH = 8192;

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// Ordering of the last-block fold, stated for the hardware (the atomics are
// relaxed, so C++ ordering alone would allow the count to pass the partials):
// every partial is an agent-scope atomic store, which writes through to the
// device-coherent level; s_waitcnt(0) returns only after the storing wave's
// stores are acknowledged there, and the workgroup barrier (where used) puts
// every wave's wait before tid 0's count increment. The block that takes the
// last count therefore reads, with agent-scope atomic loads (which bypass the
// non-coherent caches), partials that were all acknowledged before any count
// that preceded its own. An acq_rel increment would add an L2 write-back per
// block (agent-scope release on gfx950) for stores already written through.
//
// NORM: x is the fp32 residual row and the block applies the final RMSNorm
// itself (sf_row_inv_rms, then x * inv * norm_w rounded to XDT, the values
// sf_rmsnorm would have stored in an XDT buffer).
template <int XDT, bool NORM>
__global__ void __launch_bounds__(kThreads)
k_lm_head_argmax(const uint16_t *__restrict__ w, const void *__restrict__ x,
                 const float *__restrict__ norm_w, float eps, float *__restrict__ logits, int V,
                 int H, int32_t *__restrict__ token_out, int *__restrict__ pos_inc,
                 int32_t *__restrict__ hist, float *part_val, int *part_idx, unsigned *counter) {
  __shared__ __attribute__((aligned(16))) float xs[kHeadMaxH];
  __shared__ float bv_s[kThreads / 64];
  __shared__ int bi_s[kThreads / 64];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nch = H >> 3;  // 16-byte chunks per row
  const int n_waves = gridDim.x * (kThreads / 64);
  const int gw = blockIdx.x * (kThreads / 64) + wave;
  constexpr int RU = 4;   // rows per wave and pass
  constexpr int CPL = 2;  // chunks per lane (H <= 1024 in one pass)
  // a pass's rows: two passes in flight (the next pass's loads go out before
  // this pass's arithmetic), the first before the activations' norm, which
  // they do not depend on; nontemporal, the table is streamed once
  u32x4 cb[2][RU][CPL];
  auto load_rows = [&](int r0, u32x4 (&c)[RU][CPL]) {
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int row = min(r0 + u * n_waves, V - 1);
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int ch = min(lane + 64 * j, nch - 1);
        c[u][j] = __builtin_nontemporal_load((const u32x4 *)(w + (size_t)row * H + (size_t)ch * 8));
      }
    }
  };
  if (gw < V) load_rows(gw, cb[0]);
  if constexpr (NORM) {
    const float *xf = (const float *)x;
    const float inv = sf_row_inv_rms(xf, nullptr, H, eps);
    for (int h = tid; h < H; h += kThreads) xs[h] = sf_round_as<XDT>(xf[h] * inv * norm_w[h]);
  } else {
    for (int h = tid; h < H; h += kThreads) xs[h] = sf_load_as_f32<XDT>(x, h);
  }
  __syncthreads();
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  // one pass: the RU rows r0 + u * n_waves from c
  auto pass = [&](int r0, const u32x4 (&c)[RU][CPL]) {
    // rows longer than CPL * 64 chunks: the rest, one pass at a time
    float acc[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int ch = lane + 64 * j;
        if (ch < nch) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t p = c[u][j][e];
            a = fmaf(sf_bitcast<float>(p << 16), xs[ch * 8 + 2 * e], a);
            a = fmaf(sf_bitcast<float>(p & 0xffff0000u), xs[ch * 8 + 2 * e + 1], a);
          }
        }
      }
      const int row = r0 + u * n_waves;
      for (int ch = lane + 64 * CPL; ch < nch; ch += 64) {
        const u32x4 q = __builtin_nontemporal_load((const u32x4 *)(w + (size_t)min(row, V - 1) * H + (size_t)ch * 8));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a = fmaf(sf_bitcast<float>(q[e] << 16), xs[ch * 8 + 2 * e], a);
          a = fmaf(sf_bitcast<float>(q[e] & 0xffff0000u), xs[ch * 8 + 2 * e + 1], a);
        }
      }
      acc[u] = a;
    }
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const float a = sf_wave_sum(acc[u]);
      const int row = r0 + u * n_waves;
      if (row < V) {
        if (lane == 0 && logits) logits[row] = a;
        if (better(a, row, best, best_i)) {
          best = a;
          best_i = row;
        }
      }
    }
  };
  const int step = RU * n_waves;
  for (int r0 = gw; r0 < V; r0 += 2 * step) {  // two passes per turn: static buffers
    if (r0 + step < V) load_rows(r0 + step, cb[1]);
    pass(r0, cb[0]);
    if (r0 + step >= V) break;
    if (r0 + 2 * step < V) load_rows(r0 + 2 * step, cb[0]);
    pass(r0 + step, cb[1]);
  }
  if (lane == 0) {
    bv_s[wave] = best;
    bi_s[wave] = best_i;
  }
  __syncthreads();
  if (tid == 0) {
    float b = bv_s[0];
    int bi = bi_s[0];
    for (int k = 1; k < kThreads / 64; ++k)
      if (better(bv_s[k], bi_s[k], b, bi)) {
        b = bv_s[k];
        bi = bi_s[k];
      }
    __hip_atomic_store((uint32_t *)(part_val + blockIdx.x), sf_bitcast<uint32_t>(b),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(part_idx + blockIdx.x, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the partial is stored before the count (see above)
    const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  float b = -INFINITY;
  int bi = 0x7fffffff;
  for (int k = tid; k < (int)gridDim.x; k += kThreads) {
    const float v = sf_bitcast<float>(__hip_atomic_load((const uint32_t *)(part_val + k),
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    const int i = __hip_atomic_load(part_idx + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (better(v, i, b, bi)) {
      b = v;
      bi = i;
    }
  }
  // fold (value, index) over the block
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(b, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (better(ov, oi, b, bi)) {
      b = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    bv_s[wave] = b;
    bi_s[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float fb = bv_s[0];
    int fi = bi_s[0];
    for (int k = 1; k < kThreads / 64; ++k)
      if (better(bv_s[k], bi_s[k], fb, fi)) {
        fb = bv_s[k];
        fi = bi_s[k];
      }
    const int tok = fi == 0x7fffffff ? 0 : fi;
    token_out[0] = tok;
    if (pos_inc) {
      const int p = pos_inc[0];
      if (hist) hist[p] = tok;
      pos_inc[0] = p + 1;
    }
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// Logits and greedy tokens of B <= 8 rows at once (a speculative verify's K+1
// positions): one pass over the bf16 table for all rows, x staged in LDS as
// fp32 [B][H]. Each row's dot products are the same fma chains and DPP tree as
// k_lm_head_argmax, so a row's logits equal the single-row kernel's bit for
// bit; per-row (value, index) partials and a last-block fold per row. x stays
// in its own type in LDS (fp16 / bf16 widen exactly when read).
constexpr int kRowsMax = 8;
constexpr size_t kRowsLdsBytes = 65536;  // B * H * sizeof(x element)

template <int XDT>
__global__ void __launch_bounds__(kThreads)
k_lm_head_rows(const uint16_t *__restrict__ w, const void *__restrict__ x,
               float *__restrict__ logits, int V, int H, int B, int32_t *__restrict__ tokens_out,
               float *part_val, int *part_idx, unsigned *counter) {
  using XS = std::conditional_t<XDT == SF_F32, float, uint16_t>;
  extern __shared__ __attribute__((aligned(16))) unsigned char xs_raw[];
  XS *xs = (XS *)xs_raw;  // [B][H]
  __shared__ float bv_s[kRowsMax][kThreads / 64];
  __shared__ int bi_s[kRowsMax][kThreads / 64];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < B * H; i += kThreads) xs[i] = ((const XS *)x)[i];
  __syncthreads();
  const int nch = H >> 3;
  const int n_waves = gridDim.x * (kThreads / 64);
  const int gw = blockIdx.x * (kThreads / 64) + wave;
  float best[kRowsMax];
  int best_i[kRowsMax];
#pragma unroll
  for (int b = 0; b < kRowsMax; ++b) {
    best[b] = -INFINITY;
    best_i[b] = 0x7fffffff;
  }
  constexpr int RU = 4, CPL = 2;  // as k_lm_head_argmax
  for (int r0 = gw; r0 < V; r0 += RU * n_waves) {
    u32x4 c[RU][CPL];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int row = min(r0 + u * n_waves, V - 1);
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        const int ch = min(lane + 64 * j, nch - 1);
        c[u][j] = __builtin_nontemporal_load((const u32x4 *)(w + (size_t)row * H + (size_t)ch * 8));
      }
    }
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int row = r0 + u * n_waves;
      for (int b = 0; b < B; ++b) {
        const XS *xb = xs + (size_t)b * H;
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const int ch = lane + 64 * j;
          if (ch < nch) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t p = c[u][j][e];
              a = fmaf(sf_bitcast<float>(p << 16), sf_load_as_f32<XDT>(xb, ch * 8 + 2 * e), a);
              a = fmaf(sf_bitcast<float>(p & 0xffff0000u), sf_load_as_f32<XDT>(xb, ch * 8 + 2 * e + 1), a);
            }
          }
        }
        for (int ch = lane + 64 * CPL; ch < nch; ch += 64) {
          const u32x4 qv =
              __builtin_nontemporal_load((const u32x4 *)(w + (size_t)min(row, V - 1) * H + (size_t)ch * 8));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a = fmaf(sf_bitcast<float>(qv[e] << 16), sf_load_as_f32<XDT>(xb, ch * 8 + 2 * e), a);
            a = fmaf(sf_bitcast<float>(qv[e] & 0xffff0000u), sf_load_as_f32<XDT>(xb, ch * 8 + 2 * e + 1), a);
          }
        }
        a = sf_wave_sum(a);
        if (row < V) {
          if (lane == 0 && logits) logits[(size_t)b * V + row] = a;
          // runtime b: select into the compile-time slots
#pragma unroll
          for (int k = 0; k < kRowsMax; ++k)
            if (k == b && better(a, row, best[k], best_i[k])) {
              best[k] = a;
              best_i[k] = row;
            }
        }
      }
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < kRowsMax; ++k) {
      bv_s[k][wave] = best[k];
      bi_s[k][wave] = best_i[k];
    }
  }
  __syncthreads();
  if (tid < B) {
    float bb = bv_s[tid][0];
    int bi = bi_s[tid][0];
    for (int k = 1; k < kThreads / 64; ++k)
      if (better(bv_s[tid][k], bi_s[tid][k], bb, bi)) {
        bb = bv_s[tid][k];
        bi = bi_s[tid][k];
      }
    __hip_atomic_store((uint32_t *)(part_val + (size_t)tid * gridDim.x + blockIdx.x),
                       sf_bitcast<uint32_t>(bb), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(part_idx + (size_t)tid * gridDim.x + blockIdx.x, bi, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the partials are stored before the count (ordering argument above k_lm_head_argmax)
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  // the last block folds each row's partials: wave w takes rows w, w + 4
  {
    for (int b = wave; b < B; b += kThreads / 64) {
      float bb = -INFINITY;
      int bi = 0x7fffffff;
      for (int k = lane; k < (int)gridDim.x; k += 64) {
        const float v = sf_bitcast<float>(__hip_atomic_load(
            (const uint32_t *)(part_val + (size_t)b * gridDim.x + k), __ATOMIC_RELAXED,
            __HIP_MEMORY_SCOPE_AGENT));
        const int i = __hip_atomic_load(part_idx + (size_t)b * gridDim.x + k, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
        if (better(v, i, bb, bi)) {
          bb = v;
          bi = i;
        }
      }
      for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bb, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (better(ov, oi, bb, bi)) {
          bb = ov;
          bi = oi;
        }
      }
      if (lane == 0) tokens_out[b] = bi == 0x7fffffff ? 0 : bi;
    }
  }
  __syncthreads();
  if (tid == 0)  // ready for the next call on this workspace
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// The same B <= 8 rows on MFMA (fp16 / bf16 activations, H % 32 == 0,
// H <= 2048): v_mfma_f32_16x16x32_bf16 with the batch as the A operand, each
// activation split exactly into a bf16 high part (A rows 0..7) and the
// remainder (rows 8..15; an fp16 value has 11 significant bits, so the
// remainder has at most 3 and is exact in bf16, a bf16 one has none), and 16
// table rows as the B operand. Products are exact (bf16 x bf16) and summed in
// fp32; logit = C[b] + C[8 + b]. The VALU kernel above spends 8 fma per table
// element at B = 8; here the MFMA does that work and the kernel streams the
// table. The activations sit in LDS in fragment order: fragment
// (ks * 4 + kg) * 16 + i is the 8 bf16 of A row i at k = 32 ks + 8 kg .. +7,
// so lane l reads fragment (ks * 4 + l / 16) * 16 + l % 16: one linear 16-byte
// read per lane, no bank conflict.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

template <int XDT>
__global__ void __launch_bounds__(kThreads)
k_lm_head_rows_mfma(const uint16_t *__restrict__ w, const void *__restrict__ x,
                    float *__restrict__ logits, int V, int H, int B,
                    int32_t *__restrict__ tokens_out, float *part_val, int *part_idx,
                    unsigned *counter) {
  extern __shared__ __attribute__((aligned(16))) u32x4 xa[];  // [H / 32 * 4][16] fragments
  __shared__ float bv_s[kRowsMax][kThreads / 64];
  __shared__ int bi_s[kRowsMax][kThreads / 64];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nks = H >> 5;
  for (int f = tid; f < nks * 64; f += kThreads) {
    const int i = f & 15, kgs = f >> 4;
    const int b = i & 7;
    uint32_t pk[4];
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      uint32_t h2[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int k = kgs * 8 + e2 * 2 + t;
        const float v = b < B ? sf_load_as_f32<XDT>(x, (size_t)b * H + k) : 0.f;
        const uint32_t hi = sf_bitcast<uint32_t>(v) & 0xffff0000u;
        h2[t] = i < 8 ? hi >> 16 : sf_bitcast<uint32_t>(v - sf_bitcast<float>(hi)) >> 16;
      }
      pk[e2] = h2[0] | h2[1] << 16;
    }
    xa[f] = u32x4{pk[0], pk[1], pk[2], pk[3]};
  }
  __syncthreads();

  const int nt = (V + 15) >> 4;
  const int n_waves = gridDim.x * (kThreads / 64);
  const int gw = blockIdx.x * (kThreads / 64) + wave;
  const int i16 = lane & 15, kg = lane >> 4;
  // lane l < 32 tracks batch rows 4 (l / 16) + r, r = 0..3
  float best[4];
  int best_i[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    best[r] = -INFINITY;
    best_i[r] = 0x7fffffff;
  }
  constexpr int KQ = 8;  // table loads in flight per lane
  for (int t = gw; t < nt; t += n_waves) {
    const int v0 = t * 16;
    const uint16_t *wr = w + (size_t)min(v0 + i16, V - 1) * H + kg * 8;
    float4_t c = {0.f, 0.f, 0.f, 0.f};
    for (int ks0 = 0; ks0 < nks; ks0 += KQ) {
      u32x4 wv[KQ];
#pragma unroll
      for (int q = 0; q < KQ; ++q)
        wv[q] = __builtin_nontemporal_load((const u32x4 *)(wr + (size_t)min(ks0 + q, nks - 1) * 32));
#pragma unroll
      for (int q = 0; q < KQ; ++q) {
        if (ks0 + q >= nks) break;  // uniform
        const u32x4 a = xa[((ks0 + q) * 4 + kg) * 16 + i16];
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sf_bitcast<bf16x8_t>(a),
                                                    sf_bitcast<bf16x8_t>(wv[q]), c, 0, 0, 0);
      }
    }
    // lane l holds C[4 (l / 16) + r][l % 16]: rows 0..7 are the high parts,
    // 8..15 the remainders of the same batch rows, 32 lanes apart
    const int vv = v0 + i16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float sum = c[r] + __shfl_xor(c[r], 32, 64);
      const int b = 4 * (kg & 1) + r;
      if (kg < 2 && b < B && vv < V) {
        if (logits) logits[(size_t)b * V + vv] = sum;
        if (better(sum, vv, best[r], best_i[r])) {
          best[r] = sum;
          best_i[r] = vv;
        }
      }
    }
  }
  // fold each batch row over its 16 lanes, then the waves through LDS
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      const float ov = __shfl_xor(best[r], off, 64);
      const int oi = __shfl_xor(best_i[r], off, 64);
      if (better(ov, oi, best[r], best_i[r])) {
        best[r] = ov;
        best_i[r] = oi;
      }
    }
  }
  if (lane == 0 || lane == 16) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      bv_s[4 * (lane >> 4) + r][wave] = best[r];
      bi_s[4 * (lane >> 4) + r][wave] = best_i[r];
    }
  }
  __syncthreads();
  if (tid < B) {
    float bb = bv_s[tid][0];
    int bi = bi_s[tid][0];
    for (int k = 1; k < kThreads / 64; ++k)
      if (better(bv_s[tid][k], bi_s[tid][k], bb, bi)) {
        bb = bv_s[tid][k];
        bi = bi_s[tid][k];
      }
    __hip_atomic_store((uint32_t *)(part_val + (size_t)tid * gridDim.x + blockIdx.x),
                       sf_bitcast<uint32_t>(bb), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(part_idx + (size_t)tid * gridDim.x + blockIdx.x, bi, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the partials are stored before the count (ordering argument above k_lm_head_argmax)
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  for (int b = wave; b < B; b += kThreads / 64) {
    float bb = -INFINITY;
    int bi = 0x7fffffff;
    for (int k = lane; k < (int)gridDim.x; k += 64) {
      const float v = sf_bitcast<float>(__hip_atomic_load(
          (const uint32_t *)(part_val + (size_t)b * gridDim.x + k), __ATOMIC_RELAXED,
          __HIP_MEMORY_SCOPE_AGENT));
      const int i = __hip_atomic_load(part_idx + (size_t)b * gridDim.x + k, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
      if (better(v, i, bb, bi)) {
        bb = v;
        bi = i;
      }
    }
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bb, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (better(ov, oi, bb, bi)) {
        bb = ov;
        bi = oi;
      }
    }
    if (lane == 0) tokens_out[b] = bi == 0x7fffffff ? 0 : bi;
  }
  __syncthreads();
  if (tid == 0)  // ready for the next call on this workspace
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" int sf_embed(const int32_t *ids, const void *table, int table_dtype, float *out,
                        int rows, int H, int V, void *stream) {
  SF_REQUIRE(rows > 0 && H > 0 && V > 0, SF_EINVAL, "invalid embedding shape rows=%d H=%d V=%d",
             rows, H, V);
  SF_REQUIRE(ids && table && out, SF_EINVAL, "null pointer argument");
  SF_REQUIRE(table_dtype >= SF_F32 && table_dtype <= SF_BF16, SF_EINVAL, "bad table dtype %d",
             table_dtype);
  k_embed<<<rows, kThreads, 0, (hipStream_t)stream>>>(ids, table, table_dtype, out, H, V);
  return sf_check_launch("sf_embed");
}

extern "C" int sf_rmsnorm(float *x, const float *delta, const void *w, int w_dtype, void *out,
                          int out_dtype, int rows, int H, float eps, void *stream) {
  SF_REQUIRE(rows > 0 && H > 0, SF_EINVAL, "invalid rmsnorm shape rows=%d H=%d", rows, H);
  SF_REQUIRE(x && w && out, SF_EINVAL, "null pointer argument");
  SF_REQUIRE(w_dtype >= SF_F32 && w_dtype <= SF_BF16 && out_dtype >= SF_F32 && out_dtype <= SF_BF16,
             SF_EINVAL, "bad rmsnorm dtype");
  k_rmsnorm<<<rows, kThreads, 0, (hipStream_t)stream>>>(x, delta, w, w_dtype, out, out_dtype, H,
                                                         eps);
  return sf_check_launch("sf_rmsnorm");
}

extern "C" int sf_rmsnorm_partials(float *x, const float *part, int n_parts, const void *w,
                                   int w_dtype, void *out, int out_dtype, int rows, int H, float eps,
                                   void *stream) {
  SF_REQUIRE(rows > 0 && H > 0 && n_parts > 0, SF_EINVAL,
             "invalid rmsnorm shape rows=%d H=%d n_parts=%d", rows, H, n_parts);
  SF_REQUIRE(x && part && w && out, SF_EINVAL, "null pointer argument");
  SF_REQUIRE(w_dtype >= SF_F32 && w_dtype <= SF_BF16 && out_dtype >= SF_F32 && out_dtype <= SF_BF16,
             SF_EINVAL, "bad rmsnorm dtype");
  k_rmsnorm_parts<<<rows, kThreads, 0, (hipStream_t)stream>>>(x, part, n_parts, (size_t)rows * H, w,
                                                              w_dtype, out, out_dtype, H, eps);
  return sf_check_launch("sf_rmsnorm_partials");
}

extern "C" int sf_rope_kv_append(const float *qkv, const float *cos_t, const float *sin_t,
                                 int max_pos, void *q_out, int q_dtype, int8_t *k_codes,
                                 void *k_scales, int8_t *v_codes, void *v_scales, int scale_dtype,
                                 int rows, int H, int KVH, int D, int T_cap, const int *pos_dev,
                                 int pos_host, void *stream) {
  SF_REQUIRE(rows > 0 && H > 0 && KVH > 0 && D > 0 && T_cap > 0 && max_pos > 0, SF_EINVAL,
             "invalid rope/append shape rows=%d H=%d KVH=%d D=%d T_cap=%d", rows, H, KVH, D,
             T_cap);
  SF_REQUIRE(D % 2 == 0 && D <= 256, SF_EUNSUPPORTED, "head_dim=%d: need an even D <= 256", D);
  SF_REQUIRE(qkv && cos_t && sin_t && q_out && k_codes && k_scales && v_codes && v_scales,
             SF_EINVAL, "null pointer argument");
  SF_REQUIRE(q_dtype >= SF_F32 && q_dtype <= SF_BF16, SF_EINVAL, "bad q dtype %d", q_dtype);
  SF_REQUIRE(scale_dtype == SF_F16 || scale_dtype == SF_F32, SF_EINVAL, "bad scale dtype %d",
             scale_dtype);
  if (!pos_dev)
    SF_REQUIRE(pos_host >= 0 && pos_host + rows <= T_cap && pos_host + rows <= max_pos, SF_EINVAL,
               "positions %d..%d exceed the cache capacity %d or the RoPE table %d", pos_host,
               pos_host + rows - 1, T_cap, max_pos);
  dim3 grid(rows, H + 2 * KVH);
  const SfRopeAppend a{cos_t, sin_t, max_pos, q_out, q_dtype, k_codes, k_scales, v_codes,
                       v_scales, scale_dtype, H, KVH, D, T_cap};
  k_rope_kv_append<<<grid, 64, 0, (hipStream_t)stream>>>(qkv, a, pos_dev, pos_host);
  return sf_check_launch("sf_rope_kv_append");
}

extern "C" int sf_rope_kv_append_partials(const float *part, int n_parts, const void *bias,
                                          int bias_dtype, const float *cos_t, const float *sin_t,
                                          int max_pos, void *q_out, int q_dtype, int8_t *k_codes,
                                          void *k_scales, int8_t *v_codes, void *v_scales,
                                          int scale_dtype, int rows, int H, int KVH, int D,
                                          int T_cap, const int *pos_dev, int pos_host,
                                          void *stream) {
  SF_REQUIRE(n_parts > 0, SF_EINVAL, "invalid n_parts=%d", n_parts);
  SF_REQUIRE(!bias || (bias_dtype >= SF_F32 && bias_dtype <= SF_BF16), SF_EINVAL,
             "bad bias dtype %d", bias_dtype);
  SF_REQUIRE(rows > 0 && H > 0 && KVH > 0 && D > 0 && T_cap > 0 && max_pos > 0, SF_EINVAL,
             "invalid rope/append shape rows=%d H=%d KVH=%d D=%d T_cap=%d", rows, H, KVH, D,
             T_cap);
  SF_REQUIRE(D % 2 == 0 && D <= 256, SF_EUNSUPPORTED, "head_dim=%d: need an even D <= 256", D);
  SF_REQUIRE(part && cos_t && sin_t && q_out && k_codes && k_scales && v_codes && v_scales,
             SF_EINVAL, "null pointer argument");
  SF_REQUIRE(q_dtype >= SF_F32 && q_dtype <= SF_BF16, SF_EINVAL, "bad q dtype %d", q_dtype);
  SF_REQUIRE(scale_dtype == SF_F16 || scale_dtype == SF_F32, SF_EINVAL, "bad scale dtype %d",
             scale_dtype);
  if (!pos_dev)
    SF_REQUIRE(pos_host >= 0 && pos_host + rows <= T_cap && pos_host + rows <= max_pos, SF_EINVAL,
               "positions %d..%d exceed the cache capacity %d or the RoPE table %d", pos_host,
               pos_host + rows - 1, T_cap, max_pos);
  dim3 grid(rows, H + 2 * KVH);
  const SfRopeAppend a{cos_t, sin_t, max_pos, q_out, q_dtype, k_codes, k_scales, v_codes,
                       v_scales, scale_dtype, H, KVH, D, T_cap};
  const size_t MN = (size_t)rows * (H + 2 * KVH) * D;
  k_rope_kv_append_parts<<<grid, 64, 0, (hipStream_t)stream>>>(part, n_parts, MN, bias,
                                                               bias_dtype, a, pos_dev, pos_host);
  return sf_check_launch("sf_rope_kv_append_partials");
}

extern "C" int sf_silu_mul(const float *gu, void *out, int out_dtype, int rows, int I,
                           void *stream) {
  SF_REQUIRE(rows > 0 && I > 0, SF_EINVAL, "invalid silu_mul shape rows=%d I=%d", rows, I);
  SF_REQUIRE(gu && out, SF_EINVAL, "null pointer argument");
  SF_REQUIRE(out_dtype >= SF_F32 && out_dtype <= SF_BF16, SF_EINVAL, "bad out dtype %d", out_dtype);
  const long long n = (long long)rows * I;
  long long blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 4096) blocks = 4096;
  k_silu_mul<<<(unsigned)blocks, kThreads, 0, (hipStream_t)stream>>>(gu, out, out_dtype, I, n);
  return sf_check_launch("sf_silu_mul");
}

extern "C" size_t sf_lm_head_workspace_bytes(int V) {
  (void)V;
  // counter (256 B slot), then kHeadBlocks (value, index) partials
  return 256 + (size_t)kHeadBlocks * (sizeof(float) + sizeof(int));
}

static int lm_head_launch(const void *w, const void *x, int x_dtype, const float *norm_w,
                          float eps, float *logits, int V, int H, int32_t *token_out, int *pos_inc,
                          int32_t *hist, void *workspace, size_t workspace_bytes, void *stream) {
  SF_REQUIRE(V > 0 && H > 0, SF_EINVAL, "invalid lm_head shape V=%d H=%d", V, H);
  SF_REQUIRE(H % 8 == 0 && H <= kHeadMaxH, SF_EUNSUPPORTED,
             "hidden=%d: need a multiple of 8 up to %d", H, kHeadMaxH);
  SF_REQUIRE(w && x && token_out && workspace, SF_EINVAL, "null pointer argument");
  SF_REQUIRE(!hist || pos_inc, SF_EINVAL, "a token history needs the device position");
  SF_REQUIRE(x_dtype >= SF_F32 && x_dtype <= SF_BF16, SF_EINVAL, "bad x dtype %d", x_dtype);
  SF_REQUIRE(workspace_bytes >= sf_lm_head_workspace_bytes(V), SF_EINVAL,
             "lm_head workspace too small: %zu < %zu", workspace_bytes,
             sf_lm_head_workspace_bytes(V));
  SF_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)workspace & 255) == 0, SF_EINVAL,
             "weights must be 16-byte and workspace 256-byte aligned");
  unsigned *counter = (unsigned *)workspace;
  float *pv = (float *)((char *)workspace + 256);
  int *pi = (int *)(pv + kHeadBlocks);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *wb = (const uint16_t *)w;
#define SF_HEAD(XD, NM)                                                                        \
  k_lm_head_argmax<XD, NM><<<kHeadBlocks, kThreads, 0, st>>>(wb, x, norm_w, eps, logits, V, H, \
                                                             token_out, pos_inc, hist, pv, pi, \
                                                             counter)
  if (norm_w) {
    if (x_dtype == SF_F32) SF_HEAD(SF_F32, true);
    else if (x_dtype == SF_F16) SF_HEAD(SF_F16, true);
    else SF_HEAD(SF_BF16, true);
  } else {
    if (x_dtype == SF_F32) SF_HEAD(SF_F32, false);
    else if (x_dtype == SF_F16) SF_HEAD(SF_F16, false);
    else SF_HEAD(SF_BF16, false);
  }
#undef SF_HEAD
  return SF_OK;
}

extern "C" int sf_lm_head_argmax(const void *w, const void *x, int x_dtype, float *logits, int V,
                                 int H, int32_t *token_out, int *pos_inc, int32_t *hist,
                                 void *workspace, size_t workspace_bytes, void *stream) {
  const int rc = lm_head_launch(w, x, x_dtype, nullptr, 0.f, logits, V, H, token_out, pos_inc,
                                hist, workspace, workspace_bytes, stream);
  return rc ? rc : sf_check_launch("sf_lm_head_argmax");
}

extern "C" int sf_lm_head_argmax_rmsnorm(const void *w, const float *h, const float *norm_w,
                                         float eps, int act_dtype, float *logits, int V, int H,
                                         int32_t *token_out, int *pos_inc, int32_t *hist,
                                         void *workspace, size_t workspace_bytes, void *stream) {
  SF_REQUIRE(norm_w, SF_EINVAL, "null norm weight");
  const int rc = lm_head_launch(w, h, act_dtype, norm_w, eps, logits, V, H, token_out, pos_inc,
                                hist, workspace, workspace_bytes, stream);
  return rc ? rc : sf_check_launch("sf_lm_head_argmax_rmsnorm");
}

extern "C" size_t sf_lm_head_rows_workspace_bytes(int V, int B) {
  (void)V;
  if (B < 1 || B > kRowsMax) return 0;
  // counter (256 B slot), then per row kHeadBlocks (value, index) partials
  return 256 + (size_t)B * kHeadBlocks * (sizeof(float) + sizeof(int));
}

extern "C" int sf_lm_head_argmax_rows(const void *w, const void *x, int x_dtype, float *logits,
                                      int V, int H, int B, int32_t *tokens_out, void *workspace,
                                      size_t workspace_bytes, void *stream) {
  SF_REQUIRE(V > 0 && H > 0 && B >= 1 && B <= kRowsMax, SF_EINVAL,
             "invalid lm_head rows shape V=%d H=%d B=%d (B must be 1..%d)", V, H, B, kRowsMax);
  SF_REQUIRE(x_dtype >= SF_F32 && x_dtype <= SF_BF16, SF_EINVAL, "bad x dtype %d", x_dtype);
  const size_t lds = (size_t)B * H * (x_dtype == SF_F32 ? 4 : 2);
  SF_REQUIRE(H % 8 == 0 && lds <= kRowsLdsBytes, SF_EUNSUPPORTED,
             "hidden=%d x rows=%d: need a multiple of 8 and the rows in %zu bytes", H, B,
             kRowsLdsBytes);
  SF_REQUIRE(w && x && tokens_out && workspace, SF_EINVAL, "null pointer argument");
  SF_REQUIRE(workspace_bytes >= sf_lm_head_rows_workspace_bytes(V, B), SF_EINVAL,
             "lm_head workspace too small: %zu < %zu", workspace_bytes,
             sf_lm_head_rows_workspace_bytes(V, B));
  SF_REQUIRE(((uintptr_t)w & 15) == 0 && ((uintptr_t)workspace & 255) == 0, SF_EINVAL,
             "weights must be 16-byte and workspace 256-byte aligned");
  unsigned *counter = (unsigned *)workspace;
  float *pv = (float *)((char *)workspace + 256);
  int *pi = (int *)(pv + (size_t)B * kHeadBlocks);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *wb = (const uint16_t *)w;
  // MFMA from 3 rows (measured at V = 151936, H = 896: 86 / 99 us at 4 / 8
  // rows against 96 / 162 on the VALU; at 1-2 rows the VALU's contiguous
  // table reads win, 56 / 66 against 80 / 85)
  if (B >= 3 && x_dtype != SF_F32 && H % 32 == 0 && (size_t)H * 32 <= kRowsLdsBytes) {
    const size_t lds_a = (size_t)H * 32;  // 16 A rows of bf16 fragments
    if (x_dtype == SF_F16)
      k_lm_head_rows_mfma<SF_F16><<<kHeadBlocks, kThreads, lds_a, st>>>(wb, x, logits, V, H, B,
                                                                        tokens_out, pv, pi, counter);
    else
      k_lm_head_rows_mfma<SF_BF16><<<kHeadBlocks, kThreads, lds_a, st>>>(wb, x, logits, V, H, B,
                                                                         tokens_out, pv, pi, counter);
    return sf_check_launch("sf_lm_head_argmax_rows");
  }
  if (x_dtype == SF_F32)
    k_lm_head_rows<SF_F32><<<kHeadBlocks, kThreads, lds, st>>>(wb, x, logits, V, H, B, tokens_out,
                                                               pv, pi, counter);
  else if (x_dtype == SF_F16)
    k_lm_head_rows<SF_F16><<<kHeadBlocks, kThreads, lds, st>>>(wb, x, logits, V, H, B, tokens_out,
                                                               pv, pi, counter);
  else
    k_lm_head_rows<SF_BF16><<<kHeadBlocks, kThreads, lds, st>>>(wb, x, logits, V, H, B, tokens_out,
                                                                pv, pi, counter);
  return sf_check_launch("sf_lm_head_argmax_rows");
}
