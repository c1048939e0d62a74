// split_merge.h — the combine of split-T attention partials, shared by the merge
// launch of the decode attention (kv_attn.hip) and by the o-projection GEMV that
// folds the merge into its activation staging (q4_gemv_blk.h).
//
// Split s of a row's T tokens leaves (m_s, l_s, acc_s[D]): the running max of
// its base-2 scores, the sum of 2^(score - m_s) and the sum of 2^(score - m_s) v.
// The output row is
//   M = max_s m_s,  w_s = 2^(m_s - M),  out = (sum_s w_s acc_s) / (sum_s w_s l_s),
// the reference's combine (/root/reference/siliconfer/kernels/metal/
// q4_attention.py:63-70, 256-261, there in base e). Both sums run over the
// fp32 products w_s acc_s and w_s l_s, each rounded on its own, as a pairwise
// tree: over the indices [0, P), P the smallest power of two >= S, terms at
// s >= S being +0, the first level adds the pairs (2i, 2i + 1), every next
// level the pairs of the level before. A consumer evaluates that tree in
// registers (sf_tree_sum) or across P lanes with xor butterflies (the two
// lanes of a pair add the same two values), so every consumer of the
// partials computes the same bits.
// An empty split (no tokens) has m = -inf, l = 0, acc = 0 and weighs 0; a row
// with no tokens at all comes out as zeros.
//
// Workspace layout: acc [rows][S][D] fp32 at offset 0, then (m, l) [rows][S][2]
// fp32 at a 256-byte aligned offset; rows = B * H, row b * H + h.
#pragma once
#include "sf_common.h"

// Splits the GEMV's folded merge holds in registers at once.
constexpr int kMergeFoldMaxSplits = 8;

__host__ __device__ inline size_t sf_split_ws_parts(int rows, int D, int S, size_t *acc_off,
                                                    size_t *ml_off) {
  const size_t n = (size_t)rows * S;
  *acc_off = 0;
  *ml_off = ((n * D * sizeof(float)) + 255) & ~(size_t)255;
  return *ml_off + n * 2 * sizeof(float);
}

// The reference point of the weights: M, or 0 when every split is empty.
__device__ __forceinline__ float sf_merge_mref(float M) { return M == -INFINITY ? 0.f : M; }

// The weight 2^(m_s - M) of one split (exp2(-inf) = 0 for an empty split).
__device__ __forceinline__ float sf_merge_weight(float m, float mref) {
  return __builtin_amdgcn_exp2f(m - mref);
}

// One term of a sum: the rounded product x w (never contracted with the
// tree's adds into an fma: the multiply carries no contraction flag).
__device__ __forceinline__ float sf_merge_term(float x, float w) {
#pragma clang fp contract(off)
  return x * w;
}

// The tree's span: the smallest power of two >= S.
__host__ __device__ inline int sf_merge_span(int S) {
  int P = 1;
  while (P < S) P <<= 1;
  return P;
}

// The pairwise tree over t[0, P) (P a power of two <= N; t[s] = +0 past the
// terms): t[0] on return. Entries at or past P are left unused.
template <int N>
__device__ __forceinline__ float sf_tree_sum(float (&t)[N], int P) {
#pragma unroll
  for (int off = 1; off < N; off <<= 1)
#pragma unroll
    for (int i = 0; i < N; i += 2 * off)
      if (off < P) t[i] = t[i] + t[i + off];
  return t[0];
}

// The merged value from the weighted sums, as a rounded fp32 product (opaque,
// so that a consumer's next operation cannot contract it into an fma).
__device__ __forceinline__ float sf_merge_finish(float L, float v) {
  const float inv = L > 0.f ? 1.f / L : 0.f;
  return sf_opaque(v * inv);
}
