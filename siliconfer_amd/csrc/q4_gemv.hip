// q4_gemv.hip — C entry points of the int4 decode GEMV (kernels in q4_gemv_blk.h).
#include "q4_gemv_blk.h"

using namespace sf_gemv;

namespace {

void launch(const BlkPlan &p, const GemvArgs &g, int xdt, int pre, const float *pre_w, float eps,
            const SfRopeAppend *rope = nullptr, const int *pos_dev = nullptr) {
  if (xdt == SF_F16) {
    if (g.asym) launch_blk<SF_F16, true>(p, g, pre, pre_w, eps, rope, pos_dev);
    else launch_blk<SF_F16, false>(p, g, pre, pre_w, eps, rope, pos_dev);
  } else if (xdt == SF_BF16) {
    if (g.asym) launch_blk<SF_BF16, true>(p, g, pre, pre_w, eps, rope, pos_dev);
    else launch_blk<SF_BF16, false>(p, g, pre, pre_w, eps, rope, pos_dev);
  } else {
    if (g.asym) launch_blk<SF_F32, true>(p, g, pre, pre_w, eps, rope, pos_dev);
    else launch_blk<SF_F32, false>(p, g, pre, pre_w, eps, rope, pos_dev);
  }
}

int check_shape(int N, int K, int g) {
  SF_REQUIRE(N > 0 && K > 0 && g > 0, SF_EINVAL, "invalid shape N=%d K=%d group_size=%d", N, K, g);
  SF_REQUIRE(K % g == 0, SF_EINVAL, "in_features must be divisible by group_size");
  return SF_OK;
}

int check_out(int y_dtype, const void *bias, int bias_dtype) {
  SF_REQUIRE(y_dtype == SF_F16 || y_dtype == SF_BF16 || y_dtype == SF_F32, SF_EINVAL,
             "bad output dtype %d", y_dtype);
  SF_REQUIRE(!bias || bias_dtype == SF_F16 || bias_dtype == SF_BF16 || bias_dtype == SF_F32,
             SF_EINVAL, "bad bias dtype %d", bias_dtype);
  return SF_OK;
}

GemvArgs make_args(const void *blob, const void *x, void *y, int ydt, float *y32, const void *bias,
                   int bdt, int B, int N, int K, int g, int has_zeros, void *stream) {
  BlobLayout L;
  sf_blob_layout(N, K, g, has_zeros, &L);
  const uint8_t *w = (const uint8_t *)blob;
  return GemvArgs{w, (const f16 *)(w + L.s_off), has_zeros ? w + L.z_off : nullptr, x, y, ydt, y32,
                  bias, bdt, B, N, K, L.G, g, has_zeros != 0, (hipStream_t)stream};
}

}  // namespace

int sf_q4_anyg(const void *blob, const void *x, int x_dtype, void *y, int y_dtype, float *y_f32,
               const void *bias, int bias_dtype, int M, int N, int K, int g, int has_zeros, void *stream);

// Whether the MFMA GEMV takes this shape in one pass over the batch (the other
// shapes run on the any-group-size kernel, or, fp32 activations, in batch
// slices).
extern "C" int sf_q4_gemv_supported(int B, int N, int K, int group_size, int x_dtype) {
  if (B < 1 || B > 8 || N <= 0 || K <= 0 || group_size <= 0 || K % group_size || group_size % 32 ||
      (x_dtype != SF_F16 && x_dtype != SF_BF16 && x_dtype != SF_F32))
    return 0;
  BlkPlan p;
  return plan_blk(B, N, K, group_size, x_dtype, PRE_NONE, false, &p) ? 1 : 0;
}

extern "C" int sf_q4_gemv(const void *blob, const void *x, int x_dtype, void *y, int y_dtype,
                          float *y_f32, const void *bias, int bias_dtype, int B, int N, int K,
                          int group_size, int has_zeros, void *stream) {
  int rc = check_shape(N, K, group_size);
  if (rc) return rc;
  SF_REQUIRE(B >= 1 && B <= 8, SF_EINVAL, "GEMV batch must be 1..8 (got %d)", B);
  SF_REQUIRE(blob && x && (y || y_f32), SF_EINVAL, "null pointer argument");
  SF_REQUIRE(x_dtype == SF_F16 || x_dtype == SF_BF16 || x_dtype == SF_F32, SF_EINVAL,
             "bad activation dtype %d", x_dtype);
  if ((rc = check_out(y_dtype, bias, bias_dtype))) return rc;
  SF_REQUIRE(((uintptr_t)blob & 255) == 0 && ((uintptr_t)x & 15) == 0, SF_EINVAL,
             "blob must be 256-byte aligned and x 16-byte aligned");
  if (group_size % 32)
    return sf_q4_anyg(blob, x, x_dtype, y, y_dtype, y_f32, bias, bias_dtype, B, N, K, group_size,
                      has_zeros, stream);
  const GemvArgs args =
      make_args(blob, x, y, y_dtype, y_f32, bias, bias_dtype, B, N, K, group_size, has_zeros, stream);
  BlkPlan p;
  if (plan_blk(B, N, K, group_size, x_dtype, PRE_NONE, false, &p)) {
    launch(p, args, x_dtype, PRE_NONE, nullptr, 0.f);
    return sf_check_launch("sf_q4_gemv");
  }
  // fp32 activations stage their high and low bf16 rows in LDS: run the batch
  // in the largest slices that fit
  int bs = 0;
  if (x_dtype == SF_F32)
    for (int b = B - 1; b >= 1 && !bs; --b)
      if (plan_blk(b, N, K, group_size, x_dtype, PRE_NONE, false, &p)) bs = b;
  if (bs == 0)  // fp32 activations at a K whose staged rows exceed the LDS
    return sf_q4_anyg(blob, x, x_dtype, y, y_dtype, y_f32, bias, bias_dtype, B, N, K, group_size,
                      has_zeros, stream);
  const size_t ysz = y_dtype == SF_F32 ? 4 : 2;
  for (int b0 = 0; b0 < B; b0 += bs) {
    GemvArgs sl = args;
    sl.B = B - b0 < bs ? B - b0 : bs;
    sl.x = (const float *)x + (size_t)b0 * K;
    if (y) sl.y = (char *)y + (size_t)b0 * N * ysz;
    if (y_f32) sl.y32 = y_f32 + (size_t)b0 * N;
    if (bias && bias == (const void *)y_f32) sl.bias = sl.y32;  // per-row residual
    plan_blk(sl.B, N, K, group_size, x_dtype, PRE_NONE, false, &p);
    launch(p, sl, x_dtype, PRE_NONE, nullptr, 0.f);
  }
  return sf_check_launch("sf_q4_gemv");
}

extern "C" int sf_q4_gemv_fused_rows_supported(int op, int B, int N, int K, int group_size,
                                               int has_zeros, int act_dtype) {
  (void)has_zeros;
  if ((op != SF_PRE_RMSNORM && op != SF_PRE_SILU_MUL) || N <= 0 || K <= 0 || group_size <= 0 ||
      K % group_size || group_size % 32 || B < 1 || B > 8 ||
      (act_dtype != SF_F16 && act_dtype != SF_BF16 && act_dtype != SF_F32))
    return 0;
  BlkPlan p;
  return plan_blk(B, N, K, group_size, act_dtype, op == SF_PRE_RMSNORM ? PRE_RMSNORM : PRE_SILU,
                  false, &p);
}

extern "C" int sf_q4_gemv_fused_rows(const void *blob, const float *src, int op,
                                     const float *norm_w, float eps, int act_dtype, void *y,
                                     int y_dtype, float *y_f32, const void *bias, int bias_dtype,
                                     int B, int N, int K, int group_size, int has_zeros,
                                     void *stream) {
  int rc = check_shape(N, K, group_size);
  if (rc) return rc;
  SF_REQUIRE(B >= 1 && B <= 8, SF_EINVAL, "GEMV batch must be 1..8 (got %d)", B);
  SF_REQUIRE(op == SF_PRE_RMSNORM || op == SF_PRE_SILU_MUL, SF_EINVAL, "bad fused op %d", op);
  SF_REQUIRE(blob && src && (y || y_f32) && (op != SF_PRE_RMSNORM || norm_w), SF_EINVAL,
             "null pointer argument");
  SF_REQUIRE(act_dtype == SF_F16 || act_dtype == SF_BF16 || act_dtype == SF_F32, SF_EINVAL,
             "bad activation dtype %d", act_dtype);
  if ((rc = check_out(y_dtype, bias, bias_dtype))) return rc;
  SF_REQUIRE(((uintptr_t)blob & 255) == 0 && ((uintptr_t)src & 15) == 0 &&
                 ((uintptr_t)norm_w & 15) == 0,
             SF_EINVAL, "blob must be 256-byte aligned, src and norm_w 16-byte aligned");
  const int pre = op == SF_PRE_RMSNORM ? PRE_RMSNORM : PRE_SILU;
  BlkPlan p;
  SF_REQUIRE(plan_blk(B, N, K, group_size, act_dtype, pre, false, &p), SF_EUNSUPPORTED,
             "fused op %d at batch %d (N=%d K=%d group_size=%d act dtype %d): the activations "
             "do not fit this GEMV's LDS staging; run sf_rmsnorm / sf_silu_mul and sf_q4_gemv "
             "instead",
             op, B, N, K, group_size, act_dtype);
  const GemvArgs args = make_args(blob, src, y, y_dtype, y_f32, bias, bias_dtype, B, N, K,
                                  group_size, has_zeros, stream);
  launch(p, args, act_dtype, pre, norm_w, eps);
  return sf_check_launch("sf_q4_gemv_fused_rows");
}

extern "C" int sf_q4_gemv_fused(const void *blob, const float *src, int op, const float *norm_w,
                                float eps, int act_dtype, void *y, int y_dtype, float *y_f32,
                                const void *bias, int bias_dtype, int N, int K, int group_size,
                                int has_zeros, void *stream) {
  return sf_q4_gemv_fused_rows(blob, src, op, norm_w, eps, act_dtype, y, y_dtype, y_f32, bias,
                               bias_dtype, 1, N, K, group_size, has_zeros, stream);
}

extern "C" int sf_q4_gemv_attn_merge_supported(int B, int N, int H, int D, int n_splits,
                                               int group_size, int act_dtype) {
  if (B < 1 || B > 8 || N <= 0 || H <= 0 || D <= 0 || D % 8 || n_splits < 2 ||
      n_splits > kMergeFoldMaxSplits || group_size <= 0 || (H * D) % group_size ||
      group_size % 32 || (act_dtype != SF_F16 && act_dtype != SF_BF16 && act_dtype != SF_F32))
    return 0;
  BlkPlan p;
  return plan_blk(B, N, H * D, group_size, act_dtype, PRE_MERGE, false, &p) ? 1 : 0;
}

extern "C" int sf_q4_gemv_attn_merge(const void *blob, const void *workspace,
                                     size_t workspace_bytes, int n_splits, int H, int D,
                                     int act_dtype, void *y, int y_dtype, float *y_f32,
                                     const void *bias, int bias_dtype, int B, int N,
                                     int group_size, int has_zeros, void *stream) {
  const int K = H * D;
  int rc = check_shape(N, K, group_size);
  if (rc) return rc;
  SF_REQUIRE(blob && workspace && (y || y_f32), SF_EINVAL, "null pointer argument");
  if ((rc = check_out(y_dtype, bias, bias_dtype))) return rc;
  SF_REQUIRE(((uintptr_t)blob & 255) == 0 && ((uintptr_t)workspace & 255) == 0, SF_EINVAL,
             "blob and workspace must be 256-byte aligned");
  SF_REQUIRE(sf_q4_gemv_attn_merge_supported(B, N, H, D, n_splits, group_size, act_dtype),
             SF_EUNSUPPORTED,
             "folded attention merge at batch %d (N=%d H=%d head_dim=%d splits=%d group_size=%d "
             "act dtype %d): not taken by this GEMV; run sf_attn_decode_i8kv and sf_q4_gemv "
             "instead",
             B, N, H, D, n_splits, group_size, act_dtype);
  size_t acc_off, ml_off;
  const size_t need = sf_split_ws_parts(B * H, D, n_splits, &acc_off, &ml_off);
  SF_REQUIRE(workspace_bytes >= need, SF_EINVAL, "attention workspace too small: %zu < %zu",
             workspace_bytes, need);
  GemvArgs args = make_args(blob, (const char *)workspace + acc_off, y, y_dtype, y_f32, bias,
                            bias_dtype, B, N, K, group_size, has_zeros, stream);
  args.mml = (const float *)((const char *)workspace + ml_off);
  args.ms = n_splits;
  args.md = D;
  BlkPlan p;
  plan_blk(B, N, K, group_size, act_dtype, PRE_MERGE, false, &p);
  launch(p, args, act_dtype, PRE_MERGE, nullptr, 0.f);
  return sf_check_launch("sf_q4_gemv_attn_merge");
}

extern "C" int sf_q4_gemv_fused_rope_supported(int N, int K, int group_size, int H, int KVH, int D,
                                               int act_dtype) {
  if (N <= 0 || K <= 0 || group_size <= 0 || K % group_size || group_size % 32 || H <= 0 ||
      KVH <= 0 || D != 64 || N != (H + 2 * KVH) * D ||
      (act_dtype != SF_F16 && act_dtype != SF_BF16 && act_dtype != SF_F32))
    return 0;
  BlkPlan p;
  return plan_blk(1, N, K, group_size, act_dtype, PRE_RMSNORM, true, &p) &&
         p.BPW <= (group_size % 64 ? 2 : 4);
}

extern "C" int sf_q4_gemv_fused_rope(const void *blob, const float *h, const float *norm_w,
                                     float eps, int act_dtype, const void *bias, int bias_dtype,
                                     const float *cos_t, const float *sin_t, int max_pos,
                                     void *q_out, int q_dtype, int8_t *k_codes, void *k_scales,
                                     int8_t *v_codes, void *v_scales, int scale_dtype, int H,
                                     int KVH, int D, int T_cap, const int *pos_dev, int N, int K,
                                     int group_size, int has_zeros, void *stream) {
  SF_REQUIRE(blob && h && norm_w && cos_t && sin_t && q_out && k_codes && k_scales && v_codes &&
                 v_scales && pos_dev,
             SF_EINVAL, "null pointer argument");
  SF_REQUIRE(q_dtype >= SF_F32 && q_dtype <= SF_BF16, SF_EINVAL, "bad q dtype %d", q_dtype);
  SF_REQUIRE(scale_dtype == SF_F16 || scale_dtype == SF_F32, SF_EINVAL, "bad scale dtype %d",
             scale_dtype);
  SF_REQUIRE(!bias || bias_dtype == SF_F16 || bias_dtype == SF_BF16 || bias_dtype == SF_F32,
             SF_EINVAL, "bad bias dtype %d", bias_dtype);
  SF_REQUIRE(T_cap > 0 && max_pos > 0, SF_EINVAL, "invalid cache capacity %d / RoPE table %d",
             T_cap, max_pos);
  SF_REQUIRE(((uintptr_t)blob & 255) == 0 && ((uintptr_t)h & 15) == 0 &&
                 ((uintptr_t)norm_w & 15) == 0,
             SF_EINVAL, "blob must be 256-byte aligned, h and norm_w 16-byte aligned");
  SF_REQUIRE(sf_q4_gemv_fused_rope_supported(N, K, group_size, H, KVH, D, act_dtype),
             SF_EUNSUPPORTED,
             "qkv projection N=%d K=%d group_size=%d heads %d/%d x %d: the folded RoPE takes "
             "head_dim 64 (one 64-row head per workgroup) and in_features <= 4096; run "
             "sf_q4_gemv_fused and sf_rope_kv_append instead",
             N, K, group_size, H, KVH, D);
  BlkPlan p;
  plan_blk(1, N, K, group_size, act_dtype, PRE_RMSNORM, true, &p);
  const GemvArgs args = make_args(blob, h, nullptr, SF_F32, nullptr, bias, bias_dtype, 1, N, K,
                                  group_size, has_zeros, stream);
  const SfRopeAppend rope{cos_t, sin_t, max_pos, q_out, q_dtype, k_codes, k_scales, v_codes,
                          v_scales, scale_dtype, H, KVH, D, T_cap};
  launch(p, args, act_dtype, PRE_RMSNORM, norm_w, eps, &rope, pos_dev);
  return sf_check_launch("sf_q4_gemv_fused_rope");
}
