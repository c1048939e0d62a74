// q4_gemv.hip — C entry point of the int4 decode GEMV (kernels in q4_gemv_kernel.h).
#include "q4_gemv_kernel.h"

namespace sf_gemv {
bool mfma_gemv_applies(int B, int K, int g, int xdt);
bool mfma_gemv_pre_applies(int B, int N, int K, int g, bool asym, int pre);
int launch_mfma_gemv(const GemvArgs &a, int g, int pre, const float *pre_w, float eps);
extern template void launch_x<SF_F16>(const GemvPlan &, const GemvArgs &);
extern template void launch_x<SF_BF16>(const GemvPlan &, const GemvArgs &);
extern template void launch_x<SF_F32>(const GemvPlan &, const GemvArgs &);
extern template void launch_pre<SF_F16>(const GemvPlan &, const GemvArgs &, int, const float *, float);
extern template void launch_pre<SF_BF16>(const GemvPlan &, const GemvArgs &, int, const float *, float);
extern template void launch_pre<SF_F32>(const GemvPlan &, const GemvArgs &, int, const float *, float);
extern template void launch_pre_rope<SF_F16>(const GemvPlan &, const GemvArgs &, const float *, float,
                                             const SfRopeAppend &, const int *);
extern template void launch_pre_rope<SF_BF16>(const GemvPlan &, const GemvArgs &, const float *,
                                              float, const SfRopeAppend &, const int *);
extern template void launch_pre_rope<SF_F32>(const GemvPlan &, const GemvArgs &, const float *, float,
                                             const SfRopeAppend &, const int *);
}  // namespace sf_gemv

using namespace sf_gemv;

static bool mfma_gemv_enabled() {
  static const bool ok = [] {
    const char *e = getenv("SF_GEMV_MFMA");
    return !(e && e[0] == '0');
  }();
  return ok;
}

extern "C" int sf_q4_gemv(const void *blob, const void *x, int x_dtype, void *y, int y_dtype,
                          float *y_f32, const void *bias, int bias_dtype, int B, int N, int K,
                          int group_size, int has_zeros, void *stream) {
  SF_REQUIRE(N > 0 && K > 0 && group_size > 0, SF_EINVAL, "invalid shape N=%d K=%d group_size=%d",
             N, K, group_size);
  SF_REQUIRE(K % group_size == 0, SF_EINVAL, "in_features must be divisible by group_size");
  SF_REQUIRE(group_size % 32 == 0, SF_EUNSUPPORTED,
             "group_size=%d: this build's kernels need a multiple of 32", group_size);
  SF_REQUIRE(B >= 1 && B <= 8, SF_EINVAL, "GEMV batch must be 1..8 (got %d)", B);
  SF_REQUIRE(blob && x && (y || y_f32), SF_EINVAL, "null pointer argument");
  SF_REQUIRE(x_dtype == SF_F16 || x_dtype == SF_BF16 || x_dtype == SF_F32, SF_EINVAL,
             "bad activation dtype %d", x_dtype);
  SF_REQUIRE(y_dtype == SF_F16 || y_dtype == SF_BF16 || y_dtype == SF_F32, SF_EINVAL,
             "bad output dtype %d", y_dtype);
  SF_REQUIRE(!bias || bias_dtype == SF_F16 || bias_dtype == SF_BF16 || bias_dtype == SF_F32,
             SF_EINVAL, "bad bias dtype %d", bias_dtype);
  SF_REQUIRE(((uintptr_t)blob & 255) == 0 && ((uintptr_t)x & 15) == 0, SF_EINVAL,
             "blob must be 256-byte aligned and x 16-byte aligned");
  BlobLayout L;
  sf_blob_layout(N, K, group_size, has_zeros, &L);
  GemvPlan pl;
  int rc = plan_gemv(B, N, K, group_size, x_dtype, &pl);
  if (rc) return rc;
  const uint8_t *w = (const uint8_t *)blob;
  const f16 *st = (const f16 *)(w + L.s_off);
  const uint8_t *zt = has_zeros ? w + L.z_off : nullptr;
  GemvArgs args{w, st, zt, x, y, y_dtype, y_f32, bias, bias_dtype, B, N, K, L.G, has_zeros != 0,
                (hipStream_t)stream};
  // batch 3..8, fp16 activations, groups of 64 or 128: the MFMA kernel
  // (SF_GEMV_MFMA=0 keeps the VALU one)
  if (mfma_gemv_enabled() && mfma_gemv_applies(B, K, group_size, x_dtype)) {
    launch_mfma_gemv(args, group_size, PRE_NONE, nullptr, 0.f);
  } else if (x_dtype == SF_F16) {
    launch_x<SF_F16>(pl, args);
  } else if (x_dtype == SF_BF16) {
    launch_x<SF_BF16>(pl, args);
  } else {
    // fp32 activations run in slices of <= 2 batch rows
    const size_t ysz = y_dtype == SF_F32 ? 4 : 2;
    for (int b0 = 0; b0 < B; b0 += 2) {
      GemvArgs sl = args;
      sl.B = B - b0 < 2 ? B - b0 : 2;
      sl.x = (const float *)x + (size_t)b0 * K;
      if (y) sl.y = (char *)y + (size_t)b0 * N * ysz;
      if (y_f32) sl.y32 = y_f32 + (size_t)b0 * N;
      if (bias && bias == (const void *)y_f32) sl.bias = sl.y32;  // per-row residual
      GemvPlan p2;
      plan_gemv(sl.B, N, K, group_size, x_dtype, &p2);
      launch_x<SF_F32>(p2, sl);
    }
  }
  return sf_check_launch("sf_q4_gemv");
}

extern "C" int sf_q4_gemv_fused(const void *blob, const float *src, int op, const float *norm_w,
                                float eps, int act_dtype, void *y, int y_dtype, float *y_f32,
                                const void *bias, int bias_dtype, int N, int K, int group_size,
                                int has_zeros, void *stream) {
  SF_REQUIRE(N > 0 && K > 0 && group_size > 0, SF_EINVAL, "invalid shape N=%d K=%d group_size=%d",
             N, K, group_size);
  SF_REQUIRE(K % group_size == 0, SF_EINVAL, "in_features must be divisible by group_size");
  SF_REQUIRE(group_size % 32 == 0, SF_EUNSUPPORTED,
             "group_size=%d: this build's kernels need a multiple of 32", group_size);
  SF_REQUIRE(op == SF_PRE_RMSNORM || op == SF_PRE_SILU_MUL, SF_EINVAL, "bad fused op %d", op);
  SF_REQUIRE(blob && src && (y || y_f32) && (op != SF_PRE_RMSNORM || norm_w), SF_EINVAL,
             "null pointer argument");
  SF_REQUIRE(act_dtype == SF_F16 || act_dtype == SF_BF16 || act_dtype == SF_F32, SF_EINVAL,
             "bad activation dtype %d", act_dtype);
  SF_REQUIRE(y_dtype == SF_F16 || y_dtype == SF_BF16 || y_dtype == SF_F32, SF_EINVAL,
             "bad output dtype %d", y_dtype);
  SF_REQUIRE(!bias || bias_dtype == SF_F16 || bias_dtype == SF_BF16 || bias_dtype == SF_F32,
             SF_EINVAL, "bad bias dtype %d", bias_dtype);
  SF_REQUIRE(((uintptr_t)blob & 255) == 0 && ((uintptr_t)src & 15) == 0 &&
                 ((uintptr_t)norm_w & 15) == 0,
             SF_EINVAL, "blob must be 256-byte aligned, src and norm_w 16-byte aligned");
  BlobLayout L;
  sf_blob_layout(N, K, group_size, has_zeros, &L);
  GemvPlan pl;
  int rc = plan_gemv(1, N, K, group_size, act_dtype, &pl, 8);
  if (rc) return rc;
  const uint8_t *w = (const uint8_t *)blob;
  const f16 *st = (const f16 *)(w + L.s_off);
  const uint8_t *zt = has_zeros ? w + L.z_off : nullptr;
  GemvArgs args{w, st, zt, src, y, y_dtype, y_f32, bias, bias_dtype, 1, N, K, L.G, has_zeros != 0,
                (hipStream_t)stream};
  const int pre = op == SF_PRE_RMSNORM ? PRE_RMSNORM : PRE_SILU;
  if (act_dtype == SF_F16) launch_pre<SF_F16>(pl, args, pre, norm_w, eps);
  else if (act_dtype == SF_BF16) launch_pre<SF_BF16>(pl, args, pre, norm_w, eps);
  else launch_pre<SF_F32>(pl, args, pre, norm_w, eps);
  return sf_check_launch("sf_q4_gemv_fused");
}

extern "C" int sf_q4_gemv_fused_rows_supported(int op, int B, int N, int K, int group_size,
                                               int has_zeros, int act_dtype) {
  if ((op != SF_PRE_RMSNORM && op != SF_PRE_SILU_MUL) || N <= 0 || K <= 0 || group_size <= 0 ||
      K % group_size || group_size % 32)
    return 0;
  if (B == 1) return 1;
  return mfma_gemv_enabled() && act_dtype == SF_F16 &&
         mfma_gemv_pre_applies(B, N, K, group_size, has_zeros != 0,
                               op == SF_PRE_RMSNORM ? PRE_RMSNORM : PRE_SILU);
}

extern "C" int sf_q4_gemv_fused_rows(const void *blob, const float *src, int op,
                                     const float *norm_w, float eps, int act_dtype, void *y,
                                     int y_dtype, float *y_f32, const void *bias, int bias_dtype,
                                     int B, int N, int K, int group_size, int has_zeros,
                                     void *stream) {
  SF_REQUIRE(B >= 1 && B <= 8, SF_EINVAL, "GEMV batch must be 1..8 (got %d)", B);
  if (B == 1)
    return sf_q4_gemv_fused(blob, src, op, norm_w, eps, act_dtype, y, y_dtype, y_f32, bias,
                            bias_dtype, N, K, group_size, has_zeros, stream);
  SF_REQUIRE(N > 0 && K > 0 && group_size > 0, SF_EINVAL, "invalid shape N=%d K=%d group_size=%d",
             N, K, group_size);
  SF_REQUIRE(K % group_size == 0, SF_EINVAL, "in_features must be divisible by group_size");
  SF_REQUIRE(op == SF_PRE_RMSNORM || op == SF_PRE_SILU_MUL, SF_EINVAL, "bad fused op %d", op);
  SF_REQUIRE(blob && src && (y || y_f32) && (op != SF_PRE_RMSNORM || norm_w), SF_EINVAL,
             "null pointer argument");
  SF_REQUIRE(y_dtype == SF_F16 || y_dtype == SF_BF16 || y_dtype == SF_F32, SF_EINVAL,
             "bad output dtype %d", y_dtype);
  SF_REQUIRE(!bias || bias_dtype == SF_F16 || bias_dtype == SF_BF16 || bias_dtype == SF_F32,
             SF_EINVAL, "bad bias dtype %d", bias_dtype);
  SF_REQUIRE(((uintptr_t)blob & 255) == 0 && ((uintptr_t)src & 15) == 0 &&
                 ((uintptr_t)norm_w & 15) == 0,
             SF_EINVAL, "blob must be 256-byte aligned, src and norm_w 16-byte aligned");
  SF_REQUIRE(sf_q4_gemv_fused_rows_supported(op, B, N, K, group_size, has_zeros, act_dtype),
             SF_EUNSUPPORTED,
             "fused op %d at batch %d (N=%d K=%d group_size=%d act dtype %d): this build folds "
             "the producer at batch 1, and at 3..8 for fp16 activations on plans of at most four "
             "MFMAs per lane; run sf_rmsnorm / sf_silu_mul and sf_q4_gemv instead",
             op, B, N, K, group_size, act_dtype);
  BlobLayout L;
  sf_blob_layout(N, K, group_size, has_zeros, &L);
  const uint8_t *w = (const uint8_t *)blob;
  const f16 *st = (const f16 *)(w + L.s_off);
  const uint8_t *zt = has_zeros ? w + L.z_off : nullptr;
  GemvArgs args{w, st, zt, src, y, y_dtype, y_f32, bias, bias_dtype, B, N, K, L.G, has_zeros != 0,
                (hipStream_t)stream};
  launch_mfma_gemv(args, group_size, op == SF_PRE_RMSNORM ? PRE_RMSNORM : PRE_SILU, norm_w, eps);
  return sf_check_launch("sf_q4_gemv_fused_rows");
}

extern "C" int sf_q4_gemv_fused_rope_supported(int N, int K, int group_size, int H, int KVH, int D,
                                               int act_dtype) {
  if (N <= 0 || K <= 0 || group_size <= 0 || K % group_size || group_size % 32 || H <= 0 ||
      KVH <= 0 || D <= 0 || D % 2 || D > 256 || N != (H + 2 * KVH) * D || K % 32 ||
      (act_dtype != SF_F16 && act_dtype != SF_BF16 && act_dtype != SF_F32))
    return 0;
  GemvPlan pl;
  if (plan_gemv(1, N, K, group_size, act_dtype, &pl, 8)) return 0;
  return pl.Q == 32 && pl.P == 32 && pl.RS * pl.R == D;
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
             "qkv projection N=%d K=%d group_size=%d heads %d/%d x %d: the folded RoPE needs one "
             "head per workgroup of the batch-1 plan (in_features <= 1024); run sf_q4_gemv_fused "
             "and sf_rope_kv_append instead",
             N, K, group_size, H, KVH, D);
  BlobLayout L;
  sf_blob_layout(N, K, group_size, has_zeros, &L);
  GemvPlan pl;
  int rc = plan_gemv(1, N, K, group_size, act_dtype, &pl, 8);
  if (rc) return rc;
  const uint8_t *w = (const uint8_t *)blob;
  const f16 *st = (const f16 *)(w + L.s_off);
  const uint8_t *zt = has_zeros ? w + L.z_off : nullptr;
  GemvArgs args{w, st, zt, h, nullptr, SF_F32, nullptr, bias, bias_dtype, 1, N, K, L.G,
                has_zeros != 0, (hipStream_t)stream};
  const SfRopeAppend rope{cos_t, sin_t, max_pos, q_out, q_dtype, k_codes, k_scales, v_codes,
                          v_scales, scale_dtype, H, KVH, D, T_cap};
  if (act_dtype == SF_F16) launch_pre_rope<SF_F16>(pl, args, norm_w, eps, rope, pos_dev);
  else if (act_dtype == SF_BF16) launch_pre_rope<SF_BF16>(pl, args, norm_w, eps, rope, pos_dev);
  else launch_pre_rope<SF_F32>(pl, args, norm_w, eps, rope, pos_dev);
  return sf_check_launch("sf_q4_gemv_fused_rope");
}
