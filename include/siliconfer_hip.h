/* siliconfer_hip.h — C ABI of the MI355X (gfx950) quantized-inference hot path.
 *
 * One shared library, libsiliconfer_hip.so, built from the HIP sources in siliconfer_amd/csrc.
 * Conventions for every entry point:
 *   - all data pointers are DEVICE memory owned by the caller;
 *   - `stream` is a hipStream_t (NULL = the legacy default stream); work is
 *     enqueued and the call returns without synchronising;
 *   - nothing allocates device memory; kernels that need scratch take a
 *     caller-provided workspace whose size a *_workspace_bytes() call reports;
 *   - return 0 on success, a negative SF_E* code otherwise; sf_last_error()
 *     then holds a message for the calling thread. Shape errors reuse the
 *     reference's message texts ("scales shape mismatch", "in_features must
 *     be divisible by group_size", ...) from
 *     /root/reference/siliconfer/kernels/neon/bindings.cpp:24-40.
 *
 * Weight format at the boundary is the reference's canonical one
 * (siliconfer/kernels/neon/__init__.py:42-81, quant/primitives.py:332-349):
 * packed uint8 [N, K/2], byte (i,j) = q[i,2j] | q[i,2j+1] << 4; symmetric codes
 * are two's-complement nibbles, asymmetric codes unsigned. Scales are fp16
 * [N, K/g]; zero-points are integral values 0..15 given as uint8 [N, K/g].
 * sf_q4_repack turns that into the device blob every GEMV/GEMM call reads.
 */
#ifndef SILICONFER_HIP_H
#define SILICONFER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SF_ABI_VERSION 1

/* return codes */
#define SF_OK 0
#define SF_EINVAL (-1)       /* bad shape / argument (reference: std::runtime_error) */
#define SF_EUNSUPPORTED (-2) /* valid for the reference, outside this build's kernels */
#define SF_EHIP (-3)         /* a HIP runtime call or launch failed */

/* element types for activations, KV inputs, attention q/out and KV scales */
#define SF_F32 0
#define SF_F16 1
#define SF_BF16 2

/* ---- library ------------------------------------------------------------ */

/* Message for the last failing call on this thread ("" if none). */
const char *sf_last_error(void);

/* SF_ABI_VERSION of the loaded library. */
int sf_abi_version(void);

/* 1 if `device` is a gfx950 (MI355X-class) device, 0 otherwise, <0 on error. */
int sf_device_arch_ok(int device);

/* ---- int4 weights: canonical -> device blob ----------------------------- */

/* Bytes of the device blob for an N x K int4 matrix with group size g.
 * Replaces the reference's packed-array allocation in pack_weights_sym/asym
 * (siliconfer/kernels/neon/__init__.py:42-81); 0 if the shape is invalid. */
size_t sf_q4_blob_bytes(int N, int K, int group_size, int has_zeros);

/* Canonical (packed u8 [N,K/2], scales f16 [N,K/g], zeros u8 [N,K/g] or NULL)
 * -> blob. has_zeros = (zeros != NULL) selects asymmetric codes. Same
 * validation as check_gemv (bindings.cpp:24-40): any group_size dividing K. */
int sf_q4_repack(const uint8_t *packed, const void *scales_f16, const uint8_t *zeros_u8,
                 int N, int K, int group_size, void *blob, size_t blob_bytes, void *stream);

/* Blob -> canonical (inverse of sf_q4_repack; zeros_u8 may be NULL for sym). */
int sf_q4_unpack(const void *blob, int N, int K, int group_size, int has_zeros,
                 uint8_t *packed, void *scales_f16, uint8_t *zeros_u8, void *stream);

/* ---- decode GEMV (batch 1..8) -------------------------------------------
 * y[b, n] = sum_g s[n,g] * sum_{k in g} (q[n,k] - z[n,g]) x[b,k]   (z = 0 sym)
 * Replaces q4_gemv_sym / q4_gemv_asym (bindings.cpp:45-93) and, through
 * Q4Linear at T<=8 rows, q4_gemm_sym / q4_gemm_asym (bindings.cpp:98-150).
 * x: [B, K] of x_dtype (SF_F16, SF_BF16 or SF_F32). Outputs: y [B, N] of y_dtype
 * (SF_F16 / SF_BF16 / SF_F32), and/or y_f32 [B, N]; either may be NULL but
 * not both. bias: NULL, [N] of bias_dtype (added before the store), or y_f32
 * itself (fp32: each output adds its own previous value, per batch row — a
 * residual add). fp32 accumulation throughout. Any K and group size the
 * reference takes (K % group_size == 0): group sizes that are a multiple of 32
 * run on MFMA (long K in per-wave chunks), the others — and fp32 activations
 * whose staged rows exceed the LDS at very long K — on a VALU kernel. */
int sf_q4_gemv(const void *blob, const void *x, int x_dtype, void *y, int y_dtype, float *y_f32,
               const void *bias, int bias_dtype, int B, int N, int K, int group_size,
               int has_zeros, void *stream);
/* 1 when sf_q4_gemv runs this shape on the MFMA GEMV in one pass over the
 * batch, 0 when it takes the VALU kernel or batch slices (callers choosing
 * between the batch GEMV and sf_q4_gemm for a few rows ask this). No
 * counterpart in the reference. */
int sf_q4_gemv_supported(int B, int N, int K, int group_size, int x_dtype);

/* The decode GEMV (batch 1) with the operation that produces its input folded
 * into the activation load, for the decoder step (no counterpart in the
 * reference, which runs RMSNorm / SwiGLU and the Q4Linear as separate ops:
 * /root/reference/siliconfer/model/layers.py:14-21, 143-144):
 *   op SF_PRE_RMSNORM:  x = src[0:K] * rsqrt(mean(src^2) + eps) * norm_w
 *                       (src the fp32 residual row [K], norm_w fp32 [K]);
 *   op SF_PRE_SILU_MUL: x[k] = silu(src[k]) * src[K + k]
 *                       (src the fp32 gate|up row [2K]; norm_w unused).
 * x is rounded to act_dtype (SF_F16 / SF_BF16 / SF_F32) before the product,
 * and the result is bit-identical to sf_rmsnorm / sf_silu_mul writing an
 * act_dtype buffer followed by sf_q4_gemv on it. Outputs as sf_q4_gemv. */
#define SF_PRE_RMSNORM 1
#define SF_PRE_SILU_MUL 2
int sf_q4_gemv_fused(const void *blob, const float *src, int op, const float *norm_w, float eps,
                     int act_dtype, void *y, int y_dtype, float *y_f32, const void *bias,
                     int bias_dtype, int N, int K, int group_size, int has_zeros, void *stream);

/* sf_q4_gemv_fused over B = 1..8 rows (src [B][K], or [B][2K] gate|up): the
 * target's verify rows of speculative decoding (engine/speculative.py:280)
 * with each RMSNorm / SwiGLU folded into the next projection as the decode
 * step does. B = 1 is sf_q4_gemv_fused. The producer runs while the GEMV
 * stages its activations, and the result equals sf_rmsnorm / sf_silu_mul
 * followed by sf_q4_gemv bit for bit. Shapes whose B rows of activations do
 * not fit the staging (or whose RMSNorm plan exceeds its wave budget) return
 * SF_EUNSUPPORTED; sf_q4_gemv_fused_rows_supported says which (1 = supported).
 * bias may be y_f32 itself (each row adds its own previous value), as for
 * sf_q4_gemv. */
int sf_q4_gemv_fused_rows_supported(int op, int B, int N, int K, int group_size, int has_zeros,
                                    int act_dtype);
int sf_q4_gemv_fused_rows(const void *blob, const float *src, int op, const float *norm_w,
                          float eps, int act_dtype, void *y, int y_dtype, float *y_f32,
                          const void *bias, int bias_dtype, int B, int N, int K, int group_size,
                          int has_zeros, void *stream);

/* The decode step's qkv projection with the input RMSNorm folded into its
 * activation load (sf_q4_gemv_fused, SF_PRE_RMSNORM) and RoPE + the KV-cache
 * append (sf_rope_kv_append at the device position *pos_dev) folded into its
 * epilogue: q_out [H][D] and the cache row at *pos_dev get the same bits as
 * those two calls; the fp32 q|k|v rows are not stored. Needs D = 64 (one
 * 64-row head per workgroup) and a batch-1 plan of at most four weight units
 * per wave (in_features <= 4096 for groups of 64 / 128);
 * sf_q4_gemv_fused_rope_supported says so (1), else SF_EUNSUPPORTED. No
 * counterpart in the reference (layers.py:93-112 runs these as separate ops). */
int sf_q4_gemv_fused_rope_supported(int N, int K, int group_size, int H, int KVH, int D,
                                    int act_dtype);
int sf_q4_gemv_fused_rope(const void *blob, const float *h, const float *norm_w, float eps,
                          int act_dtype, const void *bias, int bias_dtype, const float *cos_t,
                          const float *sin_t, int max_pos, void *q_out, int q_dtype,
                          int8_t *k_codes, void *k_scales, int8_t *v_codes, void *v_scales,
                          int scale_dtype, int H, int KVH, int D, int T_cap, const int *pos_dev,
                          int N, int K, int group_size, int has_zeros, void *stream);

/* ---- prefill GEMM (M rows) ------------------------------------------------
 * Y[m, n] = X[m, :] . dequant(W)[n, :] for M rows; replaces q4_gemm_sym /
 * q4_gemm_asym (bindings.cpp:98-150; q4_gemm.cpp:12-51). bf16/f16 MFMA on
 * integer-valued int4 codes, fp32 per-(row, group) scale epilogue; group sizes
 * that are not a multiple of 32 run on the VALU kernel sf_q4_gemv uses for them.
 * Up to 16 rows the call runs as sf_q4_gemv over 8-row slices (the same bits
 * as those calls; the reference's GEMM is a loop of GEMVs too), unless y_f32
 * doubles as the bias. workspace: sf_q4_gemm_workspace_bytes(...) bytes (may
 * be 0 -> NULL ok). */
size_t sf_q4_gemm_workspace_bytes(int M, int N, int K, int group_size);
int sf_q4_gemm(const void *blob, const void *x, int x_dtype, void *y, int y_dtype, float *y_f32,
               const void *bias, int bias_dtype, int M, int N, int K, int group_size,
               int has_zeros, void *workspace, size_t workspace_bytes, void *stream);

/* The prefill GEMM with its K-split partials left for the next op (no
 * counterpart in the reference, whose q4_gemm returns Y; here the decoder's
 * prompt path folds the residual delta into the RMSNorm that follows).
 * sf_q4_gemm_splits: the number of K splits sf_q4_gemm runs for this shape
 * (1: unsplit; 0: invalid shape or a group size that is not a multiple of 32).
 * sf_q4_gemm_partials: for a shape with 2+ splits, writes split s's fp32
 * partial of Y[m, n] at workspace[s * M * N + m * N + n] and launches nothing
 * else; SF_EINVAL for an unsplit shape. The partials summed in split order
 * from 0 are the sums sf_q4_gemm's own reduce forms. */
int sf_q4_gemm_splits(int M, int N, int K, int group_size);
int sf_q4_gemm_partials(const void *blob, const void *x, int x_dtype, int M, int N, int K,
                        int group_size, int has_zeros, void *workspace, size_t workspace_bytes,
                        void *stream);

/* ---- int8 KV cache ----------------------------------------------------------
 * Quantize T_new new tokens and write them at positions [T_off, T_off+T_new)
 * of a preallocated cache. Replaces quantize_kv + the concatenation in
 * QuantizedKVCache.update (siliconfer/model/kv_cache.py:49-63, 90-105).
 * k_new/v_new: [B, KVH, T_new, D] of in_dtype, contiguous.
 * codes: int8 [B, KVH, T_cap, D]; scales: [B, KVH, T_cap] of scale_dtype
 * (SF_F16 or SF_F32). Per (b, h, t): s = max|x|/127 (1 if 0), computed in
 * fp32; code = clip(rint(x/s), -128, 127); the stored scale is s rounded to
 * scale_dtype. */
int sf_kv_quant_append(const void *k_new, const void *v_new, int in_dtype, int8_t *k_codes,
                       void *k_scales, int8_t *v_codes, void *v_scales, int scale_dtype,
                       int B, int KVH, int T_new, int T_off, int T_cap, int D, void *stream);

/* ---- fused decode attention over the int8 cache ----------------------------
 * out[b, h, :] = softmax(scale * q[b,h] . K[b, h/(H/KVH), :T]^T) V[...]
 * with K = k_codes * k_scales per token (likewise V). Replaces
 * fused_quantized_attention_decode (siliconfer/kernels/metal/q4_attention.py:
 * 200-261). q: [B, H, D] of q_dtype; out: [B, H, D] of out_dtype. n_splits is
 * the split-T count (the reference's n_tiles; <=0 picks a default; at most
 * 512). D <= 256 (the reference's bound, q4_attention.py:78,227-228) and
 * D % 8 == 0. One split is one launch; more splits write their partials
 * (m, l, acc) to the workspace and a second launch merges them with the
 * reference's combine rule (q4_attention.py:63-70, 256-261), each sum a
 * pairwise tree over the splits in order.
 * workspace: sf_attn_workspace_bytes(B, H, D, n_splits) bytes, 256-byte
 * aligned (NULL for one split), no initial contents needed: acc
 * [B*H][n_splits][D] fp32 at offset 0, then (m, l) [B*H][n_splits][2] fp32
 * at the next 256-byte boundary. Calls that share a workspace must not
 * overlap (use one workspace per stream). */
size_t sf_attn_workspace_bytes(int B, int H, int D, int n_splits);
/* Default split count (the reference's _choose_n_tiles, q4_attention.py:183-197,
 * re-tuned for MI355X): one split up to 160 cached tokens, then 32 tokens per
 * split up to 2048 tokens and 64 above, 8 to 128 splits (any head_dim).
 * sf_attn_default_splits is the same rule. */
int sf_attn_default_splits(int B, int KVH, int T);
int sf_attn_default_splits_d(int B, int KVH, int T, int D);
int sf_attn_decode_i8kv(const void *q, int q_dtype, const int8_t *k_codes, const void *k_scales,
                        const int8_t *v_codes, const void *v_scales, int scale_dtype, void *out,
                        int out_dtype, void *workspace, size_t workspace_bytes, int B, int H,
                        int KVH, int T, int T_cap, int D, float scale, int n_splits,
                        void *stream);

/* No counterpart in the reference: sf_attn_decode_i8kv for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Same arguments and result, without the workspace: the
 * split partials live in a fixed device array of
 * sf_attn_noalloc_max_bytes() (4 MiB) per GPU, held until the process ends;
 * shapes whose workspace would exceed it (sf_attn_workspace_bytes) return
 * SF_EINVAL. The call allocates nothing. Calls that overlap on one GPU (two
 * streams at once) race on the shared array. */
size_t sf_attn_noalloc_max_bytes(void);
int sf_attn_decode_i8kv_noalloc(const void *q, int q_dtype, const int8_t *k_codes,
                                const void *k_scales, const int8_t *v_codes, const void *v_scales,
                                int scale_dtype, void *out, int out_dtype, int B, int H, int KVH,
                                int T, int T_cap, int D, float scale, int n_splits, void *stream);

/* The same attention with its length in device memory: T = *T_dev + T_add
 * (for decode steps replayed from a HIP graph, where the length grows by one
 * token per replay). n_splits (<= 0: sf_attn_default_splits_d at T_max) and the
 * workspace are fixed for T <= T_max. Same reference interface as above. */
int sf_attn_decode_i8kv_dev(const void *q, int q_dtype, const int8_t *k_codes,
                            const void *k_scales, const int8_t *v_codes, const void *v_scales,
                            int scale_dtype, void *out, int out_dtype, void *workspace,
                            size_t workspace_bytes, int B, int H, int KVH, const int *T_dev,
                            int T_add, int T_max, int T_cap, int D, float scale, int n_splits,
                            void *stream);

/* sf_attn_decode_i8kv_dev without the merge launch, for a consumer that merges
 * the split partials itself (sf_q4_gemv_attn_merge, the decoder's o
 * projection): leaves the partials of n_splits (2..512) splits in the
 * workspace in the layout above and writes no output. No counterpart in the
 * reference (its decode kernel merges in the same dispatch,
 * q4_attention.py:256-261). */
int sf_attn_decode_i8kv_partials_dev(const void *q, int q_dtype, const int8_t *k_codes,
                                     const void *k_scales, const int8_t *v_codes,
                                     const void *v_scales, int scale_dtype, void *workspace,
                                     size_t workspace_bytes, int B, int H, int KVH,
                                     const int *T_dev, int T_add, int T_max, int T_cap, int D,
                                     float scale, int n_splits, void *stream);

/* The decoder's o projection with the attention's split merge folded into its
 * activation load: x[b, h*D + d] is the merged attention output of the split
 * partials in `workspace` (sf_attn_decode_i8kv_partials_dev, B rows of H heads,
 * n_splits = 2..8), rounded to act_dtype, and y = W x as sf_q4_gemv (K = H*D).
 * Bit-identical to sf_attn_decode_i8kv writing an act_dtype output followed by
 * sf_q4_gemv on it. sf_q4_gemv_attn_merge_supported says which shapes (1);
 * others return SF_EUNSUPPORTED. No counterpart in the reference, which runs
 * the attention and Q4Linear o_proj as separate ops
 * (/root/reference/siliconfer/model/layers.py:120-133). */
int sf_q4_gemv_attn_merge_supported(int B, int N, int H, int D, int n_splits, int group_size,
                                    int act_dtype);
int sf_q4_gemv_attn_merge(const void *blob, const void *workspace, size_t workspace_bytes,
                          int n_splits, int H, int D, int act_dtype, void *y, int y_dtype,
                          float *y_f32, const void *bias, int bias_dtype, int B, int N,
                          int group_size, int has_zeros, void *stream);

/* Causal prefill attention over a batch-1 int8 cache: query row i of q
 * [T_q][H][D] attends to the first T0 + i + 1 cached tokens (the prompt's own
 * keys already appended). Replaces the reference's prompt path, which
 * dequantizes the whole cache and runs SDPA with an additive causal mask
 * (/root/reference/siliconfer/model/layers.py:108-126). Output [T_q][H][D]. */
int sf_attn_prefill_i8kv(const void *q, int q_dtype, const int8_t *k_codes, const void *k_scales,
                         const int8_t *v_codes, const void *v_scales, int scale_dtype, void *out,
                         int out_dtype, int T_q, int H, int KVH, int T0, int T_cap, int D,
                         float scale, void *stream);

/* The same causal attention with T0 in device memory (*T0_dev, read when the
 * kernel runs): the verify rows of speculative decoding replayed from a HIP
 * graph at a position the host does not know when it records the launch.
 * n_splits (<= 0: sf_attn_default_splits_d(T_q, KVH, T_max, D)) and the workspace
 * (sf_attn_workspace_bytes(T_q, H, D, n_splits)) are fixed for T0 + T_q <= T_max;
 * rows past T_cap see T_cap tokens. */
int sf_attn_prefill_i8kv_dev(const void *q, int q_dtype, const int8_t *k_codes,
                             const void *k_scales, const int8_t *v_codes, const void *v_scales,
                             int scale_dtype, void *out, int out_dtype, void *workspace,
                             size_t workspace_bytes, int T_q, int H, int KVH, const int *T0_dev,
                             int T_max, int T_cap, int D, float scale, int n_splits, void *stream);

/* ---- decoder step operations (model runner) -------------------------------
 * The per-token work of the reference's TransformerBlock / LlamaModel around
 * the projections (/root/reference/siliconfer/model/layers.py:14-163,
 * model/llama.py:38-83). Row-major fp32 residual stream. */

/* Embedding gather: out[r][:] = table[ids[r]][:] (nn.Embedding, llama.py:55).
 * ids int32 on the device (out-of-range ids are clamped). */
int sf_embed(const int32_t *ids, const void *table, int table_dtype, float *out, int rows, int H,
             int V, void *stream);

/* RMSNorm (layers.py:14-21, mx.fast.rms_norm): if delta, x += delta in place
 * (the residual add of layers.py:160-162); then
 * out[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * w. */
int sf_rmsnorm(float *x, const float *delta, const void *w, int w_dtype, void *out, int out_dtype,
               int rows, int H, float eps, void *stream);

/* sf_rmsnorm with delta given as the n_parts K-split partials of
 * sf_q4_gemm_partials for rows x H outputs (partial s at
 * part[s * rows * H + r * H + h]): delta = the partials summed in split order
 * from 0. x and out get the bits of sf_q4_gemm into a delta buffer followed
 * by sf_rmsnorm(x, delta), with one launch less (the same layers.py:14-21,
 * 160-162). */
int sf_rmsnorm_partials(float *x, const float *part, int n_parts, const void *w, int w_dtype,
                        void *out, int out_dtype, int rows, int H, float eps, void *stream);

/* RoPE (layers.py:58-66, rotate-half) of the q and k heads of the fused q|k|v
 * projection rows qkv [rows][(H + 2 KVH) * D] at positions pos0 + r, then the
 * int8 quantize-append of k and v into a batch-1 cache [KVH][T_cap][D] with the
 * rule of sf_kv_quant_append (kv_cache.py:49-63, 90-105). cos_t / sin_t are
 * fp32 [max_pos][D/2] tables of position * freq (layers.py:24-33). pos0 is
 * *pos_dev when pos_dev is not NULL (device-side decode position), else
 * pos_host. Rotated q goes to q_out [rows][H][D]. */
int sf_rope_kv_append(const float *qkv, const float *cos_t, const float *sin_t, int max_pos,
                      void *q_out, int q_dtype, int8_t *k_codes, void *k_scales, int8_t *v_codes,
                      void *v_scales, int scale_dtype, int rows, int H, int KVH, int D, int T_cap,
                      const int *pos_dev, int pos_host, void *stream);

/* sf_rope_kv_append with the q|k|v rows given as the n_parts K-split partials
 * of sf_q4_gemm_partials (partial s at part[s * rows * W + r * W + c],
 * W = (H + 2 KVH) * D) plus the projection's bias [W] (or NULL): each value
 * summed in split order from 0, then the bias added. The same bits as
 * sf_q4_gemm(..., bias) into a qkv buffer followed by sf_rope_kv_append, with
 * one launch less (no counterpart in the reference; layers.py:99-112). */
int sf_rope_kv_append_partials(const float *part, int n_parts, const void *bias, int bias_dtype,
                               const float *cos_t, const float *sin_t, int max_pos, void *q_out,
                               int q_dtype, int8_t *k_codes, void *k_scales, int8_t *v_codes,
                               void *v_scales, int scale_dtype, int rows, int H, int KVH, int D,
                               int T_cap, const int *pos_dev, int pos_host, void *stream);

/* SwiGLU activation (layers.py:143-144): out[r][i] = silu(gu[r][i]) *
 * gu[r][I + i] for the fused gate|up projection rows gu [rows][2 I]. */
int sf_silu_mul(const float *gu, void *out, int out_dtype, int rows, int I, void *stream);

/* Tied-embedding logits and greedy token (llama.py:77-79 `as_linear`,
 * generate.py:45-46 argmax): logits[v] = sum_k W[v][k] x[k] for bf16 W [V][H],
 * written as fp32 when logits is not NULL; *token_out = argmax (lowest index
 * on ties). When pos_inc is not NULL: hist[*pos_inc] = token (if hist is not
 * NULL), then *pos_inc += 1 — the device-side decode position. The workspace
 * (sf_lm_head_workspace_bytes, 256-byte aligned) must be zero-filled before
 * its first use; each call leaves it so. */
size_t sf_lm_head_workspace_bytes(int V);
int sf_lm_head_argmax(const void *w, const void *x, int x_dtype, float *logits, int V, int H,
                      int32_t *token_out, int *pos_inc, int32_t *hist, void *workspace,
                      size_t workspace_bytes, void *stream);

/* sf_lm_head_argmax with the final RMSNorm (llama.py:76) folded in: x =
 * h * rsqrt(mean(h^2) + eps) * norm_w for the fp32 residual row h [H], rounded
 * to act_dtype; bit-identical to sf_rmsnorm into an act_dtype buffer followed
 * by sf_lm_head_argmax on it. */
int sf_lm_head_argmax_rmsnorm(const void *w, const float *h, const float *norm_w, float eps,
                              int act_dtype, float *logits, int V, int H, int32_t *token_out,
                              int *pos_inc, int32_t *hist, void *workspace, size_t workspace_bytes,
                              void *stream);

/* Logits and greedy tokens of B = 1..8 rows at once: the target model's
 * verify of K+1 = B positions in greedy speculative decoding
 * (/root/reference/siliconfer/engine/speculative.py:166-189, which takes the
 * argmax of each verify row of `t_log`). x [B, H] (x_dtype); logits [B, V]
 * fp32 or NULL; tokens_out[b] = argmax of row b (lowest index on ties).
 * From 3 rows, fp16 / bf16 rows with H % 32 == 0 and H <= 2048 run on MFMA
 * (exact products, fp32 sums); the others on the VALU, where each row's logits equal
 * sf_lm_head_argmax's for that row alone, bit for bit. Needs
 * B * H * sizeof(x element) <= 65536. The workspace
 * (sf_lm_head_rows_workspace_bytes, 256-byte aligned) is zero-filled before
 * its first use; each call leaves it so. */
size_t sf_lm_head_rows_workspace_bytes(int V, int B);
int sf_lm_head_argmax_rows(const void *w, const void *x, int x_dtype, float *logits, int V, int H,
                           int B, int32_t *tokens_out, void *workspace, size_t workspace_bytes,
                           void *stream);

/* ---- a chain of dependent decode GEMVs in one persistent launch (no
 * counterpart in the reference, which runs each Q4Linear of a layer as its own
 * call, /root/reference/siliconfer/model/layers.py:93-95, 133, 139-144) -------
 * y = W_{n-1} f(... f(W_1 f(W_0 x0))): phase p multiplies the symmetric int4
 * blob blobs[p] ([N[p], K[p]], group group[p]: 64 or a multiple of 128; K[p] a
 * multiple of 128 up to 12288) by its input, at batch 1. Phase 0 reads x0
 * (fp16 [K[0]]); phase p > 0 reads the first K[p] of phase p-1's fp32 outputs
 * rounded to fp16 (in_kind[p] = SF_CHAIN_IN_PREV, N[p-1] >= K[p]) or silu(gate) * up of them
 * (SF_CHAIN_IN_SWIGLU: gate = outputs [0, K[p]), up = [K[p], 2 K[p]),
 * N[p-1] == 2 K[p]); in_kind[0] = SF_CHAIN_IN_X0. The last phase's fp32 output
 * goes to y_f32. One workgroup per CU runs every phase; a workgroup issues a
 * phase's weight loads before it waits for the phase's input, which it reads
 * from the workspace as tagged words (value + launch tag in one 8-byte atomic
 * word). The workspace (sf_q4_chain_workspace_bytes(N, nph), 256-byte aligned)
 * must be zero-filled once before its first call and then kept: it holds the
 * launch counter the tags come from. Calls that overlap on one workspace race.
 * Every wait is bounded by spin_cap rounds (~1-2 us each; 1 << 20 for
 * production use): on expiry the kernel records an error in the workspace and
 * exits normally with wrong results; sf_q4_chain_error (synchronous) returns
 * that error (0: none) and the workspace keeps it. drop_phase >= 0 is a test
 * hook: that phase's outputs are not published, so its consumers' waits
 * expire (-1 for normal use). */
#define SF_CHAIN_MAX_PHASES 8
#define SF_CHAIN_IN_X0 0
#define SF_CHAIN_IN_PREV 1
#define SF_CHAIN_IN_SWIGLU 2
size_t sf_q4_chain_workspace_bytes(const int *N, int nph);
int sf_q4_chain(const void *const *blobs, const int *N, const int *K, const int *group,
                const int *in_kind, int nph, const void *x0_f16, float *y_f32, void *workspace,
                size_t workspace_bytes, int spin_cap, int drop_phase, void *stream);
int sf_q4_chain_error(const void *workspace, int *err_out, void *stream);

/* ---- measurement floor (no counterpart in the reference: the reference only
 * assumes a peak bandwidth, scripts/benchmark.py:26) ----------------------
 * sf_floor_empty: one empty one-wave launch (the per-launch cost of the queue).
 * sf_floor_read: a plain read of `bytes` (a multiple of 16, 16-byte aligned)
 * from device memory, one 16-byte load per lane; `sink` is a device word it
 * writes only in a case random data does not produce. bench.py times both
 * beside the GEMV so each case's rate is reported against this GPU's own
 * read of the same size. */
int sf_floor_empty(void *stream);
int sf_floor_read(const void *buf, size_t bytes, uint32_t *sink, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* SILICONFER_HIP_H */
