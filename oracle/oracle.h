/*
 * oracle.h -- CPU restatement of typhoon-ocr-server's INT8 linear kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links, loads or calls
 * this code.  It is the checker used by tests/, by the smoke check and by the
 * CPU-baseline leg of bench.py.
 *
 * Naming follows the reference's ABI: N ("M" in the reference signatures) is
 * the number of output features (rows of W), K the number of input features,
 * batch the number of tokens (rows of X and Y).
 *
 * Each function cites the reference lines it restates.  Parity status of each
 * function (what pins it) is recorded in the header comment of oracle.c.
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Per-row symmetric quantizer (kernel/w8a32_kernel.c:63-108,
 * kernel/w8a8_kernel.c:54-100, kernel/w8a16_kernel.c:44-65 and, with
 * clamp_main=0, the activation quantizer kernel/w8a32_kernel.c:139-178). */
void orc_quantize_rows(const float *src, int8_t *dst, float *scales,
                       int rows, int cols, int clamp_main);

/* Exact int32 accumulators acc[b*N+n] = sum_k x_q[b*K+k] * w[n*K+k]. */
void orc_int_acc(const int8_t *x_q, const int8_t *w, int32_t *acc,
                 int batch, int N, int K, int threads);

/* w8a32_linear (kernel/w8a32_kernel.c:355-370).  scratch is ignored exactly
 * as in the reference (:364).  If codes/xscale/acc are non-NULL and batch==1
 * they receive the M=1 intermediates (activation codes, activation scale,
 * int32 accumulators). */
void orc_w8a32_linear(const float *X, const int8_t *w, const float *scales,
                      const float *bias, float *Y, int batch, int N, int K,
                      int threads, int8_t *codes, float *xscale, int32_t *acc);

/* w8a8_linear (kernel/w8a8_kernel.c:270-275). */
void orc_w8a8_linear(const int8_t *x_q, const float *x_scales,
                     const int8_t *w, const float *w_scales, const float *bias,
                     float *Y, int batch, int N, int K, int threads);

/* w8a16_linear (kernel/w8a16_kernel.c:218-223); X is raw bf16 bits. */
void orc_w8a16_linear(const uint16_t *x_bf16, const int8_t *w,
                      const float *w_scales, const float *bias, float *Y,
                      int batch, int N, int K, int threads);

/* Same-formula CPU GEMV timed as the CPU baseline: the reference's M=1
 * decode path (activation quantization, int8 dot per row, fp32 epilogue),
 * parallel over rows like _sdot_gemv_worker (w8a32_kernel.c:205-275). */
void orc_w8a32_gemv_timed(const float *x, const int8_t *w, const float *scales,
                          float *y, int N, int K, int threads);

/* ---- decoder layer step (decoder_ref.c) -------------------------------- */
/* Arm FRECPE / FRSQRTE estimates and their Newton steps (positive normal x). */
float orc_frecpe(float x);
float orc_frsqrte(float x);
float orc_frecps(float a, float b);
float orc_frsqrts(float a, float b);
/* rmsnorm_f32 (kernel/ops.c:22-56); out may alias x. */
void orc_rmsnorm(float *out, const float *x, const float *w, int dim, float eps);
/* mrope_precompute (kernel/ops.c:150-177), tables [max_seq x head_dim/2]. */
void orc_mrope_precompute(float *cos_tab, float *sin_tab, int max_seq, int head_dim, float theta);
/* mrope_apply (kernel/ops.c:233-289), in place. */
void orc_mrope_apply(float *q, float *k, const float *cos_tab, const float *sin_tab, int num_q_heads,
                     int num_kv_heads, int head_dim, int pos);
/* fast_exp_f32 (kernel/ops.c:478-491), silu of the vector loop, and
 * silu_mul_inplace (kernel/ops.c:493-531). */
float orc_fast_exp(float x);
float orc_silu_fast(float g);
void orc_silu_mul(float *gate, const float *up, int n);
/* attention_decode_gqa (kernel/attention.c:172-224); cache per kv head
 * [max_seq x 128], positions 0..S-1. */
void orc_attention_decode(const float *q, const float *Kc, const float *Vc, float *out, int num_q_heads,
                          int num_kv_heads, int max_seq, int S, float scale);
/* decoder_layer_forward in DECODE_MODE (kernel/decoder.c:33-157). */
void orc_decode_layer(const int8_t *const *w, const float *const *s, const float *input_ln,
                      const float *post_attn_ln, const float *q_norm, const float *k_norm, float *Kc,
                      float *Vc, int max_seq, float *hidden, const float *cos_tab, const float *sin_tab,
                      int cache_len, int rope_pos, int hidden_dim, int ffn_dim, int num_q_heads,
                      int num_kv_heads, int threads);

/* ---- prefill (decoder_ref.c) ------------------------------------------ */
/* mrope_build_cos_sin_3d (kernel/ops.c:188-223), pos_ids [3 x seq_len]. */
void orc_mrope_build_3d(float *cos_out, float *sin_out, const int *pos_ids, int seq_len, int head_dim,
                        const int sections[3], float theta);
/* attention_prefill_gqa / _flash_worker (kernel/attention.c:252-344). */
void orc_attention_prefill(const float *q, const float *k, const float *v, float *out, int Sq, int nq, int nkv,
                           float scale);
/* decoder_layer_forward in PREFILL_MODE / PREFILL_3D_MODE (kernel/decoder.c:33-157). */
void orc_prefill_layer(const int8_t *const *w, const float *const *s, const float *input_ln,
                       const float *post_attn_ln, const float *q_norm, const float *k_norm, float *Kc, float *Vc,
                       int max_seq, float *hidden, int S, const float *cos_tab, const float *sin_tab,
                       const float *token_cos, const float *token_sin, int cache_len, int hidden_dim, int ffn_dim,
                       int num_q_heads, int num_kv_heads, int threads, int w8a8);

/* CPU baseline (baseline.c): the reference's M>1 tile decompositions on a
 * blocked fp32 SGEMM, and the W8A16 batch-1 GEMV, for timing beside the GPU. */
void orc_base_w8a32_gemm(const float *X, const int8_t *w, const float *ws, const float *bias, float *Y,
                         int M, int N, int K, int threads);
void orc_base_w8a8_gemm(const int8_t *xq, const float *xs, const int8_t *w, const float *ws, const float *bias,
                        float *Y, int M, int N, int K, int threads);
void orc_base_w8a16_linear(const uint16_t *xb, const int8_t *w, const float *ws, const float *bias, float *Y,
                           int M, int N, int K, int threads);

#ifdef __cplusplus
}
#endif
