/*
 * typhoon_linear.h -- C ABI of the MI355X (gfx950) INT8 weight-quantized
 * linear layers: libtyphoon_linear.so.
 *
 * Part 1 is a drop-in for the reference's linear-layer entry points: same
 * names, same signatures, same argument meaning, same `void` returns, host
 * pointers borrowed for the duration of the call, Y fully written when the
 * call returns.  "M" in these signatures is the number of output features
 * (rows of W) and "batch" the number of tokens, as in the reference.
 * Numerics follow the reference's batch-dependent branches:
 *   w8a32_linear batch==1: per-token int8 activation quantization, exact
 *     int32 dot, y = fl(fl(fl(acc)*ws)*xs) (+bias)          (bit-exact)
 *   w8a32_linear batch>1 : fp32 X times dequantized weights (fp32 accuracy)
 *   w8a8_linear  batch==1: exact int32 dot, fma(fl(fl(acc)*ws), xs, bias|0)
 *   w8a8_linear  batch>1 : exact int32 dot, fl(fl(fl(acc)*ws)*xs) (+bias)
 *   w8a16_linear         : bf16 X, int8 W exact in bf16, fp32 accumulate,
 *                          fp32 per-row scale, fp32 Y
 * Quantized weights are uploaded once into HBM as 16x64 int8 tiles with
 * their fp32 scales (a registry keyed by the host weight pointer, its scale
 * pointer and shape, validated by a sampled content fingerprint).
 *
 * Errors: the reference functions return void and report nothing.  Here a
 * failed call prints one line to stderr and records a message that
 * tl_last_error() returns (per calling thread); the outputs are then
 * unspecified.
 *
 * Part 2 (tl_*) has no counterpart in the reference: device-resident weights
 * and stream-ordered calls on device pointers for callers that keep
 * activations in HBM (a device-resident decoder loop, benchmarks, tests).
 */
#ifndef TYPHOON_LINEAR_H
#define TYPHOON_LINEAR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ======================================================================== */
/* Part 1 -- reference entry points                                          */
/* ======================================================================== */

/* Replaces w8a32_quantize, kernel/w8a32_kernel.c:63-68 (bound in decoder.py
 * at :146-150).  Per-row symmetric quantization, codes in [-127, 127]. */
void w8a32_quantize(const float *w_fp32, int8_t *w_int8, float *scales, int rows, int cols);

/* Replaces w8a32_linear, kernel/w8a32_kernel.c:355-363 (declared for the
 * decoder at kernel/decoder.h:13-21, bound in decoder.py at :153-157).
 * X [batch x K] fp32, w_int8 [M x K], scales [M], bias [M] or NULL,
 * Y [batch x M] fp32.  scratch is ignored, as in the reference (:364). */
void w8a32_linear(const float *X, const int8_t *w_int8, const float *scales, const float *bias,
                  float *Y, float *scratch, int batch, int M, int K);

/* Replaces w8a8_quantize_weights, kernel/w8a8_kernel.c:102-107. */
void w8a8_quantize_weights(const float *w_fp32, int8_t *w_int8, float *w_scales, int rows,
                           int cols);

/* Replaces w8a8_quantize_activations, kernel/w8a8_kernel.c:109-114.
 * Per-token (per-row) quantization of X [batch x K]. */
void w8a8_quantize_activations(const float *x_fp32, int8_t *x_int8, float *x_scales, int batch,
                               int K);

/* Replaces w8a8_linear, kernel/w8a8_kernel.c:270-272. */
void w8a8_linear(const int8_t *x_int8, const float *x_scales, const int8_t *w_int8,
                 const float *w_scales, const float *bias, float *Y, int batch, int M, int K);

/* Replaces w8a16_quantize_weights, kernel/w8a16_kernel.c:44. */
void w8a16_quantize_weights(const float *w_fp32, int8_t *w_int8, float *scales, int rows,
                            int cols);

/* Replaces w8a16_linear, kernel/w8a16_kernel.c:218-219.  x_bf16_raw holds
 * raw bf16 bits [batch x K]; Y is fp32 [batch x M]. */
void w8a16_linear(const uint16_t *x_bf16_raw, const int8_t *w_int8, const float *w_scales,
                  const float *bias, float *Y, int batch, int M, int K);

/* ======================================================================== */
/* Part 2 -- extensions (no reference counterpart)                           */
/* ======================================================================== */

/* Message of the calling thread's last failed call, or NULL.  Cleared by
 * tl_clear_error() and at the start of every call. */
const char *tl_last_error(void);
void tl_clear_error(void);

/* Library version string and the number of visible GPUs (0 if none). */
const char *tl_version(void);
int tl_device_count(void);

/* Host-weight registry (Part 1 calls fill it lazily).  tl_register_weights
 * uploads eagerly (what a decoder's weight-registration call would do);
 * tl_evict_weights drops every entry whose weight pointer is w_int8. */
int tl_register_weights(const int8_t *w_int8, const float *scales, int rows, int cols);
int tl_evict_weights(const int8_t *w_int8);
void tl_registry_clear(void);
size_t tl_registry_bytes(void);
int tl_registry_entries(void);

/* Tuning override of the M=1 GEMV decomposition for every later call in the
 * process: rows per work-group (16, or 8 = half of a 16-row tile group) and
 * weight load instructions per batch (2, 4, 8, 12 with 16 rows; 2, 4, 6, 8
 * with 8 rows).  Zeros restore the built-in planner. */
int tl_gemv_set_plan(int rows, int u);

/* Tuning override of the int8 MFMA GEMM (W8A8, M > 16) for every later call
 * in the process: -1 restores the planner; 0..2 stage both operands through
 * LDS (tiles 128x192, 64x128, 128x128); 3..7 load weight tiles straight into
 * registers (128x192 with prefetch 3, 5, 7 stages; 64x128 and 128x128 with
 * prefetch 7). */
int tl_gemm_i8_set_cfg(int cfg);

/* Tuning override of the same GEMM's K slices for every later call in the
 * process: 0 restores the planner (slices where a shape has fewer than 128
 * tiles), 1..64 force that many work-groups per tile (on the LDS-staged
 * kernel), whose exact int32 partial sums the last to arrive adds. */
int tl_gemm_i8_set_split(int split);

/* Tuning override of the 16-bit MFMA GEMM (W8A16, M > 16 on the tiled
 * kernel) for every later call in the process: cfg -1 restores the planner's
 * kernel and tile, 0..2 force 128x192, 64x128 or 32x64 tiles of the
 * LDS-staged kernel, 4..8 the column-split kernel's 128x192 (5- or 7-deep
 * ring), 128x128, 64x192 or 64x128 tiles (K a multiple of 64; other K run
 * cfg 0), 3 forces the
 * streamed small-M kernel (M <= 256, weights read once per work-group of
 * token rows; with cfg 3 a split of 100 R + 10 TG + U picks its work-group
 * shape: R, TG in {1, 2, 4} weight / token row groups, U in {2, 4} tiles per
 * load batch); split 0 restores the
 * planner's K slices, 1..64 force that many (work-groups per tile, whose fp32
 * partial sums the last to arrive adds in slice order). */
int tl_gemm_b16_set_plan(int cfg, int split);

/* Tuning override of the 2..8-row kernel of w8a32_linear (int8 digit planes
 * of the fp32 activations) for every later call in the process: 1..64 K
 * slices per weight row group (at least as many as its LDS and registers
 * need), 0 restores the planner, -1 switches the kernel off (the bf16-term
 * small-batch kernel then takes those batches). */
int tl_rows_set_split(int split);

/* Tuning override of the same kernel: 1..3 16-row weight groups per
 * work-group, sharing one split of the activations (taken only where a K
 * slice holds at most 32 k-blocks; 1 elsewhere), 0 restores the planner. */
int tl_rows_set_groups(int groups);

/* Tuning switch of w8a16_linear at batch 1 for every later call in the
 * process: 1 (the default) runs it on the GEMV's weight stream with x as four
 * int8 digit rows; 0 on the bf16 / fp16 MFMA small-batch kernel. */
int tl_w8a16_set_gemv(int on);

/* Tuning switch of w8a32_linear at batch 2..4 for every later call in the
 * process: on the GEMV's weight stream with four int8 digit rows per token
 * where measured faster (1, the default: batch 2 at every shape, 3..4 below
 * 32768 weight rows, K <= 8192), wherever the kernel takes the shape (2:
 * batch 2 up to K = 16384, 3..4 up to K = 8192), or never (0: the digit-row
 * MFMA kernel of batches 2..8 or the planes GEMM, the same arithmetic as the
 * former at one K slice). */
int tl_w8a32_set_gemv2(int on);

/* Measurement aid, no counterpart in the reference: one streaming read of
 * `bytes` device bytes (a multiple of 16, p 16-byte aligned) by `grid`
 * work-groups with u (4 or 8) 16-byte loads in flight per lane, the loads
 * of the GEMV weight stream and nothing else.  Its launch time is the floor
 * a launch reading that many bytes reaches on the device, against which the
 * GEMV times are set (bench.py).  sink: one device word, written only if the
 * bytes fold to a fixed improbable value. */
int tl_stream_read_dev(const void *p, size_t bytes, int grid, int u, uint32_t *sink, void *stream);

/* Tuning override of the decode attention for every later launch or graph
 * capture in the process: cache positions per work-group, 32, 64 or 128; 0
 * restores the built-in choice. */
int tl_attn_set_chunk(int positions);

/* ---- device-resident weights ------------------------------------------- */
typedef struct tl_weights tl_weights;

/* Packs int8 weights [rows x cols] (row-major, host or device memory) and
 * their fp32 scales into HBM tiles on the current device.  NULL on error. */
tl_weights *tl_weights_create(const int8_t *w_int8, const float *scales, int rows, int cols,
                              int src_on_device);
/* Quantizes fp32 weights held in device memory (per row, as w8a32_quantize)
 * straight into tiles; optionally also returns row-major codes/scales
 * (device pointers, may be NULL).  NULL on error. */
tl_weights *tl_weights_quantize_dev(const float *w_fp32, int rows, int cols, int8_t *codes_out,
                                    float *scales_out, void *stream);
void tl_weights_destroy(tl_weights *w);

/* Packed-weight cache file (no counterpart in the reference, which
 * re-quantizes every fp32 matrix at load: decoder.py:248-260 through
 * w8a32_quantize, kernel/w8a32_kernel.c:63-108).  A file is a sequence of
 * named records, each holding one matrix's HBM tiles and scales exactly as
 * resident, with a checksum; loading is a copy into HBM with no kernel.
 *   tl_weights_save   writes W as record `name` (append != 0 adds it at the
 *                     end of an existing file, else the file is replaced)
 *   tl_weights_load   reads the first record called `name` into HBM on the
 *                     current device; NULL on error (missing record, bad
 *                     magic/version/sizes, checksum mismatch)
 *   tl_weights_cache_list  number of records (-1 on error); their names,
 *                     one per line, into names when it is non-NULL */
int tl_weights_save(const tl_weights *W, const char *path, const char *name, int append);
tl_weights *tl_weights_load(const char *path, const char *name);
int tl_weights_cache_list(const char *path, char *names, size_t names_len);

/* Copies W's codes out as row-major int8 [rows x cols] and its fp32 scales
 * [rows] (either may be NULL), into host or device memory. */
int tl_weights_export(const tl_weights *W, int8_t *codes, float *scales, int dst_on_device);

/* Makes W the device copy the host-pointer entry points use for the host
 * arrays (w_int8 [rows x cols], scales [rows]), which must hold W's codes
 * and scales (e.g. from tl_weights_export): later calls on those arrays
 * upload nothing.  On success the registry owns W (do not destroy it). */
int tl_registry_adopt(const int8_t *w_int8, const float *scales, tl_weights *W);
int tl_weights_rows(const tl_weights *w);
int tl_weights_cols(const tl_weights *w);
size_t tl_weights_bytes(const tl_weights *w);

/* ---- stream-ordered device calls (all pointers device memory) ----------
 * stream is a hipStream_t (NULL = default stream).  Return 0 on success,
 * -1 on error (see tl_last_error).  Work-space for split reductions is
 * owned by the library per (device, stream); calls that overlap on one
 * stream are ordered by it. */
enum { TL_F32 = 0, TL_BF16 = 1, TL_F16 = 2 };

/* w8a32_linear semantics (batch==1: fused per-token int8 GEMV; batch>1:
 * fp32-accurate GEMM). */
int tl_w8a32_linear_dev(const float *X, const tl_weights *W, const float *bias, float *Y,
                        int batch, void *stream);
/* Per-token quantization, row-major codes (w8a8_quantize_activations). */
int tl_quantize_rows_dev(const float *src, int8_t *codes, float *scales, int rows, int cols,
                         int clamp127, void *stream);
/* w8a8_linear semantics on row-major device codes. */
int tl_w8a8_linear_dev(const int8_t *x_int8, const float *x_scales, const tl_weights *W,
                       const float *bias, float *Y, int batch, void *stream);
/* W8A8 prefill: fp32 X quantized per token on the GPU (into int8 tiles),
 * then the int8 MFMA GEMM with the fp32 epilogue. */
int tl_w8a8_linear_f32_dev(const float *X, const tl_weights *W, const float *bias, float *Y,
                           int batch, void *stream);

/* The two halves of tl_w8a8_linear_f32_dev at batch > 1, for callers that
 * quantize once and reuse the codes, or time the GEMM alone (no reference
 * counterpart: the reference's w8a8_quantize_activations / w8a8_linear,
 * w8a8_kernel.c:109-114, :259-275, on row-major codes):
 * tl_w8a8_quantize_tiles_dev writes the per-token int8 codes of X [batch][K]
 * in the library's 16x64 activation tile layout (tl_w8a8_tiles_bytes bytes)
 * and the token scales (ceil(batch/16)*16 floats of room); the codes are
 * those of w8a8_quantize_activations.  tl_w8a8_linear_tiles_dev runs the
 * int8 MFMA GEMM on them with the fp32 epilogue fl(fl(fl(acc) ws) xs)
 * (+ bias as its own rounding). */
size_t tl_w8a8_tiles_bytes(int batch, int K);
int tl_w8a8_quantize_tiles_dev(const float *X, int batch, int K, uint8_t *x_tiles, float *x_scales,
                               void *stream);
int tl_w8a8_linear_tiles_dev(const uint8_t *x_tiles, const float *x_scales, const tl_weights *W,
                             const float *bias, float *Y, int batch, void *stream);
/* W8A16: X bf16 or fp16 [batch x K], Y fp32, bf16 or fp16 [batch x N]. */
int tl_w8a16_linear_dev(const void *X, int x_type, const tl_weights *W, const float *bias,
                        void *Y, int y_type, int batch, void *stream);

/* Greedy next token from the last hidden row, the steps of decoder.py:443-464
 * (_get_logits, then the greedy branch of _sample) in one stream-ordered
 * call: x = (h / sqrt(mean(h*h) + 1e-6)) * norm_w in numpy's float32 order
 * (norm_w may be NULL: no weight), lm_head logits = w8a32_linear(x, W)
 * (stored only if logits != NULL), *token = first index of the largest
 * logit, *max_logit = that logit (may be NULL).  K = W's columns must be a
 * power of two in [128, 16384].  No reference counterpart: the reference
 * returns all 151936 logits to Python and takes the argmax there. */
int tl_lm_head_argmax_dev(const float *h, const float *norm_w, const tl_weights *W, float *logits,
                          int32_t *token, float *max_logit, void *stream);
/* No reference counterpart.  tl_lm_head_argmax_dev for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the same launches and results, with the
 * work-space in a device array inside the library -- the argmax keys of up to
 * 262144 lm_head rows and one normalised row of up to 16384 floats, 192 KiB,
 * one copy per device, held until the process ends.  The call allocates
 * nothing; larger lm_heads are rejected with an error.  Calls that overlap on
 * one device share the array and race. */
int tl_lm_head_argmax_noalloc_dev(const float *h, const float *norm_w, const tl_weights *W, float *logits,
                                  int32_t *token, float *max_logit, void *stream);
/* The same on host pointers (weights through the registry, like
 * w8a32_linear); returns the token in *token, logits optional. */
int tl_lm_head_argmax(const float *h, const float *norm_w, const int8_t *w_int8, const float *scales,
                      int N, int K, float *logits, int32_t *token);
/* Test hook: the normalised row alone (device pointers). */
int tl_rmsnorm_np_dev(const float *h, const float *norm_w, float *out, int K, void *stream);

/* Test hooks: the exact int32 accumulators of the fused M=1 GEMV (and the
 * activation scale it derived), and of the int8 MFMA GEMM on row-major
 * codes. */
int tl_w8a32_gemv_acc_dev(const float *x, const tl_weights *W, int32_t *acc, float *x_scale,
                          void *stream);
int tl_w8a8_gemm_acc_dev(const int8_t *x_int8, const tl_weights *W, int32_t *acc, int batch,
                         void *stream);
/* The M=1 GEMV with the decoder's fusions (device pointers): norm 0 none,
 * 1 numpy final RMSNorm, 2 the decoder's RMSNorm (kernel/ops.c:22-56) of x
 * with norm_w first; epi 0 W8A32 (+ bias as its own rounding; bias may be y
 * itself: the residual add of decoder.c:122-123), 4 SwiGLU over gate/up rows
 * interleaved per 16-row group (y[8b + r] = silu(gate) * up, kernel/ops.c:
 * 493-531, N/2 outputs). */
int tl_gemv_fused_dev(const float *x, const tl_weights *W, const float *bias, float *y, int epi, int norm,
                      const float *norm_w, void *stream);

/* ==========================================================================
 * Part 3 -- the decoder loop (kernel/decoder.h, kernel/decoder.c:300-526)
 *
 * The reference's decoder handles and entry points, same names, signatures
 * and void returns, with the layer loop resident on the GPU: weights are
 * packed into HBM at decoder_set_layer_weights*, the KV cache and scratch
 * live in HBM, and each decode step is one replay of a captured HIP graph.
 * Dimensions are the reference's (decoder.h, scratch.h): hidden 2048, FFN
 * 6144, 16 q / 8 kv heads of 128; layers run from 0 to the first layer not
 * set (the reference always runs its 28).  Host pointers are borrowed for the
 * call.  Failures set tl_last_error().
 * ========================================================================== */
typedef struct ModelWeights ModelWeights;
typedef struct KVCache KVCache;
typedef struct DecoderScratch DecoderScratch;

ModelWeights *decoder_model_alloc(void);                      /* decoder.c:322 */
void decoder_model_free(ModelWeights *m);                     /* decoder.c:327 */
KVCache *decoder_cache_alloc(int max_seq);                    /* decoder.c:332 */
void decoder_cache_free(KVCache *c);                          /* decoder.c:337 */
void decoder_cache_clear(KVCache *c);                         /* decoder.c:342 */
void decoder_cache_set_rope_offset(KVCache *c, int offset);   /* decoder.c:347 */
DecoderScratch *decoder_scratch_alloc_fn(int max_seq);        /* decoder.c:352 */
void decoder_scratch_free_fn(DecoderScratch *s);              /* decoder.c:357 */

/* decoder.c:363-391: int8 codes row-major + fp32 scales per projection, the
 * two RMSNorm weights [2048] and the q/k head norms [128]; copied into HBM
 * (Q||K||V fused; gate/up interleaved per 16-row group for the fused SwiGLU). */
void decoder_set_layer_weights(ModelWeights *model, int layer_idx, const int8_t *q_w, const float *q_s,
                               const int8_t *k_w, const float *k_s, const int8_t *v_w, const float *v_s,
                               const int8_t *o_w, const float *o_s, const int8_t *gate_w, const float *gate_s,
                               const int8_t *up_w, const float *up_s, const int8_t *down_w, const float *down_s,
                               const float *input_ln, const float *post_attn_ln, const float *q_norm,
                               const float *k_norm);
/* decoder.c:393-424: as above, with the fused Q||K||V [4096 x 2048] and
 * gate||up [12288 x 2048] (decoder.py:290-302); when given, the fused arrays
 * are the source of those rows (gate||up re-laid out per 16-row group) and
 * the separate q/k/v and gate/up arrays are not read. */
void decoder_set_layer_weights_v32(ModelWeights *model, int layer_idx, const int8_t *q_w, const float *q_s,
                                   const int8_t *k_w, const float *k_s, const int8_t *v_w, const float *v_s,
                                   const int8_t *o_w, const float *o_s, const int8_t *gate_w,
                                   const float *gate_s, const int8_t *up_w, const float *up_s,
                                   const int8_t *down_w, const float *down_s, const float *input_ln,
                                   const float *post_attn_ln, const float *q_norm, const float *k_norm,
                                   const int8_t *qkv_w, const float *qkv_s, const int8_t *gate_up_w,
                                   const float *gate_up_s);
/* decoder.c:509-516 -> ops.c:150-177: sequential-position rope tables
 * [max_seq x head_dim/2] on the host. */
void decoder_precompute_rope(float *cos_tab, float *sin_tab, int max_seq, int head_dim, const int sections[3],
                             const float theta_bases[3]);
/* decoder.c:426-435: one decode step of every set layer on hidden [2048]
 * (host, in/out); the tables are the host arrays decoder_precompute_rope
 * filled for the cache's max_seq (copied to HBM once, re-checked by a
 * sampled fingerprint). */
void decoder_decode_step(const ModelWeights *model, KVCache *cache, float *hidden, DecoderScratch *scratch,
                         const float *cos_tab, const float *sin_tab);

/* decoder.c:437-447: prefill of seq_len tokens (hidden [seq_len x 2048],
 * host, in/out) through every layer: token t rotated at position
 * seq_len_of_cache + t, K/V appended, causal attention within the new tokens
 * (PREFILL_MODE); the cache advances by seq_len. */
void decoder_prefill_step(const ModelWeights *model, KVCache *cache, float *hidden, DecoderScratch *scratch,
                          const float *cos_tab, const float *sin_tab, int seq_len);
/* decoder.c:449-474: the same in chunks of chunk_size tokens, each attending
 * to every cached position (CHUNKED_PREFILL_MODE). */
void decoder_chunked_prefill_step(const ModelWeights *model, KVCache *cache, float *hidden, DecoderScratch *scratch,
                                  const float *cos_tab, const float *sin_tab, int total_seq_len, int chunk_size);
/* decoder.c:476-493: equal to decoder_prefill_step (the reference chunks only
 * its GEMMs; chunk_size is accepted and unused). */
void decoder_hybrid_chunked_prefill_step(const ModelWeights *model, KVCache *cache, float *hidden,
                                         DecoderScratch *scratch, const float *cos_tab, const float *sin_tab,
                                         int seq_len, int chunk_size);
/* decoder.c:495-507: prefill with per-token rope tables [seq_len x 64] (host),
 * built by decoder_build_rope_3d from 3-D position ids (PREFILL_3D_MODE). */
void decoder_prefill_step_3d(const ModelWeights *model, KVCache *cache, float *hidden, DecoderScratch *scratch,
                             const float *token_cos, const float *token_sin, int seq_len);
/* decoder.c:518-526 -> ops.c:188-223: per-token tables from pos_ids [3 x
 * seq_len] (temporal, height, width), on the host. */
void decoder_build_rope_3d(float *cos_out, float *sin_out, const int *pos_ids, int seq_len, int head_dim,
                           const int sections[3], const float theta_bases[3]);

/* Extensions (no reference counterpart). */
int tl_decoder_num_layers(const ModelWeights *model);
int tl_decoder_cache_len(const KVCache *cache);
/* Prefill linear layers: 0 (default) w8a32_linear at batch seq_len, the
 * reference decoder's fp32 activations (decoder.c:56-155); 1 W8A8, per-token
 * int8 activations (w8a8_quantize_activations, kernel/w8a8_kernel.c:109-114)
 * and the exact int8 GEMM. */
int tl_decoder_set_prefill_w8a8(ModelWeights *model, int on);
/* Tuning switch of the prefill for every later prefill in the process: 1
 * (default) the layer's RMSNorms and SwiGLU write their output rows directly
 * as the linears' activations (W8A8: int8 codes and scales; fp32 linears at
 * more than 32 tokens: the four int8 planes per row and their exponents); 0
 * each linear converts its stored fp32 input in its own launch.  The
 * activations are the same either way. */
int tl_prefill_set_fused_quant(int on);
/* Copies one layer's K and V cache ([8][max_seq][128] fp32 each; either may
 * be NULL) to host memory. */
int tl_decoder_read_cache(const KVCache *cache, int layer, float *k, float *v);
/* Device-resident greedy generation (the decode loop of decoder.py:494-507
 * with do_sample=False): from first_token, n_steps steps of
 *   hidden = embed[token]; every layer; lm_head logits of the numpy final
 *   RMSNorm (final_norm, host [2048], may be NULL); token = argmax
 * as graph replays with no host round trip; the n_steps tokens go to tokens
 * (host).  embed: device [vocab x 2048] fp32.  The cache advances by
 * n_steps. */
int tl_decoder_generate(const ModelWeights *model, KVCache *cache, DecoderScratch *scratch,
                        const tl_weights *lm_head, const float *final_norm, const float *embed, int first_token,
                        int n_steps, int32_t *tokens, const float *cos_tab, const float *sin_tab);

/* Test hooks (device pointers, synchronous on `stream`): one launch of the
 * decoder's attention kernels on caller buffers, so attention can be checked
 * alone against the reference's attention (kernel/attention.c).
 *   tl_attn_decode_dev: the decode-mode attention step of decoder.c:72-118
 *     for one token: qkv [16*128 | 8*128 | 8*128] is the QKV projection;
 *     q and k heads get their RMSNorm (q_norm, k_norm [128]) and the rotation
 *     at row rope_pos of cos_tab / sin_tab ([max_seq x 64]); k and v go to
 *     row pos of k_cache / v_cache ([8][max_seq][128]); out [16*128] is the
 *     GQA attention over rows 0..pos (kernel/attention.c:172-224).
 *   tl_attn_prefill_dev: the causal attention of S queries (q heads of the
 *     token-major qkv [S x 4096], already normalised and rotated) over cache
 *     rows key0 .. key0 + qoff + t for query t (PREFILL_MODE: key0 = row of
 *     the first query, qoff = 0; CHUNKED_PREFILL_MODE: key0 = 0, qoff = rows
 *     before the chunk); out [S x 2048].  split != 0 lets the longest query
 *     tiles run as two halves of their key range (the decoder's default). */
int tl_attn_decode_dev(const float *qkv, const float *q_norm, const float *k_norm, const float *cos_tab,
                       const float *sin_tab, float *k_cache, float *v_cache, int max_seq, int pos, int rope_pos,
                       float *out, void *stream);
int tl_attn_prefill_dev(const float *qkv, const float *k_cache, const float *v_cache, float *out, int S,
                        int max_seq, int key0, int qoff, int split, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* TYPHOON_LINEAR_H */
