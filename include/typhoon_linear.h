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

#ifdef __cplusplus
}
#endif
#endif /* TYPHOON_LINEAR_H */
