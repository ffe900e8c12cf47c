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

#ifdef __cplusplus
}
#endif
