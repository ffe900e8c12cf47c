/*
 * oracle.c -- CPU restatement of typhoon-ocr-server's INT8 linear kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, the smoke check and the CPU
 * baseline leg of bench.py may load this file's library, and only as the
 * checker or as the timed CPU baseline, never as a product path.
 *
 * The reference (kernel/w8a32_kernel.c, kernel/w8a8_kernel.c,
 * kernel/w8a16_kernel.c) is AArch64 NEON/i8mm/bf16 code over Apple
 * Accelerate and libdispatch; it cannot be compiled in this image, so this
 * file restates its arithmetic in portable C, function by function.
 *
 * Built with -ffp-contract=off: every fused multiply-add below is an explicit
 * fmaf() standing for a contraction the reference's compiler performs
 * (clang's default -ffp-contract=on fuses a*b+c inside one expression; the
 * reference Makefile, kernel/Makefile:2-3, does not change that default).
 *
 * Parity status (what pins each function; tests/test_oracle.py holds the
 * checks):
 *   orc_quantize_rows  -- pinned: closed forms (s == fl(absmax/127), codes in
 *       [-127,127], argmax element -> +-127, |x - q*s| <= s/2 (1+2^-22)),
 *       exact-tie cases (ties-to-even in the vector region, ties-away in the
 *       K%16 tail), x*fl(1/s) vs x/s discriminating cases, all-zero rows,
 *       NaN/Inf rows, and golden vectors computed independently in Python.
 *       A row whose absmax is so small that fl(absmax/127) < 2^-128 has
 *       inv = +inf, and its K%16 tail evaluates (int)lroundf(+-inf), which C
 *       leaves unspecified.  That value is taken from how the reference's
 *       AArch64 build evaluates it (fcvtas_x_low32 below), pinned by the
 *       Arm architecture's FCVTAS definition in tests/test_oracle.py.
 *   orc_int_acc        -- pinned: brute-force Python integer dot products.
 *   orc_w8a32_linear   -- batch==1 pinned: closed form
 *       fl(fl(fl(acc)*ws)*xs) (+ bias as its own rounding) recomputed in
 *       numpy float32 from the pinned codes and accumulators.
 *       batch>1: the reference's arithmetic lives in Accelerate's
 *       cblas_sgemm, whose summation order is not published ("parity
 *       unpinned" at that boundary); pinned instead to a float64 brute force
 *       of dequant-then-dot, to linearity in X, and to the M=1 rows.
 *   orc_w8a8_linear    -- batch==1 pinned as w8a32 batch==1 (epilogue
 *       fma(fl(acc*ws), xs, bias|0)); batch>1 as w8a32 batch>1.
 *   orc_w8a16_linear   -- batch==1: the reference accumulates with Arm
 *       BFMMLA/BFDOT, whose internal rounding is architecture-defined; here
 *       the sum is exact (float64) and rounded once, pinned to a float64
 *       brute force; batch>1 as w8a32 batch>1.  Tolerance-pinned, not
 *       bit-pinned.
 */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------- */
/* scalar models of the NEON conversions used by the quantizers            */
/* ---------------------------------------------------------------------- */

static inline uint32_t f2u(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static inline float u2f(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

/* FCVTNS (vcvtnq_s32_f32): round to nearest, ties to even, saturate to int32,
 * NaN -> 0. */
static inline int32_t fcvtns(float v)
{
    if (v != v) return 0;
    float r = nearbyintf(v);             /* default rounding mode: RNE */
    if (r >= 2147483648.0f) return INT32_MAX;
    if (r < -2147483648.0f) return INT32_MIN;
    return (int32_t)r;
}

/* (int)lroundf(v) as the reference's AArch64 build evaluates it: clang
 * lowers lroundf (long is 64-bit there, math-errno off) to FCVTAS Xd, Sn --
 * round to nearest with ties away from zero, saturating to int64, NaN -> 0
 * (Arm ARM FPToFixed) -- and the conversion to int keeps the low 32 bits of
 * the register.  Every finite v has |v| <= 127 (1 + 2^-21) here, so only the
 * non-finite cases of an overflowing reciprocal reach the saturation:
 * +inf -> INT64_MAX -> -1, -inf -> INT64_MIN -> 0. */
static inline int32_t fcvtas_x_low32(float v)
{
    if (v != v) return 0;
    if (v >= 9223372036854775808.0f) return -1;           /* low half of INT64_MAX */
    if (v < -9223372036854775808.0f) return 0;            /* low half of INT64_MIN */
    int64_t r = (int64_t)roundf(v);                        /* exact: |v| < 2^63 */
    return (int32_t)(uint32_t)(uint64_t)r;
}

/* SQXTN s32->s16 then s16->s8 (vqmovn_s32, vqmovn_s16): saturating narrow. */
static inline int32_t sqxtn8(int32_t v)
{
    if (v > 127) return 127;
    if (v < -128) return -128;
    return v;
}

/* absmax of one row, w8a32_kernel.c:73-83 (also w8a8_kernel.c:64-73,
 * w8a16_kernel.c:47-53): a NaN-propagating vector max (vmaxq_f32/vmaxvq_f32)
 * over the 16-aligned prefix starting from +0, then a scalar `v > absmax`
 * scan of the tail, which does not propagate NaN.  For non-negative floats
 * the IEEE bit patterns order like unsigned integers, and every NaN pattern
 * sorts above +Inf, so an unsigned max of |v|'s bits is that vector max. */
static float row_absmax(const float *src, int cols)
{
    int main_end = cols & ~15;
    uint32_t mx = 0;
    for (int k = 0; k < main_end; k++) {
        uint32_t b = f2u(src[k]) & 0x7fffffffu;
        if (b > mx) mx = b;
    }
    float absmax = u2f(mx);
    for (int k = main_end; k < cols; k++) {
        float v = fabsf(src[k]);
        if (v > absmax) absmax = v;
    }
    return absmax;
}

/* ---------------------------------------------------------------------- */
/* quantizers                                                               */
/* ---------------------------------------------------------------------- */

/* Restates w8a32_quantize (w8a32_kernel.c:63-108), _quantize_rows
 * (w8a8_kernel.c:54-100) and w8a16_quantize_weights (w8a16_kernel.c:44-65)
 * with clamp_main=1, and _quantize_activation_i8 (w8a32_kernel.c:139-178)
 * with clamp_main=0 (that one has no [-127,127] clamp in its vector loop,
 * :161-172).
 *   scale = absmax > 0 ? absmax/127 : 1;  inv = 1/scale          (:85-87)
 *   k <  cols&~15:  q = sat8(FCVTNS(x*inv)), clamped to +-127    (:90-101)
 *   k >= cols&~15:  q = clamp(lroundf(x*inv), -127, 127)         (:102-106)
 */
void orc_quantize_rows(const float *src, int8_t *dst, float *scales,
                       int rows, int cols, int clamp_main)
{
    int main_end = cols & ~15;
    for (int r = 0; r < rows; r++) {
        const float *row = src + (size_t)r * cols;
        int8_t *out = dst + (size_t)r * cols;
        float absmax = row_absmax(row, cols);
        float scale = (absmax > 0.0f) ? absmax / 127.0f : 1.0f;
        scales[r] = scale;
        float inv = 1.0f / scale;
        for (int k = 0; k < main_end; k++) {
            int32_t q = sqxtn8(fcvtns(row[k] * inv));
            if (clamp_main) {
                if (q < -127) q = -127;
                if (q > 127) q = 127;
            }
            out[k] = (int8_t)q;
        }
        for (int k = main_end; k < cols; k++) {
            float v = row[k] * inv;
            int q = fcvtas_x_low32(v);
            if (q > 127) q = 127;
            if (q < -127) q = -127;
            out[k] = (int8_t)q;
        }
    }
}

/* ---------------------------------------------------------------------- */
/* exact integer accumulation                                               */
/* ---------------------------------------------------------------------- */

static inline int32_t dot_i8(const int8_t *a, const int8_t *b, int K)
{
    int32_t s = 0;
    for (int k = 0; k < K; k++) s += (int32_t)a[k] * (int32_t)b[k];
    return s;
}

void orc_int_acc(const int8_t *x_q, const int8_t *w, int32_t *acc,
                 int batch, int N, int K, int threads)
{
    if (threads < 1) threads = 1;
    for (int b = 0; b < batch; b++) {
        const int8_t *xr = x_q + (size_t)b * K;
        int32_t *ar = acc + (size_t)b * N;
#pragma omp parallel for num_threads(threads) schedule(static)
        for (int n = 0; n < N; n++) ar[n] = dot_i8(w + (size_t)n * K, xr, K);
    }
}

/* ---------------------------------------------------------------------- */
/* fp32 "dequant then SGEMM" branch (batch > 1)                            */
/* ---------------------------------------------------------------------- */

/* Y[b,n] = fl( sum_k Xd[b,k] * Wd[n,k] ) with Wd = fl(w*s) as
 * _dequant_neon (w8a32_kernel.c:114-131) / _dequant_row (w8a8_kernel.c:
 * 119-136, w8a16_kernel.c:75-85) produce it, the sum taken in float64 (the
 * products of two floats are exact there), then the bias added as its own
 * fp32 rounding after the product (w8a32_kernel.c:321-330).  The reference
 * sums inside cblas_sgemm (w8a32_kernel.c:314-319) in an unpublished order. */
static void dequant_gemm(const float *Xd, const int8_t *w, const float *ws,
                         const float *bias, float *Y, int batch, int N, int K,
                         int threads)
{
    float *wd = (float *)malloc((size_t)K * sizeof(float) * (size_t)threads);
    if (!wd) abort();
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int n = 0; n < N; n++) {
        int t = 0;
#ifdef _OPENMP
        t = omp_get_thread_num();
#endif
        float *row = wd + (size_t)t * K;
        const int8_t *wr = w + (size_t)n * K;
        for (int k = 0; k < K; k++) row[k] = (float)wr[k] * ws[n];
        for (int b = 0; b < batch; b++) {
            const float *xr = Xd + (size_t)b * K;
            double s = 0.0;
            for (int k = 0; k < K; k++) s += (double)xr[k] * (double)row[k];
            float y = (float)s;
            if (bias) y = y + bias[n];
            Y[(size_t)b * N + n] = y;
        }
    }
    free(wd);
}

/* ---------------------------------------------------------------------- */
/* w8a32_linear                                                             */
/* ---------------------------------------------------------------------- */

/* batch == 1: w8a32_gemv (w8a32_kernel.c:248-275) -> activation quantizer
 * (:139-178) and _sdot_gemv_worker (:205-246):
 *   y[n] = fl(fl(fl(dot) * ws[n]) * x_scale);  if bias: y[n] = fl(y[n]+b[n])
 * batch > 1: w8a32_gemm_tiled (:336-350) -> dequant_gemm above. */
void orc_w8a32_linear(const float *X, const int8_t *w, const float *scales,
                      const float *bias, float *Y, int batch, int N, int K,
                      int threads, int8_t *codes, float *xscale, int32_t *acc)
{
    if (threads < 1) threads = 1;
    if (batch == 1) {
        int8_t *q = (int8_t *)malloc((size_t)K);
        if (!q) abort();
        float xs;
        orc_quantize_rows(X, q, &xs, 1, K, 0);
#pragma omp parallel for num_threads(threads) schedule(static)
        for (int n = 0; n < N; n++) {
            int32_t dot = dot_i8(w + (size_t)n * K, q, K);
            float r = (float)dot * scales[n];
            r = r * xs;
            if (bias) r = r + bias[n];
            Y[n] = r;
            if (acc) acc[n] = dot;
        }
        if (codes) memcpy(codes, q, (size_t)K);
        if (xscale) *xscale = xs;
        free(q);
    } else {
        dequant_gemm(X, w, scales, bias, Y, batch, N, K, threads);
    }
}

/* ---------------------------------------------------------------------- */
/* w8a8_linear                                                              */
/* ---------------------------------------------------------------------- */

/* batch == 1: w8a8_gemv (w8a8_kernel.c:231-237) -> _gemv_slice (:141-223):
 *   y[n] = fma(fl(fl(acc) * ws[n]), x_scale, bias ? bias[n] : 0)   (:181-188)
 * batch > 1: w8a8_gemm (:259-268): X dequantized to fl(q*xs) (:262), W to
 * fl(w*ws) per tile (:246-247), SGEMM, bias added afterwards (:249-256). */
void orc_w8a8_linear(const int8_t *x_q, const float *x_scales,
                     const int8_t *w, const float *w_scales, const float *bias,
                     float *Y, int batch, int N, int K, int threads)
{
    if (threads < 1) threads = 1;
    if (batch == 1) {
        float xs = x_scales[0];
#pragma omp parallel for num_threads(threads) schedule(static)
        for (int n = 0; n < N; n++) {
            int32_t a = dot_i8(w + (size_t)n * K, x_q, K);
            float t = (float)a * w_scales[n];
            Y[n] = fmaf(t, xs, bias ? bias[n] : 0.0f);
        }
    } else {
        float *xd = (float *)malloc((size_t)batch * K * sizeof(float));
        if (!xd) abort();
        for (int b = 0; b < batch; b++)
            for (int k = 0; k < K; k++)
                xd[(size_t)b * K + k] = (float)x_q[(size_t)b * K + k] * x_scales[b];
        dequant_gemm(xd, w, w_scales, bias, Y, batch, N, K, threads);
        free(xd);
    }
}

/* ---------------------------------------------------------------------- */
/* w8a16_linear                                                             */
/* ---------------------------------------------------------------------- */

static inline float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* batch == 1: w8a16_gemv (w8a16_kernel.c:176-182) -> _gemv_slice (:90-168):
 * r = sum_k bf16(w)*x (BFMMLA/BFDOT, products exact), then
 *   y[n] = fma(r, ws[n], bias ? bias[n] : 0)                       (:134)
 * Here r is the exact sum rounded once to fp32.
 * batch > 1: w8a16_gemm (:203-216): X widened to fp32 (:206-210), W
 * dequantized to fl(w*ws), SGEMM, bias afterwards (:193-200). */
void orc_w8a16_linear(const uint16_t *x_bf16, const int8_t *w,
                      const float *w_scales, const float *bias, float *Y,
                      int batch, int N, int K, int threads)
{
    if (threads < 1) threads = 1;
    float *xd = (float *)malloc((size_t)batch * K * sizeof(float));
    if (!xd) abort();
    for (size_t i = 0; i < (size_t)batch * K; i++) xd[i] = bf16_to_f32(x_bf16[i]);
    if (batch == 1) {
#pragma omp parallel for num_threads(threads) schedule(static)
        for (int n = 0; n < N; n++) {
            const int8_t *wr = w + (size_t)n * K;
            double s = 0.0;
            for (int k = 0; k < K; k++) s += (double)wr[k] * (double)xd[k];
            Y[n] = fmaf((float)s, w_scales[n], bias ? bias[n] : 0.0f);
        }
    } else {
        dequant_gemm(xd, w, w_scales, bias, Y, batch, N, K, threads);
    }
    free(xd);
}

/* ---------------------------------------------------------------------- */
/* CPU baseline: the reference's M=1 decode GEMV on host cores             */
/* ---------------------------------------------------------------------- */

/* Row chunking as adaptive_chunk (w8a32_kernel.c:51-58): chunk = ceil(N/P)
 * rounded up to a multiple of 8, at least 64 rows; one task per chunk. */
void orc_w8a32_gemv_timed(const float *x, const int8_t *w, const float *scales,
                          float *y, int N, int K, int threads)
{
    if (threads < 1) threads = 1;
    int8_t *q = (int8_t *)malloc((size_t)K);
    if (!q) abort();
    float xs;
    orc_quantize_rows(x, q, &xs, 1, K, 0);
    int chunk = (N + threads - 1) / threads;
    chunk = (chunk + 7) & ~7;
    if (chunk < 64) chunk = 64;
    int ntasks = (N + chunk - 1) / chunk;
#pragma omp parallel for num_threads(threads) schedule(static, 1)
    for (int t = 0; t < ntasks; t++) {
        int n0 = t * chunk, n1 = n0 + chunk;
        if (n1 > N) n1 = N;
        for (int n = n0; n < n1; n++) {
            int32_t dot = dot_i8(w + (size_t)n * K, q, K);
            float r = (float)dot * scales[n];
            y[n] = r * xs;
        }
    }
    free(q);
}
