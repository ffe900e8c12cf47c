/*
 * baseline.c -- the CPU baseline that bench.py times beside the GPU.
 *
 * TEST INFRASTRUCTURE ONLY, like oracle.c: only bench.py's CPU-baseline leg
 * and tests/ call these functions, never a product path.
 *
 * The reference's M>1 branches dequantize a tile of weight rows into fp32
 * and multiply it with Apple Accelerate's cblas_sgemm; Accelerate and
 * AArch64 are absent here, so these functions restate the same decomposition
 * on the host cores with a blocked fp32 SGEMM of this file:
 *   w8a32_linear, batch > 1  (kernel/w8a32_kernel.c:297-350): 64-row weight
 *       tiles, one task per tile (dispatch_apply_f over tiles), X fp32 as is;
 *   w8a8_linear, batch > 1   (kernel/w8a8_kernel.c:243-268): X dequantized to
 *       fl(q * xs) once, 128-row weight tiles;
 *   w8a16_linear             (kernel/w8a16_kernel.c:176-223): batch 1 is a
 *       GEMV over row chunks of ceil(N / P) rounded to 8, at least 64 rows
 *       (adaptive_chunk, w8a32_kernel.c:51-58); batch > 1 converts X from
 *       bf16 to fp32 once, then 128-row weight tiles.
 * Every weight tile is dequantized as fl(w * ws) (the reference's
 * _dequant_row / _dequant_neon), and the bias, when given, is added after the
 * product as its own rounding.  The SGEMM sums in its own blocked order (the
 * reference's order lives inside Accelerate and is unpublished), so results
 * agree with the oracle's float64-accumulated checker to a tolerance
 * (tests/test_oracle.py), not bit for bit.
 *
 * This file is compiled with -ffp-contract=fast (oracle/Makefile): the
 * SGEMM's a*b+c are fused multiply-adds, as in any tuned SGEMM.
 */
#include "oracle.h"

#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef float v16 __attribute__((vector_size(64)));   /* 16 floats: one AVX-512 or two AVX2 registers */
static inline float hsum16(const v16 *v)
{
    float s = 0.0f;
    for (int j = 0; j < 16; j++) s += (*v)[j];
    return s;
}

static inline float bf16_f(uint16_t b)
{
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* C[m][0..nt) = A[m][0..K) . B[n][0..K) for m < M, with B given as the
 * transposed dequantized tile Bt[k][0..ntp) (ntp = nt rounded up to 32, zero
 * columns past nt); C has row stride ldc.  4 x 32 register blocks: per k,
 * two 16-float loads of Bt and eight fused multiply-adds; a 32-column block
 * of Bt (K x 128 bytes) stays in L2 while the row blocks of A pass. */
static void sgemm_tile(const float *A, int M, int K, const float *Bt, int nt, int ntp, float *C, int ldc)
{
    float cbuf[4][32];
    for (int m0 = 0; m0 < M; m0 += 4) {
        const int mr = M - m0 < 4 ? M - m0 : 4;
        for (int n0 = 0; n0 < ntp; n0 += 32) {
            v16 acc[4][2];
            for (int i = 0; i < 4; i++) acc[i][0] = acc[i][1] = (v16){0};
            for (int k = 0; k < K; k++) {
                v16 b0, b1;
                memcpy(&b0, Bt + (size_t)k * ntp + n0, 64);
                memcpy(&b1, Bt + (size_t)k * ntp + n0 + 16, 64);
                for (int i = 0; i < 4; i++) {
                    const float a = i < mr ? A[(size_t)(m0 + i) * K + k] : 0.0f;
                    acc[i][0] += a * b0;
                    acc[i][1] += a * b1;
                }
            }
            for (int i = 0; i < mr; i++) {
                memcpy(cbuf[i], &acc[i][0], 64);
                memcpy(cbuf[i] + 16, &acc[i][1], 64);
                const int nn = nt - n0 < 32 ? nt - n0 : 32;
                if (nn > 0) memcpy(C + (size_t)(m0 + i) * ldc + n0, cbuf[i], (size_t)nn * 4);
            }
        }
    }
}

/* Small batches: C[m][n] = A[m] . Wd[n] with the tile dequantized row-major
 * (Wd[nt][K]), 16-lane partial sums along K */
static void dot_tile(const float *A, int M, int K, const float *Wd, int nt, float *C, int ldc)
{
    for (int r = 0; r < nt; r++) {
        const float *wr = Wd + (size_t)r * K;
        for (int m = 0; m < M; m++) {
            const float *ar = A + (size_t)m * K;
            v16 acc = {0};
            int k = 0;
            for (; k + 16 <= K; k += 16) {
                v16 a, b;
                memcpy(&a, ar + k, 64);
                memcpy(&b, wr + k, 64);
                acc += a * b;
            }
            float s = hsum16(&acc);
            for (; k < K; k++) s += ar[k] * wr[k];
            C[(size_t)m * ldc + r] = s;
        }
    }
}

/* Y[M][N] = X[M][K] . (fl(w * ws))^T (+ bias): one task per `tile` weight rows */
static void dequant_sgemm(const float *X, int M, int K, const int8_t *w, const float *ws, const float *bias,
                          int N, int tile, float *Y, int threads)
{
    const int ntiles = (N + tile - 1) / tile;
    const int ntp = (tile + 31) & ~31;
#pragma omp parallel num_threads(threads)
    {
        float *Bt = (float *)aligned_alloc(64, (size_t)K * ntp * sizeof(float));
        if (!Bt) abort();
#pragma omp for schedule(dynamic, 1)
        for (int t = 0; t < ntiles; t++) {
            const int n0 = t * tile;
            const int nt = N - n0 < tile ? N - n0 : tile;
            if (M <= 16) {
                /* few rows of X: the dequantized tile row-major, dot products */
                for (int r = 0; r < nt; r++) {
                    const int8_t *wr = w + (size_t)(n0 + r) * K;
                    const float s = ws[n0 + r];
                    for (int k = 0; k < K; k++) Bt[(size_t)r * K + k] = (float)wr[k] * s;
                }
                dot_tile(X, M, K, Bt, nt, Y + n0, N);
            } else {
                memset(Bt, 0, (size_t)K * ntp * sizeof(float));
                for (int r = 0; r < nt; r++) {
                    const int8_t *wr = w + (size_t)(n0 + r) * K;
                    const float s = ws[n0 + r];
                    for (int k = 0; k < K; k++) Bt[(size_t)k * ntp + r] = (float)wr[k] * s;
                }
                sgemm_tile(X, M, K, Bt, nt, ntp, Y + n0, N);
            }
            if (bias)
                for (int m = 0; m < M; m++)
                    for (int r = 0; r < nt; r++) Y[(size_t)m * N + n0 + r] = Y[(size_t)m * N + n0 + r] + bias[n0 + r];
        }
        free(Bt);
    }
}

void orc_base_w8a32_gemm(const float *X, const int8_t *w, const float *ws, const float *bias, float *Y,
                         int M, int N, int K, int threads)
{
    if (threads < 1) threads = 1;
    dequant_sgemm(X, M, K, w, ws, bias, N, 64, Y, threads);
}

void orc_base_w8a8_gemm(const int8_t *xq, const float *xs, const int8_t *w, const float *ws, const float *bias,
                        float *Y, int M, int N, int K, int threads)
{
    if (threads < 1) threads = 1;
    float *Xd = (float *)malloc((size_t)M * K * sizeof(float));
    if (!Xd) abort();
    for (int m = 0; m < M; m++)
        for (int k = 0; k < K; k++) Xd[(size_t)m * K + k] = (float)xq[(size_t)m * K + k] * xs[m];
    dequant_sgemm(Xd, M, K, w, ws, bias, N, 128, Y, threads);
    free(Xd);
}

void orc_base_w8a16_linear(const uint16_t *xb, const int8_t *w, const float *ws, const float *bias, float *Y,
                           int M, int N, int K, int threads)
{
    if (threads < 1) threads = 1;
    float *Xd = (float *)malloc((size_t)M * K * sizeof(float));
    if (!Xd) abort();
    for (size_t i = 0; i < (size_t)M * K; i++) Xd[i] = bf16_f(xb[i]);
    if (M > 1) {
        dequant_sgemm(Xd, M, K, w, ws, bias, N, 128, Y, threads);
        free(Xd);
        return;
    }
    /* GEMV over row chunks (adaptive_chunk): fp32 dot products of the
     * widened weights, 16 lanes, then the per-row scale and the bias */
    int chunk = (N + threads - 1) / threads;
    chunk = (chunk + 7) & ~7;
    if (chunk < 64) chunk = 64;
    const int ntasks = (N + chunk - 1) / chunk;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int t = 0; t < ntasks; t++) {
        const int n1 = (t + 1) * chunk < N ? (t + 1) * chunk : N;
        for (int n = t * chunk; n < n1; n++) {
            const int8_t *wr = w + (size_t)n * K;
            float acc[16] = {0};               /* 16 lanes: the compiler widens and fuses per lane */
            int k = 0;
            for (; k + 16 <= K; k += 16)
                for (int j = 0; j < 16; j++) acc[j] += (float)wr[k + j] * Xd[k + j];
            float s = 0.0f;
            for (int j = 0; j < 16; j++) s += acc[j];
            for (; k < K; k++) s += (float)wr[k] * Xd[k];
            float y = s * ws[n];
            if (bias) y = y + bias[n];
            Y[n] = y;
        }
    }
    free(Xd);
}
