/*
 * decoder_ref.c -- CPU restatement of the reference's decoder layer step.
 *
 * TEST INFRASTRUCTURE ONLY (the same rules as oracle.c: only tests/ and the
 * smoke check load it, as the checker).
 *
 * Restates, function by function, the decode-mode layer of
 * kernel/decoder.c:33-157 (seq_len == 1) with the NEON operators it calls:
 * rmsnorm_f32 (kernel/ops.c:22-56), mrope_precompute (:150-177), mrope_apply
 * (:233-289), silu_mul_inplace with its fast exp (:478-531), the decode GQA
 * attention (kernel/attention.c:99-134 dot128 / fmadd4, :172-224) and the KV
 * cache append/advance (kernel/kv_cache.c:53-64, :108-112).  The linear
 * layers are orc_w8a32_linear at batch 1 (oracle.c).
 *
 * NEON semantics used below:
 *   vfmaq_f32 / vfmsq_f32  -> fmaf (fused, one rounding)
 *   vaddvq_f32             -> (l0 + l1) + (l2 + l3)  (two FADDP steps)
 *   vcvtq_s32_f32          -> round toward zero, saturating
 *   vrecpeq / vrsqrteq     -> FRECPE / FRSQRTE, restated below from the Arm
 *                             architecture pseudocode (FPRecipEstimate,
 *                             FPRSqrtEstimate; 8-bit estimates, no
 *                             increased-precision extension, FZ = 0)
 *   vrecpsq / vrsqrtsq     -> 2 - a*b and (3 - a*b) / 2, each one rounding
 *
 * Parity status: no Arm machine is available to run the reference, so the
 * estimate instructions are pinned only by their mathematical bounds
 * (|frecpe(x) x - 1| < 2^-8, |frsqrte(x) sqrt(x) - 1| < 2^-8, after the
 * reference's Newton steps 2^-16 and ~2^-23; tests/test_decoder_oracle.py)
 * and by exact values at powers of two; the operators are pinned against
 * float64 numpy restatements of their formulas (tolerance), the fast exp
 * against its closed form (exact).  Summation orders follow the reference
 * literally.
 */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static inline float u2f(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

/* ---------------------------------------------------------------------- */
/* Arm reciprocal and reciprocal-square-root estimates and steps            */
/* ---------------------------------------------------------------------- */

/* RecipEstimate: a in [256, 512) (a fixed-point value in [0.5, 1) in units of
 * 1/512) -> r in [256, 512) (1/value in [1, 2) in units of 1/256) */
static uint32_t recip_estimate(uint32_t a)
{
    a = a * 2 + 1;                     /* midpoint, units of 1/1024 */
    uint32_t b = (1u << 19) / a;
    return (b + 1) / 2;                /* round to nearest */
}

/* RecipSqrtEstimate: a in [128, 512) (a value in [0.25, 1) in units of 1/512)
 * -> r in [256, 512) (1/sqrt(value) in units of 1/256) */
static uint32_t rsqrt_estimate(uint32_t a)
{
    if (a < 256) {
        a = a * 2 + 1;                 /* [0.25, 0.5): 9-bit midpoint */
    } else {
        a = (a >> 1) << 1;             /* [0.5, 1): 8 bits, then the midpoint */
        a = (a + 1) * 2;
    }
    uint32_t b = 512;                  /* largest b with a * b^2 < 2^28 */
    while ((uint64_t)a * (b + 1) * (b + 1) < (1ull << 28)) b++;
    return (b + 1) / 2;
}

/* FRECPE for a positive normal x (the decoder only passes 1 + e >= 1) */
float orc_frecpe(float x)
{
    const uint32_t u = f2u(x);
    const int exp = (int)((u >> 23) & 0xff);
    const uint32_t frac = u & 0x7fffff;
    const uint32_t est = recip_estimate(256 + (frac >> 15)) & 0xff;
    int rexp = 253 - exp;
    uint32_t rfrac;
    if (rexp == 0) {
        rfrac = (1u << 22) | (est << 14);          /* subnormal result */
    } else if (rexp == -1) {
        rfrac = (1u << 21) | (est << 13);
        rexp = 0;
    } else {
        rfrac = est << 15;
    }
    return u2f((u & 0x80000000u) | ((uint32_t)rexp << 23) | rfrac);
}

/* FRSQRTE for a positive normal x */
float orc_frsqrte(float x)
{
    const uint32_t u = f2u(x);
    const int exp = (int)((u >> 23) & 0xff);
    const uint32_t frac = u & 0x7fffff;
    /* scaled to [0.25, 1) in steps of 1/512 keeping the parity of the
     * (biased) exponent: '01' + 7 fraction bits (odd), '1' + 8 bits (even) */
    const uint32_t scaled = (exp & 1) ? 128 + (frac >> 16) : 256 + (frac >> 15);
    const uint32_t est = rsqrt_estimate(scaled) & 0xff;
    const int rexp = (380 - exp) / 2;
    return u2f(((uint32_t)rexp << 23) | (est << 15));
}

float orc_frecps(float a, float b) { return fmaf(-a, b, 2.0f); }
float orc_frsqrts(float a, float b) { return fmaf(-a, b, 3.0f) * 0.5f; }

/* ---------------------------------------------------------------------- */
/* RMSNorm (ops.c:22-56)                                                    */
/* ---------------------------------------------------------------------- */
void orc_rmsnorm(float *out, const float *x, const float *w, int dim, float eps)
{
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    int i = 0;
    for (; i + 15 < dim; i += 16)
        for (int v = 0; v < 4; v++)
            for (int j = 0; j < 4; j++) acc[j] = fmaf(x[i + 4 * v + j], x[i + 4 * v + j], acc[j]);
    float sum_sq = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    for (; i < dim; i++) sum_sq = fmaf(x[i], x[i], sum_sq);   /* contracted scalar tail */
    const float rms_sq = sum_sq / (float)dim + eps;
    float r = orc_frsqrte(rms_sq);
    r = r * orc_frsqrts(rms_sq * r, r);
    r = r * orc_frsqrts(rms_sq * r, r);
    for (i = 0; i < dim; i++) out[i] = (x[i] * r) * w[i];
}

/* ---------------------------------------------------------------------- */
/* M-RoPE (ops.c:150-177 sequential tables, :233-289 apply)                 */
/* ---------------------------------------------------------------------- */
void orc_mrope_precompute(float *cos_tab, float *sin_tab, int max_seq, int head_dim, float theta)
{
    const int half = head_dim / 2;
    for (int pos = 0; pos < max_seq; pos++)
        for (int j = 0; j < half; j++) {
            const float inv_freq = 1.0f / powf(theta, (float)(2 * j) / (float)head_dim);
            const float angle = (float)pos * inv_freq;
            cos_tab[(size_t)pos * half + j] = cosf(angle);
            sin_tab[(size_t)pos * half + j] = sinf(angle);
        }
}

static void rope_heads(float *x, const float *co, const float *si, int heads, int head_dim)
{
    const int half = head_dim / 2;
    for (int h = 0; h < heads; h++) {
        float *xh = x + (size_t)h * head_dim;
        for (int j = 0; j < half; j++) {
            const float lo = xh[j], hi = xh[j + half];
            xh[j] = lo * co[j] - hi * si[j];
            xh[j + half] = hi * co[j] + lo * si[j];
        }
    }
}

void orc_mrope_apply(float *q, float *k, const float *cos_tab, const float *sin_tab, int num_q_heads,
                     int num_kv_heads, int head_dim, int pos)
{
    const int half = head_dim / 2;
    rope_heads(q, cos_tab + (size_t)pos * half, sin_tab + (size_t)pos * half, num_q_heads, head_dim);
    rope_heads(k, cos_tab + (size_t)pos * half, sin_tab + (size_t)pos * half, num_kv_heads, head_dim);
}

/* ---------------------------------------------------------------------- */
/* SwiGLU with the Schraudolph exponent-only exp (ops.c:478-531)            */
/* ---------------------------------------------------------------------- */
static inline int32_t fcvtzs(float v)
{
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;                 /* C conversion truncates */
}

float orc_fast_exp(float x)
{
    x = fmaxf(x, -88.f);
    x = fminf(x, 88.f);
    const int32_t i = fcvtzs(fmaf(x, 1.4426950408889634f, 126.94269504f));
    return u2f((uint32_t)i << 23);
}

float orc_silu_fast(float g)
{
    const float d = 1.0f + orc_fast_exp(-g);
    const float r0 = orc_frecpe(d);
    return (g * r0) * orc_frecps(d, r0);
}

void orc_silu_mul(float *gate, const float *up, int n)
{
    int i = 0;
    for (; i + 15 < n; i += 16)
        for (int j = 0; j < 16; j++) gate[i + j] = orc_silu_fast(gate[i + j]) * up[i + j];
    for (; i < n; i++) {                 /* scalar tail: exact expf */
        const float g = gate[i];
        gate[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

/* ---------------------------------------------------------------------- */
/* decode GQA attention (attention.c:99-134, :172-224)                      */
/* ---------------------------------------------------------------------- */
#define HD 128

static float dot128(const float *a, const float *b)
{
    float acc[4][4] = {{0}};
    for (int i = 0; i < HD; i += 16)
        for (int k = 0; k < 4; k++)
            for (int j = 0; j < 4; j++) acc[k][j] = fmaf(a[i + 4 * k + j], b[i + 4 * k + j], acc[k][j]);
    float t[4];
    for (int j = 0; j < 4; j++) t[j] = (acc[0][j] + acc[1][j]) + (acc[2][j] + acc[3][j]);
    return (t[0] + t[1]) + (t[2] + t[3]);
}

/* q [num_q_heads x 128]; Kc/Vc per kv head [max_seq x 128] at head stride
 * max_seq*128; out [num_q_heads x 128]; positions 0..S-1 */
void orc_attention_decode(const float *q, const float *Kc, const float *Vc, float *out, int num_q_heads,
                          int num_kv_heads, int max_seq, int S, float scale)
{
    const int group = num_q_heads / num_kv_heads;
    float *scores = (float *)malloc((size_t)S * sizeof(float));
    if (!scores) abort();
    for (int kvh = 0; kvh < num_kv_heads; kvh++) {
        const float *K = Kc + (size_t)kvh * max_seq * HD;
        const float *V = Vc + (size_t)kvh * max_seq * HD;
        for (int g = 0; g < group; g++) {
            const int qh = kvh * group + g;
            const float *qv = q + (size_t)qh * HD;
            float max_s = -1e38f;
            for (int t = 0; t < S; t++) {
                scores[t] = dot128(qv, K + (size_t)t * HD) * scale;
                if (scores[t] > max_s) max_s = scores[t];
            }
            float sum = 0.f;
            for (int t = 0; t < S; t++) {
                scores[t] = expf(scores[t] - max_s);
                sum += scores[t];
            }
            const float inv = 1.f / sum;
            for (int t = 0; t < S; t++) scores[t] *= inv;
            float *o = out + (size_t)qh * HD;
            memset(o, 0, HD * sizeof(float));
            for (int t = 0; t < S; t++)
                for (int d = 0; d < HD; d++) o[d] = fmaf(scores[t], V[(size_t)t * HD + d], o[d]);
        }
    }
    free(scores);
}

/* ---------------------------------------------------------------------- */
/* one decode-mode layer (decoder.c:33-157, seq_len == 1)                   */
/* ---------------------------------------------------------------------- */
/* w/s: the seven projections in the order q, k, v, o, gate, up, down
 * (row-major int8 codes, fp32 scales); norms: input_ln [H], post_attn_ln [H],
 * q_norm [128], k_norm [128].  Kc/Vc: this layer's cache, [kv_heads][max_seq]
 * [128].  hidden [H] in/out.  cache_len: positions already in the cache (the
 * new K/V go to position cache_len); rope_pos: the rotary position. */
void orc_decode_layer(const int8_t *const *w, const float *const *s, const float *input_ln,
                      const float *post_attn_ln, const float *q_norm, const float *k_norm, float *Kc,
                      float *Vc, int max_seq, float *hidden, const float *cos_tab, const float *sin_tab,
                      int cache_len, int rope_pos, int hidden_dim, int ffn_dim, int num_q_heads,
                      int num_kv_heads, int threads)
{
    const int H = hidden_dim, KV = num_kv_heads * HD, F = ffn_dim;
    float *residual = (float *)malloc((size_t)H * 4);
    float *xn = (float *)malloc((size_t)H * 4);
    float *q = (float *)malloc((size_t)H * 4);
    float *k = (float *)malloc((size_t)KV * 4);
    float *v = (float *)malloc((size_t)KV * 4);
    float *attn = (float *)malloc((size_t)H * 4);
    float *gate = (float *)malloc((size_t)F * 4);
    float *up = (float *)malloc((size_t)F * 4);
    float *y = (float *)malloc((size_t)H * 4);
    if (!residual || !xn || !q || !k || !v || !attn || !gate || !up || !y) abort();

    memcpy(residual, hidden, (size_t)H * 4);
    orc_rmsnorm(xn, hidden, input_ln, H, 1e-6f);
    orc_w8a32_linear(xn, w[0], s[0], NULL, q, 1, H, H, threads, NULL, NULL, NULL);
    orc_w8a32_linear(xn, w[1], s[1], NULL, k, 1, KV, H, threads, NULL, NULL, NULL);
    orc_w8a32_linear(xn, w[2], s[2], NULL, v, 1, KV, H, threads, NULL, NULL, NULL);
    for (int h = 0; h < num_q_heads; h++) orc_rmsnorm(q + h * HD, q + h * HD, q_norm, HD, 1e-6f);
    for (int h = 0; h < num_kv_heads; h++) orc_rmsnorm(k + h * HD, k + h * HD, k_norm, HD, 1e-6f);
    orc_mrope_apply(q, k, cos_tab, sin_tab, num_q_heads, num_kv_heads, HD, rope_pos);
    for (int h = 0; h < num_kv_heads; h++) {
        memcpy(Kc + ((size_t)h * max_seq + cache_len) * HD, k + h * HD, HD * 4);
        memcpy(Vc + ((size_t)h * max_seq + cache_len) * HD, v + h * HD, HD * 4);
    }
    orc_attention_decode(q, Kc, Vc, attn, num_q_heads, num_kv_heads, max_seq, cache_len + 1,
                         0.08838834764831843f);
    orc_w8a32_linear(attn, w[3], s[3], NULL, y, 1, H, H, threads, NULL, NULL, NULL);
    for (int i = 0; i < H; i++) hidden[i] = y[i] + residual[i];

    memcpy(residual, hidden, (size_t)H * 4);
    orc_rmsnorm(xn, hidden, post_attn_ln, H, 1e-6f);
    orc_w8a32_linear(xn, w[4], s[4], NULL, gate, 1, F, H, threads, NULL, NULL, NULL);
    orc_w8a32_linear(xn, w[5], s[5], NULL, up, 1, F, H, threads, NULL, NULL, NULL);
    orc_silu_mul(gate, up, F);
    orc_w8a32_linear(gate, w[6], s[6], NULL, y, 1, H, F, threads, NULL, NULL, NULL);
    for (int i = 0; i < H; i++) hidden[i] = y[i] + residual[i];

    free(residual); free(xn); free(q); free(k); free(v); free(attn); free(gate); free(up); free(y);
}

/* ---------------------------------------------------------------------- */
/* prefill (decoder.c:33-157 in PREFILL_MODE / PREFILL_3D_MODE)            */
/* ---------------------------------------------------------------------- */

/* mrope_build_cos_sin_3d (ops.c:188-223) with the section map of
 * _init_section_map (ops.c:128-146): dims j < 3 * min(s1, s2) cycle T, H, W;
 * the rest are T.  pos_ids [3 x seq_len]. */
void orc_mrope_build_3d(float *cos_out, float *sin_out, const int *pos_ids, int seq_len, int head_dim,
                        const int sections[3], float theta)
{
    const int half = head_dim / 2;
    int min_s = sections[1] < sections[2] ? sections[1] : sections[2];
    for (int t = 0; t < seq_len; t++)
        for (int j = 0; j < half; j++) {
            const int sect = j < 3 * min_s ? j % 3 : 0;
            const int pos = pos_ids[sect * seq_len + t];
            const float inv_freq = 1.0f / powf(theta, (float)(2 * j) / (float)head_dim);
            const float angle = (float)pos * inv_freq;
            cos_out[(size_t)t * half + j] = cosf(angle);
            sin_out[(size_t)t * half + j] = sinf(angle);
        }
}

/* exp_f32_poly4 (attention.c:57-91): Cody-Waite reduction, degree-5 Horner,
 * 2^n through the exponent field */
static float exp_poly4(float x)
{
    x = fmaxf(x, -88.0f);
    x = fminf(x, 88.0f);
    const float n = roundf(x * 1.4426950408889634f);            /* vrndaq: ties away */
    float r = fmaf(-n, 6.93147182464599609375e-1f, x);
    r = fmaf(-n, -1.90465429995776716e-9f, r);
    float p = 1.0f / 120.0f;
    p = fmaf(r, p, 1.0f / 24.0f);
    p = fmaf(r, p, 1.0f / 6.0f);
    p = fmaf(r, p, 1.0f / 2.0f);
    p = fmaf(r, p, 1.0f);
    p = fmaf(r, p, 1.0f);
    const int32_t ni = (int32_t)n;
    return p * u2f((uint32_t)(ni + 127) << 23);
}

#define TQ 32
#define TKV 256

/* _flash_worker (attention.c:252-344), token-major q [Sq x nq x 128],
 * k/v [Sk x nkv x 128], causal within the chunk (key j <= query i) */
void orc_attention_prefill(const float *q, const float *k, const float *v, float *out, int Sq, int nq, int nkv,
                           float scale)
{
    const int group = nq / nkv;
    const int qs = nq * HD, ks = nkv * HD;
    float *s_tile = (float *)malloc((size_t)TQ * TKV * sizeof(float));
    float *o_tile = (float *)malloc((size_t)TQ * HD * sizeof(float));
    if (!s_tile || !o_tile) abort();
    float m_tile[TQ], l_tile[TQ];
    const int ntq = (Sq + TQ - 1) / TQ;
    for (int kvh = 0; kvh < nkv; kvh++)
        for (int qt = 0; qt < ntq; qt++) {
            const int t_q0 = qt * TQ;
            const int t_q1 = t_q0 + TQ < Sq ? t_q0 + TQ : Sq;
            const int tq = t_q1 - t_q0;
            for (int g = 0; g < group; g++) {
                const int qh = kvh * group + g;
                for (int qi = 0; qi < tq; qi++) { m_tile[qi] = -1e38f; l_tile[qi] = 0.f; }
                memset(o_tile, 0, (size_t)tq * HD * sizeof(float));
                for (int kv0 = 0; kv0 < t_q1; kv0 += TKV) {
                    const int kv1 = kv0 + TKV < Sq ? kv0 + TKV : Sq;
                    const int tkv = kv1 - kv0;
                    for (int qi = 0; qi < tq; qi++) {
                        const int qpos = t_q0 + qi;
                        const float *qv = q + (size_t)qpos * qs + (size_t)qh * HD;
                        float *sp = s_tile + qi * TKV;
                        for (int ki = 0; ki < tkv; ki++) {
                            const int kpos = kv0 + ki;
                            if (kpos > qpos) { sp[ki] = -1e38f; continue; }
                            sp[ki] = dot128(qv, k + (size_t)kpos * ks + (size_t)kvh * HD) * scale;
                        }
                    }
                    for (int qi = 0; qi < tq; qi++) {
                        float *sp = s_tile + qi * TKV;
                        const float m_old = m_tile[qi];
                        float m_new = m_old;
                        for (int ki = 0; ki < tkv; ki++)
                            if (sp[ki] > m_new) m_new = sp[ki];
                        const float rescale = expf(m_old - m_new);
                        float l_new = l_tile[qi] * rescale;
                        float *oi = o_tile + (size_t)qi * HD;
                        for (int d = 0; d < HD; d++) oi[d] = oi[d] * rescale;
                        int ki = 0;
                        for (; ki + 3 < tkv; ki += 4) {
                            float e[4];
                            for (int jj = 0; jj < 4; jj++) {
                                e[jj] = exp_poly4(sp[ki + jj] - m_new);
                                sp[ki + jj] = e[jj];
                            }
                            l_new += (e[0] + e[1]) + (e[2] + e[3]);
                        }
                        for (; ki < tkv; ki++) {
                            sp[ki] = expf(sp[ki] - m_new);
                            l_new += sp[ki];
                        }
                        for (ki = 0; ki < tkv; ki++) {
                            const float *vt = v + (size_t)(kv0 + ki) * ks + (size_t)kvh * HD;
                            for (int d = 0; d < HD; d++) oi[d] = fmaf(sp[ki], vt[d], oi[d]);
                        }
                        m_tile[qi] = m_new;
                        l_tile[qi] = l_new;
                    }
                }
                for (int qi = 0; qi < tq; qi++) {
                    const float inv_l = l_tile[qi] > 0.f ? 1.f / l_tile[qi] : 0.f;
                    float *o = out + (size_t)(t_q0 + qi) * qs + (size_t)qh * HD;
                    for (int d = 0; d < HD; d++) o[d] = o_tile[(size_t)qi * HD + d] * inv_l;
                }
            }
        }
    free(s_tile);
    free(o_tile);
}

/* decoder_layer_forward with seq_len = S > 1 (decoder.c:33-157):
 * PREFILL_MODE when token_cos is NULL (token t rotated at position
 * cache_len + t of cos_tab/sin_tab), PREFILL_3D_MODE otherwise (row t of
 * token_cos/token_sin).  Fused Q||K||V and gate||up GEMMs are row
 * concatenations of the separate weights; orc_w8a32_linear at batch S is the
 * float64 dequant-then-dot restatement.  hidden [S x H] in/out; the cache rows
 * cache_len .. cache_len + S - 1 of Kc/Vc receive k and v. */
/* batch-S linear of the prefill: w8a32_linear (fp32 activations), or with
 * w8a8 set per-token activation codes (w8a8_quantize_activations,
 * w8a8_kernel.c:109-114) and w8a8_linear (:259-268) */
static void prefill_linear(const float *x, const int8_t *w, const float *s, float *y, int S, int N, int K, int w8a8,
                           int threads)
{
    if (!w8a8) {
        orc_w8a32_linear(x, w, s, NULL, y, S, N, K, threads, NULL, NULL, NULL);
        return;
    }
    int8_t *q = (int8_t *)malloc((size_t)S * K);
    float *xs = (float *)malloc((size_t)S * sizeof(float));
    if (!q || !xs) abort();
    orc_quantize_rows(x, q, xs, S, K, 1);
    orc_w8a8_linear(q, xs, w, s, NULL, y, S, N, K, threads);
    free(q);
    free(xs);
}

void orc_prefill_layer(const int8_t *const *w, const float *const *s, const float *input_ln,
                       const float *post_attn_ln, const float *q_norm, const float *k_norm, float *Kc, float *Vc,
                       int max_seq, float *hidden, int S, const float *cos_tab, const float *sin_tab,
                       const float *token_cos, const float *token_sin, int cache_len, int hidden_dim, int ffn_dim,
                       int num_q_heads, int num_kv_heads, int threads, int w8a8)
{
    const int H = hidden_dim, KV = num_kv_heads * HD, F = ffn_dim;
    const size_t SH = (size_t)S * H;
    float *residual = (float *)malloc(SH * 4), *xn = (float *)malloc(SH * 4);
    float *q = (float *)malloc(SH * 4), *k = (float *)malloc((size_t)S * KV * 4);
    float *v = (float *)malloc((size_t)S * KV * 4), *attn = (float *)malloc(SH * 4);
    float *gate = (float *)malloc((size_t)S * F * 4), *up = (float *)malloc((size_t)S * F * 4);
    float *y = (float *)malloc(SH * 4);
    if (!residual || !xn || !q || !k || !v || !attn || !gate || !up || !y) abort();

    memcpy(residual, hidden, SH * 4);
    for (int t = 0; t < S; t++) orc_rmsnorm(xn + (size_t)t * H, hidden + (size_t)t * H, input_ln, H, 1e-6f);
    prefill_linear(xn, w[0], s[0], q, S, H, H, w8a8, threads);
    prefill_linear(xn, w[1], s[1], k, S, KV, H, w8a8, threads);
    prefill_linear(xn, w[2], s[2], v, S, KV, H, w8a8, threads);
    for (int r = 0; r < S * num_q_heads; r++) orc_rmsnorm(q + (size_t)r * HD, q + (size_t)r * HD, q_norm, HD, 1e-6f);
    for (int r = 0; r < S * num_kv_heads; r++) orc_rmsnorm(k + (size_t)r * HD, k + (size_t)r * HD, k_norm, HD, 1e-6f);
    for (int t = 0; t < S; t++) {
        float *qt = q + (size_t)t * H, *kt = k + (size_t)t * KV;
        if (token_cos) {
            rope_heads(qt, token_cos + (size_t)t * (HD / 2), token_sin + (size_t)t * (HD / 2), num_q_heads, HD);
            rope_heads(kt, token_cos + (size_t)t * (HD / 2), token_sin + (size_t)t * (HD / 2), num_kv_heads, HD);
        } else {
            orc_mrope_apply(qt, kt, cos_tab, sin_tab, num_q_heads, num_kv_heads, HD, cache_len + t);
        }
    }
    for (int t = 0; t < S; t++)
        for (int h = 0; h < num_kv_heads; h++) {
            memcpy(Kc + ((size_t)h * max_seq + cache_len + t) * HD, k + (size_t)t * KV + h * HD, HD * 4);
            memcpy(Vc + ((size_t)h * max_seq + cache_len + t) * HD, v + (size_t)t * KV + h * HD, HD * 4);
        }
    orc_attention_prefill(q, k, v, attn, S, num_q_heads, num_kv_heads, 0.08838834764831843f);
    prefill_linear(attn, w[3], s[3], y, S, H, H, w8a8, threads);
    for (size_t i = 0; i < SH; i++) hidden[i] = y[i] + residual[i];

    memcpy(residual, hidden, SH * 4);
    for (int t = 0; t < S; t++) orc_rmsnorm(xn + (size_t)t * H, hidden + (size_t)t * H, post_attn_ln, H, 1e-6f);
    prefill_linear(xn, w[4], s[4], gate, S, F, H, w8a8, threads);
    prefill_linear(xn, w[5], s[5], up, S, F, H, w8a8, threads);
    orc_silu_mul(gate, up, S * F);
    prefill_linear(gate, w[6], s[6], y, S, H, F, w8a8, threads);
    for (size_t i = 0; i < SH; i++) hidden[i] = y[i] + residual[i];

    free(residual); free(xn); free(q); free(k); free(v); free(attn); free(gate); free(up); free(y);
}
