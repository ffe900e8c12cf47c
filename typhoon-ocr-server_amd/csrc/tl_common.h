// tl_common.h -- device-side building blocks shared by the INT8 linear kernels
// (gfx950 / CDNA4, wave64).
//
// Weight tile layout ("16x64 tiles"), used for every weight matrix held in
// HBM and for the int8 activation codes fed to the int8 MFMA:
//
//   tile (g, kb) covers rows 16g .. 16g+15 and columns 64kb .. 64kb+63; it is
//   1 KiB, lane-major: byte b of lane l holds  W[16g + (l & 15)][64kb + 16(l >> 4) + b].
//   tiles are stored k-block-major: offset(g, kb) = (kb * NG + g) * 1024,
//   NG = ceil(rows/16).  One K slice of all row groups is then contiguous, so
//   the tiles a GEMM stage reads spread over all L2 channels (with g-major
//   order they sat KB KiB apart and fell on the same few channels).
//
// One 16-byte load per lane reads a whole tile, perfectly coalesced.  The
// layout is the operand layout of v_mfma_i32_16x16x64_i8 (A or B): lane l
// supplies row (l & 15), lane group (l >> 4) supplies a 16-wide slice of K.
// An MFMA only needs A and B to agree on which K index sits in which (lane
// group, byte) slot, and they do because both are packed this way.  For the
// bf16 MFMA (v_mfma_f32_16x16x32_bf16, 8 values per lane) bytes 0-7 and 8-15
// of a lane become two bf16 operands for two MFMAs over K halves.
//
// Rows beyond N and columns beyond K are zero in the packed buffer, so a
// padded K contributes exactly 0 to every integer or float dot product.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tl_kernels.h"

#define TL_TILE_ROWS 16
#define TL_TILE_K 64
#define TL_TILE_BYTES 1024

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v8s __attribute__((ext_vector_type(8)));

namespace tl {

// ---------------------------------------------------------------------------
// quantizer primitives (reference: kernel/w8a32_kernel.c:63-108, :139-178)
// ---------------------------------------------------------------------------

// |v| as raw bits; for non-negative floats the unsigned order of the bits is
// the numeric order and every NaN sorts above +Inf, so an unsigned max of
// these is the NaN-propagating vmaxq_f32/vmaxvq_f32 max of the reference's
// 16-aligned prefix.
__device__ inline uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7fffffffu; }

// scale = absmax > 0 ? fl(absmax / 127) : 1  (NaN > 0 is false -> 1)
__device__ inline float quant_scale(float absmax) {
  return (absmax > 0.0f) ? __fdiv_rn(absmax, 127.0f) : 1.0f;
}
__device__ inline float quant_inv(float scale) { return __fdiv_rn(1.0f, scale); }

// FCVTNS + saturating narrow to int8 (vector region): round half to even,
// NaN -> 0.  clamp127 additionally limits to [-127, 127] (weight quantizers).
__device__ inline int code_rne(float v, bool clamp127) {
  float r = __builtin_rintf(v);
  r = (v != v) ? 0.0f : r;
  r = __builtin_fminf(__builtin_fmaxf(r, clamp127 ? -127.0f : -128.0f), 127.0f);
  return (int)r;
}

// (int)lroundf + clamp to [-127, 127] (scalar tail k >= K & ~15): half away
// from 0.  lroundf is FCVTAS into a 64-bit register on the reference's
// AArch64 build (NaN -> 0, saturating), and the conversion to int keeps the
// low 32 bits; an overflowing reciprocal (fl(absmax/127) < 2^-128) makes
// v = +-inf, so +inf -> low half of INT64_MAX = -1 and -inf -> 0.  Finite v
// here has |v| <= 127 (1 + 2^-21).
__device__ inline int code_tail(float v) {
  float r = __builtin_roundf(v);
  r = (v != v) ? 0.0f : r;
  r = (v == __builtin_inff()) ? -1.0f : r;
  r = (v == -__builtin_inff()) ? 0.0f : r;
  r = __builtin_fminf(__builtin_fmaxf(r, -127.0f), 127.0f);
  return (int)r;
}

// code for element k of a row of length K with reciprocal scale inv
__device__ inline int code_at(float x, float inv, int k, int K, bool clamp127) {
  float v = x * inv;
  return (k < (K & ~15)) ? code_rne(v, clamp127) : code_tail(v);
}

__device__ inline uint32_t pack4(int a, int b, int c, int d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)(d & 0xff) << 24);
}

// ---------------------------------------------------------------------------
// wave reductions (wave64)
// ---------------------------------------------------------------------------
__device__ inline uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t t = (uint32_t)__shfl_xor((int)v, o, 64);
    v = v > t ? v : t;
  }
  return v;
}

__device__ inline float wave_maxf_nonnan(float v) {  // max ignoring NaN (tail scan)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float t = __shfl_xor(v, o, 64);
    v = (t > v) ? t : v;
  }
  return v;
}

// block-wide absmax of a 256-thread block with the reference's NaN semantics:
// mx = max |x| bits over the 16-aligned prefix (NaN-propagating), tail = max
// over the K%16 tail ignoring NaN; the tail is compared against the prefix max
// the way `if (v > absmax) absmax = v` does (kernel/w8a32_kernel.c:153).
__device__ inline float block_absmax_256(uint32_t mx, float tail, uint32_t* s_mx, float* s_tail) {
  mx = wave_max_u32(mx);
  tail = wave_maxf_nonnan(tail);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_mx[w] = mx;
    s_tail[w] = tail;
  }
  __syncthreads();
  uint32_t m = s_mx[0];
  float t = s_tail[0];
#pragma unroll
  for (int i = 1; i < 4; i++) {
    m = s_mx[i] > m ? s_mx[i] : m;
    t = s_tail[i] > t ? s_tail[i] : t;
  }
  const float vec = __uint_as_float(m);
  return (t > vec) ? t : vec;
}

// ---------------------------------------------------------------------------
// DPP wave reductions and the fast RNE code packer
// ---------------------------------------------------------------------------
// DPP row operations (gfx9 encodings): quad permutations, mirrors
enum : int { DPP_QP_1032 = 0xB1, DPP_QP_2301 = 0x4E, DPP_ROW_HALF_MIRROR = 0x141, DPP_ROW_MIRROR = 0x140 };

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

// wave-wide unsigned max, returned wave-uniform: max within each row of 16
// lanes through DPP, then the 4 row results through readlane
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
  uint32_t t;
  t = dpp_u32<DPP_QP_1032>(v);         v = v > t ? v : t;
  t = dpp_u32<DPP_QP_2301>(v);         v = v > t ? v : t;
  t = dpp_u32<DPP_ROW_HALF_MIRROR>(v); v = v > t ? v : t;
  t = dpp_u32<DPP_ROW_MIRROR>(v);      v = v > t ? v : t;
  uint32_t m = __builtin_amdgcn_readlane(v, 0);
  uint32_t r1 = __builtin_amdgcn_readlane(v, 16), r2 = __builtin_amdgcn_readlane(v, 32),
           r3 = __builtin_amdgcn_readlane(v, 48);
  m = m > r1 ? m : r1;
  m = m > r2 ? m : r2;
  return m > r3 ? m : r3;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}

// sum over each row of 16 lanes, returned to every lane of the row: quad
// pairs, quads, then the two halves of each 8 and of the row, all through DPP
// (a fixed order, the same in every row)
__device__ __forceinline__ float row16_sum(float v) {
  v = __fadd_rn(v, dpp_f32<DPP_QP_1032>(v));
  v = __fadd_rn(v, dpp_f32<DPP_QP_2301>(v));
  v = __fadd_rn(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
  return __fadd_rn(v, dpp_f32<DPP_ROW_MIRROR>(v));
}

// wave-wide sum, returned wave-uniform: row sums, then (r0 + r1) + (r2 + r3)
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  const float r0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
  const float r1 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16));
  const float r2 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32));
  const float r3 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48));
  return __fadd_rn(__fadd_rn(r0, r1), __fadd_rn(r2, r3));
}

// wave-wide fmaxf, returned wave-uniform
__device__ __forceinline__ float wave_fmax(float v) {
  v = fmaxf(v, dpp_f32<DPP_QP_1032>(v));
  v = fmaxf(v, dpp_f32<DPP_QP_2301>(v));
  v = fmaxf(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_f32<DPP_ROW_MIRROR>(v));
  const float r0 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
  const float r1 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16));
  const float r2 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32));
  const float r3 = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// max ignoring NaN (the tail scan), for non-negative inputs
__device__ __forceinline__ float wave_fmax_nonnan(float v) {
  float t;
  t = __uint_as_float(dpp_u32<DPP_QP_1032>(__float_as_uint(v)));         v = (t > v) ? t : v;
  t = __uint_as_float(dpp_u32<DPP_QP_2301>(__float_as_uint(v)));         v = (t > v) ? t : v;
  t = __uint_as_float(dpp_u32<DPP_ROW_HALF_MIRROR>(__float_as_uint(v))); v = (t > v) ? t : v;
  t = __uint_as_float(dpp_u32<DPP_ROW_MIRROR>(__float_as_uint(v)));      v = (t > v) ? t : v;
  float m = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
#pragma unroll
  for (int r = 16; r < 64; r += 16) {
    const float o = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), r));
    m = (o > m) ? o : m;
  }
  return m;
}

// Four int8 codes of fl(v * inv) rounded to nearest even, packed: adding
// 1.5 * 2^23 leaves rint(p) in the low mantissa bits of the (exact for
// |p| < 2^22) sum, so the low byte of the sum's bits is the two's-complement
// code; v_perm_b32 gathers the four low bytes.  Valid when inv is finite and
// every |v| <= absmax (then |p| <= 127 (1 + 2^-22)).
__device__ __forceinline__ uint32_t codes4_rne(float4 v, float inv) {
  const float M = 12582912.0f;
  const uint32_t a = __float_as_uint(__fadd_rn(__fmul_rn(v.x, inv), M));
  const uint32_t b = __float_as_uint(__fadd_rn(__fmul_rn(v.y, inv), M));
  const uint32_t c = __float_as_uint(__fadd_rn(__fmul_rn(v.z, inv), M));
  const uint32_t d = __float_as_uint(__fadd_rn(__fmul_rn(v.w, inv), M));
  const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);   // a.b0, b.b0, 0, 0
  const uint32_t hi = __builtin_amdgcn_perm(d, c, 0x04000c0cu);   // 0, 0, c.b0, d.b0
  return lo | hi;
}

// ---------------------------------------------------------------------------
// W8A32 batches on the int8 MFMA: each fp32 token row is four int8 planes
// (split_i8x4_kernel), x = 2^e (q0 + q1/254 + q2/254^2 + q3/254^3)
// ---------------------------------------------------------------------------
constexpr int kXeNonFinite = -100000;   // exponent marking a row with Inf / NaN

// The fp32 value of sum_k x[k] w[n][k] over k in [k0, k1) for a row slice
// that holds Inf or NaN, as the reference's fp32 sums give it (X times the
// dequantized weights, code x scale with scale > 0, kernel/w8a32_kernel.c:
// 297-350; bf16 x times bf16 codes, w8a16_kernel.c:90-182): NaN when the
// slice holds a NaN, when an infinite x meets a zero code (inf * 0), or when
// the infinite terms have both signs; otherwise the infinite terms' common
// sign times Inf, which no finite term changes.  Partial sums of K slices
// combine the same way under IEEE addition.  x is fp32 (xt 0), bf16 (1) or
// fp16 (2) at element offset `off` of x; w is in the 16x64 tile layout with NG
// row groups.  Called only for rows the kernels flag as non-finite, so it
// reads the slice element by element.
__device__ __forceinline__ float nonfinite_dot(const void* x, int xt, size_t off, int k0, int k1,
                                                               const uint8_t* wt, int NG, int n) {
  bool pos = false, neg = false;
  const int g = n >> 4, r = n & 15;
  for (int k = k0; k < k1; k++) {
    float v;
    if (xt == 0) {
      v = static_cast<const float*>(x)[off + k];
    } else {
      const uint16_t h = static_cast<const uint16_t*>(x)[off + k];
      v = xt == 1 ? __uint_as_float((uint32_t)h << 16) : (float)__builtin_bit_cast(_Float16, h);
    }
    if (v != v) return __builtin_nanf("");
    if (__builtin_fabsf(v) != __builtin_inff()) continue;
    const int kb = k >> 6, kk = k & 63;
    const int8_t c = (int8_t)wt[((size_t)kb * NG + g) * 1024 + (size_t)(r + 16 * (kk >> 4)) * 16 + (kk & 15)];
    if (c == 0) return __builtin_nanf("");
    if ((v > 0.0f) == (c > 0)) pos = true;
    else neg = true;
  }
  if (pos == neg) return __builtin_nanf("");   // both signs (or, defensively, no Inf found)
  return pos ? __builtin_inff() : -__builtin_inff();
}

// 2^s as a float, s in [-126, 127]
__device__ __forceinline__ float pow2f(int s) { return __uint_as_float((uint32_t)(s + 127) << 23); }

// x 2^sh for sh in [-126, 227] as two multiplications by powers of two,
// 2^s1 with s1 = min(sh, 100), then 2^(sh - s1).  When the second factor is
// not 1, |x| 2^100 >= 2^-49 for every nonzero float x, so the first product is
// exact and the result is rounded at most once, in the second: the value of
// ldexpf(x, sh) (exact when normal, the same round-to-nearest-even when
// subnormal).  The per-element conversions use this instead of ldexpf: on
// gfx950 ldexpf followed by the digit clamp measured several times slower
// (the two-row GEMV's digit prologue 1.2-2.7 us per launch against 0.1-0.6 us).
struct Pow2 {
  float a, b;
};
__device__ __forceinline__ Pow2 pow2_split(int sh) {
  const int s1 = min(sh, 100);
  return Pow2{pow2f(s1), pow2f(sh - s1)};
}
__device__ __forceinline__ float mul_pow2(float x, Pow2 p) { return __fmul_rn(__fmul_rn(x, p.a), p.b); }

// the four int8 planes of 4 values of a row with exponent e (v = x 2^-e
// exact, |v| < 64): dword p holds plane p of the 4 values, one byte each
__device__ __forceinline__ void planes4_i8(const float (&v)[4], int e, uint32_t (&code)[4]) {
#pragma unroll
  for (int p = 0; p < 4; p++) code[p] = 0u;
  const Pow2 sc = pow2_split(-e);
#pragma unroll
  for (int q = 0; q < 4; q++) {
    float r = mul_pow2(v[q], sc);
    float c = rintf(r);
    const uint32_t b0 = (uint32_t)((int)c & 0xff);
    r = __fsub_rn(r, c);
    uint32_t bp[3];
#pragma unroll
    for (int p = 0; p < 3; p++) {
      const float sv = __fmul_rn(r, 254.0f);
      c = rintf(sv);
      bp[p] = (uint32_t)((int)c & 0xff);
      r = __fsub_rn(sv, c);
    }
    code[0] |= b0 << (8 * q);
    code[1] |= bp[0] << (8 * q);
    code[2] |= bp[1] << (8 * q);
    code[3] |= bp[2] << (8 * q);
  }
}
// the row exponent of the planes: frexp exponent of the absmax - 6 (0 for a
// zero row), or kXeNonFinite when the row holds Inf or NaN
__device__ __forceinline__ int planes_exponent(uint32_t absmax_bits) {
  if (absmax_bits >= 0x7f800000u) return kXeNonFinite;
  int e = 0;
  if (absmax_bits != 0) {
    int ex;
    (void)frexpf(__uint_as_float(absmax_bits), &ex);
    e = ex - 6;
  }
  return e;
}

// the four plane accumulators of one output: a0 + a1/254 + a2/254^2 +
// a3/254^3, Horner from the smallest term, each step rounded
__device__ __forceinline__ float planes_sum(int a0, int a1, int a2, int a3) {
  const float k = 1.0f / 254.0f;
  float t = __fadd_rn(__fmul_rn((float)a3, k), (float)a2);
  t = __fadd_rn(__fmul_rn(t, k), (float)a1);
  return __fadd_rn(__fmul_rn(t, k), (float)a0);
}
// fl(t * ws) scaled by 2^e (exact unless the result leaves the float range);
// NaN for a row that held Inf or NaN
__device__ __forceinline__ float planes_scale(float t, float ws, int e) {
  return e == kXeNonFinite ? __builtin_nanf("") : ldexpf(__fmul_rn(t, ws), e);
}

// ---------------------------------------------------------------------------
// fp32 activations as four int8 digit rows (fp32-semantics products on int8
// dot products): q = x 2^sh truncated (|q| < 2^30 for |x| < 2^(30 - sh)) is
// d0 2^24 + d1 2^16 + d2 2^8 + d3 with signed digits d1..d3 in [-128, 127]
// and d0 in [-64, 64]: the bytes of q + 0x808080, the low three flipped by
// 0x80.  Digit sums a_p = sum_k w_k d_p,k are exact int32, and
// sum_k w_k x_k = 2^(24 - sh) (a0 + 2^-8 (a1 + 2^-8 (a2 + 2^-8 a3))).
// ---------------------------------------------------------------------------
// biased digit word of one activation: (q + 0x808080) with q = x 2^sh
// truncated toward zero, sc = pow2_split(sh) (x 2^sh is exact wherever
// |q| >= 1, and |x 2^sh| < 2^30 for a finite slice; the clamp keeps Inf and
// NaN, whose token's outputs are NaN anyway, in the int range)
__device__ __forceinline__ uint32_t digit_word(float x, Pow2 sc) {
  return (uint32_t)(int)__builtin_amdgcn_fmed3f(mul_pow2(x, sc), -0x1p30f, 0x1p30f) + 0x808080u;
}

// four biased digit words (k .. k+3) -> the four digit-plane dwords:
// plane p holds byte 3 - p of each word (p = 0 the most significant digit);
// the low three bytes are flipped by 0x80 back to signed digits
__device__ __forceinline__ void digit_planes(uint32_t y0, uint32_t y1, uint32_t y2, uint32_t y3, uint32_t (&pl)[4]) {
  const uint32_t t0 = __builtin_amdgcn_perm(y1, y0, 0x05010400u);   // y0.b0 y1.b0 y0.b1 y1.b1
  const uint32_t t1 = __builtin_amdgcn_perm(y1, y0, 0x07030602u);   // y0.b2 y1.b2 y0.b3 y1.b3
  const uint32_t t2 = __builtin_amdgcn_perm(y3, y2, 0x05010400u);
  const uint32_t t3 = __builtin_amdgcn_perm(y3, y2, 0x07030602u);
  pl[3] = __builtin_amdgcn_perm(t2, t0, 0x05040100u) ^ 0x80808080u;  // byte 0 of each word
  pl[2] = __builtin_amdgcn_perm(t2, t0, 0x07060302u) ^ 0x80808080u;  // byte 1
  pl[1] = __builtin_amdgcn_perm(t3, t1, 0x05040100u) ^ 0x80808080u;  // byte 2
  pl[0] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);                // byte 3 (top digit)
}

// a0 + 2^-8 (a1 + 2^-8 (a2 + 2^-8 a3)), each step rounded
__device__ __forceinline__ float digits_sum(int a0, int a1, int a2, int a3) {
  float t = __fadd_rn(__fmul_rn((float)a3, 0x1p-8f), (float)a2);
  t = __fadd_rn(__fmul_rn(t, 0x1p-8f), (float)a1);
  return __fadd_rn(__fmul_rn(t, 0x1p-8f), (float)a0);
}


// ---------------------------------------------------------------------------
// argmax keys: the float's bits made monotonic in the high word, the index
// complemented in the low word, so the largest key is the largest value and,
// among equal values, the lowest index (torch.argmax's first-max rule)
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t argmax_key(float v, int n) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)o << 32) | (uint64_t)(0xffffffffu - (uint32_t)n);
}
__device__ __forceinline__ int argmax_key_index(uint64_t k) { return (int)(0xffffffffu - (uint32_t)k); }
__device__ __forceinline__ float argmax_key_value(uint64_t k) {
  const uint32_t o = (uint32_t)(k >> 32);
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

// ---------------------------------------------------------------------------
// int8 dot products
// ---------------------------------------------------------------------------
__device__ inline int dot16(uint4 w, uint4 x, int acc) {
  acc = __builtin_amdgcn_sdot4((int)w.x, (int)x.x, acc, false);
  acc = __builtin_amdgcn_sdot4((int)w.y, (int)x.y, acc, false);
  acc = __builtin_amdgcn_sdot4((int)w.z, (int)x.z, acc, false);
  acc = __builtin_amdgcn_sdot4((int)w.w, (int)x.w, acc, false);
  return acc;
}

// ---------------------------------------------------------------------------
// bf16 helpers
// ---------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32)
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
// fp32 -> bf16 bits, round to nearest even
__device__ inline uint32_t f32_to_bf16_rne(float f) { return pack_bf16x2(f, 0.0f) & 0xffffu; }
__device__ inline float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// 8 fp32 -> three packed bf16 terms with x == t0 + t1 + t2 to within 2^-24 |x|:
// t0 = bf16(x), t1 = bf16(x - t0), t2 = bf16(x - t0 - t1); both differences
// are exact in fp32 (each term holds the leading bits of the remainder).
__device__ inline void split3x8(const float* x, uint4& t0, uint4& t1, uint4& t2) {
  uint32_t a[4], b[4], c[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const float x0 = x[2 * q], x1 = x[2 * q + 1];
    a[q] = pack_bf16x2(x0, x1);
    const float r0 = x0 - __uint_as_float(a[q] << 16), r1 = x1 - __uint_as_float(a[q] & 0xffff0000u);
    b[q] = pack_bf16x2(r0, r1);
    const float s0 = r0 - __uint_as_float(b[q] << 16), s1 = r1 - __uint_as_float(b[q] & 0xffff0000u);
    c[q] = pack_bf16x2(s0, s1);
  }
  t0 = make_uint4(a[0], a[1], a[2], a[3]);
  t1 = make_uint4(b[0], b[1], b[2], b[3]);
  t2 = make_uint4(c[0], c[1], c[2], c[3]);
}

// 4 signed int8 (one dword) -> 4 bf16 (two dwords), exact for |w| <= 128
__device__ inline uint2 i8x4_to_bf16x4(uint32_t w) {
  float f0 = (float)(int8_t)(w & 0xff);
  float f1 = (float)(int8_t)((w >> 8) & 0xff);
  float f2 = (float)(int8_t)((w >> 16) & 0xff);
  float f3 = (float)(int8_t)(w >> 24);
  // integers |v| <= 128 are exact in bf16: the high halves of the floats,
  // paired by one byte permute (bytes 2, 3 of the first, then of the second)
  uint2 r;
  r.x = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  r.y = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  return r;
}

// ---------------------------------------------------------------------------
// The reference decoder's NEON estimate arithmetic (kernel/ops.c:22-56 RMSNorm
// rsqrt, :478-531 SwiGLU), restated from the Arm architecture pseudocode
// (FPRecipEstimate / FPRSqrtEstimate: 8-bit estimates, FZ = 0) for positive
// normal inputs, the only inputs the decoder gives them.
// ---------------------------------------------------------------------------
// FRECPE: 1/x to 8 bits
__device__ __forceinline__ float arm_frecpe(float x) {
  const uint32_t u = __float_as_uint(x);
  const int e = (int)((u >> 23) & 0xff);
  const uint32_t a = 2u * (256u + ((u & 0x7fffffu) >> 15)) + 1u;   // midpoint, units of 1/1024
  // floor(2^19 / a) from the hardware reciprocal: for odd a in [513, 1023]
  // the quotient's fraction is at least 1/a, far above the product's error
  // (< 2e-4), so the truncation is the floor (the two checks below keep it
  // exact regardless)
  uint32_t b = (uint32_t)(524288.0f * __builtin_amdgcn_rcpf((float)a));
  if (b * a > 524288u) b--;
  if ((b + 1u) * a <= 524288u) b++;
  const uint32_t est = ((b + 1u) >> 1) & 0xffu;
  int re = 253 - e;
  uint32_t rf;
  if (re == 0) {
    rf = (1u << 22) | (est << 14);
  } else if (re == -1) {
    rf = (1u << 21) | (est << 13);
    re = 0;
  } else {
    rf = est << 15;
  }
  return __uint_as_float((u & 0x80000000u) | ((uint32_t)re << 23) | rf);
}

// FRSQRTE: 1/sqrt(x) to 8 bits
__device__ __forceinline__ float arm_frsqrte(float x) {
  const uint32_t u = __float_as_uint(x);
  const int e = (int)((u >> 23) & 0xff);
  const uint32_t f = u & 0x7fffffu;
  uint32_t a = (e & 1) ? 128u + (f >> 16) : 256u + (f >> 15);      // [0.25, 1) in units of 1/512
  if (a < 256u) a = a * 2u + 1u;
  else a = ((a >> 1) << 1) * 2u + 2u;
  // b = largest integer with a b^2 < 2^28
  uint32_t b = (uint32_t)sqrtf(268435456.0f / (float)a);
  while ((uint64_t)a * b * b >= (1ull << 28)) b--;
  while ((uint64_t)a * (b + 1) * (b + 1) < (1ull << 28)) b++;
  const uint32_t est = ((b + 1u) >> 1) & 0xffu;
  const int re = (380 - e) / 2;
  return __uint_as_float(((uint32_t)re << 23) | (est << 15));
}

// FRECPS / FRSQRTS: one rounding each
__device__ __forceinline__ float arm_frecps(float a, float b) { return __fmaf_rn(-a, b, 2.0f); }
__device__ __forceinline__ float arm_frsqrts(float a, float b) { return __fmul_rn(__fmaf_rn(-a, b, 3.0f), 0.5f); }

// rsqrt as rmsnorm_f32 computes it: estimate and two Newton steps
__device__ __forceinline__ float ref_rsqrt(float v) {
  float r = arm_frsqrte(v);
  r = __fmul_rn(r, arm_frsqrts(__fmul_rn(v, r), r));
  r = __fmul_rn(r, arm_frsqrts(__fmul_rn(v, r), r));
  return r;
}

// fast_exp_f32 (Schraudolph, exponent bits only): 2^(trunc(x log2 e + 126.94) - 127)
__device__ __forceinline__ float ref_fast_exp(float x) {
  x = fminf(fmaxf(x, -88.0f), 88.0f);
  const int i = (int)__fmaf_rn(x, 1.4426950408889634f, 126.94269504f);   // truncates toward zero
  return __uint_as_float((uint32_t)i << 23);
}

// silu of silu_mul_inplace's vector loop: (g * r0) * (2 - d r0), d = 1 + e^-g
__device__ __forceinline__ float ref_silu(float g) {
  const float d = __fadd_rn(1.0f, ref_fast_exp(-g));
  const float r0 = arm_frecpe(d);
  return __fmul_rn(__fmul_rn(g, r0), arm_frecps(d, r0));
}

// ---------------------------------------------------------------------------
// global -> LDS tile copies and explicit waits (LDS-staged GEMMs)
// ---------------------------------------------------------------------------
// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0]+[15:14], expcnt[6:4],
// lgkmcnt[11:8]); unnamed counters at their maximum
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | (((N >> 4) & 3) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x3 << 14)); }

// 16-byte output store that streams past the caches (non-temporal): large
// GEMM outputs are written once and read by the next launch, so keeping them
// out of L2 saves the write-back of dirty lines at the kernel's end
__device__ __forceinline__ void st_stream(float* p, float4 v) {
  typedef float v4f_t __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(v4f_t{v.x, v.y, v.z, v.w}, reinterpret_cast<v4f_t*>(p));
}
__device__ __forceinline__ void st_stream(int32_t* p, int4 v) {
  typedef int v4i_t __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(v4i_t{v.x, v.y, v.z, v.w}, reinterpret_cast<v4i_t*>(p));
}

// Partials handed between work-groups of one launch, which may sit on
// different XCDs: stored with agent-scope atomic stores (they bypass the
// XCD's non-coherent L2 path; a store is visible device-wide once vmcnt
// acknowledges it) and read with agent-scope atomic loads.
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes with the same device-scope write-through (sc1) the agent-scope
// atomic store above gets, in one vector store: a wave's 64 lanes at
// consecutive 16-byte slots write whole lines instead of 4-byte pieces.  Not
// counted by the compiler's own waits: callers wait with wait_vm<0>().  A
// store of more than 8 bytes needs one wait state before a VALU instruction
// may overwrite its data registers; the compiler inserts it for its own
// stores but cannot see into this one, so the s_nop is part of it.
__device__ __forceinline__ void st_agent4(float* p, v4f v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" : : "v"(p), "v"(v) : "memory");
}

// One 1 KiB tile global -> LDS: lane l's 16 bytes land at lds_base + 16 l.
// Issued as volatile asm with a memory clobber so the compiler neither moves
// it across the stage barrier nor adds its own (conservative) vmcnt waits in
// front of LDS reads; every wait on these copies is explicit.
__device__ __forceinline__ void dma_tile(const uint4* gsrc, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds_base), "v"(gsrc)
               : "memory");
}
// the same copy with the source split into a uniform 64-bit base (SGPRs) and a
// per-lane 32-bit byte offset, so a stage's source needs no per-lane address
// arithmetic
__device__ __forceinline__ void dma_tile_s(uint32_t voff, const void* sbase, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds_base), "v"(voff), "s"(sbase)
               : "memory");
}
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Work-group b -> token row for kernels that write one token's int8 codes
// per work-group into the 16x64 tile layout.  A 128-byte line of a tile holds
// tile lanes 8i .. 8i+7, i.e. 8 consecutive code rows (8 tokens, or 2 tokens
// of four planes each); dispatch is round-robin over the 8 XCDs (work-group b
// on XCD b % 8), so rows 8g .. 8g+7 go to work-groups of one XCD and their
// partial-line stores merge in that XCD's L2 instead of reaching memory as 8
// partial writes.  A bijection of [0, 64 n); grids are rounded up to 64.
__device__ __forceinline__ int xcd_grouped_row(int b) {
  const int x = b & 7, j = b >> 3;
  return 64 * (j >> 3) + 8 * x + (j & 7);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) void*)p));
}

}  // namespace tl
