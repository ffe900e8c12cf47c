// gemm_small.hip -- M <= 64 token rows over int8 weight tiles (decode rows
// M = 2..8 of w8a32_linear, W8A16 at M = 1..64, W8A8 batches of 2..64).
//
// HBM-bound like the M = 1 GEMV, and organised the same way: a work-group
// owns one 16-row weight group, its 4 waves split K, each wave streams its
// 1 KiB weight tiles with two batches of U tiles in flight (branch-free,
// clamped tail tiles get their activations zeroed), and the token rows ride along
// as the second MFMA operand (L2-resident: 16 rows x K).  Each wave keeps one
// 16x16 accumulator D[n][m] (weights as the first MFMA operand, so a lane
// holds 4 consecutive n of one token row m); the 4 partial accumulators are
// summed through LDS in a fixed order and wave 0 applies the epilogue.
//
//   A_I8    codes as 16x64 tiles (one row group), v_mfma_i32_16x16x64_i8
//   A_BF16  bf16 rows, v_mfma_f32_16x16x32_bf16 (two per 64-wide K block)
//   A_F16   fp16 rows, v_mfma_f32_16x16x32_f16
//   A_F32X3 fp32 rows split exactly into three bf16 terms (six MFMAs per block)
// Token rows >= M read row M-1 (their output columns are never stored); K
// positions >= K are zero in the weight tiles and are zeroed in X as well.
#include <algorithm>
#include <atomic>

#include "tl_common.h"
#include "tl_kernels.h"

typedef _Float16 v8h_s __attribute__((ext_vector_type(8)));

namespace tl {

struct GemmSmallArgs {
  const void* A;        // A_I8: code tiles [KB][1]; else row-major [M][lda]
  int lda;
  const uint8_t* Bt;    // weight tiles [KB][NG]
  const float* ws;
  const float* xs;      // per-token scales (A_I8)
  const int* xe;        // OUT_F32_X4: per-token exponents
  const float* xraw;    // OUT_F32_X4: the fp32 token rows (null: NaN for a non-finite row)
  int ldxr;
  const float* bias;
  void* Y;
  int ldy;
  int M, N, K, KB, NG;
  int MG;               // 16-row token groups: ceil(M / 16) (A_I8 tile rows)
  int ep, out;
};

template <int AMODE>
struct AFrag {
  // A_I8: 1 x uint4; 16-bit: 2 x uint4 (K halves); fp32: 4 x uint4 (16 floats)
  uint4 v[AMODE == A_I8 ? 1 : (AMODE == A_F32X3 ? 4 : 2)];
};

// activation fragment of k-block kb for token group tg (rows 16 tg ..)
template <int AMODE>
__device__ inline AFrag<AMODE> load_a(const GemmSmallArgs& a, int kb, int tg, int lane) {
  AFrag<AMODE> f;
  if constexpr (AMODE == A_I8) {
    f.v[0] = reinterpret_cast<const uint4*>(a.A)[((size_t)kb * a.MG + min(tg, a.MG - 1)) * 64 + lane];
  } else {
    constexpr int ESZ = (AMODE == A_F32X3) ? 4 : 2;
    constexpr int NV = (AMODE == A_F32X3) ? 4 : 2;
    constexpr int EPV = 16 / ESZ;                     // elements per uint4
    // only lanes of real rows load (the rest hold zeros, whose output rows are
    // never stored): at M = 2 this cuts the activation requests, which share
    // the CU's load path with the weight stream, eightfold
    const int row = tg * 16 + (lane & 15);
    const int k0 = kb * 64 + 16 * (lane >> 4);
    const char* base = static_cast<const char*>(a.A) + (size_t)min(row, a.M - 1) * a.lda * ESZ;
#pragma unroll
    for (int v = 0; v < NV; v++) f.v[v] = make_uint4(0, 0, 0, 0);
    if (row < a.M) {
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const int k = k0 + EPV * v;
        const int kc = min(k, a.K - EPV);             // in-bounds address
        const uint4 u = *reinterpret_cast<const uint4*>(base + (size_t)kc * ESZ);
        if (k < a.K) f.v[v] = u;
      }
    }
  }
  return f;
}

__device__ inline void widen_bf16(uint4 w, uint4& h0, uint4& h1) {
  uint2 p0 = i8x4_to_bf16x4(w.x), p1 = i8x4_to_bf16x4(w.y);
  uint2 p2 = i8x4_to_bf16x4(w.z), p3 = i8x4_to_bf16x4(w.w);
  h0 = make_uint4(p0.x, p0.y, p1.x, p1.y);
  h1 = make_uint4(p2.x, p2.y, p3.x, p3.y);
}

__device__ inline uint32_t f16x2(float a, float b) {
  const _Float16 ha = (_Float16)a, hb = (_Float16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}
__device__ inline void widen_f16(uint4 w, uint4& h0, uint4& h1) {
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
  uint32_t o[8];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    o[2 * q] = f16x2((float)(int8_t)(d[q] & 0xff), (float)(int8_t)((d[q] >> 8) & 0xff));
    o[2 * q + 1] = f16x2((float)(int8_t)((d[q] >> 16) & 0xff), (float)(int8_t)(d[q] >> 24));
  }
  h0 = make_uint4(o[0], o[1], o[2], o[3]);
  h1 = make_uint4(o[4], o[5], o[6], o[7]);
}


template <int AMODE>
using acc_small_t = typename std::conditional<AMODE == A_I8, v4i, v4f>::type;

// MFMA operands of one activation fragment (for fp32 activations: the
// three bf16 terms of each K half)
template <int AMODE>
struct XOps {
  // A_I8: 1 operand; 16-bit: 2 (K halves); fp32: 6 (3 terms x 2 K halves)
  static constexpr int NX = AMODE == A_I8 ? 1 : (AMODE == A_F32X3 ? 6 : 2);
  uint4 v[NX];
};

template <int AMODE>
__device__ inline XOps<AMODE> prepare_x(const AFrag<AMODE>& x) {
  XOps<AMODE> o;
  if constexpr (AMODE == A_F32X3) {
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      const uint4 u0 = x.v[2 * hh], u1 = x.v[2 * hh + 1];
      const float f[8] = {__uint_as_float(u0.x), __uint_as_float(u0.y), __uint_as_float(u0.z), __uint_as_float(u0.w),
                          __uint_as_float(u1.x), __uint_as_float(u1.y), __uint_as_float(u1.z), __uint_as_float(u1.w)};
      split3x8(f, o.v[3 * hh], o.v[3 * hh + 1], o.v[3 * hh + 2]);
    }
  } else {
#pragma unroll
    for (int q = 0; q < XOps<AMODE>::NX; q++) o.v[q] = x.v[q];
  }
  return o;
}

// MFMA operands of one weight tile: int8 as loaded, or widened to two
// 16-bit K halves (exact), once per tile for all token groups
template <int AMODE>
struct WOps {
  uint4 v[AMODE == A_I8 ? 1 : 2];
};

template <int AMODE>
__device__ inline WOps<AMODE> prepare_w(uint4 w) {
  WOps<AMODE> o;
  if constexpr (AMODE == A_I8) o.v[0] = w;
  else if constexpr (AMODE == A_F16) widen_f16(w, o.v[0], o.v[1]);
  else widen_bf16(w, o.v[0], o.v[1]);
  return o;
}

// one prepared weight tile against one prepared activation fragment
template <int AMODE>
__device__ inline acc_small_t<AMODE> mma_x(const WOps<AMODE>& w, const XOps<AMODE>& x, acc_small_t<AMODE> c) {
  if constexpr (AMODE == A_I8) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, w.v[0]), __builtin_bit_cast(v4i, x.v[0]), c, 0, 0, 0);
  } else if constexpr (AMODE == A_BF16) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, w.v[0]), __builtin_bit_cast(v8bf, x.v[0]), c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, w.v[1]), __builtin_bit_cast(v8bf, x.v[1]), c, 0, 0, 0);
  } else if constexpr (AMODE == A_F16) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h_s, w.v[0]), __builtin_bit_cast(v8h_s, x.v[0]), c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h_s, w.v[1]), __builtin_bit_cast(v8h_s, x.v[1]), c, 0, 0, 0);
  } else {
    // smallest term first: the three products of a K half are added to the
    // fp32 accumulator in increasing magnitude
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, w.v[hh]), __builtin_bit_cast(v8bf, x.v[3 * hh + 2]), c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, w.v[hh]), __builtin_bit_cast(v8bf, x.v[3 * hh + 1]), c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, w.v[hh]), __builtin_bit_cast(v8bf, x.v[3 * hh]), c, 0, 0, 0);
    }
    return c;
  }
}

// R row groups per work-group share every activation fragment (loaded and,
// for fp32 activations, split into bf16 terms once per k-block), so the
// activation work per weight byte falls by R for large N.  TG token groups of
// 16 rows ride along on every weight tile: the weights are streamed once for
// all of them.  Work-group (x, y) takes row groups R x .. R x + R - 1 and
// token groups TG y .. TG y + TG - 1, so the grid's y extent spreads the
// token rows over more work-groups where one would re-read all of them.
template <int AMODE, int U, int R, int TG>
__global__ __launch_bounds__(256) void gemm_small_kernel(GemmSmallArgs a) {
  using acc_t = acc_small_t<AMODE>;
  __shared__ acc_t s_part[R][TG][4][64];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g0 = blockIdx.x * R;                       // first weight row group
  const int tg0 = blockIdx.y * TG;                     // first token group
  const int kb0 = (wv * a.KB) / 4, kb1 = ((wv + 1) * a.KB) / 4;
  const int n_t = kb1 - kb0;                           // may be 0 when KB < 4
  const int last = max(n_t - 1, 0);
  const size_t tstride = (size_t)a.NG * 64;
  const uint4* wbase = reinterpret_cast<const uint4*>(a.Bt) + (size_t)kb0 * tstride + lane;
  int goff[R];                                         // row groups past NG re-read a valid one
#pragma unroll
  for (int r = 0; r < R; r++) goff[r] = min(g0 + r, a.NG - 1) * 64;

  acc_t acc[R][TG];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int g = 0; g < TG; g++) acc[r][g] = acc_t{0, 0, 0, 0};
  uint4 b0[U][R], b1[U][R];
  AFrag<AMODE> x0[U][TG], x1[U][TG];
  auto load = [&](uint4 (&b)[U][R], AFrag<AMODE> (&x)[U][TG], int t0) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int t = min(t0 + u, last);
#pragma unroll
      for (int r = 0; r < R; r++) {
        // each weight tile is read once per launch: non-temporal (streaming)
        // loads, as the GEMV's (lm_head at M = 2: 66 -> 60 us)
        typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
        const v4u_t w = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(wbase + (size_t)t * tstride + goff[r]));
        b[u][r] = make_uint4(w.x, w.y, w.z, w.w);
      }
#pragma unroll
      for (int g = 0; g < TG; g++) x[u][g] = load_a<AMODE>(a, min(kb0 + t, a.KB - 1), tg0 + g, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto consume = [&](const uint4 (&b)[U][R], const AFrag<AMODE> (&x)[U][TG], int t0) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      WOps<AMODE> wo[R];
#pragma unroll
      for (int r = 0; r < R; r++) wo[r] = prepare_w<AMODE>(b[u][r]);
#pragma unroll
      for (int g = 0; g < TG; g++) {
        // clamped repeats add exactly 0: their activations are zeroed (the
        // weights are finite int8, so 0 * w == 0 even when X holds Inf/NaN)
        AFrag<AMODE> xv = x[u][g];
        if (!(t0 + u < n_t)) {
#pragma unroll
          for (int q = 0; q < (int)(sizeof(xv.v) / sizeof(uint4)); q++) xv.v[q] = make_uint4(0, 0, 0, 0);
        }
        const XOps<AMODE> xo = prepare_x<AMODE>(xv);
#pragma unroll
        for (int r = 0; r < R; r++) acc[r][g] = mma_x<AMODE>(wo[r], xo, acc[r][g]);
      }
    }
  };

  load(b0, x0, 0);
  load(b1, x1, U);
  // the epilogue's per-column scales (and, for int8 codes, the per-token
  // exponent or scale), issued behind the first tiles instead of as
  // dependent loads after the reduction: columns past N read column N-1,
  // token rows past M row M-1 (neither is stored)
  float wsv[R][4];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int q = 0; q < 4; q++) wsv[r][q] = a.ws ? a.ws[min((g0 + r) * 16 + 4 * (lane >> 4) + q, a.N - 1)] : 0.0f;
  int xev[TG];
  float xsv[TG];
#pragma unroll
  for (int g = 0; g < TG; g++) {
    const int m = min((tg0 + g) * 16 + (lane & 15), a.M - 1);
    xev[g] = 0;
    xsv[g] = 0.0f;
    if constexpr (AMODE == A_I8) {
      if (a.out == OUT_F32_X4) xev[g] = a.xe[m >> 2];
      else if (a.out != OUT_I32) xsv[g] = a.xs[m];
    }
  }
  int t = 0;
  for (; t + 2 * U < n_t; t += 2 * U) {
    consume(b0, x0, t);
    load(b0, x0, t + 2 * U);
    consume(b1, x1, t + U);
    load(b1, x1, t + 3 * U);
  }
  consume(b0, x0, t);
  consume(b1, x1, t + U);

#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int g = 0; g < TG; g++) s_part[r][g][wv][lane] = acc[r][g];
  __syncthreads();
  // Epilogue: the R x TG (row group, token group) pairs are spread over the
  // 4 waves, pair TG rg + tg on wave (TG rg + tg) mod 4 (wave-uniform).
  if constexpr (AMODE == A_I8) {
    if (a.out == OUT_F32_X4) {
      // rows 4t .. 4t+3 are the planes of token t: the lane quad 4t .. 4t+3
      // (mod 16) holds them; its first lane combines and stores row t
      const bool vec = (a.ldy & 3) == 0 && (((uintptr_t)a.Y) & 15) == 0;
#pragma unroll
      for (int tg = 0; tg < TG; tg++)
#pragma unroll
        for (int rg = 0; rg < R; rg++) {
          if ((TG * rg + tg) % 4 != wv) continue;
          acc_t tot = s_part[rg][tg][0][lane];
#pragma unroll
          for (int w = 1; w < 4; w++) {
            const acc_t p = s_part[rg][tg][w][lane];
#pragma unroll
            for (int q = 0; q < 4; q++) tot[q] += p[q];
          }
          float y[4];
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const int a1 = __shfl_xor(tot[q], 1, 64), a2 = __shfl_xor(tot[q], 2, 64), a3 = __shfl_xor(tot[q], 3, 64);
            y[q] = planes_sum(tot[q], a1, a2, a3);
          }
          const int m = (tg0 + tg) * 16 + (lane & 15);
          const int n0 = (g0 + rg) * 16 + 4 * (lane >> 4);
          if ((lane & 3) != 0 || m >= a.M || n0 >= a.N) continue;
          const int t = m >> 2;
#pragma unroll
          for (int q = 0; q < 4; q++) {
            y[q] = planes_scale(y[q], wsv[rg][q], xev[tg]);
            if (a.bias && n0 + q < a.N) y[q] = __fadd_rn(y[q], a.bias[n0 + q]);
          }
          float* yp = reinterpret_cast<float*>(a.Y) + (size_t)t * a.ldy + n0;
          if (vec && n0 + 4 <= a.N) {
            *reinterpret_cast<float4*>(yp) = make_float4(y[0], y[1], y[2], y[3]);
          } else {
            for (int q = 0; q < 4 && n0 + q < a.N; q++) yp[q] = y[q];
          }
        }
      // a token flagged kXeNonFinite got NaN above: the lane stores its
      // outputs again with the reference's fp32 value (nonfinite_dot over the
      // fp32 row in a.xraw), one copy out of the unrolled loops, which carry
      // no flag for it (the token flags are read again here)
      if (a.xraw && (lane & 3) == 0) {
#pragma unroll 1
        for (int tg = 0; tg < TG; tg++) {
          const int m = (tg0 + tg) * 16 + (lane & 15);
          if (m >= a.M || a.xe[m >> 2] != kXeNonFinite) continue;
          const int t = m >> 2;
#pragma unroll 1
          for (int rg = 0; rg < R; rg++) {
            if ((TG * rg + tg) % 4 != wv) continue;   // another wave's pair
            const int n0 = (g0 + rg) * 16 + 4 * (lane >> 4);
#pragma unroll 1
            for (int q = 0; q < 4; q++) {
              const int n = n0 + q;
              if (n >= a.N) break;
              float v = nonfinite_dot(a.xraw, 0, (size_t)t * a.ldxr, 0, a.K, a.Bt, a.NG, n);
              if (a.bias) v = __fadd_rn(v, a.bias[n]);
              reinterpret_cast<float*>(a.Y)[(size_t)t * a.ldy + n] = v;
            }
          }
        }
      }
      return;
    }
  }
  // lane holds D[n .. n+3][m]: m = 16 (tg0 + tg) + (lane & 15), n = 16 g + 4 (lane >> 4);
  // the 4 consecutive outputs of row m go out as one 16-byte (fp32, int32) or
  // 8-byte (bf16, fp16) store where the row stride and base allow it
  const int esz = (a.out == OUT_BF16 || a.out == OUT_F16) ? 2 : 4;
  const bool vec = (a.ldy & 3) == 0 && (((uintptr_t)a.Y) & (4 * esz - 1)) == 0;
  int nan_sum = 0;        // A_F32X3: an output of this lane summed to NaN (an int: no lane-mask merges)
#pragma unroll
  for (int tg = 0; tg < TG; tg++)
#pragma unroll
  for (int rg = 0; rg < R; rg++) {
    if ((TG * rg + tg) % 4 != wv) continue;
    const int m = (tg0 + tg) * 16 + (lane & 15);
    const int n0 = (g0 + rg) * 16 + 4 * (lane >> 4);
    if (m >= a.M || n0 >= a.N) continue;
    acc_t tot = s_part[rg][tg][0][lane];
#pragma unroll
    for (int w = 1; w < 4; w++) {
      const acc_t p = s_part[rg][tg][w][lane];
#pragma unroll
      for (int q = 0; q < 4; q++) tot[q] += p[q];
    }
    const bool full = vec && n0 + 4 <= a.N;
    const size_t o = (size_t)m * a.ldy + n0;
    if constexpr (AMODE == A_I8) {
      if (a.out == OUT_I32) {
        if (full) {
          *reinterpret_cast<v4i*>(reinterpret_cast<int32_t*>(a.Y) + o) = tot;
        } else {
          for (int q = 0; q < 4 && n0 + q < a.N; q++) reinterpret_cast<int32_t*>(a.Y)[o + q] = tot[q];
        }
        continue;
      }
    }
    float y[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int n = min(n0 + q, a.N - 1);
      if constexpr (AMODE == A_I8) {
        y[q] = __fmul_rn(__fmul_rn((float)tot[q], wsv[rg][q]), xsv[tg]);
        if (a.bias) y[q] = __fadd_rn(y[q], a.bias[n]);
      } else {
        if (a.ep == EP_SCALE_FMA) {
          y[q] = __fmaf_rn(tot[q], wsv[rg][q], a.bias ? a.bias[n] : 0.0f);
        } else {
          y[q] = __fmul_rn(tot[q], wsv[rg][q]);
          if (a.bias) y[q] = __fadd_rn(y[q], a.bias[n]);
        }
        if constexpr (AMODE == A_F32X3) nan_sum |= (int)(tot[q] != tot[q] && n0 + q < a.N);
      }
    }
    if (a.out == OUT_F32) {
      float* yp = reinterpret_cast<float*>(a.Y) + o;
      if (full) {
        *reinterpret_cast<float4*>(yp) = make_float4(y[0], y[1], y[2], y[3]);
      } else {
        for (int q = 0; q < 4 && n0 + q < a.N; q++) yp[q] = y[q];
      }
    } else {
      uint16_t h[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        if (a.out == OUT_BF16) {
          h[q] = (uint16_t)f32_to_bf16_rne(y[q]);
        } else {
          const _Float16 f = (_Float16)y[q];
          h[q] = __builtin_bit_cast(uint16_t, f);
        }
      }
      uint16_t* yp = reinterpret_cast<uint16_t*>(a.Y) + o;
      if (full) {
        *reinterpret_cast<uint2*>(yp) = make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16),
                                                   (uint32_t)h[2] | ((uint32_t)h[3] << 16));
      } else {
        for (int q = 0; q < 4 && n0 + q < a.N; q++) yp[q] = h[q];
      }
    }
  }
  if constexpr (AMODE == A_F32X3) {
    // a row holding Inf or NaN sums to NaN above (the bf16 split of an
    // infinite x makes Inf - Inf): the lane finds those outputs among its own
    // stores (a NaN read back) and stores them again with the reference's
    // fp32 value, NaN or +-Inf from x and the weight codes (nonfinite_dot; a
    // finite row whose terms overflowed finds no Inf and stays NaN), one copy
    // out of the unrolled loops
    if (nan_sum) {
#pragma unroll 1
      for (int b = 0; b < 4 * R * TG; b++) {
        const int tg = b / (4 * R), rg = (b >> 2) % R, q = b & 3;
        if ((TG * rg + tg) % 4 != wv) continue;   // another wave's pair
        const int m = (tg0 + tg) * 16 + (lane & 15);
        const int n = (g0 + rg) * 16 + 4 * (lane >> 4) + q;
        if (m >= a.M || n >= a.N) continue;
        const size_t o = (size_t)m * a.ldy + n;
        bool was_nan;
        if (a.out == OUT_F32) {
          was_nan = __builtin_isnan(reinterpret_cast<const float*>(a.Y)[o]);
        } else {
          const uint16_t h = reinterpret_cast<const uint16_t*>(a.Y)[o];
          was_nan = a.out == OUT_BF16 ? (h & 0x7fff) > 0x7f80 : (h & 0x7fff) > 0x7c00;
        }
        if (!was_nan) continue;
        float y = nonfinite_dot(a.A, 0, (size_t)m * a.lda, 0, a.K, a.Bt, a.NG, n);
        if (a.bias) y = __fadd_rn(y, a.bias[n]);
        if (a.out == OUT_F32) {
          reinterpret_cast<float*>(a.Y)[o] = y;
        } else if (a.out == OUT_BF16) {
          reinterpret_cast<uint16_t*>(a.Y)[o] = (uint16_t)f32_to_bf16_rne(y);
        } else {
          const _Float16 h = (_Float16)y;
          reinterpret_cast<uint16_t*>(a.Y)[o] = __builtin_bit_cast(uint16_t, h);
        }
      }
    }
  }
}

bool gemm_small_supported(const GemmLaunch& L) {
  const int max_rows = (L.amode == A_BF16 || L.amode == A_F16) ? 256 : 64;
  if (L.M < 1 || L.M > max_rows) return false;
  if (L.amode == A_I8) return true;                    // code tiles, any K
  const int epv = (L.amode == A_F32X3) ? 4 : 8;        // elements per 16 bytes
  if (L.K % epv != 0 || L.lda % epv != 0) return false;
  return (((uintptr_t)L.A) & 15) == 0;
}

template <int AMODE, int R, int TG>
static void launch_small_rt(const GemmSmallArgs& a, int u, hipStream_t st) {
  if constexpr (AMODE == A_F32X3 && R * TG > 8) {
    // never planned (fp32 rows run here only below 512 weight row groups, one
    // per work-group); the instance would pass 512 VGPRs
    launch_small_rt<AMODE, 8 / TG, TG>(a, u, st);
  } else {
    const dim3 grid(cdiv(a.NG, R), cdiv(a.MG, TG)), block(256);
    // batches of 4 tiles exist for one token group, and for 16-bit rows up to
    // 8 row x token groups per work-group (wider ones pass 512 VGPRs)
    if constexpr (TG == 1 || ((AMODE == A_BF16 || AMODE == A_F16) && R * TG <= 8)) {
      if (u == 4) {
        hipLaunchKernelGGL((gemm_small_kernel<AMODE, 4, R, TG>), grid, block, 0, st, a);
        return;
      }
    }
    hipLaunchKernelGGL((gemm_small_kernel<AMODE, 2, R, TG>), grid, block, 0, st, a);
  }
}

template <int AMODE, int R>
static void launch_small_r(const GemmSmallArgs& a, int u, int tg, hipStream_t st) {
  if (tg == 1) launch_small_rt<AMODE, R, 1>(a, u, st);
  else if (tg == 2) launch_small_rt<AMODE, R, 2>(a, u, st);
  else launch_small_rt<AMODE, R, 4>(a, u, st);
}

template <int AMODE>
static void launch_small_mode(const GemmSmallArgs& a, int u, int r, int tg, hipStream_t st) {
  if (r == 4) launch_small_r<AMODE, 4>(a, u, tg, st);
  else if (r == 2) launch_small_r<AMODE, 2>(a, u, tg, st);
  else launch_small_r<AMODE, 1>(a, u, tg, st);
}

// tuning override of the 16-bit rows' work-group shape: 100 R + 10 TG + U
// (R, TG in {1, 2, 4}, U in {2, 4}), 0 = the planner in launch_gemm_small
static std::atomic<int> g_small_b16_shape{0};
void gemm_small_set_b16_shape(int code) { g_small_b16_shape.store(code, std::memory_order_relaxed); }

hipError_t launch_gemm_small(const GemmLaunch& L, hipStream_t st) {
  if (!gemm_small_supported(L)) return hipErrorInvalidValue;
  GemmSmallArgs a;
  a.A = L.A;
  a.lda = L.lda;
  a.Bt = L.Bt;
  a.ws = L.ws;
  a.xs = L.xs;
  a.xe = L.xe;
  a.xraw = L.xraw;
  a.ldxr = L.ldxr;
  a.bias = L.bias;
  a.Y = L.Y;
  a.ldy = L.ldy;
  a.M = L.M;
  a.N = L.N;
  a.K = L.K;
  a.KB = cdiv(L.K, 64);
  a.NG = cdiv(L.N, 16);
  a.MG = cdiv(L.M, 16);
  a.ep = L.ep;
  a.out = L.out;
  if (L.out == OUT_F32_X4 && (L.amode != A_I8 || !L.xe || L.M % 4 != 0)) return hipErrorInvalidValue;
  if (L.amode == A_I8 && L.out != OUT_I32 && L.out != OUT_F32_X4 && !L.xs) return hipErrorInvalidValue;
  const int n_t = cdiv(a.KB, 4);
  // four row groups per work-group once there are work-groups to spare
  // (>= 2048 row groups: the lm_head), else one
  int r = a.NG >= 2048 ? 4 : 1;
  int tg = a.MG <= 1 ? 1 : (a.MG <= 2 ? 2 : 4);
  const bool b16 = L.amode == A_BF16 || L.amode == A_F16;
  int u_force = 0;
  if (!b16) {
    if (a.NG >= 2048) {
      // weights far past the caches (the lm_head): every token group rides
      // on each weight tile, so the tiles are streamed once; four row groups
      // per work-group, batches of 2 tiles (lm_head planes at 2 tokens 51.2
      // -> 46.7 us against batches of 4)
      u_force = 2;
    } else {
      // weights within the caches: one token group per work-group (the
      // grid's y extent over the token groups) and the most row groups that
      // still leave >= 192 work-groups; batches of 4 tiles for one row group
      // (and two of int8 codes).  Measured over every shape (R, TG, U) at
      // K = 2048 / 6144: the best or within 3 % at every point, e.g. W8A32
      // at 32 tokens, N = 2048: 14.4 -> 8.6 us (all token groups on one
      // work-group before); W8A8 at 64 rows, N = 2048: 7.7 -> 6.3 us; the
      // int8 planes of 8 tokens over 2048 x 6144: 10.9 -> 9.0 us
      tg = 1;
      r = 1;
      for (int cr = 4; cr > 1; cr >>= 1)
        if ((long long)cdiv(a.NG, cr) * a.MG >= 192) {
          r = cr;
          break;
        }
      u_force = (n_t >= 8 && (r == 1 || (r == 2 && L.amode == A_I8))) ? 4 : 2;
    }
  }
  if (b16 && a.MG >= 2) {
    // 16-bit rows, 17..256 tokens: the widest work-group, most weight row
    // groups R and then most token groups TG (each 4, 2 or 1, TG at most the
    // token groups there are), that still leaves >= 192 work-groups; batches
    // of 4 tiles only below 4 (row group, token group) pairs.  Measured over
    // every shape (R, TG, U) at K = 2048 and M = 32..256, N = 2048 / 4096 /
    // 12288: the best shape or within 2 % of it at every point, e.g.
    // M = 256, N = 2048: 4 x 2 groups 9.3 us (1 x 4: 13.3, the tiled kernel
    // 11.5); M = 64, N = 4096: 4 x 1 groups 7.1 us (2 x 1: 8.7).
    r = 1;
    tg = 1;
    bool found = false;
    for (int cr = 4; cr >= 1 && !found; cr >>= 1)
      for (int ct = 4; ct >= 1; ct >>= 1)
        if (ct <= a.MG && (long long)cdiv(a.NG, cr) * cdiv(a.MG, ct) >= 192) {
          r = cr;
          tg = ct;
          found = true;
          break;
        }
    u_force = (r * tg >= 4 || n_t < 8) ? 2 : 4;
  }
  if (b16) {
    const int code = g_small_b16_shape.load(std::memory_order_relaxed);
    const int cr = code / 100, ct = (code / 10) % 10, cu = code % 10;
    if ((cr == 1 || cr == 2 || cr == 4) && (ct == 1 || ct == 2 || ct == 4) && (cu == 2 || cu == 4) &&
        (cu == 2 || ct == 1 || cr * ct <= 8)) {
      r = cr;
      tg = ct;
      u_force = cu;
    }
  }
  if (cdiv(a.MG, tg) > 65535) return hipErrorInvalidValue;
  // batches of 4 tiles only with one token group: more activation fragments
  // in flight push the waves past 256 VGPRs (one wave per SIMD); int8 codes
  // (one 16-byte fragment per tile) also with four row groups
  int u = (tg == 1 && n_t >= 8 && (r == 1 || L.amode == A_I8)) ? 4 : 2;
  if (u_force) u = u_force;
  switch (L.amode) {
    case A_I8: launch_small_mode<A_I8>(a, u, r, tg, st); break;
    case A_BF16: launch_small_mode<A_BF16>(a, u, r, tg, st); break;
    case A_F16: launch_small_mode<A_F16>(a, u, r, tg, st); break;
    default: launch_small_mode<A_F32X3>(a, u, r, tg, st); break;
  }
  return hipGetLastError();
}

}  // namespace tl
