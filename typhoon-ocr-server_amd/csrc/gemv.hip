// gemv.hip -- M=1 INT8 GEMV for decode (W8A32 batch==1 and W8A8 batch==1).
//
// Reference: kernel/w8a32_kernel.c:248-275 (w8a32_gemv) and :205-246
// (_sdot_gemv_worker); kernel/w8a8_kernel.c:141-237 (w8a8_gemv).
//   codes = per-token int8 quantization of x (fused here, see below)
//   acc[n] = sum_k W[n,k] * codes[k]                  exact int32
//   W8A32: y[n] = fl(fl(fl(acc) * ws[n]) * xs)   (+ bias[n] as its own rounding)
//   W8A8 : y[n] = fma(fl(fl(acc) * ws[n]), xs, bias ? bias[n] : 0)
//
// Work decomposition (HBM-bound: 1 weight byte per 2 ops):
//   * weights are 16x64 tiles (tl_common.h).  A work-group (4 waves) owns
//     one 16-row group at a time; wave w streams the tiles of k-blocks
//     [w*KB/4, (w+1)*KB/4) with one 16-byte load per lane per tile (1 KiB per
//     wave-load, fully coalesced), two batches of U tiles in flight; the loop
//     body is branch-free, tail tiles are read from a clamped address and
//     masked;
//   * lane l accumulates row (l & 15) over the k slice of its lane group
//     (l >> 4) with v_dot4_i32_i8; the 16 partial sums of a row (4 lane
//     groups x 4 waves) meet in LDS and are added in a fixed order.  Integer
//     sums make every decomposition bit-identical to the sequential sum.
//   * LOOP = false: one row group per work-group (NG work-groups).  Used for
//     the decode shapes, which are latency-bound: everything a wave needs is
//     issued in its first instructions (U is chosen so that the two batches
//     hold all of the wave's tiles whenever that fits).
//   * LOOP = true: a persistent grid walks the row groups (g += gridDim.x)
//     and issues the first tiles of its next row group before reducing the
//     current one, so the activation prologue runs once per work-group
//     instead of once per row group (large N: the 151936-row lm_head).
//
// Fused activation quantization (XV > 0): every work-group first issues the
// loads of x (XV float4 per thread) and of its first two batches of weight
// tiles, then reduces absmax (DPP within a wave, LDS across the 4 waves),
// derives scale/inverse exactly as the reference (w8a32_kernel.c:145-158) and
// writes the int8 codes into LDS while the weight loads are in flight.
// XV == 0 takes precomputed codes from device memory (W8A8 batch==1, or
// K > 16384).
#include "tl_common.h"
#include "tl_kernels.h"

#include <algorithm>

namespace tl {

struct GemvArgs {
  const float* x;      // fp32 activation [K]                (XV > 0)
  const uint8_t* xq;   // int8 codes zero padded to KB*64    (XV == 0)
  const float* xs_in;  // activation scale                   (XV == 0)
  const uint8_t* wt;   // weight tiles
  const float* ws;     // [N]
  const float* bias;   // [N] or null
  float* y;            // [N]
  int32_t* acc_out;    // [N] (EPI_ACC)
  float* xs_out;       // optional activation scale output
  int N, K, KB, NG, epi;
  int x_vec;           // 2: K == 1024*XV and x 16-byte aligned (unguarded loads)
};

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

__device__ __forceinline__ void gemv_epilogue(const GemvArgs& a, int n, int acc, float xs,
                                              float wsv, float bv) {
  if (a.epi == EPI_ACC) {
    a.acc_out[n] = acc;
  } else if (a.epi == EPI_W8A32) {
    float r = __fmul_rn(__fmul_rn((float)acc, wsv), xs);
    if (a.bias) r = __fadd_rn(r, bv);
    a.y[n] = r;
  } else {
    const float t = __fmul_rn((float)acc, wsv);
    a.y[n] = __fmaf_rn(t, xs, bv);
  }
}

// acc += dot(tile, codes) for U tiles starting at wave-local tile index t0;
// tiles at or beyond n_t were loaded from a clamped address and are dropped.
template <int XV, int U>
__device__ __forceinline__ int consume_batch(const uint4 (&b)[U], const uint4 (&c)[XV == 0 ? U : 1],
                                             const uint4* s_codes, int kb0, int t0, int tmax, int n_t,
                                             int lg, int acc) {
  uint4 cv[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    if constexpr (XV > 0) cv[u] = s_codes[(kb0 + min(t0 + u, tmax)) * 4 + lg];
    else cv[u] = c[u];
  }
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int d = dot16(b[u], cv[u], 0);
    acc += (t0 + u < n_t) ? d : 0;
  }
  return acc;
}

template <int XV, int U>
__device__ __forceinline__ void load_batch(uint4 (&b)[U], uint4 (&c)[XV == 0 ? U : 1], const uint4* wp,
                                           size_t tstride, const uint4* cg, int kb0, int t0, int tmax,
                                           int lg) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int t = min(t0 + u, tmax);
    b[u] = wp[(size_t)t * tstride];
    if constexpr (XV == 0) c[u] = cg[(kb0 + t) * 4 + lg];
  }
  // keep the batch issued here, ahead of the consumption that follows
  __builtin_amdgcn_sched_barrier(0);
}

template <int XV, int U, bool LOOP>
__global__ __launch_bounds__(256) void gemv_i8_kernel(GemvArgs a) {
  __shared__ uint4 s_codes[XV > 0 ? XV * 64 : 1];
  __shared__ uint32_t s_mx[4];
  __shared__ float s_tail[4];
  __shared__ int s_red[LOOP ? 2 : 1][16 * 16];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // k slice of this wave
  const int lg = lane >> 4;
  const int KB = a.KB, NG = a.NG;
  const int kb0 = (wv * KB) >> 2;
  const int n_t = ((wv + 1) * KB >> 2) - kb0;   // 0 for some waves when KB < 4
  const int tmax = n_t > 0 ? n_t - 1 : 0;        // kb0 + tmax < KB always
  const size_t tstride = (size_t)NG * 64;       // uint4 between consecutive k-blocks
  const uint4* wbase = reinterpret_cast<const uint4*>(a.wt) + (size_t)kb0 * tstride + lane;
  const uint4* cg = reinterpret_cast<const uint4*>(a.xq);
  int g = blockIdx.x;
  const uint4* wp = wbase + (size_t)g * 64;

  uint4 b0[U], b1[U];
  uint4 c0[XV == 0 ? U : 1], c1[XV == 0 ? U : 1];

  // x is read before the first weight batch is issued, so the wait for x
  // never waits for weights
  float4 xv[XV > 0 ? XV : 1];
  if constexpr (XV > 0) {
    const int K = a.K;
    if (a.x_vec == 2) {
#pragma unroll
      for (int i = 0; i < XV; i++) xv[i] = *reinterpret_cast<const float4*>(a.x + 4 * (threadIdx.x + 256 * i));
    } else {
#pragma unroll
      for (int i = 0; i < XV; i++) {
        const int k0 = 4 * (threadIdx.x + 256 * i);
        float4 v;
        v.x = (k0 < K) ? a.x[k0] : 0.f;
        v.y = (k0 + 1 < K) ? a.x[k0 + 1] : 0.f;
        v.z = (k0 + 2 < K) ? a.x[k0 + 2] : 0.f;
        v.w = (k0 + 3 < K) ? a.x[k0 + 3] : 0.f;
        xv[i] = v;
      }
    }
  }
  load_batch<XV, U>(b0, c0, wp, tstride, cg, kb0, 0, tmax, lg);
  load_batch<XV, U>(b1, c1, wp, tstride, cg, kb0, U, tmax, lg);
  // epilogue operands of this work-group's first row group
  const int r16 = lane & 15;
  float wsv = a.ws[min(g * 16 + r16, a.N - 1)];
  float bv = a.bias ? a.bias[min(g * 16 + r16, a.N - 1)] : 0.0f;

  float xs;
  if constexpr (XV > 0) {
    // ---- fused per-token activation quantization --------------------------
    const int K = a.K;
    uint32_t* sc = reinterpret_cast<uint32_t*>(s_codes);
    if ((K & 15) == 0) {
      // every element is in the 16-aligned prefix: RNE codes; elements past
      // K were loaded as zeros and do not move the max
      uint32_t mx = 0;
#pragma unroll
      for (int i = 0; i < XV; i++) {
        const uint32_t m01 = max(abs_bits(xv[i].x), abs_bits(xv[i].y));
        const uint32_t m23 = max(abs_bits(xv[i].z), abs_bits(xv[i].w));
        mx = max(mx, max(m01, m23));
      }
      mx = wave_umax(mx);
      if (lane == 0) s_mx[wv] = mx;
      __syncthreads();
      const uint32_t m = max(max(s_mx[0], s_mx[1]), max(s_mx[2], s_mx[3]));
      xs = quant_scale(__uint_as_float(m));
      const float inv = quant_inv(xs);
#pragma unroll
      for (int i = 0; i < XV; i++) {
        const float4 v = xv[i];
        sc[threadIdx.x + 256 * i] = pack4(code_rne(v.x * inv, false), code_rne(v.y * inv, false),
                                          code_rne(v.z * inv, false), code_rne(v.w * inv, false));
      }
    } else {
      // K % 16 != 0: the last K % 16 elements are the reference's scalar tail
      const int main_end = K & ~15;
      uint32_t mx = 0;
      float tail = 0.0f;
#pragma unroll
      for (int i = 0; i < XV; i++) {
        const int k0 = 4 * (threadIdx.x + 256 * i);
        const float e[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int k = k0 + q;
          const uint32_t m1 = (k < main_end) ? abs_bits(e[q]) : 0u;
          mx = m1 > mx ? m1 : mx;
          const float t1 = (k >= main_end && k < K) ? fabsf(e[q]) : 0.0f;
          tail = (t1 > tail) ? t1 : tail;
        }
      }
      mx = wave_umax(mx);
      tail = wave_fmax_nonnan(tail);
      if (lane == 0) {
        s_mx[wv] = mx;
        s_tail[wv] = tail;
      }
      __syncthreads();
      const uint32_t m = max(max(s_mx[0], s_mx[1]), max(s_mx[2], s_mx[3]));
      float t = s_tail[0];
#pragma unroll
      for (int q = 1; q < 4; q++) t = (s_tail[q] > t) ? s_tail[q] : t;
      // the tail is compared against the prefix max the way
      // `if (v > absmax) absmax = v` does (kernel/w8a32_kernel.c:153)
      const float vec = __uint_as_float(m);
      xs = quant_scale((t > vec) ? t : vec);
      const float inv = quant_inv(xs);
#pragma unroll
      for (int i = 0; i < XV; i++) {
        const int k0 = 4 * (threadIdx.x + 256 * i);
        const float4 v = xv[i];
        sc[threadIdx.x + 256 * i] = pack4(code_at(v.x, inv, k0, K, false), code_at(v.y, inv, k0 + 1, K, false),
                                          code_at(v.z, inv, k0 + 2, K, false), code_at(v.w, inv, k0 + 3, K, false));
      }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && a.xs_out) *a.xs_out = xs;
    __syncthreads();
  } else {
    xs = a.xs_in ? *a.xs_in : 1.0f;
  }

  int it = 0;
  while (true) {
    // ---- main loop: two batches of U tiles in flight -------------------------
    // Both batches were issued before this point.  The loop body is
    // straight-line code that enters and leaves with the 2U loads of b0 and
    // b1 outstanding, so the compiler keeps the wait counts exact.
    int acc = 0;
    int t = 0;
    for (; t + 2 * U < n_t; t += 2 * U) {
      acc = consume_batch<XV, U>(b0, c0, s_codes, kb0, t, tmax, n_t, lg, acc);
      load_batch<XV, U>(b0, c0, wp, tstride, cg, kb0, t + 2 * U, tmax, lg);
      acc = consume_batch<XV, U>(b1, c1, s_codes, kb0, t + U, tmax, n_t, lg, acc);
      load_batch<XV, U>(b1, c1, wp, tstride, cg, kb0, t + 3 * U, tmax, lg);
    }
    const int gcur = g;
    const float wcur = wsv, bcur = bv;
    if constexpr (LOOP) {
      // the last double batch of this row group: the loads that follow go
      // to the first tiles of the next one (clamped to a valid row group when
      // there is none; those loads are never consumed)
      g += gridDim.x;
      const int gn = min(g, NG - 1);
      wp = wbase + (size_t)gn * 64;
      acc = consume_batch<XV, U>(b0, c0, s_codes, kb0, t, tmax, n_t, lg, acc);
      load_batch<XV, U>(b0, c0, wp, tstride, cg, kb0, 0, tmax, lg);
      acc = consume_batch<XV, U>(b1, c1, s_codes, kb0, t + U, tmax, n_t, lg, acc);
      load_batch<XV, U>(b1, c1, wp, tstride, cg, kb0, U, tmax, lg);
      wsv = a.ws[min(gn * 16 + r16, a.N - 1)];
      bv = a.bias ? a.bias[min(gn * 16 + r16, a.N - 1)] : 0.0f;
    } else {
      acc = consume_batch<XV, U>(b0, c0, s_codes, kb0, t, tmax, n_t, lg, acc);
      acc = consume_batch<XV, U>(b1, c1, s_codes, kb0, t + U, tmax, n_t, lg, acc);
    }

    // ---- reduction: row r's 16 partials (wave w, lane group q) at
    //      s_red[r*16 + w*4 + q], summed in that order by wave 0 ------------
    int* red = s_red[LOOP ? (it & 1) : 0];
    red[r16 * 16 + wv * 4 + lg] = acc;
    __syncthreads();
    if (wv == 0 && lane < 16) {
      const int4* p = reinterpret_cast<const int4*>(red + lane * 16);
      const int4 q0 = p[0], q1 = p[1], q2 = p[2], q3 = p[3];
      const int tot = ((q0.x + q0.y) + (q0.z + q0.w)) + ((q1.x + q1.y) + (q1.z + q1.w)) +
                      ((q2.x + q2.y) + (q2.z + q2.w)) + ((q3.x + q3.y) + (q3.z + q3.w));
      const int n = gcur * 16 + lane;
      if (n < a.N) gemv_epilogue(a, n, tot, xs, wcur, bcur);
    }
    if constexpr (!LOOP) break;
    if (g >= NG) break;
    ++it;
  }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
template <int XV, int U, bool LOOP>
static void launch_one(const GemvArgs& a, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((gemv_i8_kernel<XV, U, LOOP>), dim3(blocks), dim3(256), 0, st, a);
}

template <int XV>
static hipError_t launch_xv(const GemvArgs& a, const GemvPlan& p, hipStream_t st) {
  if (p.loop) {
    if (p.u != 4) return hipErrorInvalidValue;
    launch_one<XV, 4, true>(a, p.blocks, st);
  } else {
    switch (p.u) {
      case 2: launch_one<XV, 2, false>(a, p.blocks, st); break;
      case 4: launch_one<XV, 4, false>(a, p.blocks, st); break;
      case 8: launch_one<XV, 8, false>(a, p.blocks, st); break;
      case 12: launch_one<XV, 12, false>(a, p.blocks, st); break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

// Number of float4 per thread needed to hold a K-long activation (0 if the
// fused prologue does not apply).
int gemv_fused_xv(int K) {
  const int kpad = cdiv(K, 64) * 64;
  if (kpad <= 2048) return 2;
  if (kpad <= 4096) return 4;
  if (kpad <= 6144) return 6;
  if (kpad <= 8192) return 8;
  if (kpad <= 16384) return 16;
  return 0;
}

static int g_force_mode = 0, g_force_grid = 0, g_force_u = 0;

void gemv_set_plan(int mode, int grid, int u) {
  g_force_mode = mode;
  g_force_grid = grid;
  g_force_u = u;
}

// Persistent grid: work-groups resident per CU x 256 CUs.
static constexpr int kLoopWgPerCu = 4;
static constexpr int kNumCu = 256;

// Measured on MI355X (graph-replayed launches over > 512 MB of rotating
// weights).  Decode shapes (NG <= 768) are latency-bound: one row group per
// work-group, with both batches holding all of a wave's tiles when that is at
// most 24 (K <= 6144), so every weight load is issued before the activation
// prologue.  Large N (the lm_head) streams on a persistent grid.
GemvPlan gemv_plan(int N, int K) {
  GemvPlan p;
  const int NG = cdiv(N, 16);
  const int KB = cdiv(K, 64);
  const int n_t = cdiv(KB, 4);
  p.loop = NG > 4 * kNumCu * kLoopWgPerCu;
  if (g_force_mode == 1) p.loop = false;
  if (g_force_mode == 2) p.loop = true;
  if (p.loop) {
    p.u = 4;
    p.blocks = std::min(NG, g_force_grid > 0 ? g_force_grid : kNumCu * kLoopWgPerCu);
  } else {
    p.blocks = NG;
    if (n_t <= 4) p.u = 2;
    else if (n_t <= 8) p.u = 4;
    else if (n_t <= 16) p.u = 8;
    else if (n_t <= 24) p.u = 12;
    else p.u = 8;
    if (g_force_u > 0) p.u = g_force_u;
  }
  return p;
}

hipError_t launch_gemv_i8(const GemvLaunch& L, hipStream_t st) {
  GemvArgs a;
  a.x = L.x;
  a.xq = L.xq;
  a.xs_in = L.xs_in;
  a.wt = L.wt;
  a.ws = L.ws;
  a.bias = L.bias;
  a.y = L.y;
  a.acc_out = L.acc_out;
  a.xs_out = L.xs_out;
  a.N = L.N;
  a.K = L.K;
  a.KB = cdiv(L.K, 64);
  a.NG = cdiv(L.N, 16);
  a.epi = L.epi;
  a.x_vec = 0;
  if (L.N <= 0 || L.K <= 0) return hipErrorInvalidValue;
  const GemvPlan p = gemv_plan(L.N, L.K);
  const int xv = L.x ? gemv_fused_xv(L.K) : 0;
  if (L.x && xv == 0) return hipErrorInvalidValue;  // caller must quantize first
  if (L.x && L.K == 1024 * xv && (((uintptr_t)L.x) & 15) == 0) a.x_vec = 2;
  if (!L.x && !L.xq) return hipErrorInvalidValue;
  switch (xv) {
    case 0: return launch_xv<0>(a, p, st);
    case 2: return launch_xv<2>(a, p, st);
    case 4: return launch_xv<4>(a, p, st);
    case 6: return launch_xv<6>(a, p, st);
    case 8: return launch_xv<8>(a, p, st);
    case 16: return launch_xv<16>(a, p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tl
