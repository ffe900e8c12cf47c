// gemm.hip -- MFMA GEMMs over int8 weight tiles (prefill and M>1 decode rows).
//
//   A_I8    W8A8:  int8 codes (16x64 tiles) x int8 weights on
//                  v_mfma_i32_16x16x64_i8, exact int32 accumulation.
//                  Reference kernel/w8a8_kernel.c:259-268 dequantizes both
//                  operands and runs cblas_sgemm; the exact integer sum with
//                  the fp32 epilogue fl(fl(fl(acc)*ws)*xs) differs from that
//                  by ~4e-7 relative L2.
//   A_BF16  W8A16: bf16 X (row-major) x int8 weights converted in registers to
//                  bf16 (exact for |w| <= 127) on v_mfma_f32_16x16x32_bf16;
//                  the fp32 scale is applied after the fp32 accumulation
//                  (kernel/w8a16_kernel.c:134 for batch==1; :187-216 batch>1).
//   A_F16   as A_BF16 with fp16 X on v_mfma_f32_16x16x32_f16.
//   A_F32X3 W8A32 batch>1 (kernel/w8a32_kernel.c:297-350, fp32 X times the
//                  dequantized weights): X is split exactly into three bf16
//                  terms x = x0 + x1 + x2 (x0 = bf16(x), x1 = bf16(x - x0),
//                  x2 = bf16(x - x0 - x1); the residual is below 2^-24 |x|), so
//                  three bf16 MFMAs per fragment reproduce the fp32 product sum
//                  with products that are exact in fp32.
//
// Layout: a wave owns a (16 TM) x (16 TN) block of Y built from 16x16 MFMA
// tiles; a work-group is WGM x WGN waves.  Fragments are loaded straight from
// HBM/L2 with one 16-byte load per lane per 1 KiB weight tile.  Output tile
// element (i, j, r) of lane l is Y[16 mg + 4 (l >> 4) + r][16 ng + (l & 15)]
// (the 16x16 MFMA accumulator layout).  Small M splits K over S work-groups;
// partial tiles are summed by the last work-group to arrive in the fixed
// order s = 0..S-1, so results do not depend on scheduling.
#include "tl_common.h"
#include "tl_kernels.h"
#include <hip/hip_fp16.h>

typedef _Float16 v8h __attribute__((ext_vector_type(8)));

namespace tl {

struct GemmArgs {
  const void* A;        // tiles (A_I8) or row-major [M][lda]
  int lda;
  const uint8_t* Bt;    // weight tiles
  const float* ws;      // [N]
  const float* xs;      // [M] activation scales (A_I8) or null
  const float* bias;    // [N] or null
  void* Y;
  int ldy;
  int M, N, K, KB, MG, NG;
  int S;
  void* part;           // [S][MG*16][NG*16] fp32 or int32
  uint32_t* cnt;        // per output tile, zero at rest
  int ep, out;
  int ntn;              // number of work-group tiles along N
};

// --------------------------------------------------------------------------
// operand helpers
// --------------------------------------------------------------------------
__device__ inline v8bf as_v8bf(uint4 u) { return __builtin_bit_cast(v8bf, u); }
__device__ inline v8h as_v8h(uint4 u) { return __builtin_bit_cast(v8h, u); }

// int8 weight tile lane -> two bf16 operands (K halves)
__device__ inline void w_to_bf16(uint4 w, uint4& h0, uint4& h1) {
  uint2 p0 = i8x4_to_bf16x4(w.x), p1 = i8x4_to_bf16x4(w.y);
  uint2 p2 = i8x4_to_bf16x4(w.z), p3 = i8x4_to_bf16x4(w.w);
  h0 = make_uint4(p0.x, p0.y, p1.x, p1.y);
  h1 = make_uint4(p2.x, p2.y, p3.x, p3.y);
}

__device__ inline uint32_t f16pair(float a, float b) {
  _Float16 ha = (_Float16)a, hb = (_Float16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}
__device__ inline void w_to_f16(uint4 w, uint4& h0, uint4& h1) {
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
  uint32_t o[8];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    float f0 = (float)(int8_t)(d[q] & 0xff), f1 = (float)(int8_t)((d[q] >> 8) & 0xff);
    float f2 = (float)(int8_t)((d[q] >> 16) & 0xff), f3 = (float)(int8_t)(d[q] >> 24);
    o[2 * q] = f16pair(f0, f1);
    o[2 * q + 1] = f16pair(f2, f3);
  }
  h0 = make_uint4(o[0], o[1], o[2], o[3]);
  h1 = make_uint4(o[4], o[5], o[6], o[7]);
}


// 16 consecutive 16-bit values of row m starting at k0 (zero outside [0,K))
__device__ inline void load_row16_b16(const uint16_t* A, int lda, int M, int K, int m, int k0,
                                      uint4& lo, uint4& hi) {
  lo = make_uint4(0, 0, 0, 0);
  hi = lo;
  if (m >= M) return;
  const uint16_t* p = A + (size_t)m * lda + k0;
  if (k0 + 16 <= K && ((((uintptr_t)p) & 15) == 0)) {
    lo = reinterpret_cast<const uint4*>(p)[0];
    hi = reinterpret_cast<const uint4*>(p)[1];
  } else {
    uint32_t v[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
      uint32_t e0 = (k0 + 2 * q < K) ? p[2 * q] : 0;
      uint32_t e1 = (k0 + 2 * q + 1 < K) ? p[2 * q + 1] : 0;
      v[q] = e0 | (e1 << 16);
    }
    lo = make_uint4(v[0], v[1], v[2], v[3]);
    hi = make_uint4(v[4], v[5], v[6], v[7]);
  }
}

__device__ inline void load_row16_f32(const float* A, int lda, int M, int K, int m, int k0, float* x) {
  if (m >= M) {
#pragma unroll
    for (int q = 0; q < 16; q++) x[q] = 0.f;
    return;
  }
  const float* p = A + (size_t)m * lda + k0;
  if (k0 + 16 <= K && ((((uintptr_t)p) & 15) == 0)) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      float4 v = reinterpret_cast<const float4*>(p)[q];
      x[4 * q] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int q = 0; q < 16; q++) x[q] = (k0 + q < K) ? p[q] : 0.f;
  }
}

// --------------------------------------------------------------------------
// epilogue
// --------------------------------------------------------------------------
__device__ inline void store_y(const GemmArgs& a, int m, int n, float v) {
  const size_t o = (size_t)m * a.ldy + n;
  if (a.out == OUT_F32) {
    reinterpret_cast<float*>(a.Y)[o] = v;
  } else if (a.out == OUT_BF16) {
    reinterpret_cast<uint16_t*>(a.Y)[o] = (uint16_t)f32_to_bf16_rne(v);
  } else {
    _Float16 h = (_Float16)v;
    reinterpret_cast<uint16_t*>(a.Y)[o] = __builtin_bit_cast(uint16_t, h);
  }
}

__device__ inline void epilogue_i(const GemmArgs& a, int m, int n, int acc) {
  if (m >= a.M || n >= a.N) return;
  if (a.out == OUT_I32) {
    reinterpret_cast<int32_t*>(a.Y)[(size_t)m * a.ldy + n] = acc;
    return;
  }
  float r = __fmul_rn(__fmul_rn((float)acc, a.ws[n]), a.xs[m]);
  if (a.bias) r = __fadd_rn(r, a.bias[n]);
  store_y(a, m, n, r);
}

__device__ inline void epilogue_f(const GemmArgs& a, int m, int n, float acc) {
  if (m >= a.M || n >= a.N) return;
  float r;
  if (a.ep == EP_SCALE_FMA) {
    r = __fmaf_rn(acc, a.ws[n], a.bias ? a.bias[n] : 0.0f);
  } else {
    r = __fmul_rn(acc, a.ws[n]);
    if (a.bias) r = __fadd_rn(r, a.bias[n]);
  }
  store_y(a, m, n, r);
}

// --------------------------------------------------------------------------
// kernel
// --------------------------------------------------------------------------
template <int AMODE, int TM, int TN, int WGM, int WGN>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
  static_assert(WGM * WGN == 4, "4 waves per work-group");
  constexpr bool INT = (AMODE == A_I8);
  typedef typename std::conditional<INT, v4i, v4f>::type acc_t;

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int wm = wv / WGN, wn = wv % WGN;
  const int tile = blockIdx.x / a.S;
  const int s = blockIdx.x - tile * a.S;
  const int tmi = tile / a.ntn, tni = tile - (tile / a.ntn) * a.ntn;
  const int mg0 = (tmi * WGM + wm) * TM;
  const int ng0 = (tni * WGN + wn) * TN;
  const int kb0 = (int)(((long long)s * a.KB) / a.S);
  const int kb1 = (int)(((long long)(s + 1) * a.KB) / a.S);

  acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = acc_t{0, 0, 0, 0};

  const uint4* Bt4 = reinterpret_cast<const uint4*>(a.Bt);
  const int row = lane & 15;
  const int kl = (lane >> 4) * 16;

  for (int kb = kb0; kb < kb1; kb++) {
    uint4 bw[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int ng = ng0 + j;
      bw[j] = (ng < a.NG) ? Bt4[((size_t)kb * a.NG + ng) * 64 + lane] : make_uint4(0, 0, 0, 0);
    }
    if constexpr (AMODE == A_I8) {
      const uint4* At4 = reinterpret_cast<const uint4*>(a.A);
      uint4 aw[TM];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int mg = mg0 + i;
        aw[i] = (mg < a.MG) ? At4[((size_t)kb * a.MG + mg) * 64 + lane] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, aw[i]),
                                                            __builtin_bit_cast(v4i, bw[j]),
                                                            acc[i][j], 0, 0, 0);
    } else if constexpr (AMODE == A_BF16 || AMODE == A_F16) {
      uint4 a0[TM], a1[TM];
#pragma unroll
      for (int i = 0; i < TM; i++)
        load_row16_b16(reinterpret_cast<const uint16_t*>(a.A), a.lda, a.M, a.K, (mg0 + i) * 16 + row,
                       kb * 64 + kl, a0[i], a1[i]);
#pragma unroll
      for (int j = 0; j < TN; j++) {
        uint4 h0, h1;
        if constexpr (AMODE == A_BF16) w_to_bf16(bw[j], h0, h1);
        else w_to_f16(bw[j], h0, h1);
#pragma unroll
        for (int i = 0; i < TM; i++) {
          if constexpr (AMODE == A_BF16) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(a0[i]), as_v8bf(h0), acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(a1[i]), as_v8bf(h1), acc[i][j], 0, 0, 0);
          } else {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_v8h(a0[i]), as_v8h(h0), acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_v8h(a1[i]), as_v8h(h1), acc[i][j], 0, 0, 0);
          }
        }
      }
    } else {  // A_F32X3
      uint4 t[TM][2][3];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        float x[16];
        load_row16_f32(reinterpret_cast<const float*>(a.A), a.lda, a.M, a.K, (mg0 + i) * 16 + row,
                       kb * 64 + kl, x);
        split3x8(x, t[i][0][0], t[i][0][1], t[i][0][2]);
        split3x8(x + 8, t[i][1][0], t[i][1][1], t[i][1][2]);
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        uint4 h[2];
        w_to_bf16(bw[j], h[0], h[1]);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int hh = 0; hh < 2; hh++) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(t[i][hh][2]), as_v8bf(h[hh]), acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(t[i][hh][1]), as_v8bf(h[hh]), acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(t[i][hh][0]), as_v8bf(h[hh]), acc[i][j], 0, 0, 0);
          }
      }
    }
  }

  const int col = lane & 15;
  const int r0 = (lane >> 4) * 4;
  if (a.S == 1) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = (mg0 + i) * 16 + r0 + r, n = (ng0 + j) * 16 + col;
          if constexpr (INT) epilogue_i(a, m, n, acc[i][j][r]);
          else epilogue_f(a, m, n, acc[i][j][r]);
        }
    return;
  }

  // ---- split-K: publish partials, last work-group reduces in order s = 0.. ----
  const size_t ldp = (size_t)a.NG * 16;
  const size_t slab = (size_t)a.MG * 16 * ldp;
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = (mg0 + i) * 16 + r0 + r, n = (ng0 + j) * 16 + col;
        if ((mg0 + i) < a.MG && (ng0 + j) < a.NG) {
          if constexpr (INT) reinterpret_cast<int32_t*>(a.part)[s * slab + m * ldp + n] = acc[i][j][r];
          else reinterpret_cast<float*>(a.part)[s * slab + m * ldp + n] = acc[i][j][r];
        }
      }
  __threadfence();
  __syncthreads();
  __shared__ uint32_t s_last;
  if (threadIdx.x == 0) s_last = atomicAdd(&a.cnt[tile], 1u);
  __syncthreads();
  if (s_last != (uint32_t)(a.S - 1)) return;
  __threadfence();
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = (mg0 + i) * 16 + r0 + r, n = (ng0 + j) * 16 + col;
        if ((mg0 + i) < a.MG && (ng0 + j) < a.NG) {
          if constexpr (INT) {
            int tot = 0;
            for (int q = 0; q < a.S; q++)
              tot += __hip_atomic_load(&reinterpret_cast<int32_t*>(a.part)[q * slab + m * ldp + n],
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            epilogue_i(a, m, n, tot);
          } else {
            float tot = 0.f;
            for (int q = 0; q < a.S; q++)
              tot += __hip_atomic_load(&reinterpret_cast<float*>(a.part)[q * slab + m * ldp + n],
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            epilogue_f(a, m, n, tot);
          }
        }
      }
  if (threadIdx.x == 0) atomicExch(&a.cnt[tile], 0u);
}

// --------------------------------------------------------------------------
// planning and launch
// --------------------------------------------------------------------------
// config ids: 0 small M (<= 16): TM=1,TN=2 over 1x4 waves  -> 16 x 128
//             1 medium (<= 64):  TM=2,TN=2 over 2x2 waves  -> 64 x 64
//             2 large:           TM=4,TN=4 over 2x2 waves  -> 128 x 128 (F32X3: TM=2 -> 64 x 128)
static void cfg_dims(int amode, int cfg, int& tm, int& tn, int& wgm, int& wgn) {
  if (cfg == 0) { tm = 1; tn = 2; wgm = 1; wgn = 4; }
  else if (cfg == 1) { tm = 2; tn = 2; wgm = 2; wgn = 2; }
  else { tm = (amode == A_F32X3) ? 2 : 4; tn = 4; wgm = 2; wgn = 2; }
}

GemmPlan gemm_plan(int amode, int M, int N, int K) {
  GemmPlan p;
  p.cfg = (M <= 16) ? 0 : (M <= 64 ? 1 : 2);
  int tm, tn, wgm, wgn;
  cfg_dims(amode, p.cfg, tm, tn, wgm, wgn);
  const int MG = cdiv(M, 16), NG = cdiv(N, 16), KB = cdiv(K, 64);
  p.ntm = cdiv(MG, tm * wgm);
  p.ntn = cdiv(NG, tn * wgn);
  const int tiles = p.ntm * p.ntn;
  int s = 1;
  const int target_blocks = 512;  // 2 work-groups per CU
  if (tiles < target_blocks) {
    s = cdiv(target_blocks, tiles);
    int max_s = KB / 2;
    if (max_s < 1) max_s = 1;
    if (s > max_s) s = max_s;
  }
  p.split = s;
  p.blocks = tiles * s;
  return p;
}

size_t gemm_workspace_bytes(int amode, int M, int N, int K) {
  GemmPlan p = gemm_plan(amode, M, N, K);
  if (p.split <= 1) return 0;
  return (size_t)p.split * cdiv(M, 16) * 16 * (size_t)cdiv(N, 16) * 16 * 4;
}

size_t gemm_counter_count(int amode, int M, int N, int K) {
  GemmPlan p = gemm_plan(amode, M, N, K);
  return (size_t)p.ntm * p.ntn;
}

template <int AMODE>
static hipError_t launch_mode(const GemmArgs& a, int cfg, int blocks, hipStream_t st) {
  if (cfg == 0)
    hipLaunchKernelGGL((gemm_kernel<AMODE, 1, 2, 1, 4>), dim3(blocks), dim3(256), 0, st, a);
  else if (cfg == 1)
    hipLaunchKernelGGL((gemm_kernel<AMODE, 2, 2, 2, 2>), dim3(blocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_kernel<AMODE, (AMODE == A_F32X3 ? 2 : 4), 4, 2, 2>), dim3(blocks), dim3(256), 0, st, a);
  return hipGetLastError();
}

// which kernel launch_gemm runs for L
enum GemmKernel { GK_SMALL, GK_I8, GK_B16, GK_GENERIC };
static GemmKernel gemm_choice(const GemmLaunch& L) {
  // up to 16 token rows always stream the weights once; more rows too while N
  // is small (N <= 4096: the tiled kernels would leave CUs idle), up to 64
  // int8 rows; for wide N the activation
  // fragments every work-group re-reads cost more than the tiled kernels' reuse,
  // except up to 32 int8 rows at lm_head width (>= 2048 row groups, four per
  // work-group share each fragment): the int8 planes of 5-8 fp32 tokens,
  // 81 -> 70 us for the lm_head at 8 tokens
  const bool b16 = L.amode == A_BF16 || L.amode == A_F16;
  if (b16) {   // tuning override: 3 the small-M kernel, 0..2 a tile of the tiled one
    const int fc = gemm_b16_forced_cfg();
    if (fc == 3 && gemm_small_supported(L)) return GK_SMALL;
    if (((fc >= 0 && fc <= 2) || fc >= 4) && L.M > 16 && gemm_b16_supported(L)) return GK_B16;
  }
  // 16-bit rows (the grid's y extent over the token groups): up to 256 rows at
  // N <= 4096 and 64 rows on wider N, measured at K = 2048 against every tile
  // of the tiled kernel (M = 96 / 128 / 192 / 256, N = 2048: 6.8 / 6.9 / 9.2 /
  // 9.3 us against 11.5 / 11.5 / 11.6 / 11.8; N = 4096: 9.4 / 9.5 / 14.9 /
  // 15.0 against 11.8 / 11.9 / 16.1 / 16.2; N = 12288 at 32 / 64 rows 10.3 /
  // 15.7 against 12.0 / 16.6; from 96 rows there the tiled kernel wins: 20.7
  // against 25.2 us)
  const int ng = cdiv(L.N, 16);
  const bool b16_small = b16 && L.M <= 256 && (ng <= 256 || L.M <= 64);
  const bool wide_i8 = L.amode == A_I8 && L.M <= 32 && ng >= 2048;
  // int8 codes and fp32 rows: up to 64 rows at N <= 6144 and 32 rows at
  // N <= 12288 (W8A8 at K = 2048, N = 6144, 24..64 rows: 8.1-11.0 us against
  // 12.7-13.7 us on the tiled kernel; N = 12288 at 24 / 32 rows 12.1 / 12.4
  // against 13.4, at 48 / 64 rows 15.4 / 16.3 against 14.2 / 14.4)
  const bool mid_i8 = !b16 && ((L.M <= 64 && ng <= 384) || (L.M <= 32 && ng <= 768));
  if (gemm_small_supported(L) && (L.M <= 16 || mid_i8 || b16_small || wide_i8))
    return GK_SMALL;
  if (L.amode == A_I8 && L.M > 16) return GK_I8;
  if (L.amode != A_I8 && L.M > 16 && gemm_b16_supported(L)) return GK_B16;
  return GK_GENERIC;
}

// split work-space of the kernel launch_gemm picks for L: partial-sum bytes
// and zeroed arrival counters (0 and 0 when it needs none)
void gemm_needs(const GemmLaunch& L, size_t* part_bytes, size_t* counters) {
  *part_bytes = 0;
  *counters = 0;
  switch (gemm_choice(L)) {
    case GK_SMALL: return;
    case GK_I8: gemm_i8_needs(L.M, L.N, L.K, part_bytes, counters); return;
    case GK_B16: gemm_b16_needs(L.M, L.N, L.K, part_bytes, counters); return;
    default: break;
  }
  GemmPlan p = gemm_plan(L.amode, L.M, L.N, L.K);
  if (L.force_split > 0) p.split = L.force_split;
  if (p.split > 1) {
    *part_bytes = (size_t)p.split * cdiv(L.M, 16) * 16 * (size_t)cdiv(L.N, 16) * 16 * 4;
    *counters = (size_t)p.ntm * p.ntn;
  }
}

hipError_t launch_gemm(const GemmLaunch& L, hipStream_t st) {
  GemmArgs a;
  a.A = L.A;
  a.lda = L.lda;
  a.Bt = L.Bt;
  a.ws = L.ws;
  a.xs = L.xs;
  a.bias = L.bias;
  a.Y = L.Y;
  a.ldy = L.ldy;
  a.M = L.M;
  a.N = L.N;
  a.K = L.K;
  a.KB = cdiv(L.K, 64);
  a.MG = cdiv(L.M, 16);
  a.NG = cdiv(L.N, 16);
  a.ep = L.ep;
  a.out = L.out;
  GemmPlan p = gemm_plan(L.amode, L.M, L.N, L.K);
  if (L.force_split > 0) {
    p.split = L.force_split;
    p.blocks = p.ntm * p.ntn * p.split;
  }
  a.S = p.split;
  a.ntn = p.ntn;
  a.part = L.part;
  a.cnt = L.cnt;
  if (L.amode == A_I8 && L.out != OUT_I32 && L.out != OUT_F32_X4 && !L.xs) return hipErrorInvalidValue;
  if (L.out == OUT_F32_X4 && L.amode != A_I8) return hipErrorInvalidValue;
  switch (gemm_choice(L)) {
    case GK_SMALL: return launch_gemm_small(L, st);
    case GK_I8: return launch_gemm_i8(L, st);
    case GK_B16: return launch_gemm_b16(L, st);
    default: break;
  }
  // the generic kernel's K split needs the work-space gemm_needs reports
  if (p.split > 1 && (!L.part || !L.cnt)) return hipErrorInvalidValue;
  switch (L.amode) {
    case A_I8: return launch_mode<A_I8>(a, p.cfg, p.blocks, st);
    case A_BF16: return launch_mode<A_BF16>(a, p.cfg, p.blocks, st);
    case A_F16: return launch_mode<A_F16>(a, p.cfg, p.blocks, st);
    case A_F32X3: return launch_mode<A_F32X3>(a, p.cfg, p.blocks, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tl

// ---------------------------------------------------------------------------
// C ABI of the launchers above (tl_kernels.h)
// ---------------------------------------------------------------------------
extern "C" {
void tlk_gemm_plan(int amode, int M, int N, int K, GemmPlan* plan) { *plan = tl::gemm_plan(amode, M, N, K); }
size_t tlk_gemm_workspace_bytes(int amode, int M, int N, int K) {
  return tl::gemm_workspace_bytes(amode, M, N, K);
}
size_t tlk_gemm_counter_count(int amode, int M, int N, int K) { return tl::gemm_counter_count(amode, M, N, K); }
hipError_t tlk_launch_gemm(const GemmLaunch* L, hipStream_t st) { return tl::launch_gemm(*L, st); }
void tlk_gemm_needs(const GemmLaunch* L, size_t* part_bytes, size_t* counters) {
  tl::gemm_needs(*L, part_bytes, counters);
}
void tlk_gemm_b16_set_plan(int cfg, int split) { tl::gemm_b16_set_plan(cfg, split); }
}  // extern "C"
