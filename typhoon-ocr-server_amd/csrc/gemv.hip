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
//   * weights are 16x64 tiles (tl_common.h); a wave streams the tiles of one
//     16-row group over a contiguous range of k-blocks with one 16-byte load
//     per lane per tile (1 KiB per wave-load, fully coalesced) and keeps two
//     batches of 8 tiles in flight (software pipeline);
//   * lane l accumulates row (l & 15) over the k slice of its lane group with
//     v_dot4_i32_i8; two xor-shuffles finish the row sums;
//   * a work-group has 4 waves = RPW row groups x (4/RPW) k-slices, reduced
//     through LDS; small N additionally splits K over S work-groups, whose
//     int32 partials are summed in a fixed order by the last work-group to
//     arrive (arrival counter in device memory, reset by that work-group, so
//     the counters are zero again when the kernel ends).  Integer sums make
//     every split bit-identical to the unsplit sum.
//
// Fused activation quantization (XV > 0): every work-group first issues its
// first batch of weight loads, then reads all of x (XV float4 per thread),
// reduces absmax, derives scale/inverse exactly as the reference
// (w8a32_kernel.c:145-158) and writes the int8 codes into LDS; the weight
// loads are in flight meanwhile.  XV == 0 takes precomputed codes from
// device memory (W8A8 batch==1, or K > 16384).
#include "tl_common.h"
#include "tl_kernels.h"

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
  int32_t* part;       // [S][NG*16] partial sums (S > 1)
  uint32_t* cnt;       // [NG] arrival counters, zero at rest
  int N, K, KB, NG, S, epi;
};

__device__ inline void gemv_epilogue(const GemvArgs& a, int n, int acc, float xs) {
  if (n >= a.N) return;
  if (a.epi == EPI_ACC) {
    a.acc_out[n] = acc;
  } else if (a.epi == EPI_W8A32) {
    float r = __fmul_rn(__fmul_rn((float)acc, a.ws[n]), xs);
    if (a.bias) r = __fadd_rn(r, a.bias[n]);
    a.y[n] = r;
  } else {
    float t = __fmul_rn((float)acc, a.ws[n]);
    a.y[n] = __fmaf_rn(t, xs, a.bias ? a.bias[n] : 0.0f);
  }
}

template <int RPW, int XV>
__global__ __launch_bounds__(256) void gemv_i8_kernel(GemvArgs a) {
  constexpr int U = 8;           // tiles per batch
  constexpr int KSW = 4 / RPW;   // waves per row group inside the work-group
  __shared__ uint4 s_codes[XV > 0 ? XV * 64 : 1];
  __shared__ uint32_t s_mx[4];
  __shared__ float s_tail[4];
  __shared__ int s_red[4][16];

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int lg = lane >> 4;
  const int blk = blockIdx.x / a.S;
  const int s = blockIdx.x - blk * a.S;
  const int g = blk * RPW + wv / KSW;
  const int ks = wv % KSW;
  const int T = a.S * KSW;
  const int j = s * KSW + ks;
  const int kb0 = (int)(((long long)j * a.KB) / T);
  const int kb1 = (int)(((long long)(j + 1) * a.KB) / T);
  const bool g_ok = g < a.NG;
  const int n_t = g_ok ? (kb1 - kb0) : 0;

  const uint4* wp = reinterpret_cast<const uint4*>(a.wt) + ((size_t)(g_ok ? g : 0) * a.KB + kb0) * 64 + lane;
  const uint4* cg = reinterpret_cast<const uint4*>(a.xq);

  uint4 b0[U], b1[U];
  uint4 c0[XV == 0 ? U : 1], c1[XV == 0 ? U : 1];
#pragma unroll
  for (int u = 0; u < U; u++)
    if (u < n_t) {
      b0[u] = wp[(size_t)u * 64];
      if constexpr (XV == 0) c0[u] = cg[(kb0 + u) * 4 + lg];
    }

  float xs;
  if constexpr (XV > 0) {
    // ---- fused per-token activation quantization --------------------------
    const int K = a.K;
    const int main_end = K & ~15;
    const bool vec = ((K & 3) == 0) && ((((uintptr_t)a.x) & 15) == 0);
    float4 xv[XV];
    uint32_t mx = 0;
    float tail = 0.0f;
#pragma unroll
    for (int i = 0; i < XV; i++) {
      const int k0 = 4 * (threadIdx.x + 256 * i);
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (vec && k0 + 3 < K) {
        v = *reinterpret_cast<const float4*>(a.x + k0);
      } else if (k0 < K) {
        v.x = a.x[k0];
        v.y = (k0 + 1 < K) ? a.x[k0 + 1] : 0.f;
        v.z = (k0 + 2 < K) ? a.x[k0 + 2] : 0.f;
        v.w = (k0 + 3 < K) ? a.x[k0 + 3] : 0.f;
      }
      xv[i] = v;
      if (k0 + 3 < main_end) {
        uint32_t m4 = max(max(abs_bits(v.x), abs_bits(v.y)), max(abs_bits(v.z), abs_bits(v.w)));
        mx = m4 > mx ? m4 : mx;
      } else {
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int k = k0 + q;
          if (k < main_end) {
            uint32_t m1 = abs_bits(e[q]);
            mx = m1 > mx ? m1 : mx;
          } else if (k < K) {
            float t = fabsf(e[q]);
            tail = (t > tail) ? t : tail;
          }
        }
      }
    }
    const float absmax = block_absmax_256(mx, tail, s_mx, s_tail);
    xs = quant_scale(absmax);
    const float inv = quant_inv(xs);
    uint32_t* sc = reinterpret_cast<uint32_t*>(s_codes);
#pragma unroll
    for (int i = 0; i < XV; i++) {
      const int k0 = 4 * (threadIdx.x + 256 * i);
      const float4 v = xv[i];
      sc[k0 >> 2] = pack4(code_at(v.x, inv, k0, K, false), code_at(v.y, inv, k0 + 1, K, false),
                          code_at(v.z, inv, k0 + 2, K, false), code_at(v.w, inv, k0 + 3, K, false));
    }
    if (blockIdx.x == 0 && threadIdx.x == 0 && a.xs_out) *a.xs_out = xs;
    __syncthreads();
  } else {
    xs = a.xs_in ? *a.xs_in : 1.0f;
  }

  // ---- main loop: two batches of U tiles in flight ---------------------------
  int acc = 0;
  for (int i = 0; i < n_t; i += 2 * U) {
#pragma unroll
    for (int u = 0; u < U; u++)
      if (i + U + u < n_t) {
        b1[u] = wp[(size_t)(i + U + u) * 64];
        if constexpr (XV == 0) c1[u] = cg[(kb0 + i + U + u) * 4 + lg];
      }
#pragma unroll
    for (int u = 0; u < U; u++)
      if (i + u < n_t) {
        uint4 c;
        if constexpr (XV > 0) c = s_codes[(kb0 + i + u) * 4 + lg];
        else c = c0[u];
        acc = dot16(b0[u], c, acc);
      }
#pragma unroll
    for (int u = 0; u < U; u++)
      if (i + 2 * U + u < n_t) {
        b0[u] = wp[(size_t)(i + 2 * U + u) * 64];
        if constexpr (XV == 0) c0[u] = cg[(kb0 + i + 2 * U + u) * 4 + lg];
      }
#pragma unroll
    for (int u = 0; u < U; u++)
      if (i + U + u < n_t) {
        uint4 c;
        if constexpr (XV > 0) c = s_codes[(kb0 + i + U + u) * 4 + lg];
        else c = c1[u];
        acc = dot16(b1[u], c, acc);
      }
  }

  // ---- reductions ------------------------------------------------------------
  acc += __shfl_xor(acc, 16, 64);
  acc += __shfl_xor(acc, 32, 64);
  if constexpr (KSW > 1) {
    if (lane < 16) s_red[wv][lane] = acc;
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int q = 1; q < KSW; q++) acc += s_red[wv + q][lane & 15];
    }
  }
  if (ks != 0 || !g_ok) return;

  const int n = g * 16 + (lane & 15);
  if (a.S == 1) {
    if (lane < 16) gemv_epilogue(a, n, acc, xs);
    return;
  }
  // split over work-groups: publish, count, last one reduces in fixed order
  const int stride = a.NG * 16;
  if (lane < 16) a.part[(size_t)s * stride + n] = acc;
  __threadfence();
  uint32_t old = 0;
  if (lane == 0) old = atomicAdd(&a.cnt[g], 1u);
  old = __shfl(old, 0, 64);
  if (old != (uint32_t)(a.S - 1)) return;
  __threadfence();
  if (lane < 16) {
    int tot = 0;
    for (int q = 0; q < a.S; q++)
      tot += __hip_atomic_load(&a.part[(size_t)q * stride + n], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    gemv_epilogue(a, n, tot, xs);
  }
  if (lane == 0) atomicExch(&a.cnt[g], 0u);
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
template <int RPW, int XV>
static void launch_rpw_xv(const GemvArgs& a, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((gemv_i8_kernel<RPW, XV>), dim3(blocks), dim3(256), 0, st, a);
}

template <int RPW>
static hipError_t launch_rpw(const GemvArgs& a, int xv, int blocks, hipStream_t st) {
  switch (xv) {
    case 0: launch_rpw_xv<RPW, 0>(a, blocks, st); break;
    case 2: launch_rpw_xv<RPW, 2>(a, blocks, st); break;
    case 4: launch_rpw_xv<RPW, 4>(a, blocks, st); break;
    case 6: launch_rpw_xv<RPW, 6>(a, blocks, st); break;
    case 8: launch_rpw_xv<RPW, 8>(a, blocks, st); break;
    case 16: launch_rpw_xv<RPW, 16>(a, blocks, st); break;
    default: return hipErrorInvalidValue;
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

GemvPlan gemv_plan(int N, int K) {
  GemvPlan p;
  const int NG = cdiv(N, 16);
  const int KB = cdiv(K, 64);
  const int target_waves = 2048;  // 8 per CU on 256 CUs
  if (NG >= 2048) {
    p.rpw = 4;
    p.split = 1;
  } else if (NG >= 512) {
    p.rpw = 2;
    p.split = 1;
  } else {
    p.rpw = 1;
    int waves = NG * 4;
    int s = cdiv(target_waves, waves);
    int max_s = KB / 4;            // at least one tile per wave
    if (max_s < 1) max_s = 1;
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    p.split = s;
  }
  p.blocks = cdiv(NG, p.rpw) * p.split;
  return p;
}

size_t gemv_workspace_bytes(int N, int K) {
  GemvPlan p = gemv_plan(N, K);
  if (p.split <= 1) return 0;
  const size_t ng = (size_t)cdiv(N, 16);
  return ng * 16 * p.split * sizeof(int32_t);
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
  GemvPlan p = gemv_plan(L.N, L.K);
  if (L.force_split > 0) {
    p.split = L.force_split;
    p.blocks = cdiv(a.NG, p.rpw) * p.split;
  }
  a.S = p.split;
  a.part = L.part;
  a.cnt = L.cnt;
  if (p.split > 1 && (!L.part || !L.cnt)) return hipErrorInvalidValue;
  const int xv = L.x ? gemv_fused_xv(L.K) : 0;
  if (L.x && xv == 0) return hipErrorInvalidValue;  // caller must quantize first
  if (!L.x && !L.xq) return hipErrorInvalidValue;
  switch (p.rpw) {
    case 1: return launch_rpw<1>(a, xv, p.blocks, st);
    case 2: return launch_rpw<2>(a, xv, p.blocks, st);
    case 4: return launch_rpw<4>(a, xv, p.blocks, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tl
