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
//     batches of U tiles in flight (software pipeline, U in {2, 4, 8} picked
//     so that the wave's tiles form whole batches); the loop body is
//     branch-free, tail tiles are read from a clamped address and masked;
//   * lane l accumulates row (l & 15) over the k slice of its lane group with
//     v_dot4_i32_i8; two xor-shuffles finish the row sums;
//   * a work-group has 4 waves = (4/KSW) row groups x KSW k-slices, reduced
//     through LDS; small N additionally splits K over S work-groups, whose
//     int32 partials are summed in a fixed order by the last work-group to
//     arrive (arrival counter in device memory, reset by that work-group, so
//     the counters are zero again when the kernel ends).  Integer sums make
//     every split bit-identical to the unsplit sum.
//
// Fused activation quantization (XV > 0): every work-group first issues the
// loads of x and of its first two batches of weight tiles, then reduces all of
// x (XV float4 per thread),
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
  int ksw;             // waves per row group in a work-group (1, 2, 4)
  int x_vec;           // 2: K == 1024*XV and x 16-byte aligned (unguarded loads)
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

// acc += dot(tile, codes) for U tiles starting at wave-local tile index t0;
// tiles at or beyond n_t were loaded from a clamped address and are dropped.
template <int XV, int U>
__device__ inline int consume_batch(const uint4 (&b)[U], const uint4 (&c)[XV == 0 ? U : 1],
                                    const uint4* s_codes, int kb0, int t0, int n_t, int lg, int acc) {
  uint4 cv[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    if constexpr (XV > 0) cv[u] = s_codes[(kb0 + min(t0 + u, n_t - 1)) * 4 + lg];
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
__device__ inline void load_batch(uint4 (&b)[U], uint4 (&c)[XV == 0 ? U : 1], const uint4* wp,
                                  size_t tstride, const uint4* cg, int kb0, int t0, int n_t, int lg) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int t = min(t0 + u, n_t - 1);
    b[u] = wp[(size_t)t * tstride];
    if constexpr (XV == 0) c[u] = cg[(kb0 + t) * 4 + lg];
  }
  // keep the batch issued here, ahead of the consumption that follows
  __builtin_amdgcn_sched_barrier(0);
}

template <int XV, int U>
__global__ __launch_bounds__(256) void gemv_i8_kernel(GemvArgs a) {
  __shared__ uint4 s_codes[XV > 0 ? XV * 64 : 1];
  __shared__ uint32_t s_mx[4];
  __shared__ float s_tail[4];
  __shared__ int s_red[4][16];

  const int KSW = a.ksw;                  // waves per row group (1, 2 or 4)
  const int RPW = 4 / KSW;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
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
  const int n_t = kb1 - kb0;              // >= 1 (host keeps T <= KB)
  const int gl = g_ok ? g : a.NG - 1;     // out-of-range row groups re-read a valid one

  const uint4* wp = reinterpret_cast<const uint4*>(a.wt) + ((size_t)kb0 * a.NG + gl) * 64 + lane;
  const size_t tstride = (size_t)a.NG * 64;   // uint4 between consecutive k-blocks
  const uint4* cg = reinterpret_cast<const uint4*>(a.xq);

  uint4 b0[U], b1[U];
  uint4 c0[XV == 0 ? U : 1], c1[XV == 0 ? U : 1];

  // x is read before the first weight batch is issued, so the wait for x
  // never waits for weights
  float4 xv[XV > 0 ? XV : 1];
  if constexpr (XV > 0) {
    const int K = a.K;
    if (a.x_vec == 2) {
      // K == 1024 * XV and x 16-byte aligned: XV unconditional float4 loads
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
  load_batch<XV, U>(b0, c0, wp, tstride, cg, kb0, 0, n_t, lg);
  load_batch<XV, U>(b1, c1, wp, tstride, cg, kb0, U, n_t, lg);

  float xs;
  if constexpr (XV > 0) {
    // ---- fused per-token activation quantization --------------------------
    const int K = a.K;
    const int main_end = K & ~15;
    uint32_t mx = 0;
    float tail = 0.0f;
#pragma unroll
    for (int i = 0; i < XV; i++) {
      const int k0 = 4 * (threadIdx.x + 256 * i);
      const float4 v = xv[i];
      const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int k = k0 + q;
        const uint32_t m1 = (k < main_end) ? abs_bits(e[q]) : 0u;
        mx = m1 > mx ? m1 : mx;
        const float t1 = (k >= main_end && k < K) ? fabsf(e[q]) : 0.0f;
        tail = (t1 > tail) ? t1 : tail;
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
  // Both batches were issued before the prologue.  The loop body is
  // straight-line code that enters and leaves with the 2U loads of b0 and b1
  // outstanding, so the compiler keeps the wait counts exact.
  int acc = 0;
  int t = 0;
  for (; t + 2 * U < n_t; t += 2 * U) {
    acc = consume_batch<XV, U>(b0, c0, s_codes, kb0, t, n_t, lg, acc);
    load_batch<XV, U>(b0, c0, wp, tstride, cg, kb0, t + 2 * U, n_t, lg);
    acc = consume_batch<XV, U>(b1, c1, s_codes, kb0, t + U, n_t, lg, acc);
    load_batch<XV, U>(b1, c1, wp, tstride, cg, kb0, t + 3 * U, n_t, lg);
  }
  acc = consume_batch<XV, U>(b0, c0, s_codes, kb0, t, n_t, lg, acc);
  acc = consume_batch<XV, U>(b1, c1, s_codes, kb0, t + U, n_t, lg, acc);

  // ---- reductions ------------------------------------------------------------
  acc += __shfl_xor(acc, 16, 64);
  acc += __shfl_xor(acc, 32, 64);
  if (KSW > 1) {
    if (lane < 16) s_red[wv][lane] = acc;
    __syncthreads();
    if (ks == 0) {
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
template <int XV, int U>
static void launch_xv_u(const GemvArgs& a, int blocks, hipStream_t st) {
  hipLaunchKernelGGL((gemv_i8_kernel<XV, U>), dim3(blocks), dim3(256), 0, st, a);
}

template <int XV>
static hipError_t launch_xv(const GemvArgs& a, int u, int blocks, hipStream_t st) {
  switch (u) {
    case 2: launch_xv_u<XV, 2>(a, blocks, st); break;
    case 4: launch_xv_u<XV, 4>(a, blocks, st); break;
    case 8: launch_xv_u<XV, 8>(a, blocks, st); break;
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

// batch depth: the largest of {8, 4, 2} that splits the wave's tiles into an
// even number of whole batches (no redundant loads), else the smallest waste
static int pick_u(int n_t) {
  for (int u : {8, 4, 2})
    if (n_t % (2 * u) == 0) return u;
  int best = 2, waste = 1 << 30;
  for (int u : {8, 4, 2}) {
    int w = (2 * u - n_t % (2 * u)) % (2 * u);
    if (w < waste) { waste = w; best = u; }
  }
  return best;
}

static int g_force_ksw = 0, g_force_split = 0, g_force_u = 0;

void gemv_set_plan(int ksw, int split, int u) {
  g_force_ksw = ksw;
  g_force_split = split;
  g_force_u = u;
}

static GemvPlan planner(int N, int K);

// the planner's choice with the process-wide tuning override applied
GemvPlan gemv_plan(int N, int K) {
  GemvPlan p = planner(N, K);
  const int NG = cdiv(N, 16), KB = cdiv(K, 64);
  if (g_force_ksw > 0 || g_force_split > 0) {
    const int ksw = g_force_ksw > 0 ? g_force_ksw : p.ksw;
    const int split = g_force_split > 0 ? g_force_split : p.split;
    if (ksw * split <= KB) {
      p.ksw = ksw;
      p.split = split;
      p.blocks = cdiv(NG, 4 / ksw) * split;
      p.u = pick_u(cdiv(KB, ksw * split));
    }
  }
  if (g_force_u > 0) p.u = g_force_u;
  return p;
}

// Measured on MI355X (graph-replayed launches over > 512 MB of rotating
// weights): one 16-row group per work-group with K split over its 4 waves is
// fastest for every decode shape, including the 151936-row lm_head; splitting
// K across work-groups (fence + counter reduction) was 1.5-2.5x slower for
// N <= 4096.  U = 4: both batches (8 tiles per wave at K = 2048) are in
// flight before the activation prologue; at K = 6144 the 24 tiles form 3
// exact double batches.
static GemvPlan planner(int N, int K) {
  GemvPlan p;
  const int NG = cdiv(N, 16);
  const int KB = cdiv(K, 64);
  p.ksw = KB >= 4 ? 4 : (KB >= 2 ? 2 : 1);
  p.split = 1;
  p.blocks = cdiv(NG, 4 / p.ksw);
  const int n_t = cdiv(KB, p.ksw);
  p.u = n_t >= 4 ? 4 : 2;
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
  a.x_vec = 0;
  GemvPlan p = gemv_plan(L.N, L.K);
  if (L.force_ksw > 0) p.ksw = L.force_ksw;
  if (L.force_split > 0) p.split = L.force_split;
  if (L.force_ksw > 0 || L.force_split > 0) {
    if (p.ksw * p.split > a.KB) return hipErrorInvalidValue;
    p.blocks = cdiv(a.NG, 4 / p.ksw) * p.split;
    p.u = pick_u(cdiv(a.KB, p.ksw * p.split));
  }
  if (L.force_u > 0) p.u = L.force_u;
  a.ksw = p.ksw;
  a.S = p.split;
  a.part = L.part;
  a.cnt = L.cnt;
  if (p.split > 1 && (!L.part || !L.cnt)) return hipErrorInvalidValue;
  const int xv = L.x ? gemv_fused_xv(L.K) : 0;
  if (L.x && xv == 0) return hipErrorInvalidValue;  // caller must quantize first
  if (L.x && L.K == 1024 * xv && (((uintptr_t)L.x) & 15) == 0) a.x_vec = 2;
  if (!L.x && !L.xq) return hipErrorInvalidValue;
  switch (xv) {
    case 0: return launch_xv<0>(a, p.u, p.blocks, st);
    case 2: return launch_xv<2>(a, p.u, p.blocks, st);
    case 4: return launch_xv<4>(a, p.u, p.blocks, st);
    case 6: return launch_xv<6>(a, p.u, p.blocks, st);
    case 8: return launch_xv<8>(a, p.u, p.blocks, st);
    case 16: return launch_xv<16>(a, p.u, p.blocks, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tl
