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
//   * weights are 16x64 tiles (tl_common.h).  A work-group (4 waves) owns RH
//     rows (16, or 8 = half a tile's rows); wave w streams k-blocks
//     [w*KB/4, (w+1)*KB/4) with one 16-byte load per lane per instruction
//     (1 KiB per wave-load, whole 128-byte lines), two batches of U load
//     instructions in flight; the loop body is branch-free, tail k-blocks are
//     read from a clamped address and masked;
//   * each lane accumulates one row over a 16-wide k sub-slice of a k-block
//     with v_dot4_i32_i8; the partial sums of a row (lane slots x 4 waves)
//     meet in LDS and are added in a fixed order.  Integer sums make every
//     decomposition bit-identical to the sequential sum.
//   * the decode shapes are latency-bound: U is chosen so that both batches
//     hold all of a wave's loads whenever that fits, so every weight load is
//     issued in the wave's first instructions; 8-row work-groups put every CU
//     to work when N has fewer than 256 tile rows.
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

constexpr int kNpNormStride = 136;   // LDS floats per 128-block of the final RMSNorm's squares

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
  uint64_t* keys;      // EPI_ARGMAX: per-work-group keys
  const float* norm_w; // RMSNorm weights (norm)
  float norm_eps;
  int norm;            // NORM_*
  int N, K, KB, NG, epi;
  int x_vec;           // 2: K == 1024*XV and x aligned to 4 elements (unguarded loads)
  int x_type = 0;      // EPI_W8A16: 0 fp32, 1 bf16, 2 fp16
  int out = OUT_F32;   // EPI_W8A16: output type
  int ntok = 1;        // EPI_W8A32_ROWS: token rows
};

// fp32 outputs go out as device-scope write-through stores (st_agent): the
// next launch of a decode step reads them on every XCD, and a plain store
// would leave the line dirty in this XCD's L2 for the kernel-end write-back
// (28-layer greedy decode 1,161 -> 1,190 tok/s, tokens identical; the
// linear benchmark's step unchanged)
__device__ __forceinline__ void gemv_epilogue(const GemvArgs& a, int n, int acc, float xs,
                                              float wsv, float bv) {
  if (a.epi == EPI_ACC) {
    a.acc_out[n] = acc;
  } else if (a.epi == EPI_W8A32) {
    float r = __fmul_rn(__fmul_rn((float)acc, wsv), xs);
    if (a.bias) r = __fadd_rn(r, bv);
    st_agent(a.y + n, r);
  } else {
    const float t = __fmul_rn((float)acc, wsv);
    st_agent(a.y + n, __fmaf_rn(t, xs, bv));
  }
}

// Per-lane view of the weight stream.  RH rows per work-group:
//   RH == 16: one 16x64 tile per load instruction, lane l = tile lane l;
//   RH == 8 : rows 8h..8h+7 of two consecutive k-blocks per load instruction
//             (lanes 0-31: k-block kb, lanes 32-63: kb + 1); within a k-block
//             lane j reads tile lane 16 (j >> 3 & 3) + 8h + (j & 7), so each 8
//             consecutive lanes read one 128-byte line.
template <int RH>
struct WStream {
  static constexpr int KPI = 16 / RH;   // k-blocks per load instruction
  const uint4* base;                    // tile lane of this lane in k-block 0
  size_t tstride;                       // uint4 between consecutive k-blocks
  int kb0, kb1, kbmax, sub;
  __device__ __forceinline__ int kb_of(int i) const { return kb0 + i * KPI + sub; }
  __device__ __forceinline__ int kb_clamped(int i) const { return min(kb_of(i), kbmax); }
};

// acc[p] += dot(tiles, codes of row p) for U load instructions starting at
// i0 (NP = 1 code row, or the 4 digit rows of the plane mode, each XV KiB of
// LDS); k-blocks at or beyond kb1 were loaded from a clamped address and are
// dropped.
template <int XV, int U, int RH, int NP>
__device__ __forceinline__ void consume_batch(const uint4 (&b)[U], const uint4 (&c)[XV == 0 ? U : 1],
                                              const uint4* s_codes, const WStream<RH>& ws, int i0, int lg,
                                              int (&acc)[NP]) {
  uint4 cv[U][NP];
#pragma unroll
  for (int u = 0; u < U; u++)
#pragma unroll
    for (int p = 0; p < NP; p++) {
      if constexpr (XV > 0) cv[u][p] = s_codes[p * XV * 64 + ws.kb_clamped(i0 + u) * 4 + lg];
      else cv[u][p] = c[u];
    }
#pragma unroll
  for (int u = 0; u < U; u++)
#pragma unroll
    for (int p = 0; p < NP; p++) {
      const int d = dot16(b[u], cv[u][p], 0);
      acc[p] += (ws.kb_of(i0 + u) < ws.kb1) ? d : 0;
    }
}

// Digit-row modes (NP = 4..16 code rows, XV > 0): NM int8 MFMAs per load
// instruction instead of NP LDS reads and 4 NP v_dot4 per lane.  The weight
// load is the MFMA's second operand as it stands.  RH == 16: lane l holds
// tile lane l (row l & 15, 16-byte k slice l >> 4), the operand layout
// itself; the first operand is code row l & 15 at the lane's own k slice
// (zero rows from NP up), and C[code row][weight row] is the dot product.
// RH == 8: lane l holds weight row 8h + (l & 7) at k-block kb + (l >> 5),
// slice (l >> 3) & 3, while the MFMA pairs lane 16 s + i of the first operand
// with lane 16 s + j of the second: virtual rows j and j + 8 are the same
// weight row over the two complementary halves of the k slices.  With code
// row l & 7 at the lane's own (k-block, slice), C[i][j] with i >> 3 == j >> 3
// is code row i & 7 times weight row j & 7 over one half, and
// C[i][j] + C[i + 8][j + 8] the whole dot product (the other entries mix
// halves and are ignored); 16 code rows take two MFMAs, rows 0-7 and 8-15.
// K-blocks at or past kb1 (clamped loads) and code rows past NP contribute
// zero operands, so the int32 sums equal the v_dot4 sums bit for bit.
template <int RH, int NP>
constexpr int gemv_nm() { return RH == 16 ? (NP + 15) / 16 : (NP + 7) / 8; }

template <int XV, int U, int RH, int NP>
__device__ __forceinline__ void consume_batch_mfma(const uint4 (&b)[U], const uint4* s_codes, const WStream<RH>& ws,
                                                   int i0, int lg, int lane, v4i (&acc)[gemv_nm<RH, NP>()]) {
  constexpr int NM = gemv_nm<RH, NP>();
#pragma unroll
  for (int mm = 0; mm < NM; mm++) {
    const int crow = RH * mm + (lane & (RH - 1));
    uint4 cv[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      // unconditional LDS read (clamped row), then a mask: a select around
      // the load would become a branch
      const uint4 c = s_codes[min(crow, NP - 1) * XV * 64 + ws.kb_clamped(i0 + u) * 4 + lg];
      const uint32_t m = (crow < NP && ws.kb_of(i0 + u) < ws.kb1) ? 0xffffffffu : 0u;
      cv[u] = make_uint4(c.x & m, c.y & m, c.z & m, c.w & m);
    }
#pragma unroll
    for (int u = 0; u < U; u++)
      acc[mm] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, cv[u]), __builtin_bit_cast(v4i, b[u]),
                                                      acc[mm], 0, 0, 0);
  }
}

template <int XV, int U, int RH>
__device__ __forceinline__ void load_batch(uint4 (&b)[U], uint4 (&c)[XV == 0 ? U : 1], const WStream<RH>& ws,
                                           const uint4* cg, int i0, int lg) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int kb = ws.kb_clamped(i0 + u);
    {
      // the weight stream is read once per launch: non-temporal (streaming)
      // loads, which keep it from displacing what later launches reuse from
      // L2 (activations, the KV cache); lm_head 52.6 -> 46.6 us, the
      // 28-layer decoder step 0.519 -> 0.492 ms
      typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
      const v4u_t t = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(ws.base + (size_t)kb * ws.tstride));
      b[u] = make_uint4(t.x, t.y, t.z, t.w);
    }
    if constexpr (XV == 0) c[u] = cg[kb * 4 + lg];
  }
  // keep the batch issued here, ahead of the consumption that follows
  __builtin_amdgcn_sched_barrier(0);
}

// Final RMSNorm of the hidden row held in xv (K == 1024 XV, a power of two),
// in numpy's float32 order (the same arithmetic as rmsnorm_np_kernel in
// lmhead.hip, decoder.py:444-446): squares through LDS, accumulator j of
// 128-block b folds x[128b + 8i + j]^2 over i in order, xor butterflies
// combine the 8 accumulators of a block and the 8 blocks of a wave, every
// thread finishes the balanced tree over the groups of 8 blocks itself.
// Then x = fl(fl(x / rms) * w).  Uses the dynamic LDS of the launch
// (kNpNormStride floats per 128-block: the 8-float pad puts the 64 lanes of a
// fold step, 8 blocks x 8 accumulators, on 64 distinct banks).
template <int XV>
__device__ void final_rmsnorm(float4 (&xv)[XV], const float4 (&nwv)[XV], bool has_w, int K, float eps) {
  extern __shared__ float s_sq[];
  __shared__ float s_grp[16];
#pragma unroll
  for (int i = 0; i < XV; i++) {
    const float4 v = xv[i];
    const int e = 4 * (threadIdx.x + 256 * i);        // element index, a multiple of 4
    *reinterpret_cast<float4*>(s_sq + kNpNormStride * (e >> 7) + (e & 127)) =
        make_float4(__fmul_rn(v.x, v.x), __fmul_rn(v.y, v.y), __fmul_rn(v.z, v.z), __fmul_rn(v.w, v.w));
  }
  __syncthreads();
  const int nb = K >> 7, ngrp = nb >> 3;     // K >= 1024 here: whole groups of 8 blocks
  for (int base = 0; base < 64 * ngrp; base += 256) {
    const int p = base + threadIdx.x;
    const int b = p >> 3, j = p & 7;
    float r = 0.0f;
    if (b < nb) {
      const float* src = s_sq + kNpNormStride * b + j;
      r = src[0];
#pragma unroll
      for (int i = 1; i < 16; i++) r = __fadd_rn(r, src[8 * i]);
    }
    // xor butterflies over lanes 1, 2, 4, 8 then 16, 32: numpy's order.  The
    // DPP quad permutes and row mirrors of wave_sum meet the same partner
    // values (each step's inputs are uniform over the previous step's group)
    // and its (r0 + r1) + (r2 + r3) is the last two steps, so the bits agree.
    r = wave_sum(r);
    if ((threadIdx.x & 63) == 0 && (p >> 6) < ngrp) s_grp[p >> 6] = r;
  }
  __syncthreads();
  float gsum[16];
#pragma unroll
  for (int i = 0; i < 16; i++) gsum[i] = i < ngrp ? s_grp[i] : 0.0f;
#pragma unroll
  for (int wdt = 1; wdt < 16; wdt <<= 1)
#pragma unroll
    for (int i = 0; i < 16; i += 2 * wdt)
      if (i + wdt < ngrp) gsum[i] = __fadd_rn(gsum[i], gsum[i + wdt]);
  const float mean = __fdiv_rn(gsum[0], (float)K);
  const float rms = sqrtf(__fadd_rn(mean, eps));   // correctly rounded (see lmhead.hip)
#pragma unroll
  for (int i = 0; i < XV; i++) {
    float4 v = xv[i];
    v.x = __fdiv_rn(v.x, rms);
    v.y = __fdiv_rn(v.y, rms);
    v.z = __fdiv_rn(v.z, rms);
    v.w = __fdiv_rn(v.w, rms);
    if (has_w) {
      v.x = __fmul_rn(v.x, nwv[i].x);
      v.y = __fmul_rn(v.y, nwv[i].y);
      v.z = __fmul_rn(v.z, nwv[i].z);
      v.w = __fmul_rn(v.w, nwv[i].w);
    }
    xv[i] = v;
  }
}

// The decoder's RMSNorm of the hidden row held in xv (kernel/ops.c:22-56):
// rms_sq = sum(x^2) / K + eps, r = FRSQRTE(rms_sq) refined by two FRSQRTS
// Newton steps, x = fl(fl(x * r) * w).  The reference sums the squares with
// four sequential fused chains; the sum here is a tree (fused squares per
// thread, DPP and LDS across the work-group), so rms_sq can differ in its
// last bits: parity with the reference is by tolerance.
template <int XV>
__device__ void decoder_rmsnorm(float4 (&xv)[XV], const float4 (&nwv)[XV], bool has_w, int K, float eps) {
  __shared__ float s_part[4];
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < XV; i++) {
    sq = __fmaf_rn(xv[i].x, xv[i].x, sq);
    sq = __fmaf_rn(xv[i].y, xv[i].y, sq);
    sq = __fmaf_rn(xv[i].z, xv[i].z, sq);
    sq = __fmaf_rn(xv[i].w, xv[i].w, sq);
  }
  sq = wave_sum(sq);
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = sq;
  __syncthreads();
  const float tot = __fadd_rn(__fadd_rn(s_part[0], s_part[1]), __fadd_rn(s_part[2], s_part[3]));
  const float r = ref_rsqrt(__fadd_rn(__fdiv_rn(tot, (float)K), eps));
#pragma unroll
  for (int i = 0; i < XV; i++) {
    float4 v = xv[i];
    v.x = __fmul_rn(v.x, r);
    v.y = __fmul_rn(v.y, r);
    v.z = __fmul_rn(v.z, r);
    v.w = __fmul_rn(v.w, r);
    if (has_w) {
      v.x = __fmul_rn(v.x, nwv[i].x);
      v.y = __fmul_rn(v.y, nwv[i].y);
      v.z = __fmul_rn(v.z, nwv[i].z);
      v.w = __fmul_rn(v.w, nwv[i].w);
    }
    xv[i] = v;
  }
}

// 4 activations at k of a row of fp32 (xt 0), bf16 (1) or fp16 (2), as fp32
__device__ __forceinline__ float4 gemv_x4(const float* x, int xt, int k) {
  if (xt == 0) return *reinterpret_cast<const float4*>(x + k);
  const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(x) + k);
  if (xt == 1)
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
  return make_float4((float)__builtin_bit_cast(_Float16, (uint16_t)(u.x & 0xffff)),
                     (float)__builtin_bit_cast(_Float16, (uint16_t)(u.x >> 16)),
                     (float)__builtin_bit_cast(_Float16, (uint16_t)(u.y & 0xffff)),
                     (float)__builtin_bit_cast(_Float16, (uint16_t)(u.y >> 16)));
}
__device__ __forceinline__ float gemv_x1(const float* x, int xt, int k) {
  if (xt == 0) return x[k];
  const uint16_t h = reinterpret_cast<const uint16_t*>(x)[k];
  return xt == 1 ? __uint_as_float((uint32_t)h << 16) : (float)__builtin_bit_cast(_Float16, h);
}

// Arguments are scalars so that the leading ones (through `flags`) are
// preloaded into SGPRs at wave launch (kernarg preload, -amdgpu-kernarg-
// preload-count in the build): the first loads need no kernarg fetch.
// flags: bits 0-1 x_vec, bits 2-4 epilogue, bit 5 bias present, bits 6-7
// RMSNorm of x first (NORM_*; K == 1024 XV a power of two, x_vec 2); plane
// mode (PL, EPI_W8A16): bits 8-9 x type (0 fp32, 1 bf16, 2 fp16), bits 10-11
// output type (OUT_F32, OUT_BF16, OUT_F16); token rows (PL >= 2,
// EPI_W8A32_ROWS): bits 12-14 their number.
//
// Plane mode: x (any of the three types, held as fp32) becomes four int8
// digit rows in LDS (digit_word / digit_planes: the row's absmax exponent
// e, q = x 2^(30-e) truncated), every weight load meets them in int8 MFMAs
// (consume_batch_mfma), and y = fma(2^(e-6) t, ws, bias) with t the digit
// sums' Horner combination: fp32-accurate products (w8a16_linear batch 1,
// kernel/w8a16_kernel.c:90-182) on the GEMV's weight stream.  PL == 2 and 4
// take up to that many fp32 token rows (x [ntok][K]) as four digit rows per
// token with the token's own e, and store y[t][n] = 2^(e_t - 6) fl(t_t ws)
// (+ bias as its own rounding): w8a32_linear at batch 2..4
// (kernel/w8a32_kernel.c:297-350, fp32 semantics) on the weight stream of
// batch 1, one weight read for every token.  Token slots past ntok repeat
// the last row; their outputs are not stored.
template <int XV, int U, int RH, int PL>
__global__ __launch_bounds__(256) void gemv_i8_kernel(const float* x, const uint8_t* wt, const float* ws,
                                                      float* y, int N, int K, int NG, int KB, int flags,
                                                      const uint8_t* xq, const float* xs_in, const float* bias,
                                                      int32_t* acc_out, float* xs_out, uint64_t* keys,
                                                      const float* norm_w, float norm_eps) {
  constexpr int SL = 64 / RH;           // lanes per row within a wave
  GemvArgs a;
  a.x = x;
  a.xq = xq;
  a.xs_in = xs_in;
  a.wt = wt;
  a.ws = ws;
  a.bias = (flags & 32) ? bias : nullptr;
  a.y = y;
  a.acc_out = acc_out;
  a.xs_out = xs_out;
  a.keys = keys;
  a.norm_w = norm_w;
  a.norm_eps = norm_eps;
  a.norm = (flags >> 6) & 3;
  a.N = N;
  a.K = K;
  a.KB = KB;
  a.NG = NG;
  a.epi = (flags >> 2) & 7;
  a.x_vec = flags & 3;
  constexpr int NTOK = PL >= 2 ? PL : 1; // token slots of x
  constexpr int NP = PL ? 4 * NTOK : 1;  // code rows: the activation codes, or 4 digit rows per token
  static_assert(NP <= 16, "at most 16 code rows");
  const int xt = PL == 1 ? (flags >> 8) & 3 : 0;
  const int ntok = PL >= 2 ? (flags >> 12) & 7 : 1;   // token rows of x and y
  __shared__ uint4 s_codes[XV > 0 ? XV * 64 * NP : 1];
  __shared__ uint32_t s_mx[4 * NTOK];
  __shared__ float s_tail[4];
  __shared__ int s_red[PL ? 1 : NP][PL ? 1 : RH * 4 * SL];
  __shared__ int s_redp[PL ? NP : 1][RH][4];   // digit-row modes: [code row][weight row][wave]

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // k slice of this wave
  const int r = lane % RH;              // row of this lane within the work-group
  const int slot = lane / RH;           // 0 .. SL-1
  const int lg = slot & 3;              // 16-wide k sub-slice of the tile
  const int row0 = blockIdx.x * RH;
  WStream<RH> st;
  {
    const int g16 = row0 >> 4, h = (row0 >> 3) & 1;
    const int lane_off = (RH == 16) ? lane : (lg * 16 + 8 * h + r);
    st.kb0 = (wv * KB) >> 2;
    st.kb1 = ((wv + 1) * KB) >> 2;
    st.kbmax = st.kb1 > st.kb0 ? st.kb1 - 1 : st.kb0;   // < KB always
    st.sub = slot >> 2;
    st.tstride = (size_t)NG * 64;
    st.base = reinterpret_cast<const uint4*>(wt) + (size_t)g16 * 64 + lane_off;
  }
  const int n_i = (st.kb1 - st.kb0 + WStream<RH>::KPI - 1) / WStream<RH>::KPI;
  const uint4* cg = reinterpret_cast<const uint4*>(a.xq);

  uint4 b0[U], b1[U];
  uint4 c0[XV == 0 ? U : 1], c1[XV == 0 ? U : 1];

  // x is read before the first weight batch is issued, so the wait for x
  // never waits for weights
  float4 xv[XV > 0 ? XV : 1];
  float4 xvt[NTOK > 1 ? NTOK - 1 : 1][XV > 0 ? XV : 1];     // token slots 1.. (PL >= 2)
  float4 nwv[XV > 0 ? XV : 1];
  const bool norm = ((flags >> 6) & 3) != NORM_NONE;   // x is a hidden row to normalise first
  if constexpr (XV > 0) {
    if (a.x_vec == 2) {
#pragma unroll
      for (int i = 0; i < XV; i++) xv[i] = gemv_x4(a.x, xt, 4 * (threadIdx.x + 256 * i));
      if constexpr (NTOK > 1) {
#pragma unroll
        for (int t = 1; t < NTOK; t++) {
          const float* xr = a.x + (size_t)min(t, ntok - 1) * K;
#pragma unroll
          for (int i = 0; i < XV; i++) xvt[t - 1][i] = *reinterpret_cast<const float4*>(xr + 4 * (threadIdx.x + 256 * i));
        }
      }
      if (norm) {
#pragma unroll
        for (int i = 0; i < XV; i++)
          nwv[i] = norm_w ? *reinterpret_cast<const float4*>(norm_w + 4 * (threadIdx.x + 256 * i))
                          : make_float4(1.f, 1.f, 1.f, 1.f);
      }
    } else {
#pragma unroll
      for (int i = 0; i < XV; i++) {
        const int k0 = 4 * (threadIdx.x + 256 * i);
        float4 v;
        v.x = (k0 < K) ? gemv_x1(a.x, xt, k0) : 0.f;
        v.y = (k0 + 1 < K) ? gemv_x1(a.x, xt, k0 + 1) : 0.f;
        v.z = (k0 + 2 < K) ? gemv_x1(a.x, xt, k0 + 2) : 0.f;
        v.w = (k0 + 3 < K) ? gemv_x1(a.x, xt, k0 + 3) : 0.f;
        xv[i] = v;
        if constexpr (NTOK > 1) {
#pragma unroll
          for (int t = 1; t < NTOK; t++) {
            const float* x1 = a.x + (size_t)min(t, ntok - 1) * K;
            xvt[t - 1][i] = make_float4((k0 < K) ? x1[k0] : 0.f, (k0 + 1 < K) ? x1[k0 + 1] : 0.f,
                                        (k0 + 2 < K) ? x1[k0 + 2] : 0.f, (k0 + 3 < K) ? x1[k0 + 3] : 0.f);
          }
        }
      }
    }
  }
  load_batch<XV, U, RH>(b0, c0, st, cg, 0, lg);
  load_batch<XV, U, RH>(b1, c1, st, cg, U, lg);
  // epilogue operands (lanes < RH use them)
  const int nr = min(row0 + r, N - 1);
  const float wsv = a.ws[nr];
  const float bv = a.bias ? a.bias[nr] : 0.0f;

  float xs;
  int px[NTOK];                          // plane mode: each row's absmax exponent, or kXeNonFinite
#pragma unroll
  for (int t = 0; t < NTOK; t++) px[t] = 0;
  if constexpr (PL) {
    // ---- digit rows of x (every element: no scalar tail in this mode) ------
#pragma unroll
    for (int t = 0; t < NTOK; t++) {
      uint32_t mx = 0;
#pragma unroll
      for (int i = 0; i < XV; i++) {
        const float4 v = t == 0 ? xv[i] : xvt[t > 0 ? t - 1 : 0][i];
        const uint32_t m01 = max(abs_bits(v.x), abs_bits(v.y));
        const uint32_t m23 = max(abs_bits(v.z), abs_bits(v.w));
        mx = max(mx, max(m01, m23));
      }
      mx = wave_umax(mx);
      if (lane == 0) s_mx[4 * t + wv] = mx;
    }
    __syncthreads();
    uint32_t* sc = reinterpret_cast<uint32_t*>(s_codes);
#pragma unroll
    for (int t = 0; t < NTOK; t++) {
      const uint32_t m = max(max(s_mx[4 * t], s_mx[4 * t + 1]), max(s_mx[4 * t + 2], s_mx[4 * t + 3]));
      int ex = 0;
      if (m < 0x7f800000u && m != 0) (void)frexpf(__uint_as_float(m), &ex);
      px[t] = m < 0x7f800000u ? ex : kXeNonFinite;
      const Pow2 ps = pow2_split(30 - ex);
#pragma unroll
      for (int i = 0; i < XV; i++) {
        const float4 v = t == 0 ? xv[i] : xvt[t > 0 ? t - 1 : 0][i];
        uint32_t d[4];
        digit_planes(digit_word(v.x, ps), digit_word(v.y, ps), digit_word(v.z, ps), digit_word(v.w, ps), d);
#pragma unroll
        for (int p = 0; p < 4; p++) sc[(4 * t + p) * XV * 256 + threadIdx.x + 256 * i] = d[p];
      }
    }
    xs = 1.0f;
    __syncthreads();
  } else if constexpr (XV > 0) {
    if (a.norm == NORM_NUMPY) final_rmsnorm<XV>(xv, nwv, norm_w != nullptr, K, norm_eps);
    else if (a.norm == NORM_DECODER) decoder_rmsnorm<XV>(xv, nwv, norm_w != nullptr, K, norm_eps);
    // ---- fused per-token activation quantization --------------------------
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
      if (m < 0x7f800000u && (__float_as_uint(inv) & 0x7f800000u) != 0x7f800000u) {
        // finite absmax and reciprocal (the usual case): |x * inv| <= 127.x
#pragma unroll
        for (int i = 0; i < XV; i++) sc[threadIdx.x + 256 * i] = codes4_rne(xv[i], inv);
      } else {
        // NaN / Inf in x, or a reciprocal that overflows
#pragma unroll
        for (int i = 0; i < XV; i++) {
          const float4 v = xv[i];
          sc[threadIdx.x + 256 * i] = pack4(code_rne(v.x * inv, false), code_rne(v.y * inv, false),
                                            code_rne(v.z * inv, false), code_rne(v.w * inv, false));
        }
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

  // ---- main loop: two batches of U load instructions in flight --------------
  // Both batches were issued before the prologue.  The loop body is
  // straight-line code that enters and leaves with the 2U loads of b0 and b1
  // outstanding, so the compiler keeps the wait counts exact.
  int acc[PL ? 1 : NP];
#pragma unroll
  for (int p = 0; p < (PL ? 1 : NP); p++) acc[p] = 0;
  constexpr int NM = gemv_nm<RH, NP>();
  v4i macc[NM];                          // digit-row modes: the MFMA accumulators
#pragma unroll
  for (int mm = 0; mm < NM; mm++) macc[mm] = v4i{0, 0, 0, 0};
  int i = 0;
  if constexpr (PL) {
    for (; i + 2 * U < n_i; i += 2 * U) {
      consume_batch_mfma<XV, U, RH, NP>(b0, s_codes, st, i, lg, lane, macc);
      load_batch<XV, U, RH>(b0, c0, st, cg, i + 2 * U, lg);
      consume_batch_mfma<XV, U, RH, NP>(b1, s_codes, st, i + U, lg, lane, macc);
      load_batch<XV, U, RH>(b1, c1, st, cg, i + 3 * U, lg);
    }
    consume_batch_mfma<XV, U, RH, NP>(b0, s_codes, st, i, lg, lane, macc);
    consume_batch_mfma<XV, U, RH, NP>(b1, s_codes, st, i + U, lg, lane, macc);
  } else {
    for (; i + 2 * U < n_i; i += 2 * U) {
      consume_batch<XV, U, RH, NP>(b0, c0, s_codes, st, i, lg, acc);
      load_batch<XV, U, RH>(b0, c0, st, cg, i + 2 * U, lg);
      consume_batch<XV, U, RH, NP>(b1, c1, s_codes, st, i + U, lg, acc);
      load_batch<XV, U, RH>(b1, c1, st, cg, i + 3 * U, lg);
    }
    consume_batch<XV, U, RH, NP>(b0, c0, s_codes, st, i, lg, acc);
    consume_batch<XV, U, RH, NP>(b1, c1, s_codes, st, i + U, lg, acc);
  }

  // ---- reduction: row r's 4*SL partials (wave w, lane slot q) at
  //      s_red[p][r*4*SL + w*SL + q], summed in that order by wave 0; in the
  //      digit-row modes each wave's C entries go to s_redp[p][row][wave]
  //      (integer sums: every order gives the same bits) ----------------------
  if constexpr (PL) {
    // lane l, register e of MFMA mm holds C[4 (l >> 4) + e][l & 15] of its
    // code rows RH mm ..
    const int q = lane >> 4;
#pragma unroll
    for (int mm = 0; mm < NM; mm++) {
      if constexpr (RH == 8) {
        v4i other;
#pragma unroll
        for (int e = 0; e < 4; e++) other[e] = __shfl(macc[mm][e], (lane + 40) & 63, 64);
        if ((lane & 8) == 0 && q < 2) {    // lanes 0-7 and 16-23: code rows 8 mm + 4q + e, weight row lane & 7
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int cr = 8 * mm + 4 * q + e;
            if (cr < NP) s_redp[min(cr, NP - 1)][lane & 7][wv] = macc[mm][e] + other[e];
          }
        }
      } else {                             // code rows 4q + e, weight row lane & 15
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int cr = 4 * q + e;
          if (cr < NP) s_redp[min(cr, NP - 1)][lane & 15][wv] = macc[mm][e];
        }
      }
    }
  } else {
#pragma unroll
    for (int p = 0; p < NP; p++) s_red[p][r * 4 * SL + wv * SL + slot] = acc[p];
  }
  __syncthreads();
  if (wv != 0) return;
  uint64_t key = 0;
  if (lane < RH) {
    int tots[NP];
    if constexpr (PL) {
#pragma unroll
      for (int pp = 0; pp < NP; pp++) {
        const int4 v = *reinterpret_cast<const int4*>(s_redp[pp][lane]);
        tots[pp] = (v.x + v.y) + (v.z + v.w);
      }
    } else {
#pragma unroll
      for (int pp = 0; pp < NP; pp++) {
        const int4* p = reinterpret_cast<const int4*>(s_red[pp] + lane * 4 * SL);
        int t = 0;
#pragma unroll
        for (int q = 0; q < SL; q++) {
          const int4 v = p[q];
          t += (v.x + v.y) + (v.z + v.w);
        }
        tots[pp] = t;
      }
    }
    const int tot = tots[0];
    const int n = row0 + lane;
    if constexpr (PL >= 2) {
      if (n < a.N) {
        uint32_t bad = 0;
#pragma unroll
        for (int t = 0; t < NTOK; t++) {
          if (t >= ntok) break;
          const float sum = digits_sum(tots[4 * t], tots[4 * t + 1], tots[4 * t + 2], tots[4 * t + 3]);
          bad |= (uint32_t)(px[t] == kXeNonFinite) << t;
          float v = px[t] == kXeNonFinite ? __builtin_nanf("") : ldexpf(__fmul_rn(sum, wsv), px[t] - 6);
          if (a.bias) v = __fadd_rn(v, bv);
          a.y[(size_t)t * a.N + n] = v;
        }
        // a token holding Inf or NaN got NaN: store the reference's fp32 sum
        // instead (NaN or +-Inf, nonfinite_dot), one copy out of the token loop
#pragma unroll 1
        for (int t = 0; bad >> t; t++) {
          if (!((bad >> t) & 1)) continue;
          float v = nonfinite_dot(a.x, 0, (size_t)t * K, 0, K, a.wt, a.NG, n);
          if (a.bias) v = __fadd_rn(v, bv);
          a.y[(size_t)t * a.N + n] = v;
        }
      }
    } else if constexpr (PL == 1) {
      if (n < a.N) {
        const float t = digits_sum(tots[0], tots[1], tots[2], tots[3]);
        const float v = px[0] == kXeNonFinite ? __fadd_rn(nonfinite_dot(a.x, xt, 0, 0, K, a.wt, a.NG, n), bv)
                                              : __fmaf_rn(ldexpf(t, px[0] - 6), wsv, bv);
        const int out = (flags >> 10) & 3;
        if (out == OUT_F32) {
          a.y[n] = v;
        } else if (out == OUT_BF16) {
          reinterpret_cast<uint16_t*>(a.y)[n] = (uint16_t)f32_to_bf16_rne(v);
        } else {
          const _Float16 h = (_Float16)v;
          reinterpret_cast<uint16_t*>(a.y)[n] = __builtin_bit_cast(uint16_t, h);
        }
      }
    } else if (a.epi == EPI_SWIGLU) {
      // RH == 16: lanes 0-7 hold gate rows 8b + lane, lanes 8-15 the matching
      // up rows; rows past N are zero rows (their value is never stored)
      const float g = __fmul_rn(__fmul_rn((float)tot, wsv), xs);
      const float u = __shfl(g, lane + 8, 64);
      const int m = (row0 >> 1) + lane;
      if (lane < 8 && m < (a.N >> 1)) st_agent(a.y + m, __fmul_rn(ref_silu(g), u));
    } else if (n < a.N) {
      if (a.epi == EPI_ARGMAX) {
        float r = __fmul_rn(__fmul_rn((float)tot, wsv), xs);
        if (a.bias) r = __fadd_rn(r, bv);
        if (a.y) a.y[n] = r;
        key = argmax_key(r, n);
      } else {
        gemv_epilogue(a, n, tot, xs, wsv, bv);
      }
    }
  }
  if (a.epi == EPI_ARGMAX) {
    // largest key of the work-group's rows (lanes >= RH hold 0); the keys of
    // all work-groups are reduced by a second kernel (a last-work-group
    // reduction needs a device-scope fence per work-group, measured 10x
    // slower on the lm_head)
#pragma unroll
    for (int o = 1; o < RH; o <<= 1) {
      const uint64_t t = __shfl_xor(key, o, 64);
      key = t > key ? t : key;
    }
    if (lane == 0) keys[blockIdx.x] = key;
  }
}

// ---------------------------------------------------------------------------
// launcher
// ---------------------------------------------------------------------------
template <int XV, int U, int RH, int PL>
static void launch_one(const GemvArgs& a, int blocks, hipStream_t st) {
  const int flags = (a.x_vec & 3) | ((a.epi & 7) << 2) | (a.bias ? 32 : 0) | ((a.norm & 3) << 6) |
                    ((a.x_type & 3) << 8) | ((a.out & 3) << 10) | ((a.ntok & 7) << 12);
  const size_t dyn = a.norm == NORM_NUMPY ? (size_t)(a.K / 128) * kNpNormStride * sizeof(float) : 0;
  hipLaunchKernelGGL((gemv_i8_kernel<XV, U, RH, PL>), dim3(blocks), dim3(256), dyn, st, a.x, a.wt, a.ws, a.y,
                     a.N, a.K, a.NG, a.KB, flags, a.xq, a.xs_in, a.bias, a.acc_out, a.xs_out, a.keys,
                     a.norm_w, a.norm_eps);
}

template <int XV, int PL = 0>
static hipError_t launch_xv(const GemvArgs& a, const GemvPlan& p, hipStream_t st) {
  if (p.rows == 16) {
    switch (p.u) {
      case 2: launch_one<XV, 2, 16, PL>(a, p.blocks, st); break;
      case 4: launch_one<XV, 4, 16, PL>(a, p.blocks, st); break;
      case 8: launch_one<XV, 8, 16, PL>(a, p.blocks, st); break;
      case 12: launch_one<XV, 12, 16, PL>(a, p.blocks, st); break;
      default: return hipErrorInvalidValue;
    }
  } else if (p.rows == 8) {
    switch (p.u) {
      case 2: launch_one<XV, 2, 8, PL>(a, p.blocks, st); break;
      case 4: launch_one<XV, 4, 8, PL>(a, p.blocks, st); break;
      case 6: launch_one<XV, 6, 8, PL>(a, p.blocks, st); break;
      case 8: launch_one<XV, 8, 8, PL>(a, p.blocks, st); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    return hipErrorInvalidValue;
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

// The in-GEMV final RMSNorm needs all of x in registers (K == 1024 XV, both
// vectors 16-byte aligned), a power-of-two K (numpy's pairwise tree is then
// balanced) and its padded squares within 64 KiB of LDS.
bool gemv_fused_norm_ok(int K, const float* x, const float* norm_w) {
  const int xv = gemv_fused_xv(K);
  if (xv == 0 || K != 1024 * xv || (K & (K - 1)) != 0) return false;
  // the padded squares must fit 64 KiB of dynamic LDS (K <= 8192)
  if ((size_t)(K / 128) * kNpNormStride * sizeof(float) > 65536) return false;
  return ((((uintptr_t)x) | ((uintptr_t)norm_w)) & 15) == 0;
}

static int g_force_rows = 0, g_force_u = 0;

void gemv_set_plan(int rows, int u) {
  g_force_rows = rows;
  g_force_u = u;
}

// batch depths built for each row mode
static bool u_ok(int rows, int u) {
  return rows == 16 ? (u == 2 || u == 4 || u == 8 || u == 12) : (u == 2 || u == 4 || u == 6 || u == 8);
}

// Measured on MI355X (graph-replayed launches over > 512 MB of rotating
// weights).  The decode shapes are latency-bound and limited by the memory
// requests a CU can keep in flight, so every CU should stream: with at most
// 256 sixteen-row groups (N <= 4096) a work-group takes 8 rows, which doubles
// the work-groups at the same bytes per wave (QKV 4096x2048: 3.42 against
// 3.49 us with 16-row work-groups).  U is the smallest
// depth whose two batches hold all of a wave's load instructions, so every
// weight load is issued before the activation prologue; longer K loops over
// batches of 8.
GemvPlan gemv_plan(int N, int K) {
  GemvPlan p;
  const int NG = cdiv(N, 16);
  const int KB = cdiv(K, 64);
  p.rows = NG <= 256 ? 8 : 16;
  if (g_force_rows == 8 || g_force_rows == 16) p.rows = g_force_rows;
  p.blocks = cdiv(N, p.rows);
  const int n_kb = cdiv(KB, 4);
  const int n_i = p.rows == 16 ? n_kb : cdiv(n_kb, 2);
  p.u = 8;
  for (int u : {2, 4, 6, 8, 12})
    if (u_ok(p.rows, u) && 2 * u >= n_i) {
      p.u = u;
      break;
    }
  if (g_force_u > 0 && u_ok(p.rows, g_force_u)) p.u = g_force_u;
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
  a.keys = L.keys;
  a.norm_w = L.norm_w;
  a.norm_eps = L.norm_eps;
  a.norm = L.norm;
  if (L.epi == EPI_ARGMAX && !L.keys) return hipErrorInvalidValue;
  if (L.epi == EPI_SWIGLU && (L.N % 16 != 0 || L.bias)) return hipErrorInvalidValue;
  a.N = L.N;
  a.K = L.K;
  a.KB = cdiv(L.K, 64);
  a.NG = cdiv(L.N, 16);
  a.epi = L.epi;
  a.x_vec = 0;
  if (L.N <= 0 || L.K <= 0) return hipErrorInvalidValue;
  GemvPlan p = gemv_plan(L.N, L.K);
  if (L.epi == EPI_SWIGLU && p.rows != 16) {
    // gate and up rows meet in one 16-row work-group
    p.rows = 16;
    p.blocks = cdiv(L.N, 16);
    const int n_i = cdiv(cdiv(L.K, 64), 4);
    p.u = 8;
    for (int u : {2, 4, 8, 12})
      if (2 * u >= n_i) {
        p.u = u;
        break;
      }
  }
  const int xv = L.x ? gemv_fused_xv(L.K) : 0;
  if (L.epi == EPI_W8A32_ROWS && L.ntok > 2 && a.NG >= 256 && g_force_rows == 0) {
    // 3..4 token rows: every work-group splits all of them into digit rows,
    // so from 256 row groups up the 16-row work-groups (half as many splits)
    // are faster: 4096x2048 at 3 / 4 tokens 5.30 / 5.39 -> 4.11 / 4.20 us
    // (2048-row weights stay faster on 8-row work-groups: 3.92 against 4.00)
    p.rows = 16;
    p.blocks = cdiv(L.N, 16);
    const int n_i = cdiv(cdiv(L.K, 64), 4);
    p.u = 8;
    for (int u : {2, 4, 8, 12})
      if (2 * u >= n_i) {
        p.u = u;
        break;
      }
    if (g_force_u > 0 && u_ok(16, g_force_u)) p.u = g_force_u;
  }
  if (L.epi == EPI_W8A32_ROWS) {
    // 2..4 fp32 token rows as four digit rows each: fused x only, no RMSNorm;
    // 3 or 4 rows (16 code rows of XV KiB of LDS each) up to K = 8192
    if (!L.x || xv == 0 || L.norm != NORM_NONE || L.x_type != 0 || L.out != OUT_F32) return hipErrorInvalidValue;
    if (L.ntok < 2 || L.ntok > 4 || (L.ntok > 2 && xv > 8)) return hipErrorInvalidValue;
    a.ntok = L.ntok;
    if (L.K == 1024 * xv && (((uintptr_t)L.x) & 15) == 0) a.x_vec = 2;
    if (L.ntok == 2) {
      switch (xv) {
        case 2: return launch_xv<2, 2>(a, p, st);
        case 4: return launch_xv<4, 2>(a, p, st);
        case 6: return launch_xv<6, 2>(a, p, st);
        case 8: return launch_xv<8, 2>(a, p, st);
        case 16: return launch_xv<16, 2>(a, p, st);
        default: return hipErrorInvalidValue;
      }
    }
    switch (xv) {
      case 2: return launch_xv<2, 4>(a, p, st);
      case 4: return launch_xv<4, 4>(a, p, st);
      case 6: return launch_xv<6, 4>(a, p, st);
      case 8: return launch_xv<8, 4>(a, p, st);
      default: return hipErrorInvalidValue;
    }
  }
  if (L.epi == EPI_W8A16) {
    // digit-plane mode: fused x only, no RMSNorm; y of type L.out
    if (!L.x || xv == 0 || L.norm != NORM_NONE || L.x_type < 0 || L.x_type > 2) return hipErrorInvalidValue;
    if (L.out != OUT_F32 && L.out != OUT_BF16 && L.out != OUT_F16) return hipErrorInvalidValue;
    a.x_type = L.x_type;
    a.out = L.out;
    const uintptr_t align = L.x_type == 0 ? 15 : 7;
    if (L.K == 1024 * xv && (((uintptr_t)L.x) & align) == 0) a.x_vec = 2;
    switch (xv) {
      case 2: return launch_xv<2, 1>(a, p, st);
      case 4: return launch_xv<4, 1>(a, p, st);
      case 6: return launch_xv<6, 1>(a, p, st);
      case 8: return launch_xv<8, 1>(a, p, st);
      case 16: return launch_xv<16, 1>(a, p, st);
      default: return hipErrorInvalidValue;
    }
  }
  if (L.x && xv == 0) return hipErrorInvalidValue;  // caller must quantize first
  if (L.x && L.K == 1024 * xv && (((uintptr_t)L.x) & 15) == 0) a.x_vec = 2;
  if (L.norm && (!gemv_fused_norm_ok(L.K, L.x, L.norm_w) || a.x_vec != 2)) return hipErrorInvalidValue;
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

// ---------------------------------------------------------------------------
// C ABI of the launchers above (tl_kernels.h)
// ---------------------------------------------------------------------------
extern "C" {
void tlk_gemv_plan(int N, int K, GemvPlan* plan) { *plan = tl::gemv_plan(N, K); }
int tlk_gemv_fused_xv(int K) { return tl::gemv_fused_xv(K); }
bool tlk_gemv_fused_norm_ok(int K, const float* x, const float* norm_w) {
  return tl::gemv_fused_norm_ok(K, x, norm_w);
}
hipError_t tlk_launch_gemv_i8(const GemvLaunch* L, hipStream_t st) { return tl::launch_gemv_i8(*L, st); }
void tlk_gemv_set_plan(int rows, int u) { tl::gemv_set_plan(rows, u); }
}  // extern "C"
