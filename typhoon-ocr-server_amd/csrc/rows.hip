// rows.hip -- 2 to 8 token rows of fp32 activations over the int8 weight
// tiles with fp32 semantics, on the int8 MFMA: w8a32_linear at batch 2..8
// (kernel/w8a32_kernel.c:297-350: X times the weights dequantized to fp32,
// through cblas_sgemm).
//
// Digit planes.  Per work-group slice of K, each token row is a 31-bit
// fixed-point vector: q = x * 2^(30-e) truncated, e the binary exponent of the
// slice's absmax (|x| < 2^e, so |q| < 2^30), and q splits into signed
// digits q = d0 2^24 + d1 2^16 + d2 2^8 + d3 (d1..d3 in [-128, 127], d0 in
// [-64, 64]): the bytes of q + 0x808080, the low three flipped by 0x80.  The
// four digit rows of a token are four int8 code rows of the MFMA's second
// operand, so a_p = sum_k w_k d_p,k are exact int32 sums and
//   sum_k w_k x_k = 2^(e-6) (a0 + 2^-8 (a1 + 2^-8 (a2 + 2^-8 a3)))
// up to the truncation of q (below one unit: 2^-30 of the slice absmax per
// element) and the roundings of the Horner steps.  The weights stay int8 (no widening),
// one MFMA per 16x64 weight tile and 4-token group.
//
// Work decomposition (HBM-bound like the GEMV: the weight bytes dominate):
//   * work-group (g, s) owns the 16 R weight rows of row groups gR .. gR+R-1
//     (R = 1..3) and the k-blocks of K slice s (S slices of kbs k-blocks);
//     its 4 waves split the slice's k-blocks and issue every weight load of
//     the slice first (all tiles in flight at once, non-temporal);
//   * meanwhile all 256 threads load the slice of the M token rows in
//     chunks of 16 consecutive k (chunk c = (kbl MP + t) 4 + kq: k-block
//     kbl, token t, k quarter kq, MP = M rounded up to a power of two;
//     thread c mod 256), find each token's absmax
//     (a DPP max over the chunk's lane quad, then an LDS max), convert to
//     digits and write each chunk's four digit rows as four 16-byte pieces
//     of the k-block's code tile, slot 16 kq + 4 (t mod 4) + (p ^ kq) (the
//     xor spreads a quad's writes over the banks; readers undo it);
//   * per weight tile: one ds_read_b128 of codes and one MFMA per token
//     group; the 4 waves' int32 accumulators meet in LDS;
//   * the (row group, token group) pairs are spread over the 4 waves; each
//     combines its pairs' four digit sums per token (lane quads), scales them
//     (y_s = 2^(e-6) fl(t ws), the scales loaded with the weight tiles), and
//     either stores the outputs (S == 1, 16 bytes per token and lane quad) or
//     stores its partials with agent-scope atomic stores and waits for their
//     acknowledgement; then one thread bumps work-group column g's arrival
//     counter; the work-group that brings it to S adds the S partials in slice
//     order, adds the bias, stores, and resets the counter.  Nothing waits on
//     another work-group.
// A token whose slice holds Inf or NaN gets that slice's fp32 sum as the
// reference gives it, NaN or +-Inf (nonfinite_dot, tl_common.h), which the
// slices' merge adds like any partial.
#include <atomic>

#include "tl_common.h"
#include "tl_kernels.h"

namespace tl {

struct RowsArgs {
  const void* X;        // row-major [M][ldx] fp32 (load_x4 also reads bf16 / fp16 rows)
  int ldx;
  const uint8_t* Bt;    // weight tiles [KB][NG]
  const float* ws;
  const float* bias;
  void* Y;
  int ldy;
  float* part;          // [S][M][N] partial outputs (S > 1)
  uint32_t* cnt;        // [NG] arrival counters, zero at rest (S > 1)
  int M, N, K, KB, NG, S, kbs;
  int NGR;              // work-groups per K slice: ceil(NG / R)
  int lmp;              // log2 of M rounded up to a power of two
  int out;
};

// 4 consecutive activations of token row `row` at k as floats (k + 4 <= K)
template <int AMODE>
__device__ __forceinline__ float4 load_x4(const void* X, size_t off) {
  if constexpr (AMODE == A_F32X3) {
    return *reinterpret_cast<const float4*>(static_cast<const float*>(X) + off);
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(X) + off);
    if constexpr (AMODE == A_BF16) {
      return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                         __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
    } else {
      const _Float16 h0 = __builtin_bit_cast(_Float16, (uint16_t)(u.x & 0xffff));
      const _Float16 h1 = __builtin_bit_cast(_Float16, (uint16_t)(u.x >> 16));
      const _Float16 h2 = __builtin_bit_cast(_Float16, (uint16_t)(u.y & 0xffff));
      const _Float16 h3 = __builtin_bit_cast(_Float16, (uint16_t)(u.y >> 16));
      return make_float4((float)h0, (float)h1, (float)h2, (float)h3);
    }
  }
}

__device__ __forceinline__ void store_out(const RowsArgs& a, size_t o, float y) {
  if (a.out == OUT_F32) {
    reinterpret_cast<float*>(a.Y)[o] = y;
  } else if (a.out == OUT_BF16) {
    reinterpret_cast<uint16_t*>(a.Y)[o] = (uint16_t)f32_to_bf16_rne(y);
  } else {
    const _Float16 h = (_Float16)y;
    reinterpret_cast<uint16_t*>(a.Y)[o] = __builtin_bit_cast(uint16_t, h);
  }
}

// After the epilogue: the outputs (slice < 0, one K slice) or slice partials
// (slice s) a lane stored for tokens whose slice holds Inf or NaN (NaN there)
// are stored again with the reference's fp32 sum over the slice, NaN or +-Inf
// (nonfinite_dot).  One copy per kernel, out of the unrolled epilogue; the
// lane rewrites its own addresses, before its partials are acknowledged.
template <int AMODE, int R, int TG>
__device__ __forceinline__ void nonfinite_fixup(const RowsArgs& a, const uint32_t* mx, int gg, int tq, int lane,
                                                int wv, int kb_lo, int nk, int slice) {
  constexpr int xt = AMODE == A_F32X3 ? 0 : (AMODE == A_BF16 ? 1 : 2);
  const int k1 = min(64 * (kb_lo + nk), a.K);
#pragma unroll 1
  for (int tg = 0; tg < TG; tg++) {
    const int t = 4 * tg + tq;
    if (t >= a.M || mx[t] < 0x7f800000u) continue;
#pragma unroll 1
    for (int r = 0; r < R; r++) {
      if ((r * TG + tg) % 4 != wv) continue;   // another wave's pair
      const int n0 = 16 * (gg * R + r) + 4 * (lane >> 4);
#pragma unroll 1
      for (int q = 0; q < 4; q++) {
        const int n = n0 + q;
        if (n >= a.N) break;
        float v = nonfinite_dot(a.X, xt, (size_t)t * a.ldx, 64 * kb_lo, k1, a.Bt, a.NG, n);
        if (slice < 0) {
          if (a.bias) v = __fadd_rn(v, a.bias[n]);
          store_out(a, (size_t)t * a.ldy + n, v);
        } else {
          st_agent(a.part + ((size_t)slice * a.M + t) * a.N + n, v);
        }
      }
    }
  }
}

// TG 4-token groups (M <= 4 TG); NKB k-blocks per slice at most (code tiles
// in LDS); CPT chunks of 16 activations per thread (MP * nk * 4 <= 256 CPT);
// R weight row groups per work-group, sharing one split of the activations
template <int AMODE, int TG, int NKB, int CPT, int R>
__global__ __launch_bounds__(256) void rows_planes_kernel(RowsArgs a) {
  constexpr int NT = NKB / 4;           // weight tiles per wave and row group at most
  __shared__ uint4 s_codes[NKB][TG][64];
  __shared__ uint32_t s_mx[TG * 4];
  __shared__ v4i s_part[R][TG][4][64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gg = blockIdx.x % a.NGR;         // row groups gg R .. gg R + R - 1
  const int s = blockIdx.x / a.NGR;
  const int kb_lo = s * a.kbs;
  const int nk = min(a.kbs, a.KB - kb_lo);   // >= 1 (the host sizes S so)
  // chunks (k-block, token, k quarter); tokens padded to MP = 2^lmp >= M so
  // that the chunk index splits with shifts (padding tokens load nothing)
  const int lmp = a.lmp, mp = 1 << lmp;
  const int nch = nk * mp * 4;
  if (tid < TG * 4) s_mx[tid] = 0;

  // ---- activation chunks: issued first, so waiting for them never waits
  //      for the weight stream (loads retire in issue order).  Chunk
  //      c = (kbl MP + t) 4 + kq holds x[t][64 (kb_lo + kbl) + 16 kq ..+16]
  float4 xr[CPT][4];
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    const int c = tid + 256 * j;
    const int kq = c & 3, t = (c >> 2) & (mp - 1), kbl = c >> (2 + lmp);
    const int k = 64 * (kb_lo + kbl) + 16 * kq;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      xr[j][i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (c < nch && t < a.M && k + 4 * i < a.K) xr[j][i] = load_x4<AMODE>(a.X, (size_t)t * a.ldx + k + 4 * i);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- this wave's weight tiles of every row group, all in flight (row
  //      groups past NG re-read the last one; their outputs are never stored)
  const int kw0 = (wv * nk) >> 2, n_t = (((wv + 1) * nk) >> 2) - kw0;
  const size_t tstride = (size_t)a.NG * 64;
  const uint4* wbase[R];
#pragma unroll
  for (int r = 0; r < R; r++)
    wbase[r] = reinterpret_cast<const uint4*>(a.Bt) + (size_t)min(gg * R + r, a.NG - 1) * 64 + lane;
  uint4 wt[R][NT];
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const int kb = n_t > 0 ? kb_lo + kw0 + min(i, n_t - 1) : kb_lo;   // clamped repeats are skipped
#pragma unroll
    for (int r = 0; r < R; r++) {
      typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
      const v4u_t w = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(wbase[r] + (size_t)kb * tstride));
      wt[r][i] = make_uint4(w.x, w.y, w.z, w.w);
    }
  }
  // ---- the scales (and bias) of this lane's output columns n0 .. n0+3 of
  //      every row group, issued after the weight tiles (loads retire in
  //      issue order, so only the epilogue waits for them) instead of as
  //      dependent loads inside it (columns past N read column N-1; their
  //      outputs are never stored)
  float wsv[R][4], bsv[R][4];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int n0 = 16 * (gg * R + r) + 4 * (lane >> 4);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int n = min(n0 + q, a.N - 1);
      wsv[r][q] = a.ws[n];
      bsv[r][q] = a.bias ? a.bias[n] : 0.0f;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();                           // s_mx cleared

  // ---- per-token absmax over the slice: a chunk's 4 k quarters are a lane
  //      quad (c = tid + 256 j), then one LDS max per quad
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    const int c = tid + 256 * j;
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 v = xr[j][i];
      m = max(m, max(max(abs_bits(v.x), abs_bits(v.y)), max(abs_bits(v.z), abs_bits(v.w))));
    }
    uint32_t o = dpp_u32<DPP_QP_1032>(m);
    m = max(m, o);
    o = dpp_u32<DPP_QP_2301>(m);
    m = max(m, o);
    const int t = (c >> 2) & (mp - 1);
    if ((c & 3) == 0 && c < nch && t < a.M) atomicMax(&s_mx[t], m);
  }
  __syncthreads();

  // ---- digits of every chunk into the code tiles: digit row p of token t
  //      sits in slot 16 kq + 4 (t % 4) + (p ^ kq) of tile (kbl, t / 4)
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    const int c = tid + 256 * j;
    const int kq = c & 3, t = (c >> 2) & (mp - 1), kbl = c >> (2 + lmp);
    if (c >= nch || t >= a.M) continue;
    const uint32_t mx = s_mx[t];
    int ex = 0;
    if (mx < 0x7f800000u && mx != 0) (void)frexpf(__uint_as_float(mx), &ex);
    const Pow2 sc = pow2_split(30 - ex);
    uint32_t pl[4][4];                       // [plane][dword]
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float4 v = xr[j][i];
      uint32_t d[4];
      digit_planes(digit_word(v.x, sc), digit_word(v.y, sc), digit_word(v.z, sc), digit_word(v.w, sc), d);
#pragma unroll
      for (int p = 0; p < 4; p++) pl[p][i] = d[p];
    }
    uint4* tile = &s_codes[kbl][t >> 2][0];
#pragma unroll
    for (int p = 0; p < 4; p++) tile[16 * kq + 4 * (t & 3) + (p ^ kq)] = make_uint4(pl[p][0], pl[p][1], pl[p][2], pl[p][3]);
  }
  __syncthreads();

  // ---- one MFMA per weight tile and token group (code rows of tokens >= M
  //      are never written: their outputs are never stored)
  v4i acc[R][TG];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int tg = 0; tg < TG; tg++) acc[r][tg] = v4i{0, 0, 0, 0};
  const int rslot = lane ^ ((lane >> 4) & 3);   // this lane's code row, as stored
#pragma unroll
  for (int i = 0; i < NT; i++) {
    if (i < n_t) {                             // uniform
#pragma unroll
      for (int tg = 0; tg < TG; tg++) {
        const uint4 c = s_codes[kw0 + i][tg][rslot];
#pragma unroll
        for (int r = 0; r < R; r++)
          acc[r][tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, wt[r][i]),
                                                             __builtin_bit_cast(v4i, c), acc[r][tg], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int tg = 0; tg < TG; tg++) s_part[r][tg][wv][lane] = acc[r][tg];
  __syncthreads();

  // ---- epilogue: the R x TG (row group, token group) pairs are spread over
  //      the 4 waves, pair r TG + tg on wave (r TG + tg) mod 4.  A lane holds
  //      D[n0 .. n0+3][m] of its pair, m = lane & 15 = 4 tq + p (digit row p of
  //      token 4 tg + tq), n0 = 16 g + 4 (lane >> 4); the quad's first lane
  //      (p = 0) combines the four digit sums and owns the token's 4 outputs
  const int tq = (lane >> 2) & 3;
  const bool owner = (lane & 3) == 0;
  const bool vec = a.out == OUT_F32 && (a.ldy & 3) == 0 && (((uintptr_t)a.Y) & 15) == 0;
  bool bad = false;                            // a token of this wave's pairs holds Inf or NaN
  float y[R][TG][4];
#pragma unroll
  for (int r = 0; r < R; r++) {
#pragma unroll
    for (int tg = 0; tg < TG; tg++) {
      if ((r * TG + tg) % 4 != wv) continue;   // wave-uniform
      v4i tot = s_part[r][tg][0][lane];
#pragma unroll
      for (int w = 1; w < 4; w++) {
        const v4i p = s_part[r][tg][w][lane];
#pragma unroll
        for (int q = 0; q < 4; q++) tot[q] += p[q];
      }
      const int t = min(4 * tg + tq, a.M - 1);
      const uint32_t mx = s_mx[t];
      bad |= mx >= 0x7f800000u;
      int ex = 0;
      if (mx < 0x7f800000u && mx != 0) (void)frexpf(__uint_as_float(mx), &ex);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int a1 = __shfl_xor(tot[q], 1, 64), a2 = __shfl_xor(tot[q], 2, 64), a3 = __shfl_xor(tot[q], 3, 64);
        const float sum = digits_sum(tot[q], a1, a2, a3);
        y[r][tg][q] = mx >= 0x7f800000u ? __builtin_nanf("") : ldexpf(__fmul_rn(sum, wsv[r][q]), ex - 6);
      }
    }
  }

  if (a.S == 1) {
    if (!owner) return;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int n0 = 16 * (gg * R + r) + 4 * (lane >> 4);
#pragma unroll
      for (int tg = 0; tg < TG; tg++) {
        if ((r * TG + tg) % 4 != wv) continue;
        const int t = 4 * tg + tq;
        if (t >= a.M || n0 >= a.N) continue;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; q++) v[q] = a.bias ? __fadd_rn(y[r][tg][q], bsv[r][q]) : y[r][tg][q];
        if (vec && n0 + 4 <= a.N) {
          // the 4 outputs of the token as one 16-byte store
          *reinterpret_cast<float4*>(static_cast<float*>(a.Y) + (size_t)t * a.ldy + n0) =
              make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; q++)
            if (n0 + q < a.N) store_out(a, (size_t)t * a.ldy + n0 + q, v[q]);
        }
      }
    }
    if (bad) nonfinite_fixup<AMODE, R, TG>(a, s_mx, gg, tq, lane, wv, kb_lo, nk, -1);
    return;
  }

  // ---- S > 1: partials, arrival, and the last work-group's merge (each
  //      wave merges its own pairs)
  if (owner) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int n0 = 16 * (gg * R + r) + 4 * (lane >> 4);
#pragma unroll
      for (int tg = 0; tg < TG; tg++) {
        if ((r * TG + tg) % 4 != wv) continue;
        const int t = 4 * tg + tq;
        if (t >= a.M) continue;
#pragma unroll
        for (int q = 0; q < 4; q++)
          if (n0 + q < a.N) st_agent(a.part + ((size_t)s * a.M + t) * a.N + n0 + q, y[r][tg][q]);
      }
    }
    if (bad) nonfinite_fixup<AMODE, R, TG>(a, s_mx, gg, tq, lane, wv, kb_lo, nk, s);
  }
  asm volatile("" ::: "memory");
  wait_vm<0>();                                // this wave's partial stores are acknowledged
  asm volatile("" ::: "memory");
  __shared__ int s_last;
  __syncthreads();                             // every wave's partials acknowledged
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(a.cnt + gg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(a.S - 1);
  __syncthreads();
  if (!s_last) return;
  // the winner's acquire: the other slices' partials are read after the
  // counter showed them all arrived (agent scope; once per row group)
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  asm volatile("" ::: "memory");
  if (owner) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int n0 = 16 * (gg * R + r) + 4 * (lane >> 4);
#pragma unroll
      for (int tg = 0; tg < TG; tg++) {
        if ((r * TG + tg) % 4 != wv) continue;
        const int t = 4 * tg + tq;
        if (t >= a.M) continue;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int n = n0 + q;
          if (n >= a.N) continue;
          float v = ld_agent(a.part + (size_t)t * a.N + n);
          for (int ss = 1; ss < a.S; ss++) v = __fadd_rn(v, ld_agent(a.part + ((size_t)ss * a.M + t) * a.N + n));
          if (a.bias) v = __fadd_rn(v, bsv[r][q]);
          store_out(a, (size_t)t * a.ldy + n, v);
        }
      }
    }
  }
  if (tid == 0) __hip_atomic_store(a.cnt + gg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// planner and launcher
// ---------------------------------------------------------------------------
// tuning overrides; atomic, since a setter may run while other threads plan launches
static std::atomic<int> g_rows_force_split{0};
static std::atomic<int> g_rows_force_groups{0};
void rows_set_split(int s) { g_rows_force_split.store(s > 0 ? s : 0, std::memory_order_relaxed); }
void rows_set_groups(int r) { g_rows_force_groups.store(r > 0 ? r : 0, std::memory_order_relaxed); }

bool rows_supported(const GemmLaunch& L) {
  if (L.M < 1 || L.M > 8 || L.N < 1 || L.K < 1) return false;
  // 16-bit X stays on the bf16 / fp16 MFMA (gemm_small.hip), measured faster
  if (L.amode != A_F32X3) return false;
  if (L.out != OUT_F32 && L.out != OUT_BF16 && L.out != OUT_F16) return false;
  if (L.K % 4 != 0 || L.lda % 4 != 0 || L.lda < L.K) return false;
  const uintptr_t align = L.amode == A_F32X3 ? 15 : 7;   // one 4-element piece per load
  return (((uintptr_t)L.A) & align) == 0;
}

// K slices: the fewest that keep a slice's code tiles within LDS (96 k-blocks
// for up to 2 tokens, 64 for one token group, 32 for two) and its activation
// chunks within 4 per thread (MP * kbs <= 256, MP = M rounded up to a power
// of 2).  One slice needs no merge; splitting further was measured slower on
// every decode shape (the down projection at 2 tokens: 7.7 us in one slice,
// 8.2 / 8.5 / 8.9 us in 2 / 3 / 4).
// Row groups per work-group: each work-group loads and splits its slice of
// the activations once for R 16-row weight groups.  R > 1 only for two token
// groups (5..8 tokens, where the split costs twice as much) and only where
// the grid still holds >= 256 work-groups, one per CU: the gate/up
// projection (12288 x 2048) at 5..8 tokens 13.4-14.4 us with R = 1, 12.7-12.9
// with R = 3; at 2..4 tokens R = 1 is fastest on every decode shape (gate/up
// 7.5 against 8.5 us at 2 tokens).
RowsPlan rows_plan(int M, int N, int K) {
  RowsPlan p;
  p.tg = M <= 4 ? 1 : 2;
  const int NG = cdiv(N, 16), KB = cdiv(K, 64);
  const int mp = M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : 8));
  const int kmax = min(p.tg == 1 ? (mp <= 2 ? 96 : 64) : 32, 256 / mp);
  int s = cdiv(KB, kmax);
  const int force_split = g_rows_force_split.load(std::memory_order_relaxed);
  if (force_split > 0) s = max(s, min(force_split, KB));
  p.kbs = cdiv(KB, s);
  p.split = cdiv(KB, p.kbs);                // every slice holds >= 1 k-block
  p.nkb = p.kbs <= 16 ? 16 : (p.kbs <= 32 ? 32 : (p.kbs <= 64 ? 64 : 96));
  const int nch = p.kbs * mp * 4;
  p.cpt = nch <= 256 ? 1 : (nch <= 512 ? 2 : 4);
  p.r = 1;
  if (p.nkb <= 32) {   // the instances built for R > 1
    const int force_groups = g_rows_force_groups.load(std::memory_order_relaxed);
    if (force_groups > 0) p.r = force_groups;
    else if (p.tg == 2)
      for (int r = 3; r > 1; r--)
        if (cdiv(NG, r) * p.split >= 256) {
          p.r = r;
          break;
        }
  }
  p.blocks = cdiv(NG, p.r) * p.split;
  return p;
}

size_t rows_workspace_bytes(int M, int N, int K) {
  const RowsPlan p = rows_plan(M, N, K);
  return p.split > 1 ? (size_t)p.split * M * N * sizeof(float) : 0;
}
size_t rows_counter_count(int N) { return (size_t)cdiv(N, 16); }

template <int AMODE, int TG, int NKB, int R>
static void launch_rows_cpt(const RowsArgs& a, const RowsPlan& p, hipStream_t st) {
  const dim3 grid(p.blocks), block(256);
  if (p.cpt == 1) hipLaunchKernelGGL((rows_planes_kernel<AMODE, TG, NKB, 1, R>), grid, block, 0, st, a);
  else if (p.cpt == 2) hipLaunchKernelGGL((rows_planes_kernel<AMODE, TG, NKB, 2, R>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((rows_planes_kernel<AMODE, TG, NKB, 4, R>), grid, block, 0, st, a);
}

template <int AMODE, int TG, int NKB>
static void launch_rows_r(const RowsArgs& a, const RowsPlan& p, hipStream_t st) {
  if (p.r == 1) launch_rows_cpt<AMODE, TG, NKB, 1>(a, p, st);
  else if (p.r == 2) launch_rows_cpt<AMODE, TG, NKB, 2>(a, p, st);
  else launch_rows_cpt<AMODE, TG, NKB, 3>(a, p, st);
}

template <int AMODE>
static void launch_rows_mode(const RowsArgs& a, const RowsPlan& p, hipStream_t st) {
  if (p.tg == 1) {
    if (p.nkb == 16) launch_rows_r<AMODE, 1, 16>(a, p, st);
    else if (p.nkb == 32) launch_rows_r<AMODE, 1, 32>(a, p, st);
    else if (p.nkb == 64) launch_rows_cpt<AMODE, 1, 64, 1>(a, p, st);
    else launch_rows_cpt<AMODE, 1, 96, 1>(a, p, st);
  } else {
    if (p.nkb == 16) launch_rows_r<AMODE, 2, 16>(a, p, st);
    else launch_rows_r<AMODE, 2, 32>(a, p, st);
  }
}

hipError_t launch_rows(const GemmLaunch& L, hipStream_t st) {
  if (!rows_supported(L)) return hipErrorInvalidValue;
  const RowsPlan p = rows_plan(L.M, L.N, L.K);
  const int lmp = L.M <= 1 ? 0 : (L.M <= 2 ? 1 : (L.M <= 4 ? 2 : 3));
  if ((p.tg == 2 && p.nkb > 32) || p.split < 1 || (p.kbs << lmp) * 4 > 256 * p.cpt) return hipErrorInvalidValue;
  if (p.r < 1 || p.r > 3 || (p.r > 1 && p.nkb > 32) || p.blocks != cdiv(cdiv(L.N, 16), p.r) * p.split)
    return hipErrorInvalidValue;
  if (p.split > 1 && (!L.part || !L.cnt)) return hipErrorInvalidValue;
  RowsArgs a;
  a.X = L.A;
  a.ldx = L.lda;
  a.Bt = L.Bt;
  a.ws = L.ws;
  a.bias = L.bias;
  a.Y = L.Y;
  a.ldy = L.ldy;
  a.part = static_cast<float*>(L.part);
  a.cnt = L.cnt;
  a.M = L.M;
  a.N = L.N;
  a.K = L.K;
  a.KB = cdiv(L.K, 64);
  a.NG = cdiv(L.N, 16);
  a.S = p.split;
  a.kbs = p.kbs;
  a.NGR = cdiv(a.NG, p.r);
  a.lmp = lmp;
  a.out = L.out;
  launch_rows_mode<A_F32X3>(a, p, st);
  return hipGetLastError();
}

}  // namespace tl

// ---------------------------------------------------------------------------
// C ABI of the launchers above (tl_kernels.h)
// ---------------------------------------------------------------------------
extern "C" {
bool tlk_rows_supported(const GemmLaunch* L) { return tl::rows_supported(*L); }
void tlk_rows_plan(int M, int N, int K, RowsPlan* plan) { *plan = tl::rows_plan(M, N, K); }
size_t tlk_rows_workspace_bytes(int M, int N, int K) { return tl::rows_workspace_bytes(M, N, K); }
size_t tlk_rows_counter_count(int N) { return tl::rows_counter_count(N); }
void tlk_rows_set_split(int s) { tl::rows_set_split(s); }
int tlk_rows_forced_split(void) { return tl::g_rows_force_split.load(std::memory_order_relaxed); }
void tlk_rows_set_groups(int r) { tl::rows_set_groups(r); }
hipError_t tlk_launch_rows(const GemmLaunch* L, hipStream_t st) { return tl::launch_rows(*L, st); }
}  // extern "C"
