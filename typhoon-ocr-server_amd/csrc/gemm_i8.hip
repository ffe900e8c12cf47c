// gemm_i8.hip -- W8A8 prefill GEMM: int8 codes x int8 weights on
// v_mfma_i32_16x16x64_i8 with K stages staged through an LDS ring.
//
// Reference: kernel/w8a8_kernel.c:259-268 (w8a8_gemm dequantizes both
// operands and calls cblas_sgemm).  Here the int32 sum is exact and the fp32
// epilogue is y = fl(fl(fl(acc) * ws[n]) * xs[m]) (+ bias[n] as its own
// rounding), ~4e-7 relative L2 from the reference's dequant-then-SGEMM.
//
// Both operands are stored as 16x64 int8 tiles (tl_common.h), so a K stage
// of the work-group's A rows and B columns is a list of whole 1 KiB tiles:
// each is copied global -> LDS directly (global_load_lds_dwordx4, no staging
// registers), and every MFMA operand is read back with one ds_read_b128 per
// lane at consecutive addresses (no bank conflicts, no swizzle needed).
// NST stage buffers form a ring, so NST-1 stages of copies are in flight while
// a stage's MFMAs run; one barrier per stage.
//
// Work-group tile (16 MT) x (16 NT); waves WM x WN each own a
// (16 MT/WM) x (16 NT/WN) block of 16x16 accumulators, each computed as the
// transposed product (weights as the MFMA's first operand) so that a lane ends
// up with 4 consecutive columns of one output row (16-byte stores).  Tiles are ordered so
// that the work-groups placed on one XCD (dispatch is round-robin over the 8
// XCDs) share a band of B columns and all of A, which then stays in that
// XCD's 4 MB L2.
#include <algorithm>
#include <atomic>

#include "tl_common.h"
#include "tl_kernels.h"

namespace tl {

struct GemmI8Args {
  const uint8_t* At;    // activation code tiles [KB][MG]
  const uint8_t* Bt;    // weight tiles [KB][NG]
  const float* ws;      // [N]
  const float* xs;      // [M]
  const int* xe;        // OUT_F32_X4: per-token exponents [M / 4]
  const float* xraw;    // OUT_F32_X4: the fp32 token rows (null: NaN for a non-finite row)
  int ldxr;
  const float* bias;    // [N] or null
  void* Y;              // fp32 [M][ldy] or int32 (OUT_I32)
  int ldy;
  int M, N, K, KB, MG, NG;
  int ntm, ntn;         // work-group tiles along M and N
  int out;
  const uint8_t* zero_tile;  // 1 KiB of zeros (source of k-blocks past K)
  int S;                // K slices per tile (LDS-staged kernel; 1 elsewhere)
  int32_t* part;        // S > 1: int32 partial tiles [tiles][S][16 MT x 16 NT]
  uint32_t* cnt;        // S > 1: zeroed arrival counters [tiles]
  int xa;               // 2: each XCD owns a block of half the tile rows (tile_of)
};

// Work-group -> tile.  Dispatch is round-robin over the 8 XCDs: work-group b
// runs on XCD b % 8 as that XCD's (b / 8)-th.  When the tile columns divide
// over the XCDs, XCD x owns a band of ntn / 8 columns and walks it in groups
// of 4 tile rows x the whole band, so the ~32 work-groups an XCD runs at once
// share 4 A panels and the band's B panels, which fit its 4 MB L2 (one column
// at a time keeps ~32 A panels live at once: past the L2 once A exceeds it,
// e.g. the 4800 plane rows of a 1200-token fp32 batch).  Otherwise each XCD
// takes a run of consecutive tiles (columns of tm).
// With xa = 2 (one tile per CU, ntm even, ntn a multiple of 4, set by the
// launcher where it fills fewer L2 lines) XCD x owns rows (x % 2) ntm / 2 ..
// and columns (x / 2) ntn / 4 .., so it fills half of A and a quarter of the
// weights into its L2 instead of all of A and an eighth of the weights:
// 20 % fewer fills at M = 1024, N = 2048, K = 6144 (50 against 63 MB), and
// 23.2-23.9 -> 22.2-22.4 us for the LDS-staged kernel in a same-run A/B.
__device__ __forceinline__ void tile_of(int b, int ntm, int ntn, int& tm, int& tn, int xa = 1) {
  if (xa == 2) {
    const int x = b % 8, j = b / 8, bm = ntm / 2, bn = ntn / 4;
    tm = (x % 2) * bm + j % bm;
    tn = (x / 2) * bn + j / bm;
    return;
  }
  if (ntn % 8 == 0) {
    const int x = b % 8, j = b / 8, bw = ntn / 8;
    const int grp = j / (4 * bw), r = j - grp * 4 * bw;
    const int rows = min(4, ntm - 4 * grp);
    tm = 4 * grp + r % rows;
    tn = x * bw + r / rows;
  } else {
    const int ntiles = ntm * ntn;
    int t = b;
    if (ntiles % 8 == 0) t = (b % 8) * (ntiles / 8) + b / 8;
    tn = t / ntm;
    tm = t - tn * ntm;
  }
}

// OUT_F32_X4 epilogue of one 16x16 accumulator tile (every lane calls it):
// rows 4t .. 4t+3 are the int8 planes of token t, held by the lane quad
// 4t .. 4t+3 (mod 16) at the same 4 columns n .. n+3; the quad's first lane
// combines them and stores row t (16 bytes when aligned and inside N).
__device__ __forceinline__ void planes_epilogue(const GemmI8Args& a, const v4i c, int m, int n, float4 ws4,
                                                float4 b4, int e, int lane, bool vec_ok) {
  float y[4];
#pragma unroll
  for (int r = 0; r < 4; r++)
    y[r] = planes_sum(c[r], __shfl_xor(c[r], 1, 64), __shfl_xor(c[r], 2, 64), __shfl_xor(c[r], 3, 64));
  if ((lane & 3) != 0 || m >= a.M || n >= a.N) return;
  const float w[4] = {ws4.x, ws4.y, ws4.z, ws4.w};
  const float b[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
  for (int r = 0; r < 4; r++) {
    y[r] = planes_scale(y[r], w[r], e);
    if (a.bias) y[r] = __fadd_rn(y[r], b[r]);
  }
  float* yp = reinterpret_cast<float*>(a.Y) + (size_t)(m >> 2) * a.ldy + n;
  if (vec_ok && n + 4 <= a.N) {
    st_stream(yp, make_float4(y[0], y[1], y[2], y[3]));
  } else {
    for (int r = 0; r < 4 && n + r < a.N; r++) yp[r] = y[r];
  }
}

// After planes_epilogue over a lane's FM x FN accumulator tiles (rows m0 + 16i,
// columns n0 + 16j): the outputs it stored for tokens flagged kXeNonFinite
// (NaN there) are stored again with the reference's fp32 value, nonfinite_dot
// over the fp32 row in a.xraw.  One copy per kernel, out of the unrolled
// epilogue, run only by a lane holding a flagged token; the same lane rewrites
// the same addresses, so its later store is the one that stays.
template <int FM, int FN>
__device__ __forceinline__ void planes_fixup(const GemmI8Args& a, int m0, int n0, int lane) {
  if ((lane & 3) != 0) return;
#pragma unroll 1
  for (int i = 0; i < FM; i++) {
    const int m = m0 + 16 * i;
    if (m >= a.M || a.xe[m >> 2] != kXeNonFinite) continue;
    float* yp = reinterpret_cast<float*>(a.Y) + (size_t)(m >> 2) * a.ldy;
#pragma unroll 1
    for (int j = 0; j < FN; j++) {
#pragma unroll 1
      for (int r = 0; r < 4; r++) {
        const int n = n0 + 16 * j + r;
        if (n >= a.N) break;
        float y = nonfinite_dot(a.xraw, 0, (size_t)(m >> 2) * a.ldxr, 0, a.K, a.Bt, a.NG, n);
        if (a.bias) y = __fadd_rn(y, a.bias[n]);
        yp[n] = y;
      }
    }
  }
}

// Stage ring of NST buffers.  Every K stage is NW*PW whole 1 KiB tiles, each
// copied global -> LDS by one wave with one global_load_lds_dwordx4 (lane l
// writes bytes 16l..16l+15 of the tile, i.e. the tile layout itself).  Stage s
// lives in buffer s % NST; the ring is unrolled so every buffer is a distinct
// LDS object and the compiler keeps only the explicit waits in `step`.  The
// MFMA fragments of a stage are read from LDS one step before its MFMAs run.
template <int MT, int NT, int KT, int NST, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_i8_lds_kernel(GemmI8Args a) {
  constexpr int NW = WM * WN;
  constexpr int TA = MT * KT, TB = NT * KT, TS = TA + TB;  // tiles per stage
  static_assert(TS % NW == 0, "stage tiles must divide evenly over the waves");
  constexpr int PW = TS / NW;                              // tiles copied per wave per stage
  constexpr int FM = MT / WM, FN = NT / WN;                // 16x16 accumulators per wave
  static_assert(MT % WM == 0 && NT % WN == 0, "wave grid must divide the tile");
  static_assert(NST >= 2 && NST <= 8 && NST % 2 == 0, "2, 4, 6 or 8 stage buffers");
  static_assert(KT == 1, "one k-block per stage");
  static_assert(PW * (NST - 1) < 64, "vmcnt range");

  // one distinct LDS object per ring slot (unused slots are 16 bytes)
  __shared__ uint4 s0[TS * 64];
  __shared__ uint4 s1[TS * 64];
  __shared__ uint4 s2[NST > 2 ? TS * 64 : 1];
  __shared__ uint4 s3[NST > 3 ? TS * 64 : 1];
  __shared__ uint4 s4[NST > 4 ? TS * 64 : 1];
  __shared__ uint4 s5[NST > 5 ? TS * 64 : 1];
  __shared__ uint4 s6[NST > 6 ? TS * 64 : 1];
  __shared__ uint4 s7[NST > 7 ? TS * 64 : 1];
  uint4* const ring[8] = {s0, s1, s2, s3, s4, s5, s6, s7};

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wv / WN, wn = wv % WN;

  // XCD-aware tile order: work-group b runs on XCD b % 8; the work-groups of
  // one XCD walk M fastest within a band of N tiles.  With K slices,
  // work-group b takes slice b / tiles of tile b % tiles.
  const int ntiles = a.ntm * a.ntn;
  const int ks = blockIdx.x / ntiles;
  const int bt = blockIdx.x - ks * ntiles;
  int tm, tn;
  tile_of(bt, a.ntm, a.ntn, tm, tn, a.xa);
  const int mg0 = tm * MT, ng0 = tn * NT;

  const uint4* A4 = reinterpret_cast<const uint4*>(a.At) + lane;
  const uint4* B4 = reinterpret_cast<const uint4*>(a.Bt) + lane;
  const uint4* Z4 = reinterpret_cast<const uint4*>(a.zero_tile) + lane;
  const int kb0 = (ks * a.KB) / a.S;                  // this work-group's k-blocks [kb0, kb0 + KB)
  const int KB = ((ks + 1) * a.KB) / a.S - kb0;
  const int nst = cdiv(KB, KT);

  // Copy source of each tile this wave copies, fixed except for the K offset:
  // rows/columns past the matrix edge re-read a valid tile (their
  // accumulators are never stored); k-blocks past K read the zero tile.
  const uint4* qsrc[PW];
  size_t qstride[PW];          // uint4 between consecutive stages
  uint32_t qlds[PW];           // byte offset of the tile inside a stage buffer
  int qk[PW];                  // k-block offset of the tile inside a stage
#pragma unroll
  for (int p = 0; p < PW; p++) {
    const int q = wv + NW * p;
    qk[p] = q % KT;
    qlds[p] = (uint32_t)q * 1024u;
    if (q < TA) {
      const int mg = min(mg0 + q / KT, a.MG - 1);
      qsrc[p] = A4 + ((size_t)(kb0 + qk[p]) * a.MG + mg) * 64;
      qstride[p] = (size_t)KT * a.MG * 64;
    } else {
      const int ng = min(ng0 + (q - TA) / KT, a.NG - 1);
      qsrc[p] = B4 + ((size_t)(kb0 + qk[p]) * a.NG + ng) * 64;
      qstride[p] = (size_t)KT * a.NG * 64;
    }
  }
  // copy p (of PW) of stage st into ring buffer buf; stages past the end of K
  // copy the zero tile, so every step issues exactly PW copies and the
  // explicit wait counts stay exact
  auto copy = [&](int st, uint32_t base, int p) {
    const uint4* g = (st * KT + qk[p] < KB) ? qsrc[p] + (size_t)st * qstride[p] : Z4;
    dma_tile(g, base + qlds[p]);
  };
  auto issue = [&](int st, uint4* buf) {
    const uint32_t base = lds_addr(buf);
#pragma unroll
    for (int p = 0; p < PW; p++) copy(st, base, p);
  };

  // Accumulator tile (i, j) is computed transposed (B fragment as the MFMA's
  // first operand): lane l holds Y[m][n .. n+3] with m = 16 mg + (l & 15) and
  // n = 16 ng + 4 (l >> 4), so the epilogue stores 16 contiguous bytes per lane.
  // Its operands are loaded first: they are older than every tile copy, so
  // the first copy wait below also covers them.
  const int mrow = lane & 15;
  const int ncol = (lane >> 4) * 4;
  float4 e_ws[FN], e_b[FN];
  float e_xs[FM];
#pragma unroll
  for (int j = 0; j < FN; j++) {
    const int n = (ng0 + wn * FN + j) * 16 + ncol;
    float w4[4], b4[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int nn = min(n + r, a.N - 1);
      w4[r] = a.ws[nn];
      b4[r] = a.bias ? a.bias[nn] : 0.0f;
    }
    e_ws[j] = make_float4(w4[0], w4[1], w4[2], w4[3]);
    e_b[j] = make_float4(b4[0], b4[1], b4[2], b4[3]);
  }
  int e_xe[FM];
#pragma unroll
  for (int i = 0; i < FM; i++) {
    const int m = min((mg0 + wm * FM + i) * 16 + mrow, a.M - 1);
    e_xs[i] = (a.out == OUT_I32 || a.out == OUT_F32_X4) ? 0.0f : a.xs[m];
    e_xe[i] = (a.out == OUT_F32_X4) ? a.xe[m >> 2] : 0;
  }

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

  // Fragments of a stage are read one step ahead of their MFMAs (two
  // register sets), so LDS latency hides behind the previous stage's MFMAs.
  uint4 fa[2][FM], fb[2][FN];
  auto read_frags = [&](const uint4* buf, int c) {
#pragma unroll
    for (int i = 0; i < FM; i++) fa[c][i] = buf[(wm * FM + i) * 64 + lane];
#pragma unroll
    for (int j = 0; j < FN; j++) fb[c][j] = buf[(TA + wn * FN + j) * 64 + lane];
  };


  // Step s: stage s's fragments are in registers (set s & 1).
  //   wait until this wave's copies of stage s+1 landed (later stages may
  //   still be in flight), and until its reads of stage s completed;
  //   barrier: stage s+1 is visible, every wave is done reading stage s;
  //   MFMAs of stage s, with the reads of stage s+1's fragments and the
  //   copies of stage s+NST (into stage s's buffer) interleaved one after
  //   each MFMA, so LDS, copy and matrix pipes work at the same time.
  auto step = [&](int st, uint4* cur, const uint4* nxt, int c) {
    wait_vm<PW * (NST - 2)>();
    wait_lgkm0();
    stage_barrier();
    const uint32_t cbase = lds_addr(cur);
    constexpr int NMEM = FM + FN + PW;
    auto mem_op = [&](int q) {
      if (q < FM) fa[c ^ 1][q] = nxt[(wm * FM + q) * 64 + lane];
      else if (q < FM + FN) fb[c ^ 1][q - FM] = nxt[(TA + wn * FN + q - FM) * 64 + lane];
      else copy(st + NST, cbase, q - FM - FN);
    };
    // (steps past the last stage multiply fragments of zero-tile stages and
    // add nothing)
#pragma unroll
    for (int m = 0; m < FM * FN; m++) {
      {
        const int i = m / FN, j = m % FN;
        acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, fb[c][j]),
                                                          __builtin_bit_cast(v4i, fa[c][i]), acc[i][j], 0, 0, 0);
      }
      // keep the source order: one MFMA, then one memory operation
      __builtin_amdgcn_sched_barrier(0);
      if (m < NMEM) mem_op(m);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q = FM * FN; q < NMEM; q++) mem_op(q);
    __builtin_amdgcn_sched_barrier(0);
  };

  // prologue: stages 0 .. NST-1 in flight, stage 0's fragments read
#pragma unroll
  for (int b = 0; b < NST; b++) issue(b, ring[b]);
  wait_vm<PW * (NST - 1)>();
  stage_barrier();
  read_frags(ring[0], 0);
  // ring unrolled NST times (NST even, so the fragment set of every step is
  // a compile-time constant too)
  for (int st = 0; st < nst; st += NST) {
#pragma unroll
    for (int b = 0; b < NST; b++) step(st + b, ring[b], ring[(b + 1) % NST], b & 1);
  }

  wait_vm<0>();   // no copy may still be landing in LDS when the work-group exits

  if (a.S > 1) {
    // K slices: every work-group of the tile stores its int32 sums (16-byte
    // write-through stores), waits for their acknowledgement and counts in;
    // the last to arrive adds the S slices (exact integer sums, so any order
    // gives the same bits; slice order here) and runs the epilogue below
    constexpr int TF = MT * 16 * NT * 16;
    int32_t* mine = a.part + ((size_t)bt * a.S + ks) * TF;
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
        st_agent4(reinterpret_cast<float*>(mine) + (((wv * FM + i) * FN + j) * 64 + lane) * 4,
                  __builtin_bit_cast(v4f, acc[i][j]));
    __shared__ int s_last;
    asm volatile("" ::: "memory");
    wait_vm<0>();                               // this thread's partial stores are acknowledged
    asm volatile("" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(a.cnt + bt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(a.S - 1);
    __syncthreads();
    if (!s_last) return;
    // the merger's acquire: the slices are read after the counter showed them
    // all arrived (agent scope, once per tile; plain 16-byte loads after it)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    constexpr int QB = FM * FN <= 8 ? 4 : (FM * FN <= 16 ? 2 : 1);   // slices in flight together
    const int32_t* slices = a.part + (size_t)bt * a.S * TF;
    for (int q0 = 0; q0 < a.S; q0 += QB) {
      v4i pv[QB][FM][FN];
#pragma unroll
      for (int u = 0; u < QB; u++)
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++)
            pv[u][i][j] = *reinterpret_cast<const v4i*>(slices + (size_t)min(q0 + u, a.S - 1) * TF +
                                                        (((wv * FM + i) * FN + j) * 64 + lane) * 4);
#pragma unroll
      for (int u = 0; u < QB; u++) {
        if (q0 + u >= a.S) break;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][j][r] = q0 + u == 0 ? pv[u][i][j][r] : acc[i][j][r] + pv[u][i][j][r];
      }
    }
    if (threadIdx.x == 0) __hip_atomic_store(a.cnt + bt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // epilogue: y = fl(fl(fl(acc) * ws[n]) * xs[m]) (+ bias[n]); 16-byte
  // streaming stores when the 4 columns are inside N and the row is 16-byte
  // aligned (the output passes the caches: 25 MB of fp32 at M = 1024,
  // N = 6144, whose write-back from L2 otherwise trails the last MFMA;
  // 23.5 -> 22.5 us per launch)
  const bool vec_ok = ((a.ldy & 3) == 0) && ((((uintptr_t)a.Y) & 15) == 0);
  if (a.out == OUT_F32_X4) {
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
        planes_epilogue(a, acc[i][j], (mg0 + wm * FM + i) * 16 + mrow, (ng0 + wn * FN + j) * 16 + ncol, e_ws[j],
                        e_b[j], e_xe[i], lane, vec_ok);
    bool bad = false;
#pragma unroll
    for (int i = 0; i < FM; i++) bad |= e_xe[i] == kXeNonFinite;
    if (bad && a.xraw) planes_fixup<FM, FN>(a, (mg0 + wm * FM) * 16 + mrow, (ng0 + wn * FN) * 16 + ncol, lane);
    return;
  }
#pragma unroll
  for (int i = 0; i < FM; i++) {
    const int m = (mg0 + wm * FM + i) * 16 + mrow;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int n = (ng0 + wn * FN + j) * 16 + ncol;
      if (n >= a.N) continue;
      const v4i c = acc[i][j];
      if (a.out == OUT_I32) {
        int32_t* yp = reinterpret_cast<int32_t*>(a.Y) + (size_t)m * a.ldy + n;
        if (vec_ok && n + 4 <= a.N) {
          st_stream(yp, make_int4(c[0], c[1], c[2], c[3]));
        } else {
          for (int r = 0; r < 4 && n + r < a.N; r++) yp[r] = c[r];
        }
        continue;
      }
      const float ws4[4] = {e_ws[j].x, e_ws[j].y, e_ws[j].z, e_ws[j].w};
      const float b4[4] = {e_b[j].x, e_b[j].y, e_b[j].z, e_b[j].w};
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        y[r] = __fmul_rn(__fmul_rn((float)c[r], ws4[r]), e_xs[i]);
        if (a.bias) y[r] = __fadd_rn(y[r], b4[r]);
      }
      float* yp = reinterpret_cast<float*>(a.Y) + (size_t)m * a.ldy + n;
      if (vec_ok && n + 4 <= a.N) {
        st_stream(yp, make_float4(y[0], y[1], y[2], y[3]));
      } else {
        for (int r = 0; r < 4 && n + r < a.N; r++) yp[r] = y[r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Column-split variant: the 4 waves of a work-group split the tile's N columns
// (wave w owns weight row groups ng0 + FN w .. ng0 + FN w + FN - 1) and all
// share its MT activation row groups.  Weight tiles are private to one wave,
// so they go from global memory straight into that wave's registers (one
// 16-byte load per lane per tile, already in MFMA operand order); only the
// shared activation tiles pass through an LDS ring.  Per 64-wide K stage and
// work-group: MT KiB copied into LDS, 4 MT KiB of LDS fragment reads, 4 FN KiB
// of register loads and 4 MT FN MFMAs (against 3 (MT + NT) KiB of LDS traffic
// in gemm_i8_lds_kernel with its 2 x 2 wave grid).
//
// Pipeline: stage s's copies and loads are issued D steps ahead (its weight
// registers are set s % (D + 1), its LDS buffer s % D).  Step s waits for
// stage s + 1, then one barrier makes its activation tiles visible and frees
// buffer s % D, whose copy for stage s + D follows; the MFMAs of stage s run
// interleaved with the fragment reads of stage s + 1 and the issue of stage
// s + D.  The loop is unrolled D + 1 times so every register set index is a
// compile-time constant.  Copies and loads are branch-free (the compiler's
// own vmcnt waits stay exact only over straight-line code): stages past the
// last one re-read the last k-block, and nothing reads what they bring in.
template <int MT, int FN, int D>
__global__ __launch_bounds__(256) void gemm_i8_wcol_kernel(GemmI8Args a) {
  constexpr int NW = 4, NT = NW * FN, PA = MT / NW;
  constexpr int NB = D + 1;          // weight register sets
  constexpr int PS = PA + FN;        // vector memory operations per wave per stage
  static_assert(MT % NW == 0, "activation copies must divide over the waves");
  static_assert(NB % 2 == 0, "fragment double buffer needs an even unroll");
  static_assert(PS * (D - 1) < 64, "vmcnt range");
  __shared__ uint4 sA[D * MT * 64];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  int tm, tn;
  tile_of(blockIdx.x, a.ntm, a.ntn, tm, tn, a.xa);
  const int mg0 = tm * MT, ng0 = tn * NT + wv * FN;

  const uint4* A4 = reinterpret_cast<const uint4*>(a.At) + lane;
  const uint4* B4 = reinterpret_cast<const uint4*>(a.Bt) + lane;
  const int KB = a.KB;
  const size_t astride = (size_t)a.MG * 64, bstride = (size_t)a.NG * 64;
  // rows / columns past the matrix edge re-read a valid tile (their
  // accumulators are never stored)
  const uint4* asrc[PA];
#pragma unroll
  for (int p = 0; p < PA; p++) asrc[p] = A4 + (size_t)min(mg0 + wv + NW * p, a.MG - 1) * 64;
  const uint4* bsrc[FN];
#pragma unroll
  for (int j = 0; j < FN; j++) bsrc[j] = B4 + (size_t)min(ng0 + j, a.NG - 1) * 64;
  const uint32_t sbase = lds_addr(sA);
  constexpr uint32_t SBYTES = MT * 1024;

  uint4 wb[NB][FN];
  auto copy_a = [&](int st, int p) {
    const uint4* g = asrc[p] + (size_t)min(st, KB - 1) * astride;
    dma_tile(g, sbase + (uint32_t)(st % D) * SBYTES + (uint32_t)(wv + NW * p) * 1024u);
  };
  auto load_b = [&](int st, int c, int j) { wb[c][j] = bsrc[j][(size_t)min(st, KB - 1) * bstride]; };

  // epilogue operands first (older than every copy, so the first wait covers them)
  const int mrow = lane & 15;
  const int ncol = (lane >> 4) * 4;
  float4 e_ws[FN], e_b[FN];
  float e_xs[MT];
#pragma unroll
  for (int j = 0; j < FN; j++) {
    const int n = (ng0 + j) * 16 + ncol;
    float w4[4], b4[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int nn = min(n + r, a.N - 1);
      w4[r] = a.ws[nn];
      b4[r] = a.bias ? a.bias[nn] : 0.0f;
    }
    e_ws[j] = make_float4(w4[0], w4[1], w4[2], w4[3]);
    e_b[j] = make_float4(b4[0], b4[1], b4[2], b4[3]);
  }
  int e_xe[MT];
#pragma unroll
  for (int i = 0; i < MT; i++) {
    const int m = min((mg0 + i) * 16 + mrow, a.M - 1);
    e_xs[i] = (a.out == OUT_I32 || a.out == OUT_F32_X4) ? 0.0f : a.xs[m];
    e_xe[i] = (a.out == OUT_F32_X4) ? a.xe[m >> 2] : 0;
  }

  v4i acc[MT][FN];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

  uint4 fa[2][MT];
  auto read_frags = [&](int st, int c) {
    const uint4* buf = sA + (size_t)(st % D) * (MT * 64);
#pragma unroll
    for (int i = 0; i < MT; i++) fa[c][i] = buf[i * 64 + lane];
  };

  // prologue: stages 0 .. D-1 in flight, stage 0 visible and its fragments read
#pragma unroll
  for (int b = 0; b < D; b++) {
#pragma unroll
    for (int p = 0; p < PA; p++) copy_a(b, p);
#pragma unroll
    for (int j = 0; j < FN; j++) load_b(b, b, j);
  }
  wait_vm<PS * (D - 1)>();
  stage_barrier();
  read_frags(0, 0);

  // step s (set b = s % NB, fragment set f = s & 1)
  auto step = [&](int st, int b, int f) {
    wait_vm<PS * (D - 2)>();   // stage s + 1 landed (this wave's part)
    wait_lgkm0();              // this wave's reads of stage s are done
    stage_barrier();           // stage s + 1 visible; buffer s % D free
    constexpr int NMEM = MT + PS;
    const int nb = (b + D) % NB;
    auto mem_op = [&](int q) {
      if (q < PA) copy_a(st + D, q);
      else if (q < PS) load_b(st + D, nb, q - PA);
      else {
        const uint4* buf = sA + (size_t)((st + 1) % D) * (MT * 64);
        fa[f ^ 1][q - PS] = buf[(q - PS) * 64 + lane];
      }
    };
#pragma unroll
    for (int m = 0; m < MT * FN; m++) {
      const int i = m / FN, j = m % FN;
      acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, wb[b][j]),
                                                        __builtin_bit_cast(v4i, fa[f][i]), acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (m < NMEM) mem_op(m);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q = MT * FN; q < NMEM; q++) mem_op(q);
    __builtin_amdgcn_sched_barrier(0);
  };
  const int kfull = KB - KB % NB;
  for (int st = 0; st < kfull; st += NB) {
#pragma unroll
    for (int b = 0; b < NB; b++) step(st + b, b, b & 1);
  }
#pragma unroll
  for (int b = 0; b < NB - 1; b++)
    if (kfull + b < KB) step(kfull + b, b, b & 1);

  wait_vm<0>();   // no copy may still be landing in LDS when the work-group exits

  const bool vec_ok = ((a.ldy & 3) == 0) && ((((uintptr_t)a.Y) & 15) == 0);
  if (a.out == OUT_F32_X4) {
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
        planes_epilogue(a, acc[i][j], (mg0 + i) * 16 + mrow, (ng0 + j) * 16 + ncol, e_ws[j], e_b[j], e_xe[i], lane,
                        vec_ok);
    bool bad = false;
#pragma unroll
    for (int i = 0; i < MT; i++) bad |= e_xe[i] == kXeNonFinite;
    if (bad && a.xraw) planes_fixup<MT, FN>(a, mg0 * 16 + mrow, ng0 * 16 + ncol, lane);
    return;
  }
#pragma unroll
  for (int i = 0; i < MT; i++) {
    const int m = (mg0 + i) * 16 + mrow;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int n = (ng0 + j) * 16 + ncol;
      if (n >= a.N) continue;
      const v4i c = acc[i][j];
      if (a.out == OUT_I32) {
        int32_t* yp = reinterpret_cast<int32_t*>(a.Y) + (size_t)m * a.ldy + n;
        if (vec_ok && n + 4 <= a.N) {
          st_stream(yp, make_int4(c[0], c[1], c[2], c[3]));
        } else {
          for (int r = 0; r < 4 && n + r < a.N; r++) yp[r] = c[r];
        }
        continue;
      }
      const float ws4[4] = {e_ws[j].x, e_ws[j].y, e_ws[j].z, e_ws[j].w};
      const float b4[4] = {e_b[j].x, e_b[j].y, e_b[j].z, e_b[j].w};
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        y[r] = __fmul_rn(__fmul_rn((float)c[r], ws4[r]), e_xs[i]);
        if (a.bias) y[r] = __fadd_rn(y[r], b4[r]);
      }
      float* yp = reinterpret_cast<float*>(a.Y) + (size_t)m * a.ldy + n;
      if (vec_ok && n + 4 <= a.N) {
        st_stream(yp, make_float4(y[0], y[1], y[2], y[3]));
      } else {
        for (int r = 0; r < 4 && n + r < a.N; r++) yp[r] = y[r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// planning and launch
// ---------------------------------------------------------------------------
// Measured on MI355X at M = 1024 (ring depth and stage width swept):
// cfg 0: 128 x 192 tiles (8 x 12 fragments), K stage 64, 4 buffers (80 KiB)
//        (N = 6144, K = 2048: 22.0 us; cfg 4 below takes its place)
// cfg 1:  64 x 128 tiles (4 x 8),  K stage 64, 8 buffers (96 KiB)
//        best for N = 2048, K = 6144 (256 work-groups)
// cfg 2: 128 x 128 tiles (8 x 8),  K stage 64, 8 buffers (128 KiB)
// cfg 3..7: column-split kernel (weights straight to registers)
//   3: 128 x 192, prefetch 3   4: 128 x 192, prefetch 5   5: 128 x 192, prefetch 7
//   6:  64 x 128, prefetch 7   7: 128 x 128, prefetch 7
static void i8_cfg(int cfg, int& mt, int& nt) {
  if (cfg == 0) { mt = 8; nt = 12; }
  else if (cfg == 1) { mt = 4; nt = 8; }
  else if (cfg == 2) { mt = 8; nt = 8; }
  else if (cfg <= 5) { mt = 8; nt = 12; }
  else if (cfg == 6) { mt = 4; nt = 8; }
  else { mt = 8; nt = 8; }
}

// tuning overrides; atomic, since a setter may run while other threads plan launches
static std::atomic<int> g_i8_force_cfg{-1};
static std::atomic<int> g_i8_force_split{0};
void gemm_i8_set_cfg(int cfg) { g_i8_force_cfg.store(cfg, std::memory_order_relaxed); }
void gemm_i8_set_split(int s) { g_i8_force_split.store(s > 0 ? s : 0, std::memory_order_relaxed); }

int gemm_i8_pick_cfg(int M, int N, int K) {
  const int force = g_i8_force_cfg.load(std::memory_order_relaxed);
  if (force >= 0) return force;
  (void)K;
  // 2048 rows and more (the 4 x 1200 plane rows of a 1200-token fp32 batch):
  // many tiles per CU, where the deepest weight prefetch on 64 x 128 tiles
  // measured best on every decoder shape (per layer 594 -> 442 us at 4800
  // rows); below, tiles that fill the CUs (at 1024-1200 rows cfg 6 was
  // faster on some shapes and slower on others)
  if (M >= 2048) return 6;
  const int MG = cdiv(M, 16), NG = cdiv(N, 16);
  // the configuration whose tile count best fills 256 CUs (at least one
  // full wave of work-groups, then the fewest idle CUs in the last wave).
  // 128 x 192 tiles run on the register-loaded weight kernel (cfg 4: 20.7 us
  // against 22.0 us for cfg 0 at M = 1024, N = 6144, K = 2048); at 64 x 128
  // the two kernels measured the same (23.7 / 24.0 us, N = 2048, K = 6144).
  int best = 2;
  double best_eff = -1.0;
  for (int cfg : {4, 1, 2}) {
    int mt, nt;
    i8_cfg(cfg, mt, nt);
    const int tiles = cdiv(MG, mt) * cdiv(NG, nt);
    const int waves = cdiv(tiles, 256);
    const double eff = (double)tiles / (waves * 256);
    if (eff > best_eff + 1e-9) {
      best_eff = eff;
      best = cfg;
    }
  }
  return best;
}

// Plan: configuration and K slices.  With fewer than 128 tiles (a few
// hundred rows over a narrow N: the int8 planes of 17..64 fp32 tokens, small
// W8A8 batches) and K >= 4096, the K range of every tile is split over up to
// 4 work-groups on the LDS-staged kernel (its configuration of the same
// tile); slices keep at least 16 k-blocks.  The merge costs three dependent
// memory round trips (partials stored, arrival counted, partials read back),
// about 3 us: at K = 2048 every split measured slower than none, at K = 4096
// and 6144 a split of 4 (3 from 64 tiles up, 2 from 96) was the fastest or
// within 3 % of it (2048 x 6144 at 128 plane rows: 28.5 -> 19.7 us).  The
// int32 partial sums are exact, so the result is the same bits for every split.
static void gemm_i8_plan(int M, int N, int K, int& cfg, int& split) {
  cfg = gemm_i8_pick_cfg(M, N, K);
  int mt, nt;
  i8_cfg(cfg, mt, nt);
  const int tiles = cdiv(cdiv(M, 16), mt) * cdiv(cdiv(N, 16), nt);
  const int KB = cdiv(K, 64);
  split = 1;
  if (tiles < 128 && KB >= 64) split = std::min(std::min(4, 256 / tiles), KB / 16);
  const int fs = g_i8_force_split.load(std::memory_order_relaxed);
  if (fs > 0) split = std::min(fs, KB);
  if (split > 1) {              // the LDS-staged kernel of the same tile
    if (cfg == 3 || cfg == 4 || cfg == 5) cfg = 0;
    else if (cfg == 6) cfg = 1;
    else if (cfg == 7) cfg = 2;
  }
}

void gemm_i8_needs(int M, int N, int K, size_t* part_bytes, size_t* counters) {
  int cfg, sp, mt, nt;
  gemm_i8_plan(M, N, K, cfg, sp);
  i8_cfg(cfg, mt, nt);
  const size_t tiles = (size_t)cdiv(cdiv(M, 16), mt) * cdiv(cdiv(N, 16), nt);
  *part_bytes = sp > 1 ? tiles * sp * (size_t)(256 * mt * nt) * sizeof(int32_t) : 0;
  *counters = sp > 1 ? tiles : 0;
}

hipError_t launch_gemm_i8(const GemmLaunch& L, hipStream_t st) {
  GemmI8Args a;
  a.At = static_cast<const uint8_t*>(L.A);
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
  a.MG = cdiv(L.M, 16);
  a.NG = cdiv(L.N, 16);
  a.out = L.out;
  a.zero_tile = L.zero_tile;
  if (L.out == OUT_F32_X4 && (!L.xe || L.M % 4 != 0)) return hipErrorInvalidValue;
  if (L.out != OUT_I32 && L.out != OUT_F32_X4 && !L.xs) return hipErrorInvalidValue;
  if (!L.zero_tile) return hipErrorInvalidValue;
  int cfg, sp;
  gemm_i8_plan(L.M, L.N, L.K, cfg, sp);
  int mt, nt;
  i8_cfg(cfg, mt, nt);
  a.ntm = cdiv(a.MG, mt);
  a.ntn = cdiv(a.NG, nt);
  a.S = sp;
  // XCD blocks of half the tile rows x a quarter of the columns where they
  // fill fewer L2 lines (rows of A plus rows of weights per XCD)
  a.xa = 1;
  if ((long long)a.ntm * a.ntn <= 256 && a.ntm % 2 == 0 && a.ntn % 4 == 0 &&
      a.ntm * mt / 2 + a.ntn * nt / 4 < a.ntm * mt + a.ntn * nt / 8)
    a.xa = 2;
  a.part = static_cast<int32_t*>(L.part);
  a.cnt = L.cnt;
  if (sp > 1 && (!a.part || !a.cnt || cfg > 2)) return hipErrorInvalidValue;
  const long long blocks_ll = (long long)a.ntm * a.ntn * sp;
  if (blocks_ll > 0x7fffffffLL) return hipErrorInvalidValue;
  const int blocks = (int)blocks_ll;
  switch (cfg) {
    case 0: hipLaunchKernelGGL((gemm_i8_lds_kernel<8, 12, 1, 4, 2, 2>), dim3(blocks), dim3(256), 0, st, a); break;
    case 1: hipLaunchKernelGGL((gemm_i8_lds_kernel<4, 8, 1, 8, 2, 2>), dim3(blocks), dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL((gemm_i8_lds_kernel<8, 8, 1, 8, 2, 2>), dim3(blocks), dim3(256), 0, st, a); break;
    case 3: hipLaunchKernelGGL((gemm_i8_wcol_kernel<8, 3, 3>), dim3(blocks), dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL((gemm_i8_wcol_kernel<8, 3, 5>), dim3(blocks), dim3(256), 0, st, a); break;
    case 5: hipLaunchKernelGGL((gemm_i8_wcol_kernel<8, 3, 7>), dim3(blocks), dim3(256), 0, st, a); break;
    case 6: hipLaunchKernelGGL((gemm_i8_wcol_kernel<4, 2, 7>), dim3(blocks), dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((gemm_i8_wcol_kernel<8, 2, 7>), dim3(blocks), dim3(256), 0, st, a); break;
  }
  return hipGetLastError();
}

}  // namespace tl

extern "C" void tlk_gemm_i8_set_cfg(int cfg) { tl::gemm_i8_set_cfg(cfg); }
extern "C" void tlk_gemm_i8_set_split(int s) { tl::gemm_i8_set_split(s); }
