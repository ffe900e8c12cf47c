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
#include "tl_common.h"
#include "tl_kernels.h"

namespace tl {

struct GemmI8Args {
  const uint8_t* At;    // activation code tiles [KB][MG]
  const uint8_t* Bt;    // weight tiles [KB][NG]
  const float* ws;      // [N]
  const float* xs;      // [M]
  const float* bias;    // [N] or null
  void* Y;              // fp32 [M][ldy] or int32 (OUT_I32)
  int ldy;
  int M, N, K, KB, MG, NG;
  int ntm, ntn;         // work-group tiles along M and N
  int out;
  const uint8_t* zero_tile;  // 1 KiB of zeros (source of k-blocks past K)
};

// Stage ring of NST buffers.  Every K stage is NW*PW whole 1 KiB tiles, each
// copied global -> LDS by one wave with one global_load_lds_dwordx4 (lane l
// writes bytes 16l..16l+15 of the tile, i.e. the tile layout itself).  Stage s
// lives in buffer s % NST; the ring is unrolled so every buffer is a distinct
// LDS object and the compiler keeps only the explicit waits below:
//   wait until this wave's copies of stage s landed (vmcnt <= later stages),
//   wait until this wave's LDS reads of stage s-1 finished (lgkmcnt 0),
//   barrier (stage s visible to all waves, buffer of stage s-1 free),
//   issue the copies of stage s+NST-1 into the freed buffer,
//   MFMAs of stage s.
template <int MT, int NT, int KT, int NST, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_i8_lds_kernel(GemmI8Args a) {
  constexpr int NW = WM * WN;
  constexpr int TA = MT * KT, TB = NT * KT, TS = TA + TB;  // tiles per stage
  static_assert(TS % NW == 0, "stage tiles must divide evenly over the waves");
  constexpr int PW = TS / NW;                              // tiles copied per wave per stage
  constexpr int FM = MT / WM, FN = NT / WN;                // 16x16 accumulators per wave
  static_assert(MT % WM == 0 && NT % WN == 0, "wave grid must divide the tile");
  static_assert(NST >= 2 && NST <= 8, "2..8 stage buffers");
  static_assert(PW * (NST - 2) < 64, "vmcnt range");

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
  // one XCD walk M fastest within a band of N tiles.
  const int ntiles = a.ntm * a.ntn;
  int t = blockIdx.x;
  if (ntiles % 8 == 0) t = (blockIdx.x % 8) * (ntiles / 8) + blockIdx.x / 8;
  const int tn = t / a.ntm, tm = t - (t / a.ntm) * a.ntm;
  const int mg0 = tm * MT, ng0 = tn * NT;

  const uint4* A4 = reinterpret_cast<const uint4*>(a.At) + lane;
  const uint4* B4 = reinterpret_cast<const uint4*>(a.Bt) + lane;
  const uint4* Z4 = reinterpret_cast<const uint4*>(a.zero_tile) + lane;
  const int KB = a.KB;
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
      qsrc[p] = A4 + ((size_t)qk[p] * a.MG + mg) * 64;
      qstride[p] = (size_t)KT * a.MG * 64;
    } else {
      const int ng = min(ng0 + (q - TA) / KT, a.NG - 1);
      qsrc[p] = B4 + ((size_t)qk[p] * a.NG + ng) * 64;
      qstride[p] = (size_t)KT * a.NG * 64;
    }
  }
  auto issue = [&](int st, uint4* buf) {
    if (st >= nst) return;            // fewer copies only makes later waits stricter
    const uint32_t base = lds_addr(buf);
#pragma unroll
    for (int p = 0; p < PW; p++) {
      const uint4* g = (st * KT + qk[p] < KB) ? qsrc[p] + (size_t)st * qstride[p] : Z4;
      dma_tile(g, base + qlds[p]);
    }
  };

  // Accumulator tile (i, j) is computed transposed (B fragment as the MFMA's
  // first operand): lane l holds Y[m][n .. n+3] with m = 16 mg + (l & 15) and
  // n = 16 ng + 4 (l >> 4), so the epilogue stores 16 contiguous bytes per lane.
  // Its operands are loaded now so their latency hides behind the K loop.
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
#pragma unroll
  for (int i = 0; i < FM; i++) {
    const int m = min((mg0 + wm * FM + i) * 16 + mrow, a.M - 1);
    e_xs[i] = (a.out == OUT_I32) ? 0.0f : a.xs[m];
  }
  wait_vm<0>();   // the explicit waits below count only the tile copies

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

  // MFMAs of one stage; the fragments of k-block kk+1 are read from LDS while
  // the MFMAs of k-block kk run
  auto compute = [&](const uint4* buf) {
    uint4 fa[2][FM], fb[2][FN];
#pragma unroll
    for (int i = 0; i < FM; i++) fa[0][i] = buf[((wm * FM + i) * KT) * 64 + lane];
#pragma unroll
    for (int j = 0; j < FN; j++) fb[0][j] = buf[(TA + (wn * FN + j) * KT) * 64 + lane];
#pragma unroll
    for (int kk = 0; kk < KT; kk++) {
      const int c = kk & 1;
      if (kk + 1 < KT) {
#pragma unroll
        for (int i = 0; i < FM; i++) fa[c ^ 1][i] = buf[((wm * FM + i) * KT + kk + 1) * 64 + lane];
#pragma unroll
        for (int j = 0; j < FN; j++) fb[c ^ 1][j] = buf[(TA + (wn * FN + j) * KT + kk + 1) * 64 + lane];
      }
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, fb[c][j]),
                                                            __builtin_bit_cast(v4i, fa[c][i]), acc[i][j], 0, 0, 0);
    }
  };

  // one ring step: stage st is in `cur`; stage st+NST-1 goes into `nxt`
  auto step = [&](int st, const uint4* cur, uint4* nxt) {
    wait_vm<PW * (NST - 2)>();
    wait_lgkm0();
    stage_barrier();
    issue(st + NST - 1, nxt);
    if (st < nst) compute(cur);
  };

  // prologue: stages 0 .. NST-2 in flight
#pragma unroll
  for (int b = 0; b < NST - 1; b++) issue(b, ring[b]);
  // ring unrolled NST times: every buffer index below is a compile-time
  // constant, so each access names one LDS object
  for (int st = 0; st < nst; st += NST) {
#pragma unroll
    for (int b = 0; b < NST; b++) step(st + b, ring[b], ring[(b + NST - 1) % NST]);
  }

  wait_vm<0>();   // no copy may still be landing in LDS when the work-group exits

  // epilogue: y = fl(fl(fl(acc) * ws[n]) * xs[m]) (+ bias[n]); 16-byte stores
  // when the 4 columns are inside N and the row is 16-byte aligned
  const bool vec_ok = ((a.ldy & 3) == 0) && ((((uintptr_t)a.Y) & 15) == 0);
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
          *reinterpret_cast<int4*>(yp) = make_int4(c[0], c[1], c[2], c[3]);
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
        *reinterpret_cast<float4*>(yp) = make_float4(y[0], y[1], y[2], y[3]);
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
//        best for N = 6144, K = 2048 (256 work-groups)
// cfg 1:  64 x 128 tiles (4 x 8),  K stage 64, 8 buffers (96 KiB)
//        best for N = 2048, K = 6144 (256 work-groups)
// cfg 2: 128 x 128 tiles (8 x 8),  K stage 64, 8 buffers (128 KiB)
static void i8_cfg(int cfg, int& mt, int& nt) {
  if (cfg == 0) { mt = 8; nt = 12; }
  else if (cfg == 1) { mt = 4; nt = 8; }
  else { mt = 8; nt = 8; }
}

static int g_i8_force_cfg = -1;
void gemm_i8_set_cfg(int cfg) { g_i8_force_cfg = cfg; }

int gemm_i8_pick_cfg(int M, int N, int K) {
  if (g_i8_force_cfg >= 0) return g_i8_force_cfg;
  (void)K;
  const int MG = cdiv(M, 16), NG = cdiv(N, 16);
  // the configuration whose tile count best fills 256 CUs (at least one
  // full wave of work-groups, then the fewest idle CUs in the last wave)
  int best = 2;
  double best_eff = -1.0;
  for (int cfg : {0, 1, 2}) {
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

hipError_t launch_gemm_i8(const GemmLaunch& L, hipStream_t st) {
  GemmI8Args a;
  a.At = static_cast<const uint8_t*>(L.A);
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
  a.out = L.out;
  a.zero_tile = L.zero_tile;
  if (L.out != OUT_I32 && !L.xs) return hipErrorInvalidValue;
  if (!L.zero_tile) return hipErrorInvalidValue;
  const int cfg = gemm_i8_pick_cfg(L.M, L.N, L.K);
  int mt, nt;
  i8_cfg(cfg, mt, nt);
  a.ntm = cdiv(a.MG, mt);
  a.ntn = cdiv(a.NG, nt);
  const int blocks = a.ntm * a.ntn;
  if (cfg == 0)
    hipLaunchKernelGGL((gemm_i8_lds_kernel<8, 12, 1, 4, 2, 2>), dim3(blocks), dim3(256), 0, st, a);
  else if (cfg == 1)
    hipLaunchKernelGGL((gemm_i8_lds_kernel<4, 8, 1, 8, 2, 2>), dim3(blocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_i8_lds_kernel<8, 8, 1, 8, 2, 2>), dim3(blocks), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace tl
