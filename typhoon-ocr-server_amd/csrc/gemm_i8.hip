// gemm_i8.hip -- W8A8 prefill GEMM: int8 codes x int8 weights on
// v_mfma_i32_16x16x64_i8 with LDS-staged, double-buffered K stages.
//
// Reference: kernel/w8a8_kernel.c:259-268 (w8a8_gemm dequantizes both
// operands and calls cblas_sgemm).  Here the int32 sum is exact and the fp32
// epilogue is y = fl(fl(fl(acc) * ws[n]) * xs[m]) (+ bias[n] as its own
// rounding), ~4e-7 relative L2 from the reference's dequant-then-SGEMM.
//
// Both operands are stored as 16x64 int8 tiles (tl_common.h), so a K stage
// of the work-group's A rows and B columns is a list of whole 1 KiB tiles:
// each is copied global -> registers -> LDS with one 16-byte load and one
// 16-byte LDS store per lane, and every MFMA operand is read back with one
// ds_read_b128 per lane at consecutive addresses (no bank conflicts, no
// swizzle needed).  The next stage's global loads are in flight while the
// current stage's MFMAs run; one barrier per stage.
//
// Work-group tile (16 MT) x (16 NT); waves WM x WN each own a
// (16 MT/WM) x (16 NT/WN) block of 16x16 accumulators.  Tiles are ordered so
// that the work-groups placed on one XCD (dispatch is round-robin over the 8
// XCDs) share a band of B columns and all of A, which then stays in that
// XCD's 4 MB L2.
#include "tl_common.h"
#include "tl_kernels.h"

namespace tl {

struct GemmI8Args {
  const uint8_t* At;    // activation code tiles [MG][KB]
  const uint8_t* Bt;    // weight tiles [NG][KB]
  const float* ws;      // [N]
  const float* xs;      // [M]
  const float* bias;    // [N] or null
  void* Y;              // fp32 [M][ldy] or int32 (OUT_I32)
  int ldy;
  int M, N, K, KB, MG, NG;
  int ntm, ntn;         // work-group tiles along M and N
  int out;
};

template <int MT, int NT, int KT, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_i8_lds_kernel(GemmI8Args a) {
  constexpr int NW = WM * WN;
  constexpr int TA = MT * KT, TB = NT * KT, TS = TA + TB;  // tiles per stage
  static_assert(TS % NW == 0, "stage tiles must divide evenly over the waves");
  constexpr int PW = TS / NW;                              // tiles copied per wave per stage
  constexpr int FM = MT / WM, FN = NT / WN;                // 16x16 accumulators per wave
  static_assert(MT % WM == 0 && NT % WN == 0, "wave grid must divide the tile");

  __shared__ uint4 lds[2][TS * 64];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wv / WN, wn = wv % WN;

  // XCD-aware tile order: work-group b runs on XCD b % 8; consecutive XCD
  // slots walk M fastest within a band of N tiles.
  const int ntiles = a.ntm * a.ntn;
  int t = blockIdx.x;
  if (ntiles % 8 == 0) t = (blockIdx.x % 8) * (ntiles / 8) + blockIdx.x / 8;
  const int tn = t / a.ntm, tm = t - (t / a.ntm) * a.ntm;
  const int mg0 = tm * MT, ng0 = tn * NT;

  // global source of stage tile q at k-block offset kb (clamped: tiles past
  // the matrix edge or past K re-read a valid tile; their products land in
  // accumulators that are never stored, or are zeroed below for K)
  const uint4* A4 = reinterpret_cast<const uint4*>(a.At) + lane;
  const uint4* B4 = reinterpret_cast<const uint4*>(a.Bt) + lane;
  const int KB = a.KB;
  auto src = [&](int q, int kb) -> const uint4* {
    const int kk = q % KT;
    const int k = min(kb + kk, KB - 1);
    if (q < TA) {
      const int mg = min(mg0 + q / KT, a.MG - 1);
      return A4 + ((size_t)mg * KB + k) * 64;
    }
    const int ng = min(ng0 + (q - TA) / KT, a.NG - 1);
    return B4 + ((size_t)ng * KB + k) * 64;
  };

  v4i acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4i{0, 0, 0, 0};

  const int nst = cdiv(KB, KT);
  uint4 st[PW];
  // stage 0
#pragma unroll
  for (int p = 0; p < PW; p++) st[p] = *src(wv + NW * p, 0);
#pragma unroll
  for (int p = 0; p < PW; p++) {
    const int q = wv + NW * p;
    const bool kin = (q % KT) < KB;            // k-block inside K
    lds[0][q * 64 + lane] = kin ? st[p] : make_uint4(0, 0, 0, 0);
  }
  __syncthreads();

  for (int s = 0; s < nst; s++) {
    const int cur = s & 1;
    // next stage's loads in flight during this stage's MFMAs
    const int kbn = (s + 1) * KT;
#pragma unroll
    for (int p = 0; p < PW; p++) st[p] = *src(wv + NW * p, kbn);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int kk = 0; kk < KT; kk++) {
      uint4 fa[FM], fb[FN];
#pragma unroll
      for (int i = 0; i < FM; i++) fa[i] = lds[cur][((wm * FM + i) * KT + kk) * 64 + lane];
#pragma unroll
      for (int j = 0; j < FN; j++) fb[j] = lds[cur][(TA + (wn * FN + j) * KT + kk) * 64 + lane];
#pragma unroll
      for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, fa[i]),
                                                            __builtin_bit_cast(v4i, fb[j]), acc[i][j], 0, 0, 0);
    }

#pragma unroll
    for (int p = 0; p < PW; p++) {
      const int q = wv + NW * p;
      const bool kin = kbn + (q % KT) < KB;
      lds[cur ^ 1][q * 64 + lane] = kin ? st[p] : make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
  }

  // epilogue: lane l of 16x16 tile (i, j) holds rows 4(l>>4)+r, column l&15
  const int col = lane & 15;
  const int r0 = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < FM; i++) {
    const int mb = (mg0 + wm * FM + i) * 16 + r0;
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int n = (ng0 + wn * FN + j) * 16 + col;
      if (n >= a.N) continue;
      const float wsn = a.ws[n];
      const float bn = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = mb + r;
        if (m >= a.M) continue;
        if (a.out == OUT_I32) {
          reinterpret_cast<int32_t*>(a.Y)[(size_t)m * a.ldy + n] = acc[i][j][r];
        } else {
          float y = __fmul_rn(__fmul_rn((float)acc[i][j][r], wsn), a.xs[m]);
          if (a.bias) y = __fadd_rn(y, bn);
          reinterpret_cast<float*>(a.Y)[(size_t)m * a.ldy + n] = y;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// planning and launch
// ---------------------------------------------------------------------------
// cfg 0: 128 x 192 tiles (8 x 12 fragments), 4 waves of 64 x 96
// cfg 1:  64 x 128 tiles (4 x 8), 4 waves of 32 x 64
// cfg 2: 128 x 128 tiles (8 x 8), 4 waves of 64 x 64
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
  for (int cfg : {0, 2, 1}) {
    int mt, nt;
    i8_cfg(cfg, mt, nt);
    const int tiles = cdiv(MG, mt) * cdiv(NG, nt);
    const int waves = cdiv(tiles, 256);
    const double eff = (double)tiles / (waves * 256) * (cfg == 1 ? 0.8 : 1.0);
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
  if (L.out != OUT_I32 && !L.xs) return hipErrorInvalidValue;
  const int cfg = gemm_i8_pick_cfg(L.M, L.N, L.K);
  int mt, nt;
  i8_cfg(cfg, mt, nt);
  a.ntm = cdiv(a.MG, mt);
  a.ntn = cdiv(a.NG, nt);
  const int blocks = a.ntm * a.ntn;
  if (cfg == 0)
    hipLaunchKernelGGL((gemm_i8_lds_kernel<8, 12, 2, 2, 2>), dim3(blocks), dim3(256), 0, st, a);
  else if (cfg == 1)
    hipLaunchKernelGGL((gemm_i8_lds_kernel<4, 8, 2, 2, 2>), dim3(blocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((gemm_i8_lds_kernel<8, 8, 2, 2, 2>), dim3(blocks), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace tl
