// gemm_b16.hip -- prefill GEMMs with 16-bit MFMAs over int8 weight tiles:
//   A_BF16  W8A16 (kernel/w8a16_kernel.c:203-216): bf16 X x int8 W (exact in
//           bf16) on v_mfma_f32_16x16x32_bf16, fp32 accumulation, fp32 scale
//           after the sum, fp32 / bf16 (RNE) / fp16 output.
//   A_F16   the same with fp16 X on v_mfma_f32_16x16x32_f16.
//
// Same skeleton as gemm_i8.hip: a ring of NST LDS stage buffers filled by
// direct global -> LDS copies (one 16-byte piece per lane per copy), one
// barrier per 64-wide K stage, transposed accumulators (weights as the MFMA's
// first operand) so each lane stores 4 consecutive output columns.
//
// Within a 64-wide K block the int8 weight tile gives lane l row (l & 15) and
// k = 16 (l >> 4) + 0..15; the bf16 MFMA consumes 8 k per lane, so the block
// is two MFMAs, half h taking k = 16 (l >> 4) + 8 h + 0..7.  X (row-major in
// memory) is copied a whole 128-byte row segment per 8 lanes into a swizzled
// row-major LDS tile (xtile_* below: 2 copies per row group and K block), and
// a wave reads each MFMA operand with one conflict-free ds_read_b128.  (Copies
// in MFMA operand order, lane l reading 16 bytes of row l & 15, spread every
// copy over 16 half-used lines: about 10 B/clk per CU against the int8
// GEMM's 22-38.)  Weight tiles stay int8 and are widened to bf16/fp16 in
// registers after the read.  Lanes whose row is past M or whose k is past K
// copy 16 bytes of zeros.
#include <algorithm>
#include <atomic>

#include "tl_common.h"
#include "tl_kernels.h"

typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));

namespace tl {

struct GemmB16Args {
  const void* X;         // row-major [M][lda], element type per AMODE
  int lda;
  const uint8_t* Bt;     // weight tiles [KB][NG]
  const float* ws;       // [N]
  const float* bias;     // [N] or null
  void* Y;
  int ldy;
  int M, N, K, KB, MG, NG;
  int ntm, ntn;
  int ep, out;
  const uint8_t* zero_tile;
  int S;                 // K slices per tile (work-groups per tile)
  float* part;           // S > 1: fp32 partial tiles [tiles][S][MT*16 x NT*16]
  uint32_t* cnt;         // S > 1: zeroed arrival counters [tiles]
};

__device__ inline v8bf as_bf(uint4 u) { return __builtin_bit_cast(v8bf, u); }
__device__ inline v8h_t as_h(uint4 u) { return __builtin_bit_cast(v8h_t, u); }

// int8 weight lane (16 values) -> two 8-wide 16-bit operands (exact)
template <int AMODE>
__device__ inline void widen(uint4 w, uint4& h0, uint4& h1) {
  const uint32_t d[4] = {w.x, w.y, w.z, w.w};
  uint32_t o[8];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const float f0 = (float)(int8_t)(d[q] & 0xff), f1 = (float)(int8_t)((d[q] >> 8) & 0xff);
    const float f2 = (float)(int8_t)((d[q] >> 16) & 0xff), f3 = (float)(int8_t)(d[q] >> 24);
    if constexpr (AMODE == A_F16) {
      const _Float16 h0f = (_Float16)f0, h1f = (_Float16)f1, h2f = (_Float16)f2, h3f = (_Float16)f3;
      o[2 * q] = (uint32_t)__builtin_bit_cast(uint16_t, h0f) | ((uint32_t)__builtin_bit_cast(uint16_t, h1f) << 16);
      o[2 * q + 1] = (uint32_t)__builtin_bit_cast(uint16_t, h2f) | ((uint32_t)__builtin_bit_cast(uint16_t, h3f) << 16);
    } else {
      // |w| <= 127 is exact in bf16: the high halves of the floats, paired by
      // one byte permute (bytes 2, 3 of f0 then bytes 2, 3 of f1)
      o[2 * q] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
      o[2 * q + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
    }
  }
  h0 = make_uint4(o[0], o[1], o[2], o[3]);
  h1 = make_uint4(o[4], o[5], o[6], o[7]);
}


template <int AMODE>
__device__ inline v4f mfma16(uint4 w, uint4 x, v4f c) {
  if constexpr (AMODE == A_F16) return __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h(w), as_h(x), c, 0, 0, 0);
  else return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(w), as_bf(x), c, 0, 0, 0);
}

// X tiles in LDS.  A row group's 64-wide K block of X (16 rows x 128 bytes)
// is two 1 KiB copies, rows 0-7 and 8-15.  Copy half j: lane l fetches row
// 8 j + (l >> 3), 16-byte chunk (l & 7) ^ (l >> 3) ^ j of the row (so every
// 8 lanes read one whole 128-byte line of X), and its 16 bytes land at
// 16 l.  The XOR swizzle spreads the chunks that one MFMA operand read takes
// from 16 rows (lane l: row l & 15, chunk 2 (l >> 4) + h) over distinct
// bank groups.  Both functions are per-lane constants.
__device__ __forceinline__ int xtile_row(int lane, int j) { return 8 * j + (lane >> 3); }
__device__ __forceinline__ int xtile_chunk(int lane, int j) { return (lane & 7) ^ (lane >> 3) ^ j; }
// uint4 index, within a row group's two copies, of lane's operand for K half h
// (X[row lane & 15][16 (lane >> 4) + 8 h .. + 7])
__device__ __forceinline__ int xtile_frag(int lane, int h) {
  const int rr = lane & 15, j = rr >> 3, r8 = rr & 7;
  const int kc = 2 * (lane >> 4) + h;
  return j * 64 + r8 * 8 + (kc ^ r8 ^ j);
}

// The end of a tile's work-group: with K slices (a.S > 1) the K-slice merge,
// then the epilogue (scale, bias, conversion, stores).  acc[i][j] holds row
// group rg0 + i (lane: row lane & 15) and column group cg0 + j (lane: columns
// 4 (lane >> 4) .. + 3); slot0 + i is this wave's slot of row i in the
// partial tile (the slots of the waves of a work-group do not overlap).
template <int FM, int FN>
__device__ __forceinline__ void b16_finish(const GemmB16Args& a, v4f (&acc)[FM][FN], int rg0, int cg0, int slot0,
                                           int bt, int ks, const float (&e_ws)[FN][4], const float (&e_b)[FN][4]) {
  const int lane = threadIdx.x & 63;
  const int mrow = lane & 15;
  const int ncol = (lane >> 4) * 4;
  if (a.S > 1) {
    // K slices: every work-group of the tile stores its fp32 sums, waits for
    // the stores' acknowledgement and counts in; the last to arrive adds the
    // S slices in slice order (its own from registers, the same sums and
    // order whichever work-group merges), then runs the epilogue below
    constexpr int TF = 4 * FM * FN * 256;         // floats per partial tile: 4 waves x FM x FN fragments
    float* mine = a.part + ((size_t)bt * a.S + ks) * TF;
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++) st_agent4(mine + (((slot0 + i) * FN + j) * 64 + lane) * 4, acc[i][j]);
    __shared__ int s_last;
    asm volatile("" ::: "memory");
    wait_vm<0>();                               // this thread's partial stores are acknowledged
    asm volatile("" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
      s_last = __hip_atomic_fetch_add(a.cnt + bt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(a.S - 1);
    __syncthreads();
    if (!s_last) return;
    // the merger's acquire: the slices are read after the counter showed
    // them all arrived (agent scope, once per tile: it invalidates this
    // CU's caches, so the plain 16-byte loads below fetch what the stores
    // wrote through).  All S slices come from memory, this work-group's own
    // too (the values it stored), one slice's loads in flight at a time and
    // added in slice order.
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // QB slices' loads are in flight together (indices past S re-read the
    // last slice and are not added)
    constexpr int QB = FM * FN <= 2 ? 8 : (FM * FN <= 8 ? 4 : 1);
    const float* slices = a.part + (size_t)bt * a.S * TF;
    for (int q0 = 0; q0 < a.S; q0 += QB) {
      v4f p[QB][FM][FN];
#pragma unroll
      for (int u = 0; u < QB; u++)
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++)
            p[u][i][j] = *reinterpret_cast<const v4f*>(slices + (size_t)min(q0 + u, a.S - 1) * TF +
                                                      (((slot0 + i) * FN + j) * 64 + lane) * 4);
#pragma unroll
      for (int u = 0; u < QB; u++) {
        if (q0 + u >= a.S) break;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 4; r++)
              acc[i][j][r] = q0 + u == 0 ? p[u][i][j][r] : __fadd_rn(acc[i][j][r], p[u][i][j][r]);
      }
    }
    if (threadIdx.x == 0) __hip_atomic_store(a.cnt + bt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  const bool vec_ok = ((a.ldy & 3) == 0) &&
                      ((((uintptr_t)a.Y) & (a.out == OUT_F32 ? 15 : 7)) == 0);
#pragma unroll
  for (int i = 0; i < FM; i++) {
    const int m = (rg0 + i) * 16 + mrow;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < FN; j++) {
      const int n = (cg0 + j) * 16 + ncol;
      if (n >= a.N) continue;
      float y[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float c = acc[i][j][r];
        if (a.ep == EP_SCALE_FMA) {
          y[r] = __fmaf_rn(c, e_ws[j][r], e_b[j][r]);
        } else {
          y[r] = __fmul_rn(c, e_ws[j][r]);
          if (a.bias) y[r] = __fadd_rn(y[r], e_b[j][r]);
        }
      }
      const size_t o = (size_t)m * a.ldy + n;
      const bool full = vec_ok && n + 4 <= a.N;
      if (a.out == OUT_F32) {
        float* yp = reinterpret_cast<float*>(a.Y) + o;
        if (full) st_stream(yp, make_float4(y[0], y[1], y[2], y[3]));   // streaming, as the int8 GEMM's
        else for (int r = 0; r < 4 && n + r < a.N; r++) yp[r] = y[r];
      } else {
        uint16_t hv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          if (a.out == OUT_BF16) {
            hv[r] = (uint16_t)f32_to_bf16_rne(y[r]);
          } else {
            const _Float16 h = (_Float16)y[r];
            hv[r] = __builtin_bit_cast(uint16_t, h);
          }
        }
        uint16_t* yp = reinterpret_cast<uint16_t*>(a.Y) + o;
        if (full) *reinterpret_cast<uint2*>(yp) = make_uint2(hv[0] | ((uint32_t)hv[1] << 16), hv[2] | ((uint32_t)hv[3] << 16));
        else for (int r = 0; r < 4 && n + r < a.N; r++) yp[r] = hv[r];
      }
    }
  }
}

// KF: K is a multiple of 64 (every copy a per-lane offset from a uniform
// per-stage base; the general path masks pieces past K and rows past M)
template <int AMODE, int MT, int NT, int NST, int WM, int WN, bool KF>
__global__ __launch_bounds__(64 * WM * WN) void gemm_b16_lds_kernel(GemmB16Args a) {
  constexpr int NW = WM * WN;
  constexpr int AP = 2;                                // A copies per (row group, K block)
  constexpr int ESZ = 2;                               // bytes per X element
  constexpr int EPC = 16 / ESZ;                        // X elements per copy per lane
  constexpr int TA = MT * AP, TB = NT, TS = TA + TB;
  static_assert(TS % NW == 0, "stage copies must divide evenly over the waves");
  constexpr int PW = TS / NW;
  constexpr int FM = MT / WM, FN = NT / WN;
  static_assert(MT % WM == 0 && NT % WN == 0, "wave grid must divide the tile");
  static_assert(NST >= 2 && NST <= 8 && NST % 2 == 0, "2, 4, 6 or 8 stage buffers");
  static_assert(PW * (NST - 1) < 64, "vmcnt range");

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

  // work-group b: K slice b / ntiles of tile b % ntiles; with ntiles a
  // multiple of 8 the tiles are grouped per XCD (b % 8) as ntiles / 8
  // consecutive tile indices
  const int ntiles = a.ntm * a.ntn;
  const int ks = blockIdx.x / ntiles;
  const int bt = blockIdx.x - ks * ntiles;
  int t = bt;
  if (ntiles % 8 == 0) t = (bt % 8) * (ntiles / 8) + bt / 8;
  const int tn = t / a.ntm, tm = t - (t / a.ntm) * a.ntm;
  const int mg0 = tm * MT, ng0 = tn * NT;

  const uint4* B4 = reinterpret_cast<const uint4*>(a.Bt) + lane;
  const uint4* Z4 = reinterpret_cast<const uint4*>(a.zero_tile);   // any 16 zero bytes
  const char* Xb = static_cast<const char*>(a.X);
  const int KB = a.KB;
  const int kb0 = (ks * KB) / a.S;                     // this work-group's K blocks [kb0, kb0 + nst)
  const int nst = ((ks + 1) * KB) / a.S - kb0;

  // per copy: source for stage 0 and its advance per stage
  const char* qsrc[PW];
  int qkoff[PW];                // X column of this lane's piece at stage 0 (A copies), -1 for B
  bool qrow_ok[PW];
  uint32_t qlds[PW];
#pragma unroll
  for (int p = 0; p < PW; p++) {
    const int q = wv + NW * p;
    qlds[p] = (uint32_t)q * 1024u;
    if (q < TA) {
      const int i = q / AP, j = q % AP;
      const int row = (mg0 + i) * 16 + xtile_row(lane, j);
      const int koff = EPC * xtile_chunk(lane, j);
      qrow_ok[p] = row < a.M;
      qkoff[p] = koff;
      qsrc[p] = Xb + ((size_t)min(row, a.M - 1) * a.lda + koff) * ESZ;
    } else {
      const int ng = min(ng0 + (q - TA), a.NG - 1);
      qrow_ok[p] = true;
      qkoff[p] = -1;
      qsrc[p] = reinterpret_cast<const char*>(B4 + (size_t)ng * 64);
    }
  }
  const size_t bstride = (size_t)a.NG * 1024;   // bytes between K blocks of the weights
  // Every call issues exactly PW copies, so the explicit vmcnt waits in `step`
  // count exactly: stages past the end of the work-group's K range re-read its
  // last K block into a buffer that no step reads again.  (Skipping those
  // copies would let the last NST-2 steps' waits return before their own
  // stage had landed; waiting for every copy there instead measured 7% slower
  // at M = 64..256.)
  // K a multiple of 64 (no piece past K) and X under 4 GiB (the launcher's
  // condition for KF): each copy is a 32-bit per-lane byte offset from a
  // uniform per-stage base (rows past M read row M - 1; their outputs are
  // never stored)
  constexpr bool kfull = KF;
  uint32_t qvo[PW];
#pragma unroll
  for (int p = 0; p < PW; p++)
    qvo[p] = (uint32_t)(qsrc[p] - (qkoff[p] >= 0 ? Xb : reinterpret_cast<const char*>(a.Bt)));
  auto issue = [&](int st, uint4* buf) {
    const int sc = kb0 + min(st, nst - 1);
    const uint32_t base = lds_addr(buf);
    if constexpr (kfull) {
      const char* sa = Xb + (size_t)sc * 64 * ESZ;
      const char* sb = reinterpret_cast<const char*>(a.Bt) + (size_t)sc * bstride;
#pragma unroll
      for (int p = 0; p < PW; p++) dma_tile_s(qvo[p], (wv + NW * p < TA) ? sa : sb, base + qlds[p]);
    } else {
#pragma unroll
      for (int p = 0; p < PW; p++) {
        const uint4* g;
        if (qkoff[p] >= 0) {
          const int k = sc * 64 + qkoff[p];
          g = (qrow_ok[p] && k < a.K) ? reinterpret_cast<const uint4*>(qsrc[p] + (size_t)sc * 64 * ESZ) : Z4;
        } else {
          g = reinterpret_cast<const uint4*>(qsrc[p] + (size_t)sc * bstride);
        }
        dma_tile(g, base + qlds[p]);
      }
    }
  };

  // prologue: stages 0 .. NST-1 in flight first
#pragma unroll
  for (int b = 0; b < NST; b++) issue(b, ring[b]);
  // epilogue operands (transposed accumulators: lane holds row m, cols
  // n..n+3), loaded behind the first copies: the stage waits below then
  // also cover them (loads complete in issue order, so the extra loads only
  // make the first waits stricter), and the loop's last wait leaves them done
  const int ncol = (lane >> 4) * 4;
  float e_ws[FN][4], e_b[FN][4];
#pragma unroll
  for (int j = 0; j < FN; j++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int n = min((ng0 + wn * FN + j) * 16 + ncol + r, a.N - 1);
      e_ws[j][r] = a.ws[n];
      e_b[j][r] = a.bias ? a.bias[n] : 0.0f;
    }

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // A stage's fragments are read from LDS into a register set one step ahead
  // of their MFMAs (two sets, so the read latency hides behind the previous
  // stage's MFMAs): set c holds the stage's A copies of this wave's row
  // groups and its raw int8 weight tiles.
  uint4 fa[2][FM * AP], fb[2][FN];
  const int xf[AP] = {xtile_frag(lane, 0), xtile_frag(lane, 1)};
  auto read_frags = [&](const uint4* buf, int c) {
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int h = 0; h < AP; h++) fa[c][i * AP + h] = buf[(wm * FM + i) * AP * 64 + xf[h]];
#pragma unroll
    for (int j = 0; j < FN; j++) fb[c][j] = buf[(TA + wn * FN + j) * 64 + lane];
  };

  // Column by column: the MFMAs of weight column j (both K halves of every
  // row group) run interleaved with the widening of column j + 1, so the
  // VALU work of the int8 -> 16-bit conversion hides under the matrix pipe
  // (all widening first, then all MFMAs, left them back to back).
  auto compute = [&](int c) {
    uint4 wcur[2], wnxt[2];
    widen<AMODE>(fb[c][0], wcur[0], wcur[1]);
#pragma unroll
    for (int j = 0; j < FN; j++) {
      if (j + 1 < FN) widen<AMODE>(fb[c][j + 1], wnxt[0], wnxt[1]);
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int i = 0; i < FM; i++) acc[i][j] = mfma16<AMODE>(wcur[h], fa[c][i * AP + h], acc[i][j]);
      if (j + 1 < FN) {
#pragma unroll
        for (int q = 0; q < 2 * FM; q++) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // then three VALU
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      wcur[0] = wnxt[0];
      wcur[1] = wnxt[1];
    }
  };

  // Step s (register set c = s & 1 holds stage s):
  //   wait until this wave's copies of stage s+1 landed (later stages may
  //   still fly) and its reads of stage s completed; barrier: stage s+1 is
  //   visible and every wave is done reading stage s's buffer;
  //   read stage s+1's fragments, refill stage s's buffer with stage s+NST,
  //   then widen and multiply stage s from registers (steps past the last
  //   stage only keep the copy count exact).
  auto step = [&](int st, uint4* cur, const uint4* nxt, int c) {
    wait_vm<PW * (NST - 2)>();
    wait_lgkm0();
    stage_barrier();
    read_frags(nxt, c ^ 1);
    issue(st + NST, cur);
    __builtin_amdgcn_sched_barrier(0);
    if (st < nst) compute(c);
    __builtin_amdgcn_sched_barrier(0);
  };

  // stage 0 landed (and the epilogue operands), its fragments read
  wait_vm<PW * (NST - 1)>();
  stage_barrier();
  read_frags(ring[0], 0);
  // ring unrolled NST times (NST even: every step's register set is a
  // compile-time constant)
  for (int st = 0; st < nst; st += NST) {
#pragma unroll
    for (int b = 0; b < NST; b++) step(st + b, ring[b], ring[(b + 1) % NST], b & 1);
  }
  wait_vm<0>();   // no copy may still be landing in LDS when the work-group exits

  b16_finish<FM, FN>(a, acc, mg0 + wm * FM, ng0 + wn * FN, wv * FM, bt, ks, e_ws, e_b);
}

// One output dword of the widening: int8 elements 2p, 2p + 1 of a lane's 16
// (dword p / 2, bytes 2 (p % 2), + 1) as two 16-bit values, exact
template <int AMODE>
__device__ __forceinline__ uint32_t widen_pair(uint4 w, int p) {
  const uint32_t d = (p >> 1) == 0 ? w.x : ((p >> 1) == 1 ? w.y : ((p >> 1) == 2 ? w.z : w.w));
  const int sh = (p & 1) * 16;
  const float f0 = (float)(int8_t)((d >> sh) & 0xff), f1 = (float)(int8_t)((d >> (sh + 8)) & 0xff);
  if constexpr (AMODE == A_F16) {
    const _Float16 h0 = (_Float16)f0, h1 = (_Float16)f1;
    return (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
  } else {
    return __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  }
}
__device__ __forceinline__ void set_dword(uint4& u, int c, uint32_t v) {
  if (c == 0) u.x = v;
  else if (c == 1) u.y = v;
  else if (c == 2) u.z = v;
  else u.w = v;
}

// Column-split variant: the 4 waves split the tile's N columns (wave w owns
// weight row groups ng0 + FN w .. + FN - 1) and share its MT row groups of X.
// Each weight tile is private to one wave, so it goes from global memory
// straight into that wave's registers (one 16-byte load per lane per tile, in
// MFMA operand order) and is widened once per work-group; only the shared X
// tiles pass through the LDS ring (2 MT KiB per stage, so the ring holds D
// stages in 2 MT D KiB).  Per 64-wide K stage and work-group: 2 MT KiB
// copied into LDS, 8 MT KiB of fragment reads, 4 FN KiB of register loads,
// 8 MT FN MFMAs.
//
// Pipeline (as the int8 column-split kernel): stage s's copies and loads are
// issued D steps ahead (weight register set s % (D + 1), LDS buffer s % D).
// Step s waits for stage s + 1, one barrier makes its X tiles visible and
// frees buffer s % D, whose copy for stage s + D follows; the MFMAs of stage
// s run interleaved with the fragment reads of stage s + 1, the issue of
// stage s + D and the widening of the next weight column, two elements at a
// time between MFMAs.  Stages past the work-group's K range re-read its last
// K block (branch-free, so every wait counts exactly); nothing reads what
// they bring in.  K is a multiple of 64.
template <int AMODE, int MT, int FN, int D>
__global__ __launch_bounds__(256) void gemm_b16_wcol_kernel(GemmB16Args a) {
  constexpr int NW = 4, NT = NW * FN, AP = 2, ESZ = 2;
  constexpr int TA = MT * AP;          // X copies (1 KiB each) per stage
  constexpr int PA = TA / NW;          // ... per wave
  constexpr int NB = D + 1;            // weight register sets
  constexpr int PS = PA + FN;          // vector memory operations per wave per stage
  static_assert(TA % NW == 0, "X copies must divide over the waves");
  static_assert(NB % 2 == 0, "fragment double buffer needs an even unroll");
  static_assert(PS * (D - 1) < 64, "vmcnt range");
  __shared__ uint4 sA[D * TA * 64];

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // work-group b: K slice b / ntiles of tile b % ntiles (XCD-grouped tile
  // order as the LDS-staged kernel's)
  const int ntiles = a.ntm * a.ntn;
  const int ks = blockIdx.x / ntiles;
  const int bt = blockIdx.x - ks * ntiles;
  int t = bt;
  if (ntiles % 8 == 0) t = (bt % 8) * (ntiles / 8) + bt / 8;
  const int tn = t / a.ntm, tm = t - (t / a.ntm) * a.ntm;
  const int mg0 = tm * MT, ng0 = tn * NT + wv * FN;
  const int KB = a.KB;
  const int kb0 = (ks * KB) / a.S;
  const int nst = ((ks + 1) * KB) / a.S - kb0;

  // X copies: copy q = wv + NW p holds rows 8 (q % AP) .. + 7 of row group
  // q / AP in the swizzled layout of xtile_row / xtile_chunk (rows past M
  // read row M - 1; their outputs are never stored)
  const char* Xb = static_cast<const char*>(a.X);
  uint32_t avo[PA];
#pragma unroll
  for (int p = 0; p < PA; p++) {
    const int q = wv + NW * p;
    const int row = min((mg0 + q / AP) * 16 + xtile_row(lane, q % AP), a.M - 1);
    avo[p] = (uint32_t)(((size_t)row * a.lda + 8 * xtile_chunk(lane, q % AP)) * ESZ);
  }
  const uint4* B4 = reinterpret_cast<const uint4*>(a.Bt) + lane;
  const uint4* bsrc[FN];
#pragma unroll
  for (int j = 0; j < FN; j++) bsrc[j] = B4 + (size_t)min(ng0 + j, a.NG - 1) * 64;
  const size_t bstride = (size_t)a.NG * 64;
  const uint32_t sbase = lds_addr(sA);
  constexpr uint32_t SBYTES = TA * 1024;

  uint4 wb[NB][FN];
  auto copy_a = [&](int st, int p) {
    const int sc = kb0 + min(st, nst - 1);
    dma_tile_s(avo[p], Xb + (size_t)sc * 64 * ESZ, sbase + (uint32_t)(st % D) * SBYTES + (uint32_t)(wv + NW * p) * 1024u);
  };
  auto load_b = [&](int st, int c, int j) { wb[c][j] = bsrc[j][(size_t)(kb0 + min(st, nst - 1)) * bstride]; };

  // epilogue operands first (older than every copy, so the first wait covers them)
  const int ncol = (lane >> 4) * 4;
  float e_ws[FN][4], e_b[FN][4];
#pragma unroll
  for (int j = 0; j < FN; j++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int n = min((ng0 + j) * 16 + ncol + r, a.N - 1);
      e_ws[j][r] = a.ws[n];
      e_b[j][r] = a.bias ? a.bias[n] : 0.0f;
    }

  v4f acc[MT][FN];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < FN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  uint4 fa[2][TA];
  const int xf[AP] = {xtile_frag(lane, 0), xtile_frag(lane, 1)};
  auto read_frags = [&](int st, int c) {
    const uint4* buf = sA + (size_t)(st % D) * (TA * 64);
#pragma unroll
    for (int i = 0; i < TA; i++) fa[c][i] = buf[(i / AP) * AP * 64 + xf[i % AP]];
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

  // step s (weight set b = s % NB, fragment set f = s & 1)
  auto step = [&](int st, int b, int f) {
    wait_vm<PS * (D - 2)>();   // stage s + 1 landed (this wave's part)
    wait_lgkm0();              // this wave's reads of stage s are done
    stage_barrier();           // stage s + 1 visible; buffer s % D free
    constexpr int NMEM = TA + PS;
    const int nb = (b + D) % NB;
    auto mem_op = [&](int q) {
      if (q < PA) copy_a(st + D, q);
      else if (q < PS) load_b(st + D, nb, q - PA);
      else fa[f ^ 1][q - PS] = sA[(size_t)((st + 1) % D) * (TA * 64) + ((q - PS) / AP) * AP * 64 + xf[(q - PS) % AP]];
    };
    uint4 wcol[2][2];          // widened weight column j (set j & 1): the two K halves
#pragma unroll
    for (int p = 0; p < 8; p++) set_dword(wcol[0][p >> 2], p & 3, widen_pair<AMODE>(wb[b][0], p));
    __builtin_amdgcn_sched_barrier(0);
    constexpr int NM = 2 * MT;           // MFMAs per weight column
#pragma unroll
    for (int j = 0; j < FN; j++) {
#pragma unroll
      for (int u = 0; u < NM; u++) {
        const int h = u / MT, i = u % MT;
        acc[i][j] = mfma16<AMODE>(wcol[j & 1][h], fa[f][i * AP + h], acc[i][j]);
        __builtin_amdgcn_sched_barrier(0);
        const int m = j * NM + u;
        if (m < NMEM) mem_op(m);
        // the next column's widening, one output dword per MFMA slot
        if (j + 1 < FN && u < 8) set_dword(wcol[(j + 1) & 1][u >> 2], u & 3, widen_pair<AMODE>(wb[b][j + 1], u));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int q = FN * NM; q < NMEM; q++) mem_op(q);
    __builtin_amdgcn_sched_barrier(0);
  };
  const int kfull = nst - nst % NB;
  for (int st = 0; st < kfull; st += NB) {
#pragma unroll
    for (int b = 0; b < NB; b++) step(st + b, b, b & 1);
  }
#pragma unroll
  for (int b = 0; b < NB - 1; b++)
    if (kfull + b < nst) step(kfull + b, b, b & 1);

  wait_vm<0>();   // no copy may still be landing in LDS when the work-group exits

  b16_finish<MT, FN>(a, acc, mg0, ng0, wv * MT, bt, ks, e_ws, e_b);
}

// ---------------------------------------------------------------------------
// planning and launch
// ---------------------------------------------------------------------------
// cfg 0  128 x 192 tiles, 4-deep ring (112 KiB)
// cfg 1   64 x 128 tiles, 8-deep ring (128 KiB)
// cfg 2   32 x  64 tiles, 8-deep ring (64 KiB)
// The smaller tiles exist for mid-size M (64 < M <= 512) with small N, where
// the larger ones leave most CUs idle.
// cfg 4  128 x 192 tiles, column-split (weights to registers), 5-deep X ring (80 KiB)
// cfg 5  128 x 192 tiles, column-split, 7-deep X ring (112 KiB)
// cfg 6  128 x 128 tiles, column-split, 7-deep X ring (112 KiB)
// cfg 7   64 x 192 tiles, column-split, 7-deep X ring (56 KiB)
// cfg 8   64 x 128 tiles, column-split, 9-deep X ring (72 KiB; two work-groups
//         share a CU.  11- and 13-deep rings measured no faster with one
//         work-group per CU and 20-35% slower where a CU runs several)
// (the column-split kernel needs K % 64 == 0; other K run cfg 0's tiles)
static void b16_cfg(int cfg, int& mt, int& nt) {
  if (cfg >= 4) {
    mt = cfg >= 7 ? 4 : 8;
    nt = (cfg == 6 || cfg == 8) ? 8 : 12;
    return;
  }
  mt = (cfg == 0) ? 8 : (cfg == 1 ? 4 : 2);
  nt = (cfg == 0) ? 12 : (cfg == 1 ? 8 : 4);
}

// Plan: tile configuration and K slices, from the measured W8A16 sweep
// (M = 64 .. 1024, N = 2048 .. 12288, K = 2048, every configuration and
// 1..8 slices).  K a multiple of 64: the column-split kernel (b16_plan).
// Other K, the LDS-staged kernel: the 32 x 64 tiles while they number at
// most 512 (two work-groups of 64 KiB share a CU), else the 64 x 128 tiles
// while they fit one wave of 256 CUs, else the 128 x 192 tiles while they
// do, else the configuration whose tile count best fills 256 CUs.  The loop is bound by
// the latency of its stage copies rather than by bytes, so K slices pay only
// where the tiles are few: at most 64 tiles are split until 256 work-groups
// run (M = 64, N = 2048: 11.4 -> 10.5 us); with more tiles the slices' store,
// arrival and reload cost more than they save.
static std::atomic<int> g_b16_force_cfg{-1};
static std::atomic<int> g_b16_force_split{0};
void gemm_b16_set_plan(int cfg, int split) {
  g_b16_force_cfg.store(cfg >= 0 && cfg <= 8 ? cfg : -1, std::memory_order_relaxed);
  // with cfg 3, split (when > 64) picks the small-M kernel's work-group shape
  gemm_small_set_b16_shape(cfg == 3 && split > 64 ? split : 0);
  if (cfg == 3) split = 0;
  g_b16_force_split.store(split > 0 ? split : 0, std::memory_order_relaxed);
}

// -1 planner, 0..2 and 4..8 a forced tile configuration of this file's
// kernels, 3 the streamed small-M kernel
int gemm_b16_forced_cfg() { return g_b16_force_cfg.load(std::memory_order_relaxed); }

static int b16_tiles(int cfg, int MG, int NG) {
  int mt, nt;
  b16_cfg(cfg, mt, nt);
  return cdiv(MG, mt) * cdiv(NG, nt);
}

static void b16_plan(int MG, int NG, int KB, bool kf, int& cfg_out, int& split_out) {
  int best;
  if (kf) {
    // column-split kernel: the configuration of least estimated time, rounds
    // of 256 work-groups times the measured time of one work-group at
    // K = 2048 (one per CU, bound by its per-CU load rate: 64 x 128 tiles
    // 16.0 us, 64 x 192 20.5, 128 x 128 23.3, 128 x 192 30.3; MI355X sweep of
    // M = 64..1024, N = 2048..12288, every configuration)
    static const int kc[4] = {8, 7, 6, 4};
    static const float kt[4] = {16.0f, 20.5f, 23.3f, 30.3f};
    best = 8;
    float tbest = 3.0e38f;
    for (int c = 0; c < 4; c++) {
      const float t = (float)cdiv(b16_tiles(kc[c], MG, NG), 256) * kt[c];
      if (t < tbest) {
        tbest = t;
        best = kc[c];
      }
    }
  } else if (b16_tiles(2, MG, NG) <= 512) best = 2;
  else if (b16_tiles(1, MG, NG) <= 256) best = 1;
  else if (b16_tiles(0, MG, NG) <= 256) best = 0;
  else {
    best = 0;
    double best_eff = -1.0;
    for (int cfg : {0, 1, 2}) {
      const int tiles = b16_tiles(cfg, MG, NG);
      const double eff = (double)tiles / (cdiv(tiles, 256) * 256);
      if (eff > best_eff + 1e-9) {
        best_eff = eff;
        best = cfg;
      }
    }
  }
  const int tiles = b16_tiles(best, MG, NG);
  int sp = 1;
  if (tiles <= 64) sp = std::min(std::max(1, 256 / tiles), std::max(1, KB / 8));
  sp = std::min(sp, 4);
  const int fc = g_b16_force_cfg.load(std::memory_order_relaxed);
  const int fs = g_b16_force_split.load(std::memory_order_relaxed);
  if ((fc >= 0 && fc <= 2) || fc >= 4) best = fc;
  if (best >= 4 && !kf) best = 0;   // the column-split kernel needs K % 64 == 0
  if (fs > 0) sp = std::min(fs, std::max(1, KB));
  cfg_out = best;
  split_out = sp;
}

// partial-sum bytes and arrival counters the launch of this shape needs (the
// larger of the two plans: whether the launch takes the K-multiple-of-64 path
// also depends on the row stride, which is not known here)
void gemm_b16_needs(int M, int N, int K, size_t* part_bytes, size_t* counters) {
  const int MG = cdiv(M, 16), NG = cdiv(N, 16);
  *part_bytes = 0;
  *counters = 0;
  for (int kf = 0; kf < 2; kf++) {
    int cfg, sp, mt, nt;
    b16_plan(MG, NG, cdiv(K, 64), kf != 0 && K % 64 == 0, cfg, sp);
    b16_cfg(cfg, mt, nt);
    const size_t tiles = (size_t)cdiv(MG, mt) * cdiv(NG, nt);
    if (sp > 1) {
      *part_bytes = std::max(*part_bytes, tiles * sp * (size_t)(256 * mt * nt) * sizeof(float));
      *counters = std::max(*counters, tiles);
    }
  }
}

template <int AMODE, bool KF>
static void launch_b16(const GemmB16Args& a, int cfg, dim3 grid, dim3 block, hipStream_t st) {
  if constexpr (KF) {
    if (cfg == 4) {
      hipLaunchKernelGGL((gemm_b16_wcol_kernel<AMODE, 8, 3, 5>), grid, block, 0, st, a);
      return;
    }
    if (cfg == 5) {
      hipLaunchKernelGGL((gemm_b16_wcol_kernel<AMODE, 8, 3, 7>), grid, block, 0, st, a);
      return;
    }
    if (cfg == 6) {
      hipLaunchKernelGGL((gemm_b16_wcol_kernel<AMODE, 8, 2, 7>), grid, block, 0, st, a);
      return;
    }
    if (cfg == 7) {
      hipLaunchKernelGGL((gemm_b16_wcol_kernel<AMODE, 4, 3, 7>), grid, block, 0, st, a);
      return;
    }
    if (cfg == 8) {
      hipLaunchKernelGGL((gemm_b16_wcol_kernel<AMODE, 4, 2, 9>), grid, block, 0, st, a);
      return;
    }
  }
  if (cfg == 0) hipLaunchKernelGGL((gemm_b16_lds_kernel<AMODE, 8, 12, 4, 2, 2, KF>), grid, block, 0, st, a);
  else if (cfg == 1) hipLaunchKernelGGL((gemm_b16_lds_kernel<AMODE, 4, 8, 8, 2, 2, KF>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((gemm_b16_lds_kernel<AMODE, 2, 4, 8, 2, 2, KF>), grid, block, 0, st, a);
}

bool gemm_b16_supported(const GemmLaunch& L) {
  if (L.amode != A_BF16 && L.amode != A_F16) return false;
  if (L.K % 8 != 0 || L.lda % 8 != 0) return false;   // 8 elements per 16-byte copy
  if ((((uintptr_t)L.A) & 15) != 0) return false;
  return L.zero_tile != nullptr;
}

hipError_t launch_gemm_b16(const GemmLaunch& L, hipStream_t st) {
  if (!gemm_b16_supported(L)) return hipErrorInvalidValue;
  GemmB16Args a;
  a.X = L.A;
  a.lda = L.lda;
  a.Bt = L.Bt;
  a.ws = L.ws;
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
  a.zero_tile = L.zero_tile;
  int best, sp;
  // K a multiple of 64, and every X byte offset fits the copies' 32-bit
  // per-lane offsets (else the general path, with 64-bit addresses)
  const bool kf = (L.K % 64) == 0 && (size_t)L.M * (size_t)L.lda * 2 < ((size_t)1 << 32);
  b16_plan(a.MG, a.NG, a.KB, kf, best, sp);
  int mt, nt;
  b16_cfg(best, mt, nt);
  a.ntm = cdiv(a.MG, mt);
  a.ntn = cdiv(a.NG, nt);
  a.S = sp;
  a.part = static_cast<float*>(L.part);
  a.cnt = L.cnt;
  if (sp > 1 && (!a.part || !a.cnt)) return hipErrorInvalidValue;
  const long long blocks_ll = (long long)a.ntm * a.ntn * sp;
  if (blocks_ll > 0x7fffffffLL) return hipErrorInvalidValue;
  const int blocks = (int)blocks_ll;
  const dim3 grid(blocks), block(256);
  if (L.amode == A_BF16) {
    if (kf) launch_b16<A_BF16, true>(a, best, grid, block, st);
    else launch_b16<A_BF16, false>(a, best, grid, block, st);
  } else {
    if (kf) launch_b16<A_F16, true>(a, best, grid, block, st);
    else launch_b16<A_F16, false>(a, best, grid, block, st);
  }
  return hipGetLastError();
}

}  // namespace tl
