// prefill.hip -- the prefill-step kernels around the batch > 1 linear layers.
//
// Reference: kernel/decoder.c:33-157 with seq_len = S > 1 (PREFILL_MODE and
// PREFILL_3D_MODE): rmsnorm_seq_f32 (kernel/ops.c:75-105), per-head QK
// RMSNorm, mrope_apply_seq / mrope_apply_seq_3d (:347-458), the KV cache
// prefill append (kernel/kv_cache.c:70-104), attention_prefill_gqa
// (kernel/attention.c:252-360), silu_mul_inplace (ops.c:493-531) and
// vec_add_f32 (:537-549).  The linear layers are the fp32-accurate batch > 1
// GEMM (four int8 planes per token on the int8 MFMA, gemm_i8.hip) or, in
// W8A8 mode, the int8 GEMM on per-token codes.
//
// Layouts: activations token-major, as the reference's scratch: hidden
// [S][2048], qkv [S][4096] (q | k | v), attention output [S][2048], gate/up
// [S][12288] in the decoder's per-16-row interleave, mlp [S][6144].  The KV
// cache is [kv head][max_seq][128] per layer.
#include <algorithm>

#include "tl_common.h"
#include "tl_kernels.h"

namespace tl {

constexpr int PHD = 128;

// out[t] = x[t] * r_t * w, the decoder's RMSNorm (estimate-based rsqrt) of
// each 2048-wide row: one work-group per row, 8 elements per thread
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                           float* __restrict__ out, int K, float eps) {
  __shared__ float s_part[4];
  const size_t row = blockIdx.x;
  const float4* xr = reinterpret_cast<const float4*>(x + row * K);
  const float4* wr = reinterpret_cast<const float4*>(w);
  const int n4 = K >> 2;
  float4 v[2], wv[2];
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int f = threadIdx.x + 256 * i;
    v[i] = f < n4 ? xr[f] : make_float4(0.f, 0.f, 0.f, 0.f);
    wv[i] = f < n4 ? wr[f] : make_float4(0.f, 0.f, 0.f, 0.f);
    sq = __fmaf_rn(v[i].x, v[i].x, sq);
    sq = __fmaf_rn(v[i].y, v[i].y, sq);
    sq = __fmaf_rn(v[i].z, v[i].z, sq);
    sq = __fmaf_rn(v[i].w, v[i].w, sq);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sq = __fadd_rn(sq, __shfl_xor(sq, o, 64));
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = sq;
  __syncthreads();
  const float tot = __fadd_rn(__fadd_rn(s_part[0], s_part[1]), __fadd_rn(s_part[2], s_part[3]));
  const float r = ref_rsqrt(__fadd_rn(__fdiv_rn(tot, (float)K), eps));
  float4* orow = reinterpret_cast<float4*>(out + row * K);
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int f = threadIdx.x + 256 * i;
    if (f < n4)
      orow[f] = make_float4(__fmul_rn(__fmul_rn(v[i].x, r), wv[i].x), __fmul_rn(__fmul_rn(v[i].y, r), wv[i].y),
                            __fmul_rn(__fmul_rn(v[i].z, r), wv[i].z), __fmul_rn(__fmul_rn(v[i].w, r), wv[i].w));
  }
}

// Per-token int8 codes of a row held in registers (float4 f = tid + 256 j of
// the row), written straight into the int8 tile layout with the row's scale:
// the arithmetic of quantize_rows_tiled_vec_kernel (quant.hip) on the same
// values, so the codes equal those of quantizing the stored row afterwards.
//
// PLANES: instead, the four int8 planes of the row as code rows 4 row + p
// (MG = ceil(4 rows / 16)) and its exponent in `xe` (split_i8x4_kernel's
// arithmetic, quant.hip), the activations of the fp32-semantics GEMM.
template <int NV, bool PLANES>
__device__ __forceinline__ void quantize_row_to_tiles(const float4 (&v)[NV], int n4, int row, int MG,
                                                      uint8_t* __restrict__ tiles, float* __restrict__ scales,
                                                      int* __restrict__ xe, uint32_t* s_mx) {
  const int tid = threadIdx.x;
  uint32_t mx = 0;
#pragma unroll
  for (int j = 0; j < NV; j++)
    if (tid + 256 * j < n4)
      mx = max(mx, max(max(abs_bits(v[j].x), abs_bits(v[j].y)), max(abs_bits(v[j].z), abs_bits(v[j].w))));
  mx = wave_umax(mx);
  if ((tid & 63) == 0) s_mx[tid >> 6] = mx;
  __syncthreads();
  mx = max(max(s_mx[0], s_mx[1]), max(s_mx[2], s_mx[3]));
  if constexpr (PLANES) {
    const int ee = planes_exponent(mx);
    const bool finite = ee != kXeNonFinite;
    const int e = finite ? ee : 0;
    if (tid == 0) xe[row] = ee;
    uint32_t* t32 = reinterpret_cast<uint32_t*>(tiles);
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const int f = tid + 256 * j;
      if (f >= n4) continue;
      const float w4[4] = {finite ? v[j].x : 0.f, finite ? v[j].y : 0.f, finite ? v[j].z : 0.f, finite ? v[j].w : 0.f};
      uint32_t code[4];
      planes4_i8(w4, e, code);
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const int rr = 4 * row + p;
        t32[(((size_t)(f >> 4) * MG + (rr >> 4)) * 64 + (rr & 15) + 16 * ((f >> 2) & 3)) * 4 + (f & 3)] = code[p];
      }
    }
    return;
  }
  const float scale = quant_scale(__uint_as_float(mx));
  const float inv = quant_inv(scale);
  if (tid == 0) scales[row] = scale;
  const bool fast = mx < 0x7f800000u && (__float_as_uint(inv) & 0x7f800000u) != 0x7f800000u;
  uint32_t* t32 = reinterpret_cast<uint32_t*>(tiles) + ((size_t)(row >> 4) * 64 + (row & 15)) * 4;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int f = tid + 256 * j;          // float4 index: k = 4f .. 4f+3
    if (f >= n4) continue;
    const uint32_t code = fast ? codes4_rne(v[j], inv)
                               : pack4(code_rne(v[j].x * inv, true), code_rne(v[j].y * inv, true),
                                       code_rne(v[j].z * inv, true), code_rne(v[j].w * inv, true));
    t32[((size_t)(f >> 4) * MG) * 256 + ((f >> 2) & 3) * 64 + (f & 3)] = code;
  }
}

// The layer's RMSNorm followed by the W8A8 per-token quantization of its
// output, one work-group per token: the normalised values of
// rmsnorm_rows_kernel, quantized in registers and written as int8 tiles and
// scales (the fp32 row is never stored; K % 64 == 0, K <= 2048).
template <bool PLANES>
__global__ __launch_bounds__(256) void rmsnorm_rows_q_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                             int rows, int K, float eps, int MG,
                                                             uint8_t* __restrict__ tiles, float* __restrict__ scales,
                                                             int* __restrict__ xe) {
  __shared__ float s_part[4];
  __shared__ uint32_t s_mx[4];
  const int rr = xcd_grouped_row(blockIdx.x);
  if (rr >= rows) return;                   // the whole work-group
  const size_t row = rr;
  const float4* xr = reinterpret_cast<const float4*>(x + row * K);
  const float4* wr = reinterpret_cast<const float4*>(w);
  const int n4 = K >> 2;
  float4 v[2], wv[2];
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int f = threadIdx.x + 256 * i;
    v[i] = f < n4 ? xr[f] : make_float4(0.f, 0.f, 0.f, 0.f);
    wv[i] = f < n4 ? wr[f] : make_float4(0.f, 0.f, 0.f, 0.f);
    sq = __fmaf_rn(v[i].x, v[i].x, sq);
    sq = __fmaf_rn(v[i].y, v[i].y, sq);
    sq = __fmaf_rn(v[i].z, v[i].z, sq);
    sq = __fmaf_rn(v[i].w, v[i].w, sq);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sq = __fadd_rn(sq, __shfl_xor(sq, o, 64));
  if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = sq;
  __syncthreads();
  const float tot = __fadd_rn(__fadd_rn(s_part[0], s_part[1]), __fadd_rn(s_part[2], s_part[3]));
  const float r = ref_rsqrt(__fadd_rn(__fdiv_rn(tot, (float)K), eps));
  float4 y[2];
#pragma unroll
  for (int i = 0; i < 2; i++)
    y[i] = make_float4(__fmul_rn(__fmul_rn(v[i].x, r), wv[i].x), __fmul_rn(__fmul_rn(v[i].y, r), wv[i].y),
                       __fmul_rn(__fmul_rn(v[i].z, r), wv[i].z), __fmul_rn(__fmul_rn(v[i].w, r), wv[i].w));
  quantize_row_to_tiles<2, PLANES>(y, n4, (int)row, MG, tiles, scales, xe, s_mx);
}

// fp32 token rows -> their four int8 planes and exponents (split_i8x4_kernel's
// result, quant.hip), one work-group per row: the row is loaded once into
// registers (float4 tid + 256 j) and quantize_row_to_tiles writes the planes,
// where split_i8x4_kernel makes one wave walk the row twice.  K = 1024 NV.
// PLANES false: the W8A8 per-token codes and scales instead
// (quantize_rows_tiled's result).
template <int NV, bool PLANES>
__global__ __launch_bounds__(256) void split_rows_planes_kernel(const float* __restrict__ x, int ldx, int rows,
                                                                int MG, uint8_t* __restrict__ tiles,
                                                                float* __restrict__ scales, int* __restrict__ xe) {
  __shared__ uint32_t s_mx[4];
  const int rr = xcd_grouped_row(blockIdx.x);
  if (rr >= rows) return;                   // the whole work-group
  const float4* xr = reinterpret_cast<const float4*>(x + (size_t)rr * ldx);
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) v[j] = xr[threadIdx.x + 256 * j];
  quantize_row_to_tiles<NV, PLANES>(v, 256 * NV, rr, MG, tiles, scales, xe, s_mx);
}

// SwiGLU of one token's interleaved gate/up row (the values of
// swiglu_rows_kernel) followed by the W8A8 per-token quantization, written as
// int8 tiles and the token's scale; one work-group per token, ffn = 1024 NV.
// The SwiGLU values wait in LDS (each thread reads back its own) while the row
// is computed in two halves: holding a whole 6144-wide row's loads and values
// in registers took 127 VGPRs, 4 work-groups per CU, and a 1200-token batch
// then ran in two rounds; at 24 KB of LDS per work-group all 1200 are resident.
template <int NV, bool PLANES>
__global__ __launch_bounds__(256) void swiglu_rows_q_kernel(const float* __restrict__ gu, int S, int ffn, int MG,
                                                            uint8_t* __restrict__ tiles, float* __restrict__ scales,
                                                            int* __restrict__ xe) {
  __shared__ uint32_t s_mx[4];
  __shared__ float4 s_y[NV][256];
  const int tt = xcd_grouped_row(blockIdx.x);
  if (tt >= S) return;                      // the whole work-group
  const size_t t = tt;
  const float* row = gu + t * 2 * ffn;
  constexpr int H = (NV + 1) / 2;
#pragma unroll
  for (int h = 0; h < 2; h++) {
    float4 g[H], u[H];
#pragma unroll
    for (int i = 0; i < H; i++) {
      const int j = h * H + i;
      if (j >= NV) continue;
      const int c = 4 * (threadIdx.x + 256 * j);  // outputs c .. c+3: gate 16b + r.., up 16b + 8 + r..
      const int b = c >> 3, r = c & 7;
      g[i] = *reinterpret_cast<const float4*>(row + 16 * b + r);
      u[i] = *reinterpret_cast<const float4*>(row + 16 * b + 8 + r);
    }
#pragma unroll
    for (int i = 0; i < H; i++) {
      const int j = h * H + i;
      if (j >= NV) continue;
      s_y[j][threadIdx.x] = make_float4(__fmul_rn(ref_silu(g[i].x), u[i].x), __fmul_rn(ref_silu(g[i].y), u[i].y),
                                        __fmul_rn(ref_silu(g[i].z), u[i].z), __fmul_rn(ref_silu(g[i].w), u[i].w));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  float4 y[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) y[j] = s_y[j][threadIdx.x];
  quantize_row_to_tiles<NV, PLANES>(y, ffn >> 2, (int)t, MG, tiles, scales, xe, s_mx);
}

// One wave per 128-wide head vector of a token: the token's nq = 2 nkv q
// heads (RMSNorm with q_norm, rotation, written back in place in qkv), then
// its nkv kv heads (k: k_norm and rotation to cache row `row0 + t`; v copied
// there), so 3 nkv waves per token and no work-group barrier.  Lane l holds
// elements l and l + 64, the two halves the rotation pairs: the squares of
// each half are summed by a butterfly over the wave and the halves added low
// half first (the order of the decode attention kernel's two-wave sum).  The
// rotation uses row t of cos / sin (the caller points them at the token's
// first row).
__global__ __launch_bounds__(256) void prefill_qk_kernel(float* __restrict__ qkv, const float* __restrict__ q_norm,
                                                         const float* __restrict__ k_norm, const float* __restrict__ cos_t,
                                                         const float* __restrict__ sin_t, float* __restrict__ kc,
                                                         float* __restrict__ vc, int max_seq, int row0, int S, int nkv,
                                                         float eps) {
  const int lane = threadIdx.x & 63;
  const int unit = blockIdx.x * 4 + (threadIdx.x >> 6);   // uniform per wave
  const int per_tok = 3 * nkv;
  const int t = unit / per_tok, k = unit - t * per_tok;
  if (t >= S) return;
  float* row = qkv + (size_t)t * 4096;
  const bool is_q = k < 2 * nkv;
  const int h = is_q ? k : k - 2 * nkv;                     // q head, or kv head
  const float* src = row + (is_q ? h * PHD : 2048 + h * PHD);
  const float* nw = is_q ? q_norm : k_norm;
  const float xl = src[lane], xh = src[lane + 64];
  const float wl = nw[lane], wh = nw[lane + 64];
  const float co = cos_t[(size_t)t * 64 + lane], si = sin_t[(size_t)t * 64 + lane];
  float vl = 0.f, vh = 0.f;
  if (!is_q) {
    vl = row[3072 + h * PHD + lane];
    vh = row[3072 + h * PHD + lane + 64];
  }
  float sl = __fmul_rn(xl, xl), sh = __fmul_rn(xh, xh);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    sl = __fadd_rn(sl, __shfl_xor(sl, o, 64));
    sh = __fadd_rn(sh, __shfl_xor(sh, o, 64));
  }
  const float r = ref_rsqrt(__fadd_rn(__fdiv_rn(__fadd_rn(sl, sh), (float)PHD), eps));
  const float nl = __fmul_rn(__fmul_rn(xl, r), wl), nh = __fmul_rn(__fmul_rn(xh, r), wh);
  const float ol = __fsub_rn(__fmul_rn(nl, co), __fmul_rn(nh, si));
  const float oh = __fadd_rn(__fmul_rn(nh, co), __fmul_rn(nl, si));
  if (is_q) {
    row[h * PHD + lane] = ol;
    row[h * PHD + lane + 64] = oh;
  } else {
    const size_t off = ((size_t)h * max_seq + row0 + t) * PHD;
    kc[off + lane] = ol;
    kc[off + lane + 64] = oh;
    vc[off + lane] = vl;
    vc[off + lane + 64] = vh;
  }
}

// Causal flash attention over one q head on fp32 MFMA
// (v_mfma_f32_16x16x4f32: exact fp32 products, fp32 accumulation).
// Work-group L takes queries [64 qt, 64 qt + 64) of q head qh (longest tiles
// first over all heads) of the S-token chunk (q rows of qkv, already
// rotated); query i attends keys j <= qoff + i, read from cache rows key0 + j
// of kv head qh / 2 (qoff = 0, key0 = chunk start: attention within the
// chunk, as PREFILL_MODE; key0 = 0, qoff = chunk start: the whole cache, as
// CHUNKED_PREFILL_MODE), in 64-key tiles with an online softmax.
constexpr int FT = 64;          // queries / keys per tile

// Wave w holds the 16 queries q0 + 16 w + c in lanes (g, c) = (lane >> 4,
// lane & 15).
//   scores   D[key][query] += K[key][d] Q[query][d]: K is the first operand,
//            Q (kept in registers) the second; MFMA t = 4u + e of a 16-key
//            block reads, in lane group g, dimension d = 16u + 4g + e (any
//            bijection of d works, this one makes every operand read a
//            float4).  The block's keys are permuted so that output row
//            4g + r is key 16b + 4r + g: lane (g, c) then holds the scores of
//            query c for keys 16b + 4r + g, r = 0..3 ...
//   P.V      ... which is exactly the second operand of the four P.V MFMAs
//            of that block (MFMA m needs key 16b + 4m + g in lane group g):
//            no transpose.  V^T is the first operand: accumulator j, operand
//            row c is dimension 64 (j >> 2) + 4c + (j & 3), so a lane's eight
//            operands for one key are two float4 of its V row, and the
//            output lane (g, c) holds O[query c][64 (j >> 2) + 16g + 4r + (j & 3)].
// The online softmax of query c runs in lanes c, c+16, c+32, c+48.
//
// K and V tiles go global -> LDS directly (global_load_lds_dwordx4: 64 lanes
// x 16 bytes land contiguously, two 512-byte rows per copy; each lane picks
// its own source, so layouts are set by source addressing), double-buffered:
// the copies of tile kt + 1 fly while tile kt is computed, one wait and one
// barrier per tile.
//   K tile  row R = 16b + c holds key 16b + 4 (c & 3) + (c >> 2) (the score
//           permutation), and its float4 slot p holds dimensions
//           4 (p ^ (R & 15)) .. + 3: the 16 lanes that read one dimension
//           group from 16 consecutive rows hit 16 different bank groups.
//   V tile  row = key, plain: the P.V reads take 16 consecutive float4 of
//           each of 4 rows.
// (On gfx950, 16 rows read at one column with a 512-byte stride run at 1/4 of
// the LDS rate; the swizzle and the 4-row pattern run at full rate.)
// Each 16-key block's K operands, and each 4-key group's V operands, are read
// into registers one block ahead of their MFMAs.
//
// Split keys: the causal work of a query tile grows with its index, so the
// last tile's work-group alone would set the kernel's length.  The longest
// query tiles (those from index qs on, each with at least 2 key tiles) become
// two work items over the two halves of their key ranges; the host picks qs
// by list-scheduling makespan (flash_split_first).  Each half
// stores its unnormalised output, running max and sum (agent-scope stores,
// acknowledged before its arrival count), and the second to arrive combines
// the two in a fixed order (half 0, then half 1) and writes the output, so
// the result does not depend on which half finishes first.  Work items run
// longest first (the unsplit tiles and the split tiles' halves, each list
// already in decreasing length, merged); the host picks how many of the
// longest tiles to split from the makespan of that order on the GPU's CUs.
constexpr int FPART = 32 * 256 + 2 * 256;   // floats of one half's partials: O (32 per lane), m, l

// Work items of one q head with query tiles qs .. ntq-1 split: list A holds
// the unsplit tiles qs-1 .. 0, list B the halves (tile ntq-1 half 0, half 1,
// tile ntq-2 half 0, ...); both are in non-increasing length (a tile's key
// tiles grow by at most one per query tile) and the launch order merges
// them, longest first, ties to A.
struct FlashPlan {
  int S, qoff, qs, ntq;
  __host__ __device__ int nkt(int t) const { return (qoff + t * FT + min(FT, S - t * FT) - 1) / FT + 1; }
  __host__ __device__ int len_a(int a) const { return nkt(qs - 1 - a); }
  __host__ __device__ int len_b(int b) const {
    const int n = nkt(ntq - 1 - (b >> 1));
    return (b & 1) ? n >> 1 : (n + 1) >> 1;
  }
  // the next item comes from A after a items of A and b of B
  __host__ __device__ bool take_a(int a, int b) const {
    return a < qs && (b >= 2 * (ntq - qs) || len_a(a) >= len_b(b));
  }
};

__global__ __launch_bounds__(256) void flash_prefill_mfma_kernel(const float* __restrict__ qkv,
                                                                 const float* __restrict__ kc,
                                                                 const float* __restrict__ vc, float* __restrict__ out,
                                                                 int S, int max_seq, int key0, int qoff, float scale,
                                                                 int nheads, int qs, float* __restrict__ part,
                                                                 int* __restrict__ cnt) {
  // work item L / nheads of q head L % nheads in the launch order above;
  // query tiles qs .. ntq-1 are split into two halves of their key range
  const FlashPlan plan{S, qoff, qs, cdiv(S, FT)};
  const int item = (int)blockIdx.x / nheads;
  int ia = 0, ib = 0;
  for (int k = 0; k < item; k++) plan.take_a(ia, ib) ? ia++ : ib++;
  const bool unsplit = plan.take_a(ia, ib);
  const int qt = unsplit ? qs - 1 - ia : plan.ntq - 1 - (ib >> 1);
  const int half = unsplit ? -1 : (ib & 1);
  const int qh = (int)blockIdx.x % nheads, h = qh >> 1;
  const int q0 = qt * FT;
  const int nq = min(FT, S - q0);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c = lane & 15;

  // [buffer][K | V][64 rows x 128 floats]
  __shared__ float4 sKV[2][2][FT * PHD / 4];

  // this lane's query and its Q operand (dimensions 16u + 4g .. 16u + 4g + 3)
  const int qloc = 16 * wv + c;                           // 0..63 within the tile
  const int qrow = min(q0 + qloc, S - 1);
  float4 qr[8];
  {
    const float4* qp = reinterpret_cast<const float4*>(qkv + (size_t)qrow * 4096 + qh * PHD);
#pragma unroll
    for (int u = 0; u < 8; u++) qr[u] = qp[4 * u + g];
  }
  const int qpos = qoff + q0 + qloc;                      // key index bound of this query
  const int Sk = qoff + S;
  const float4* kbase = reinterpret_cast<const float4*>(kc + ((size_t)h * max_seq + key0) * PHD);
  const float4* vbase = reinterpret_cast<const float4*>(vc + ((size_t)h * max_seq + key0) * PHD);

  v4f o[8];
#pragma unroll
  for (int j = 0; j < 8; j++) o[j] = v4f{0.f, 0.f, 0.f, 0.f};
  float m = -3.0e38f, l = 0.0f;

  const int nkt = (qoff + q0 + nq - 1) / FT + 1;
  const int kmid = (nkt + 1) / 2;
  const int kt_begin = half == 1 ? kmid : 0;
  const int kt_end = half == 0 ? kmid : nkt;
  // copy q (0..7) of this wave: tile rows R = 16 wv + 2q + (lane >> 5), slot
  // p = lane & 31 (every lane reads a valid row: keys past the end clamp)
  const int rsub = lane >> 5, p = lane & 31;
  auto issue_tile = [&](int kt, int buf) {
    const uint32_t kb = lds_addr(&sKV[buf][0][0]), vb = lds_addr(&sKV[buf][1][0]);
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const int R = 16 * wv + 2 * q + rsub;
      const int kkey = min(kt * FT + (R & ~15) + 4 * (R & 3) + ((R >> 2) & 3), Sk - 1);
      const int vkey = min(kt * FT + R, Sk - 1);
      const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(16 * wv + 2 * q) * (PHD * 4));
      dma_tile(reinterpret_cast<const uint4*>(kbase + (size_t)kkey * (PHD / 4) + (p ^ (R & 15))), kb + dst);
      dma_tile(reinterpret_cast<const uint4*>(vbase + (size_t)vkey * (PHD / 4) + p), vb + dst);
    }
  };
  issue_tile(kt_begin, 0);
  for (int kt = kt_begin; kt < kt_end; kt++) {
    const int cb = (kt - kt_begin) & 1;
    wait_vm<0>();                           // this wave's copies of tile kt landed
    wait_lgkm0();                           // and its reads of tile kt - 1 are done
    stage_barrier();                        // every wave's: tile kt visible, buffer of kt - 1 free
    if (kt + 1 < kt_end) issue_tile(kt + 1, cb ^ 1);
    const float* sK = reinterpret_cast<const float*>(&sKV[cb][0][0]);
    const float* sV = reinterpret_cast<const float*>(&sKV[cb][1][0]);

    // scores of the tile's four 16-key blocks (operand row c of block b is
    // tile row 16b + c; dimension group g + 4u sits in slot (g + 4u) ^ c)
    v4f sc[4];
    float4 kf[2][8];
    auto kread = [&](int b, float4 (&dst)[8]) {
      const float* kp = sK + (16 * b + c) * PHD;
#pragma unroll
      for (int u = 0; u < 8; u++) dst[u] = *reinterpret_cast<const float4*>(kp + 4 * ((g + 4 * u) ^ c));
    };
    kread(0, kf[0]);
#pragma unroll
    for (int b = 0; b < 4; b++) {
      if (b < 3) kread(b + 1, kf[(b + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);   // the next block's reads stay ahead of these MFMAs
      sc[b] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const float4 kv = kf[b & 1][u];
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x, qr[u].x, sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y, qr[u].y, sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z, qr[u].z, sc[b], 0, 0, 0);
        sc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w, qr[u].w, sc[b], 0, 0, 0);
      }
    }
    // the first V operands are read while the softmax runs
    float4 vf[2][2];
    auto vread = [&](int km, float4 (&dst)[2]) {   // keys 4 km + g
      const float* vp = sV + (4 * km + g) * PHD + 4 * c;
      dst[0] = *reinterpret_cast<const float4*>(vp);
      dst[1] = *reinterpret_cast<const float4*>(vp + 64);
    };
    vread(0, vf[0]);
    __builtin_amdgcn_sched_barrier(0);
    // mask, online softmax (query c: lanes c, c+16, c+32, c+48)
    float mx = -3.0e38f;
#pragma unroll
    for (int b = 0; b < 4; b++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int key = kt * FT + 16 * b + 4 * r + g;
        sc[b][r] = (key <= qpos && key < Sk) ? __fmul_rn(sc[b][r], scale) : -3.0e38f;
        mx = fmaxf(mx, sc[b][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx);
    const float resc = expf(__fsub_rn(m, m_new));
    float ps = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; b++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float pv = sc[b][r] > -1.0e38f ? expf(__fsub_rn(sc[b][r], m_new)) : 0.0f;
        sc[b][r] = pv;
        ps = __fadd_rn(ps, pv);
      }
    ps = __fadd_rn(ps, __shfl_xor(ps, 16, 64));
    ps = __fadd_rn(ps, __shfl_xor(ps, 32, 64));
    l = __fmaf_rn(l, resc, ps);
    m = m_new;
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) o[j][r] = __fmul_rn(o[j][r], resc);
    // O^T[d][query] += V^T[d][key] P^T[key][query], keys 4 km + g, km = 4b + mm
#pragma unroll
    for (int km = 0; km < 16; km++) {
      if (km < 15) vread(km + 1, vf[(km + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      const float pk = sc[km >> 2][km & 3];
      const float4 v0 = vf[km & 1][0], v1 = vf[km & 1][1];
      o[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0.x, pk, o[0], 0, 0, 0);
      o[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0.y, pk, o[1], 0, 0, 0);
      o[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0.z, pk, o[2], 0, 0, 0);
      o[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(v0.w, pk, o[3], 0, 0, 0);
      o[4] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1.x, pk, o[4], 0, 0, 0);
      o[5] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1.y, pk, o[5], 0, 0, 0);
      o[6] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1.z, pk, o[6], 0, 0, 0);
      o[7] = __builtin_amdgcn_mfma_f32_16x16x4f32(v1.w, pk, o[7], 0, 0, 0);
    }
  }
  if (half >= 0) {
    // store this half's partials (layout: O element e of thread t at e 256 + t)
    float* mine = part + ((size_t)(qt * nheads + qh) * 2 + half) * FPART;
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) st_agent(mine + (4 * j + r) * 256 + tid, o[j][r]);
    st_agent(mine + 32 * 256 + tid, m);
    st_agent(mine + 33 * 256 + tid, l);
    __shared__ int s_last;
    asm volatile("" ::: "memory");
    wait_vm<0>();                           // the stores are acknowledged
    asm volatile("" ::: "memory");
    __syncthreads();
    int* c = cnt + qt * nheads + qh;
    if (tid == 0) s_last = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1;
    __syncthreads();
    if (!s_last) return;
    // the merger's acquire: the other half is read after the counter showed
    // it arrived (agent scope; once per split tile)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (tid == 0) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // combine half 0 and half 1 in that order
    const float* other = part + ((size_t)(qt * nheads + qh) * 2 + (1 - half)) * FPART;
    const float mo = ld_agent(other + 32 * 256 + tid), lo = ld_agent(other + 33 * 256 + tid);
    const float m0 = half == 0 ? m : mo, m1 = half == 0 ? mo : m;
    const float l0 = half == 0 ? l : lo, l1 = half == 0 ? lo : l;
    const float M = fmaxf(m0, m1);
    const float a0 = expf(__fsub_rn(m0, M)), a1 = expf(__fsub_rn(m1, M));
    l = __fadd_rn(__fmul_rn(l0, a0), __fmul_rn(l1, a1));
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float ov = ld_agent(other + (4 * j + r) * 256 + tid);
        const float o0 = half == 0 ? o[j][r] : ov, o1 = half == 0 ? ov : o[j][r];
        o[j][r] = __fadd_rn(__fmul_rn(o0, a0), __fmul_rn(o1, a1));
      }
  }
  if (qloc < nq) {
    const float inv = __fdiv_rn(1.0f, l);
    float* op = out + (size_t)(q0 + qloc) * 2048 + qh * PHD + 16 * g;
#pragma unroll
    for (int jh = 0; jh < 2; jh++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        *reinterpret_cast<float4*>(op + 64 * jh + 4 * r) =
            make_float4(__fmul_rn(o[4 * jh][r], inv), __fmul_rn(o[4 * jh + 1][r], inv),
                        __fmul_rn(o[4 * jh + 2][r], inv), __fmul_rn(o[4 * jh + 3][r], inv));
  }
}

// mlp[t][8b + r] = silu(gu[t][16b + r]) * gu[t][16b + 8 + r] (the decoder's
// per-16-row gate/up interleave; silu as silu_mul_inplace's vector loop)
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const float* __restrict__ gu, float* __restrict__ mlp,
                                                          long long n_out, int ffn) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_out) return;
  const long long t = i / ffn;
  const int c = (int)(i - t * ffn);
  const int b = c >> 3, r = c & 7;
  const float* row = gu + t * 2 * ffn;
  mlp[i] = __fmul_rn(ref_silu(row[16 * b + r]), row[16 * b + 8 + r]);
}

// h = y + h (vec_add_f32 of the residual), float4 per thread
__global__ __launch_bounds__(256) void residual_add_kernel(const float4* __restrict__ y, float4* __restrict__ h,
                                                           long long n4) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const float4 a = y[i], b = h[i];
  h[i] = make_float4(__fadd_rn(a.x, b.x), __fadd_rn(a.y, b.y), __fadd_rn(a.z, b.z), __fadd_rn(a.w, b.w));
}

hipError_t launch_rmsnorm_rows(const float* x, const float* w, float* out, int rows, int K, float eps,
                               hipStream_t st) {
  if (K % 4 != 0 || K > 2048 || rows < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rmsnorm_rows_kernel, dim3(rows), dim3(256), 0, st, x, w, out, K, eps);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rows_q(const float* x, const float* w, uint8_t* tiles, float* scales, int* xe, int rows,
                                 int K, float eps, hipStream_t st) {
  if (K % 64 != 0 || K > 2048 || rows < 1 || (!scales == !xe)) return hipErrorInvalidValue;
  const dim3 grid(cdiv(rows, 64) * 64);     // xcd_grouped_row: whole groups of 64 rows
  if (xe)
    hipLaunchKernelGGL(rmsnorm_rows_q_kernel<true>, grid, dim3(256), 0, st, x, w, rows, K, eps, cdiv(4 * rows, 16),
                       tiles, scales, xe);
  else
    hipLaunchKernelGGL(rmsnorm_rows_q_kernel<false>, grid, dim3(256), 0, st, x, w, rows, K, eps, cdiv(rows, 16),
                       tiles, scales, xe);
  return hipGetLastError();
}

template <bool PLANES>
static hipError_t launch_rows_q(const float* x, int ldx, int rows, int K, uint8_t* tiles, float* scales, int* xe,
                                hipStream_t st) {
  if (rows < 1 || ldx < K || ldx % 4 != 0 || (((uintptr_t)x) & 15) != 0) return hipErrorInvalidValue;
  const dim3 grid(cdiv(rows, 64) * 64);     // xcd_grouped_row: whole groups of 64 rows
  const int MG = cdiv(PLANES ? 4 * rows : rows, 16);
  switch (K) {
    case 1024: hipLaunchKernelGGL((split_rows_planes_kernel<1, PLANES>), grid, dim3(256), 0, st, x, ldx, rows, MG, tiles, scales, xe); break;
    case 2048: hipLaunchKernelGGL((split_rows_planes_kernel<2, PLANES>), grid, dim3(256), 0, st, x, ldx, rows, MG, tiles, scales, xe); break;
    case 4096: hipLaunchKernelGGL((split_rows_planes_kernel<4, PLANES>), grid, dim3(256), 0, st, x, ldx, rows, MG, tiles, scales, xe); break;
    case 6144: hipLaunchKernelGGL((split_rows_planes_kernel<6, PLANES>), grid, dim3(256), 0, st, x, ldx, rows, MG, tiles, scales, xe); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_split_rows_planes(const float* x, int ldx, int rows, int K, uint8_t* tiles, int* xe,
                                    hipStream_t st) {
  return launch_rows_q<true>(x, ldx, rows, K, tiles, nullptr, xe, st);
}

hipError_t launch_quantize_rows_by_row(const float* x, int rows, int K, uint8_t* tiles, float* scales,
                                       hipStream_t st) {
  return launch_rows_q<false>(x, K, rows, K, tiles, scales, nullptr, st);
}

hipError_t launch_swiglu_rows_q(const float* gu, uint8_t* tiles, float* scales, int* xe, int S, int ffn,
                                hipStream_t st) {
  if (S < 1 || (!scales == !xe)) return hipErrorInvalidValue;
  const int MG = xe ? cdiv(4 * S, 16) : cdiv(S, 16);
  const dim3 grid(cdiv(S, 64) * 64);        // xcd_grouped_row: whole groups of 64 rows
  if (ffn == 6144 && xe)
    hipLaunchKernelGGL((swiglu_rows_q_kernel<6, true>), grid, dim3(256), 0, st, gu, S, ffn, MG, tiles, scales, xe);
  else if (ffn == 6144)
    hipLaunchKernelGGL((swiglu_rows_q_kernel<6, false>), grid, dim3(256), 0, st, gu, S, ffn, MG, tiles, scales, xe);
  else if (ffn == 2048 && xe)
    hipLaunchKernelGGL((swiglu_rows_q_kernel<2, true>), grid, dim3(256), 0, st, gu, S, ffn, MG, tiles, scales, xe);
  else if (ffn == 2048)
    hipLaunchKernelGGL((swiglu_rows_q_kernel<2, false>), grid, dim3(256), 0, st, gu, S, ffn, MG, tiles, scales, xe);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_prefill_qk(float* qkv, const float* q_norm, const float* k_norm, const float* cos_t,
                             const float* sin_t, float* kc, float* vc, int max_seq, int row0, int S, int nkv,
                             float eps, hipStream_t st) {
  if (S < 1 || row0 < 0 || row0 + S > max_seq || nkv != 8) return hipErrorInvalidValue;   // rows of 4096: 16 q + 8 k + 8 v heads
  const long long waves = (long long)S * 3 * nkv;
  hipLaunchKernelGGL(prefill_qk_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, qkv, q_norm, k_norm,
                     cos_t, sin_t, kc, vc, max_seq, row0, S, nkv, eps);
  return hipGetLastError();
}

// First query tile whose key range is split (ntq: none): the qs whose launch
// order has the shortest makespan under list scheduling on `mach` machines
// (the CUs per q head: each item runs once per head), an item costing 4 per
// key tile plus 1 for a half's partial hand-over.  Past 2 tiles per machine
// the unsplit launch is balanced already.
int flash_split_first(int S, int qoff, int mach) {
  const int ntq = cdiv(S, FT);
  if (mach < 1 || ntq > 2 * mach) return ntq;
  auto makespan = [&](int qs) {
    const FlashPlan p{S, qoff, qs, ntq};
    int load[64] = {};
    const int nm = std::min(mach, 64);
    int a = 0, b = 0, worst = 0;
    for (int k = 0; k < ntq + (ntq - qs); k++) {
      const int cost = p.take_a(a, b) ? 4 * p.len_a(a++) : 4 * p.len_b(b++) + 1;
      int* lo = std::min_element(load, load + nm);
      *lo += cost;
      worst = std::max(worst, *lo);
    }
    return worst;
  };
  int best_qs = ntq, best = makespan(ntq);
  for (int qs = ntq - 1; qs >= 0 && FlashPlan{S, qoff, qs, ntq}.nkt(qs) >= 2; qs--) {
    const int m = makespan(qs);
    if (m < best) best = m, best_qs = qs;
  }
  return best_qs;
}

size_t flash_split_floats(int S, int nq) { return (size_t)cdiv(S, FT) * nq * 2 * FPART; }
size_t flash_split_counters(int S, int nq) { return (size_t)cdiv(S, FT) * nq; }

hipError_t launch_flash_prefill(const float* qkv, const float* kc, const float* vc, float* out, int S, int nq,
                                int max_seq, int key0, int qoff, float scale, float* part, int* cnt,
                                hipStream_t st) {
  if (S < 1 || key0 < 0 || qoff < 0 || key0 + qoff + S > max_seq) return hipErrorInvalidValue;
  const int ntq = cdiv(S, FT);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return hipErrorInvalidDevice;
  const int qs = (part && cnt) ? flash_split_first(S, qoff, cus / nq) : ntq;
  const int items = ntq + (ntq - qs);
  hipLaunchKernelGGL(flash_prefill_mfma_kernel, dim3(items * nq), dim3(256), 0, st, qkv, kc, vc, out, S,
                     max_seq, key0, qoff, scale, nq, qs, part, cnt);
  return hipGetLastError();
}

hipError_t launch_swiglu_rows(const float* gu, float* mlp, int S, int ffn, hipStream_t st) {
  const long long n = (long long)S * ffn;
  hipLaunchKernelGGL(swiglu_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, gu, mlp, n, ffn);
  return hipGetLastError();
}

hipError_t launch_residual_add(const float* y, float* h, long long n, hipStream_t st) {
  if (n % 4 != 0) return hipErrorInvalidValue;
  const long long n4 = n / 4;
  hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st,
                     reinterpret_cast<const float4*>(y), reinterpret_cast<float4*>(h), n4);
  return hipGetLastError();
}

}  // namespace tl

// ---------------------------------------------------------------------------
// C ABI of the launchers above (tl_kernels.h)
// ---------------------------------------------------------------------------
extern "C" {
hipError_t tlk_launch_rmsnorm_rows(const float* x, const float* w, float* out, int rows, int K, float eps,
                                   hipStream_t st) {
  return tl::launch_rmsnorm_rows(x, w, out, rows, K, eps, st);
}
hipError_t tlk_launch_prefill_qk(float* qkv, const float* q_norm, const float* k_norm, const float* cos_t,
                                 const float* sin_t, float* kc, float* vc, int max_seq, int row0, int S, int nkv,
                                 float eps, hipStream_t st) {
  return tl::launch_prefill_qk(qkv, q_norm, k_norm, cos_t, sin_t, kc, vc, max_seq, row0, S, nkv, eps, st);
}
size_t tlk_flash_split_floats(int S, int nq) { return tl::flash_split_floats(S, nq); }
size_t tlk_flash_split_counters(int S, int nq) { return tl::flash_split_counters(S, nq); }
hipError_t tlk_launch_flash_prefill(const float* qkv, const float* kc, const float* vc, float* out, int S, int nq,
                                    int max_seq, int key0, int qoff, float scale, float* part, int* cnt,
                                    hipStream_t st) {
  return tl::launch_flash_prefill(qkv, kc, vc, out, S, nq, max_seq, key0, qoff, scale, part, cnt, st);
}
hipError_t tlk_launch_swiglu_rows(const float* gu, float* mlp, int S, int ffn, hipStream_t st) {
  return tl::launch_swiglu_rows(gu, mlp, S, ffn, st);
}
hipError_t tlk_launch_split_rows_planes(const float* x, int ldx, int rows, int K, uint8_t* tiles, int* xe,
                                        hipStream_t st) {
  return tl::launch_split_rows_planes(x, ldx, rows, K, tiles, xe, st);
}
hipError_t tlk_launch_quantize_rows_by_row(const float* x, int rows, int K, uint8_t* tiles, float* scales,
                                           hipStream_t st) {
  return tl::launch_quantize_rows_by_row(x, rows, K, tiles, scales, st);
}
hipError_t tlk_launch_rmsnorm_rows_q(const float* x, const float* w, uint8_t* tiles, float* scales, int* xe,
                                     int rows, int K, float eps, hipStream_t st) {
  return tl::launch_rmsnorm_rows_q(x, w, tiles, scales, xe, rows, K, eps, st);
}
hipError_t tlk_launch_swiglu_rows_q(const float* gu, uint8_t* tiles, float* scales, int* xe, int S, int ffn,
                                    hipStream_t st) {
  return tl::launch_swiglu_rows_q(gu, tiles, scales, xe, S, ffn, st);
}
hipError_t tlk_launch_residual_add(const float* y, float* h, long long n, hipStream_t st) {
  return tl::launch_residual_add(y, h, n, st);
}
}  // extern "C"
