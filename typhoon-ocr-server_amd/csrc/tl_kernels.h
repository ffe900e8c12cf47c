// tl_kernels.h -- the launch interface of the INT8 linear kernels: a C ABI
// (tlk_* functions, plain structs, device pointers, asynchronous on `st`)
// that the C host layer (api.c, decoder_host.c) calls, and below it, for C++
// only, the same launchers in namespace tl as the kernel sources call each
// other.  Each tlk_* function forwards to its tl:: counterpart in the source
// file that defines it; no allocation, no synchronisation.
#pragma once
#include <hip/hip_runtime_api.h>
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

// default member values in C++ (the kernel sources declare plain locals of
// these structs); C code starts from the tlk_*_init functions below
#ifdef __cplusplus
#define TLK_DEF(v) = v
#else
#define TLK_DEF(v)
#endif

#ifdef __cplusplus
extern "C" {
#endif

static inline int tlk_cdiv(int a, int b) { return (a + b - 1) / b; }

// GEMV epilogues (gemv.hip)
// EPI_ARGMAX: W8A32 outputs (optionally stored), reduced per work-group to
// the key of its largest output (argmax_key) written to keys[blockIdx.x]
// EPI_SWIGLU: W8A32 outputs of a gate/up weight interleaved per 16-row group
// (rows 16b..16b+7 = gate rows 8b.., rows 16b+8.. = up rows 8b..), written as
// y[8b + r] = fl(silu(gate) * up) with the reference's fast-exp silu
// EPI_W8A16: fp32-semantics products of a bf16 / fp16 / fp32 x (x_type) as
// four int8 digit rows, y = fma(sum, ws, bias) stored as `out`
// EPI_W8A32_ROWS: 2..4 fp32 token rows (x [ntok][K], contiguous) as four
// int8 digit rows each; y[t][n] = 2^(e_t - 6) fl(sum * ws) (+ bias as its own
// rounding), y [ntok][N]: the arithmetic of the digit-row kernel (rows.hip)
// at one K slice
enum { EPI_W8A32 = 0, EPI_W8A8 = 1, EPI_ACC = 2, EPI_ARGMAX = 3, EPI_SWIGLU = 4, EPI_W8A16 = 5,
       EPI_W8A32_ROWS = 6 };
// GEMV x prologues: the numpy final RMSNorm (decoder.py:444-446) or the
// decoder's RMSNorm (kernel/ops.c:22-56, estimate-based rsqrt)
enum { NORM_NONE = 0, NORM_NUMPY = 1, NORM_DECODER = 2 };
// GEMM A-operand modes and output types (gemm.hip)
enum { A_I8 = 0, A_BF16 = 1, A_F16 = 2, A_F32X3 = 3 };
enum { OUT_F32 = 0, OUT_BF16 = 1, OUT_F16 = 2, OUT_I32 = 3,
       OUT_F32_X4 = 4 };   // A_I8 rows 4t..4t+3 are the int8 planes of fp32 token t (split_i8x4):
                           // y[t][n] = ldexp((a0 + a1/254 + a2/254^2 + a3/254^3) * ws[n], xe[t]) (+ bias[n])
// GEMM float epilogues: fl(acc*ws) then + bias, or fma(acc, ws, bias|0)
enum { EP_SCALE = 0, EP_SCALE_FMA = 1 };
// the final RMSNorm's widest row (lmhead.hip)
enum { TLK_RMS_MAX_K = 16384 };

// ---- quantization / packing (quant.hip) ----------------------------------
hipError_t tlk_launch_quantize_rows(const float* src, int8_t* dst, float* scales, int rows, int cols,
                                    bool clamp127, hipStream_t st);
hipError_t tlk_launch_quantize_rows_tiled(const float* src, int rows, int cols, uint8_t* tiles,
                                          float* scales, bool clamp127, hipStream_t st);
hipError_t tlk_launch_pack_tiles(const int8_t* w, int rows, int cols, uint8_t* tiles, hipStream_t st);
// rows [0, rows) of w into row groups g0.. of a tile array with NGt row groups
hipError_t tlk_launch_pack_tiles_rows(const int8_t* w, int rows, int cols, int NGt, int g0, uint8_t* tiles,
                                      hipStream_t st);
// whole-matrix tiles -> row-major int8 codes
hipError_t tlk_launch_unpack_tiles(const uint8_t* tiles, int rows, int cols, int8_t* w, hipStream_t st);
// fp32 rows X [M][ldx] -> int8 code tiles of 4 M rows (tile row groups
// MG = ceil(4M / 16), k-blocks ceil(K / 64); row 4t + p is plane p of token
// t) and per-token exponents xe[M]: x = 2^e (q0 + q1/254 + q2/254^2 +
// q3/254^3) up to 2^-32 of the row's absmax; a row holding Inf or NaN gets
// xe = kXeNonFinite (tl_common.h; the GEMM epilogues given the fp32 rows in
// GemmLaunch.xraw take that row's outputs from them, nonfinite_dot, else NaN)
hipError_t tlk_launch_split_i8x4(const float* X, int ldx, int M, int K, uint8_t* tiles, int* xe, hipStream_t st);
// 4-byte-word copy by a kernel (bytes % 4 == 0), e.g. from mapped pinned host memory
hipError_t tlk_launch_copy_words(const void* src, void* dst, size_t bytes, hipStream_t st);
// dst[0, npad) = src[0, n) followed by zeros, by a kernel (src null when n == 0):
// padding that stays a kernel node when the caller captures the stream
hipError_t tlk_launch_copy_pad_bytes(const void* src, size_t n, void* dst, size_t npad, hipStream_t st);
// one streaming read of `bytes` (a multiple of 16, 16-byte aligned) by grid
// work-groups of 256 lanes with u (4 or 8) 16-byte loads in flight each
// (stream.hip): the read floor of a launch that moves those bytes
hipError_t tlk_launch_stream_read(const void* p, size_t bytes, int grid, int u, uint32_t* sink, hipStream_t st);

// ---- lm_head step (lmhead.hip) -------------------------------------------
// final RMSNorm of one hidden row, numpy's float32 order (K = 128 * 2^j)
hipError_t tlk_launch_rmsnorm_np(const float* h, const float* w, float* out, int K, float eps, hipStream_t st);
// token = argmax over the per-work-group keys of an EPI_ARGMAX GEMV
hipError_t tlk_launch_argmax_keys(const uint64_t* keys, int n, int32_t* token, float* value, hipStream_t st);
// the no-allocation work-space, a file-scope device array of lmhead.hip: its
// address on device `dev` (which must be current), looked up once per
// device; argmax keys of up to TLK_NA_MAX_ROWS lm_head rows (16-row
// work-groups), then one row of TLK_RMS_MAX_K floats at TLK_NA_KEY_BYTES
enum { TLK_NA_MAX_ROWS = 262144, TLK_NA_KEY_BYTES = 262144 / 16 * 8 };
hipError_t tlk_noalloc_workspace(int dev, uint8_t** base);

// ---- decode-step kernels (decoder.hip) ------------------------------------
typedef struct AttnDecodeArgs {
  const float* qkv TLK_DEF(nullptr);      // [nq*128 | nkv*128 | nkv*128] of the QKV GEMV
  const float* q_norm TLK_DEF(nullptr);   // [128]
  const float* k_norm TLK_DEF(nullptr);   // [128]
  const float* cos_tab TLK_DEF(nullptr);  // [max_seq x 64]
  const float* sin_tab TLK_DEF(nullptr);
  float* kc TLK_DEF(nullptr);             // this layer's cache [nkv][max_seq][128]
  float* vc TLK_DEF(nullptr);
  const int* state TLK_DEF(nullptr);      // device decode state (position, rotary position, counter)
  float* pm TLK_DEF(nullptr);             // chunk maxima [nq][C]
  float* pl TLK_DEF(nullptr);             // chunk sums [nq][C]
  float* po TLK_DEF(nullptr);             // chunk outputs [nq][C][128]
  int* count TLK_DEF(nullptr);            // arrival counters [nkv], zero between launches
  float* out TLK_DEF(nullptr);            // merged attention row [nq*128]
  int nq TLK_DEF(16), nkv TLK_DEF(8), max_seq TLK_DEF(0);
  int C TLK_DEF(0);                       // chunks per q head the partial arrays hold (>= ceil(max_seq / T))
  int T TLK_DEF(64);                      // cache positions per work-group (attn_chunk_size)
  float scale TLK_DEF(0.0f), eps TLK_DEF(1e-6f);
} AttnDecodeArgs;
static inline AttnDecodeArgs tlk_attn_decode_init(void) {
  AttnDecodeArgs a;
  memset(&a, 0, sizeof a);
  a.nq = 16;
  a.nkv = 8;
  a.T = 64;
  a.eps = 1e-6f;
  return a;
}
// records per q head the work-space must hold for any chunk size
int tlk_attn_chunks(int max_seq);
// cache positions per work-group: 64, or the tuning override (32, 64, 128)
int tlk_attn_chunk_size(int max_seq);
void tlk_attn_set_chunk(int t);
hipError_t tlk_launch_attn_decode(const AttnDecodeArgs* a, hipStream_t st);
hipError_t tlk_launch_step_end(const uint64_t* keys, int n, const float* embed, int H, float* hidden, int* state,
                               int32_t* tokens, int max_tokens, hipStream_t st);

// ---- prefill-step kernels (prefill.hip) -----------------------------------
hipError_t tlk_launch_rmsnorm_rows(const float* x, const float* w, float* out, int rows, int K, float eps,
                                   hipStream_t st);
hipError_t tlk_launch_prefill_qk(float* qkv, const float* q_norm, const float* k_norm, const float* cos_t,
                                 const float* sin_t, float* kc, float* vc, int max_seq, int row0, int S, int nkv,
                                 float eps, hipStream_t st);
// part / cnt: work-space for splitting the longest query tiles' key ranges in
// two (flash_split_floats floats, flash_split_counters ints zeroed once: the
// kernel leaves them zero); null: no split
size_t tlk_flash_split_floats(int S, int nq);
size_t tlk_flash_split_counters(int S, int nq);
hipError_t tlk_launch_flash_prefill(const float* qkv, const float* kc, const float* vc, float* out, int S, int nq,
                                    int max_seq, int key0, int qoff, float scale, float* part, int* cnt,
                                    hipStream_t st);
hipError_t tlk_launch_swiglu_rows(const float* gu, float* mlp, int S, int ffn, hipStream_t st);
// the same two steps with their output rows written as GEMM activations
// instead of fp32 rows (K % 64 == 0, K <= 2048; ffn 2048 or 6144), one of:
//   scales: the W8A8 per-token quantization, int8 code tiles (ceil(rows / 16)
//           row groups) and per-token scales, the codes of
//           launch_quantize_rows_tiled on the stored rows, bit for bit;
//   xe:     the four int8 planes per row (code rows 4t + p, ceil(4 rows / 16)
//           row groups) and exponents of launch_split_i8x4, bit for bit
hipError_t tlk_launch_rmsnorm_rows_q(const float* x, const float* w, uint8_t* tiles, float* scales, int* xe,
                                     int rows, int K, float eps, hipStream_t st);
// the result of tlk_launch_split_i8x4 with one work-group per row, for
// K = 1024, 2048, 4096 or 6144 and 16-byte aligned rows (else
// hipErrorInvalidValue)
hipError_t tlk_launch_split_rows_planes(const float* x, int ldx, int rows, int K, uint8_t* tiles, int* xe,
                                        hipStream_t st);
// the result of tlk_launch_quantize_rows_tiled (clamp127) with one
// work-group per row, for the same K and alignment
hipError_t tlk_launch_quantize_rows_by_row(const float* x, int rows, int K, uint8_t* tiles, float* scales,
                                           hipStream_t st);
hipError_t tlk_launch_swiglu_rows_q(const float* gu, uint8_t* tiles, float* scales, int* xe, int S, int ffn,
                                    hipStream_t st);
hipError_t tlk_launch_residual_add(const float* y, float* h, long long n, hipStream_t st);

// ---- M=1 GEMV (gemv.hip) --------------------------------------------------
typedef struct GemvPlan {
  int rows TLK_DEF(16);       // rows per work-group (16 or 8)
  int blocks TLK_DEF(0), u TLK_DEF(4);
} GemvPlan;
typedef struct GemvLaunch {
  const float* x TLK_DEF(nullptr);       // fp32 activation (fused quantization) or null
  const uint8_t* xq TLK_DEF(nullptr);    // precomputed codes, zero padded to ceil(K/64)*64
  const float* xs_in TLK_DEF(nullptr);   // precomputed activation scale (device scalar)
  const uint8_t* wt TLK_DEF(nullptr);    // weight tiles
  const float* ws TLK_DEF(nullptr);
  const float* bias TLK_DEF(nullptr);
  float* y TLK_DEF(nullptr);
  int32_t* acc_out TLK_DEF(nullptr);
  float* xs_out TLK_DEF(nullptr);
  uint64_t* keys TLK_DEF(nullptr);       // EPI_ARGMAX: one key per work-group (gemv_plan().blocks)
  int norm TLK_DEF(NORM_NONE);           // RMSNorm of x first (gemv_fused_norm_ok)
  const float* norm_w TLK_DEF(nullptr);  //   its weights (null: none)
  float norm_eps TLK_DEF(1e-6f);
  int N TLK_DEF(0), K TLK_DEF(0), epi TLK_DEF(EPI_W8A32);
  int x_type TLK_DEF(0);                 // EPI_W8A16: x is 0 fp32, 1 bf16, 2 fp16
  int out TLK_DEF(OUT_F32);              // EPI_W8A16: y is OUT_F32 / OUT_BF16 / OUT_F16
  int ntok TLK_DEF(1);                   // EPI_W8A32_ROWS: token rows of x and y (2..4)
} GemvLaunch;
static inline GemvLaunch tlk_gemv_launch_init(void) {
  GemvLaunch L;
  memset(&L, 0, sizeof L);
  L.norm = NORM_NONE;
  L.norm_eps = 1e-6f;
  L.epi = EPI_W8A32;
  L.out = OUT_F32;
  L.ntok = 1;
  return L;
}
void tlk_gemv_plan(int N, int K, GemvPlan* plan);
int tlk_gemv_fused_xv(int K);
bool tlk_gemv_fused_norm_ok(int K, const float* x, const float* norm_w);
hipError_t tlk_launch_gemv_i8(const GemvLaunch* L, hipStream_t st);
// process-wide override of the GEMV plan for tuning: rows per work-group
// (16 or 8) and load instructions per batch (0 = planner's choice)
void tlk_gemv_set_plan(int rows, int u);

// ---- MFMA GEMM (gemm.hip) -------------------------------------------------
typedef struct GemmPlan {
  int cfg TLK_DEF(0), ntm TLK_DEF(1), ntn TLK_DEF(1), split TLK_DEF(1), blocks TLK_DEF(0);
} GemmPlan;
typedef struct GemmLaunch {
  int amode TLK_DEF(A_I8);
  const void* A TLK_DEF(nullptr);        // A_I8: code tiles; else row-major [M][lda]
  int lda TLK_DEF(0);
  const uint8_t* Bt TLK_DEF(nullptr);    // weight tiles
  const float* ws TLK_DEF(nullptr);
  const float* xs TLK_DEF(nullptr);      // per-token scales (A_I8)
  const float* bias TLK_DEF(nullptr);
  void* Y TLK_DEF(nullptr);
  int ldy TLK_DEF(0);
  int M TLK_DEF(0), N TLK_DEF(0), K TLK_DEF(0);
  int ep TLK_DEF(EP_SCALE), out TLK_DEF(OUT_F32);
  void* part TLK_DEF(nullptr);           // split workspace (gemm_workspace_bytes)
  uint32_t* cnt TLK_DEF(nullptr);        // gemm_counter_count zeroed counters
  int force_split TLK_DEF(0);
  const uint8_t* zero_tile TLK_DEF(nullptr);   // 1 KiB of device zeros (LDS-staged int8 GEMM)
  const int* xe TLK_DEF(nullptr);        // OUT_F32_X4: per-token power-of-two exponents (split_i8x4)
  const float* xraw TLK_DEF(nullptr);    // OUT_F32_X4: the fp32 token rows [M / 4][ldxr] the planes came
  int ldxr TLK_DEF(0);                   //   from (outputs of a non-finite row from them); null: NaN
} GemmLaunch;
static inline GemmLaunch tlk_gemm_launch_init(void) {
  GemmLaunch L;
  memset(&L, 0, sizeof L);
  L.amode = A_I8;
  L.ep = EP_SCALE;
  L.out = OUT_F32;
  return L;
}
void tlk_gemm_plan(int amode, int M, int N, int K, GemmPlan* plan);
size_t tlk_gemm_workspace_bytes(int amode, int M, int N, int K);
size_t tlk_gemm_counter_count(int amode, int M, int N, int K);
// every GEMM shape: the small-M, int8 LDS-staged, 16-bit LDS-staged or
// generic MFMA kernel
hipError_t tlk_launch_gemm(const GemmLaunch* L, hipStream_t st);
// split work-space of the kernel tlk_launch_gemm picks for *L: partial-sum
// bytes (L->part) and zeroed arrival counters (L->cnt); 0 when none
void tlk_gemm_needs(const GemmLaunch* L, size_t* part_bytes, size_t* counters);
void tlk_gemm_i8_set_cfg(int cfg);   // tuning override of the int8 GEMM (-1 = planner)
void tlk_gemm_i8_set_split(int s);   // tuning override of its K slices (0 = planner)
// tuning override of the 16-bit GEMM: tile configuration 0..2 (-1 = planner)
// and K slices (0 = planner)
void tlk_gemm_b16_set_plan(int cfg, int split);

// ---- 2..8 rows of fp32 activations as int8 digit planes (rows.hip): amode
//      A_F32X3; fp32 sums of w * x, y = 2^e fl(t * ws) summed over K slices,
//      then + bias -----------------------------------------------------------
typedef struct RowsPlan {
  int tg TLK_DEF(1), nkb TLK_DEF(16), cpt TLK_DEF(1), kbs TLK_DEF(1), split TLK_DEF(1), r TLK_DEF(1),
      blocks TLK_DEF(0);
} RowsPlan;
bool tlk_rows_supported(const GemmLaunch* L);
void tlk_rows_plan(int M, int N, int K, RowsPlan* plan);
size_t tlk_rows_workspace_bytes(int M, int N, int K);   // partials when split > 1
size_t tlk_rows_counter_count(int N);                   // zeroed arrival counters
void tlk_rows_set_split(int s);                         // tuning override (0 = planner)
int tlk_rows_forced_split(void);                        // that override (0 = none)
void tlk_rows_set_groups(int r);                        // tuning override (0 = planner)
hipError_t tlk_launch_rows(const GemmLaunch* L, hipStream_t st);

#ifdef __cplusplus
}  // extern "C"

// ---------------------------------------------------------------------------
// C++ spellings between the kernel sources (namespace tl)
// ---------------------------------------------------------------------------
#include <hip/hip_runtime.h>

namespace tl {

__host__ __device__ inline int cdiv(int a, int b) { return (a + b - 1) / b; }

hipError_t launch_quantize_rows(const float* src, int8_t* dst, float* scales, int rows, int cols,
                                bool clamp127, hipStream_t st);
hipError_t launch_quantize_rows_tiled(const float* src, int rows, int cols, uint8_t* tiles,
                                      float* scales, bool clamp127, hipStream_t st);
hipError_t launch_pack_tiles(const int8_t* w, int rows, int cols, uint8_t* tiles, hipStream_t st);
hipError_t launch_pack_tiles_rows(const int8_t* w, int rows, int cols, int NGt, int g0, uint8_t* tiles,
                                  hipStream_t st);
hipError_t launch_unpack_tiles(const uint8_t* tiles, int rows, int cols, int8_t* w, hipStream_t st);
hipError_t launch_rmsnorm_np(const float* h, const float* w, float* out, int K, float eps, hipStream_t st);
hipError_t launch_argmax_keys(const uint64_t* keys, int n, int32_t* token, float* value, hipStream_t st);
hipError_t launch_split_i8x4(const float* X, int ldx, int M, int K, uint8_t* tiles, int* xe, hipStream_t st);
hipError_t launch_stream_read(const void* p, size_t bytes, int grid, int u, uint32_t* sink, hipStream_t st);
hipError_t launch_copy_words(const void* src, void* dst, size_t bytes, hipStream_t st);
hipError_t launch_copy_pad_bytes(const void* src, size_t n, void* dst, size_t npad, hipStream_t st);

int attn_chunks(int max_seq);
int attn_chunk_size(int max_seq);
void attn_set_chunk(int t);
hipError_t launch_attn_decode(const AttnDecodeArgs& a, hipStream_t st);
hipError_t launch_step_end(const uint64_t* keys, int n, const float* embed, int H, float* hidden, int* state,
                           int32_t* tokens, int max_tokens, hipStream_t st);

hipError_t launch_rmsnorm_rows(const float* x, const float* w, float* out, int rows, int K, float eps,
                               hipStream_t st);
hipError_t launch_prefill_qk(float* qkv, const float* q_norm, const float* k_norm, const float* cos_t,
                             const float* sin_t, float* kc, float* vc, int max_seq, int row0, int S, int nkv,
                             float eps, hipStream_t st);
size_t flash_split_floats(int S, int nq);
size_t flash_split_counters(int S, int nq);
hipError_t launch_flash_prefill(const float* qkv, const float* kc, const float* vc, float* out, int S, int nq,
                                int max_seq, int key0, int qoff, float scale, float* part, int* cnt,
                                hipStream_t st);
hipError_t launch_swiglu_rows(const float* gu, float* mlp, int S, int ffn, hipStream_t st);
hipError_t launch_split_rows_planes(const float* x, int ldx, int rows, int K, uint8_t* tiles, int* xe,
                                    hipStream_t st);
hipError_t launch_quantize_rows_by_row(const float* x, int rows, int K, uint8_t* tiles, float* scales,
                                       hipStream_t st);
hipError_t launch_rmsnorm_rows_q(const float* x, const float* w, uint8_t* tiles, float* scales, int* xe, int rows,
                                 int K, float eps, hipStream_t st);
hipError_t launch_swiglu_rows_q(const float* gu, uint8_t* tiles, float* scales, int* xe, int S, int ffn,
                                hipStream_t st);
hipError_t launch_residual_add(const float* y, float* h, long long n, hipStream_t st);

GemvPlan gemv_plan(int N, int K);
int gemv_fused_xv(int K);
bool gemv_fused_norm_ok(int K, const float* x, const float* norm_w);
hipError_t launch_gemv_i8(const GemvLaunch& L, hipStream_t st);
void gemv_set_plan(int rows, int u);

GemmPlan gemm_plan(int amode, int M, int N, int K);
size_t gemm_workspace_bytes(int amode, int M, int N, int K);
size_t gemm_counter_count(int amode, int M, int N, int K);
hipError_t launch_gemm(const GemmLaunch& L, hipStream_t st);

// W8A8 LDS-staged int8 MFMA GEMM (gemm_i8.hip), used for M > 16
hipError_t launch_gemm_i8(const GemmLaunch& L, hipStream_t st);
int gemm_i8_pick_cfg(int M, int N, int K);
void gemm_i8_set_cfg(int cfg);
void gemm_i8_set_split(int s);
void gemm_i8_needs(int M, int N, int K, size_t* part_bytes, size_t* counters);

// LDS-staged 16-bit MFMA GEMM (gemm_b16.hip): A_BF16 / A_F16, used for M > 16
// when X rows are 16-byte aligned pieces
bool gemm_b16_supported(const GemmLaunch& L);
hipError_t launch_gemm_b16(const GemmLaunch& L, hipStream_t st);
void gemm_b16_needs(int M, int N, int K, size_t* part_bytes, size_t* counters);
void gemm_b16_set_plan(int cfg, int split);
int gemm_b16_forced_cfg();
void gemm_small_set_b16_shape(int code);
void gemm_needs(const GemmLaunch& L, size_t* part_bytes, size_t* counters);
// M <= 16 rows (gemm_small.hip): GEMV-shaped MFMA kernel
bool gemm_small_supported(const GemmLaunch& L);
hipError_t launch_gemm_small(const GemmLaunch& L, hipStream_t st);

bool rows_supported(const GemmLaunch& L);
RowsPlan rows_plan(int M, int N, int K);
size_t rows_workspace_bytes(int M, int N, int K);
size_t rows_counter_count(int N);
void rows_set_split(int s);
void rows_set_groups(int r);
hipError_t launch_rows(const GemmLaunch& L, hipStream_t st);

}  // namespace tl
#endif
