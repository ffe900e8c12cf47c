/* decoder_host.c -- the reference's decoder C ABI (kernel/decoder.h,
 * kernel/decoder.c:300-526) with the decode loop resident on the GPU.
 *
 * Handles keep the reference's names and roles, as opaque types:
 *   ModelWeights    per layer: fused Q||K||V, O, gate/up interleaved per
 *                   16-row group (for the SwiGLU epilogue), down, as HBM tiles,
 *                   plus the four norm vectors (decoder_set_layer_weights*)
 *   KVCache         K and V [layer][kv head][max_seq][128] fp32 in HBM, the
 *                   reference's seq_len / rope_offset counters, and the
 *                   device copy of the decode state (position, rotary position,
 *                   token counter) that the kernels read
 *   DecoderScratch  activation buffers, attention partials, a stream and the
 *                   captured step graphs
 *
 * One layer of a decode step is five launches (decoder.c:33-157):
 *   1. QKV GEMV, input RMSNorm in its prologue                  -> qkv
 *   2. attention: QK RMSNorm, M-RoPE, KV append, chunk partials, and the
 *      merge in the last work-group of each kv head             -> attn
 *   3. O GEMV + residual (the residual is the GEMV bias, in place) -> hidden
 *   4. gate/up GEMV, post-attention RMSNorm prologue, SwiGLU epilogue -> mlp
 *   5. down GEMV + residual                                     -> hidden
 * The layer loop is captured once into a HIP graph per (model, cache, rope
 * tables) and replayed; the decode state is written before each replay.
 * tl_decoder_generate adds the lm_head (numpy final RMSNorm + argmax keys)
 * and step_end (token, next embedding row, position advance) to the graph, so
 * consecutive greedy steps are graph replays with no host round trip.
 *
 * Calls on one scratch must not overlap (the reference's are synchronous too). */
#include "host.h"

#include <math.h>
#include <unistd.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

enum { H = 2048, KVD = 1024, FF = 6144, NQ = 16, NKV = 8, HDIM = 128, NL = 28 };
enum { QKVD = H + 2 * KVD };
#define EPS 1e-6f
#define SCALE 0.08838834764831843f   /* 1/sqrt(128), decoder.c:28 */

typedef struct LayerDev {
  tl_weights* qkv;
  tl_weights* o;
  tl_weights* gu;     /* gate/up interleaved per 16-row group */
  tl_weights* down;
  float* norms;       /* input_ln [H] | post_attn_ln [H] | q_norm [128] | k_norm [128] */
} LayerDev;

static void layer_release(LayerDev* L) {
  tlh_weights_free(L->qkv);
  tlh_weights_free(L->o);
  tlh_weights_free(L->gu);
  tlh_weights_free(L->down);
  if (L->norms) (void)hipFree(L->norms);
  memset(L, 0, sizeof *L);
}

/* device copies of a pair of host rope tables, keyed by their addresses */
typedef struct RopeDev {
  const float* hcos;
  const float* hsin;
  float* cos;
  float* sin;
  uint64_t fp;
  uint64_t uid;       /* process-unique (tlh_next_uid), drawn at allocation */
  struct RopeDev* next;
} RopeDev;

static uint64_t mix(uint64_t h, uint64_t v) {
  h ^= v + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
  h *= 0xbf58476d1ce4e5b9ull;
  return h ^ (h >> 31);
}

/* sampled fingerprint of a rope table pair (rows x 64 floats each) */
static uint64_t rope_fp(const float* c, const float* s, int rows) {
  uint64_t h = (uint64_t)rows;
  const size_t n = (size_t)rows * 64;
  for (int i = 0; i < 64; i++) {
    const size_t k = (size_t)(((unsigned __int128)(n - 1) * (unsigned)i) / 63);
    uint32_t a, b;
    memcpy(&a, c + k, 4);
    memcpy(&b, s + k, 4);
    h = mix(mix(h, a), b);
  }
  return h;
}

struct ModelWeights {
  int dev;
  LayerDev layers[NL];
  uint64_t version;     /* process-unique, redrawn whenever a layer changes */
  bool prefill_w8a8;    /* prefill linears on per-token int8 activations */
};

static int num_layers(const ModelWeights* m) {
  int n = 0;
  while (n < NL && m->layers[n].qkv) n++;
  return n;
}

struct KVCache {
  int dev;
  int max_seq;
  int seq_len, rope_offset;   /* kv_cache.h fields */
  float* k;
  float* v;
  int* state;                 /* device: position, rotary position, token counter */
  uint64_t uid;               /* process-unique, never reused */
  RopeDev* rope;              /* device copies of host tables */
};

static size_t layer_floats(const KVCache* c) { return (size_t)NKV * c->max_seq * HDIM; }

struct DecoderScratch {
  int dev;
  int max_seq;
  hipStream_t st;
  float *hidden, *qkv, *attn, *mlp;
  float *pm, *pl, *po;        /* attention chunk partials [NQ][C](x128) */
  int* count;                 /* attention arrival counters [NKV], zero between launches */
  int C;
  DevBuf keys, tokens, fnorm;
  PinnedBuf pin;
  PinnedBuf pin_rows;         /* prefill hidden rows on their way to / from HBM */
  /* prefill activations (token-major, grown to the longest prefill) */
  DevBuf p_h, p_xn, p_qkv, p_att, p_gu, p_mlp, p_y, p_cos, p_sin;
  DevBuf p_q, p_qs;           /* int8 activation tiles, per-token scales (W8A8) or exponents (planes) */
  DevBuf p_fpart, p_fcnt;     /* prefill attention's split-key partials and counters (zero between launches) */
  /* captured graphs and what they were captured for: process-unique ids of
   * the handles whose device memory they bake in (a freed handle's successor
   * can reuse its host address, never its id) and the device pointers the
   * scratch itself owns */
  hipGraphExec_t layers_exec;
  uint64_t layers_key[4];
  hipGraphExec_t gen_exec;
  uint64_t gen_key[9];
};

static void drop_graph(hipGraphExec_t* g) {
  if (*g) (void)hipGraphExecDestroy(*g);
  *g = NULL;
}

static int rope_device(KVCache* c, const float* cos_tab, const float* sin_tab, RopeDev** out) {
  REQ(cos_tab && sin_tab, "rope tables must be non-NULL");
  const uint64_t fp = rope_fp(cos_tab, sin_tab, c->max_seq);
  RopeDev* r = c->rope;
  while (r && !(r->hcos == cos_tab && r->hsin == sin_tab)) r = r->next;
  if (!r) {
    r = (RopeDev*)calloc(1, sizeof *r);
    REQ(r, "out of host memory");
    r->hcos = cos_tab;
    r->hsin = sin_tab;
    r->next = c->rope;
    c->rope = r;
  }
  if (!r->cos) {
    HIP_TRY(hipMalloc((void**)&r->cos, (size_t)c->max_seq * 64 * 4));
    HIP_TRY(hipMalloc((void**)&r->sin, (size_t)c->max_seq * 64 * 4));
    r->uid = tlh_next_uid();
    r->fp = 0;
  }
  if (r->fp != fp) {
    HIP_TRY(hipMemcpy(r->cos, cos_tab, (size_t)c->max_seq * 64 * 4, hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(r->sin, sin_tab, (size_t)c->max_seq * 64 * 4, hipMemcpyHostToDevice));
    r->fp = fp;
  }
  *out = r;
  return 0;
}

static int check_handles(const ModelWeights* m, const KVCache* c, const DecoderScratch* s) {
  REQ(m && c && s, "NULL handle");
  int d;
  TRY(tlh_current_device(&d));
  REQ(m->dev == d && c->dev == d && s->dev == d, "handles live on another device");
  REQ(s->max_seq >= c->max_seq, "scratch max_seq is smaller than the cache's");
  REQ(num_layers(m) > 0, "no layer weights set");
  return 0;
}

static int gemv(const tl_weights* W, const float* x, float* y, const float* bias, int epi, int norm,
                const float* norm_w, hipStream_t st) {
  GemvLaunch L = tlk_gemv_launch_init();
  L.x = x;
  L.wt = W->tiles;
  L.ws = W->scales;
  L.bias = bias;
  L.y = y;
  L.N = W->rows;
  L.K = W->cols;
  L.epi = epi;
  L.norm = norm;
  L.norm_w = norm_w;
  L.norm_eps = EPS;
  HIP_TRY(tlk_launch_gemv_i8(&L, st));
  return 0;
}

/* the five launches of each layer (see the file comment) */
static int enqueue_layers(const ModelWeights* m, const KVCache* c, DecoderScratch* s, const RopeDev* r,
                          hipStream_t st) {
  const int nl = num_layers(m);
  for (int l = 0; l < nl; l++) {
    const LayerDev* L = &m->layers[l];
    TRY(gemv(L->qkv, s->hidden, s->qkv, NULL, EPI_W8A32, NORM_DECODER, L->norms, st));
    AttnDecodeArgs a = tlk_attn_decode_init();
    a.qkv = s->qkv;
    a.q_norm = L->norms + 2 * H;
    a.k_norm = L->norms + 2 * H + HDIM;
    a.cos_tab = r->cos;
    a.sin_tab = r->sin;
    a.kc = c->k + (size_t)l * layer_floats(c);
    a.vc = c->v + (size_t)l * layer_floats(c);
    a.state = c->state;
    a.pm = s->pm;
    a.pl = s->pl;
    a.po = s->po;
    a.count = s->count;
    a.out = s->attn;
    a.nq = NQ;
    a.nkv = NKV;
    a.max_seq = c->max_seq;
    a.T = tlk_attn_chunk_size(c->max_seq);
    a.C = tlk_attn_chunks(c->max_seq);
    a.scale = SCALE;
    a.eps = EPS;
    HIP_TRY(tlk_launch_attn_decode(&a, st));
    TRY(gemv(L->o, s->attn, s->hidden, s->hidden, EPI_W8A32, NORM_NONE, NULL, st));
    TRY(gemv(L->gu, s->hidden, s->mlp, NULL, EPI_SWIGLU, NORM_DECODER, L->norms + H, st));
    TRY(gemv(L->down, s->mlp, s->hidden, s->hidden, EPI_W8A32, NORM_NONE, NULL, st));
  }
  return 0;
}

static void advance(KVCache* c, int n) {   /* kv_cache_advance (kernel/kv_cache.c:108-112) */
  c->seq_len += n;
  if (c->rope_offset > 0) c->rope_offset += n;
}

/* prefill with the activation quantization / plane split fused into the
 * RMSNorm and SwiGLU kernels (default), or each linear's own launch
 * (tl_prefill_set_fused_quant) */
/* atomic, since a setter may run while other threads enqueue prefills */
static atomic_bool g_prefill_fused_quant = true;

/* Prefill of S tokens through every layer (decoder.c:33-157 with seq_len > 1):
 * token t is rotated with rows t of cos_rows / sin_rows, its K/V go to cache
 * row row0 + t, and it attends cache rows key0 .. key0 + qoff + t. */
static int enqueue_prefill(const ModelWeights* m, KVCache* c, DecoderScratch* s, int S, const float* cos_rows,
                           const float* sin_rows, int row0, int key0, int qoff, hipStream_t st) {
  float* Hd = (float*)s->p_h.p;
  float* Xn = (float*)s->p_xn.p;
  float* QKV = (float*)s->p_qkv.p;
  float* ATT = (float*)s->p_att.p;
  float* GU = (float*)s->p_gu.p;
  float* MLP = (float*)s->p_mlp.p;
  float* Y = (float*)s->p_y.p;
  const long long n = (long long)S * H;
  /* w8a32_linear at batch S (decoder.c), or W8A8 with per-token activation
   * codes.  The layer's two RMSNorms and the SwiGLU write their output rows
   * directly as the GEMM's activations (the fp32 rows are never stored): the
   * W8A8 codes and scales, or, for w8a32_linear's fp32 semantics, the four
   * int8 planes and exponents it splits a batch of more than 32 rows into
   * (S <= 32 keeps the fp32 rows: w8a32_linear takes other kernels there).
   * Only the attention output goes through its linear's own quantization. */
  const bool w8 = m->prefill_w8a8;
  const bool fused_q = atomic_load_explicit(&g_prefill_fused_quant, memory_order_relaxed) && (w8 || S > 32);
  uint8_t* Aq = (uint8_t*)s->p_q.p;
  float* As = w8 ? (float*)s->p_qs.p : NULL;
  int* Ae = w8 ? NULL : (int*)s->p_qs.p;
#define LINEAR(X, W, OUT) (w8 ? tlh_linear_w8a8(X, W, NULL, OUT, S, st) : tlh_linear_w8a32(X, W, NULL, OUT, S, st))
#define LINEAR_Q(W, OUT) \
  (w8 ? tlh_linear_w8a8_tiles(Aq, As, W, OUT, S, st) : tlh_linear_w8a32_planes(Aq, Ae, W, OUT, S, st))
  for (int l = 0; l < num_layers(m); l++) {
    const LayerDev* L = &m->layers[l];
    float* kc = c->k + (size_t)l * layer_floats(c);
    float* vc = c->v + (size_t)l * layer_floats(c);
    if (fused_q) {
      HIP_TRY(tlk_launch_rmsnorm_rows_q(Hd, L->norms, Aq, As, Ae, S, H, EPS, st));
      TRY(LINEAR_Q(L->qkv, QKV));
    } else {
      HIP_TRY(tlk_launch_rmsnorm_rows(Hd, L->norms, Xn, S, H, EPS, st));
      TRY(LINEAR(Xn, L->qkv, QKV));
    }
    HIP_TRY(tlk_launch_prefill_qk(QKV, L->norms + 2 * H, L->norms + 2 * H + HDIM, cos_rows, sin_rows, kc, vc,
                                  c->max_seq, row0, S, NKV, EPS, st));
    HIP_TRY(tlk_launch_flash_prefill(QKV, kc, vc, ATT, S, NQ, c->max_seq, key0, qoff, SCALE, (float*)s->p_fpart.p,
                                     (int*)s->p_fcnt.p, st));
    TRY(LINEAR(ATT, L->o, Y));
    HIP_TRY(tlk_launch_residual_add(Y, Hd, n, st));
    if (fused_q) {
      HIP_TRY(tlk_launch_rmsnorm_rows_q(Hd, L->norms + H, Aq, As, Ae, S, H, EPS, st));
      TRY(LINEAR_Q(L->gu, GU));
      HIP_TRY(tlk_launch_swiglu_rows_q(GU, Aq, As, Ae, S, FF, st));
      TRY(LINEAR_Q(L->down, Y));
    } else {
      HIP_TRY(tlk_launch_rmsnorm_rows(Hd, L->norms + H, Xn, S, H, EPS, st));
      TRY(LINEAR(Xn, L->gu, GU));
      HIP_TRY(tlk_launch_swiglu_rows(GU, MLP, S, FF, st));
      TRY(LINEAR(MLP, L->down, Y));
    }
    HIP_TRY(tlk_launch_residual_add(Y, Hd, n, st));
  }
#undef LINEAR
#undef LINEAR_Q
  return 0;
}

static int ensure_prefill_buffers(DecoderScratch* s, int S) {
  TRY(tlh_devbuf_ensure(&s->p_h, (size_t)S * H * 4, s->st));
  TRY(tlh_devbuf_ensure(&s->p_xn, (size_t)S * H * 4, s->st));
  TRY(tlh_devbuf_ensure(&s->p_qkv, (size_t)S * QKVD * 4, s->st));
  TRY(tlh_devbuf_ensure(&s->p_att, (size_t)S * H * 4, s->st));
  TRY(tlh_devbuf_ensure(&s->p_gu, (size_t)S * 2 * FF * 4, s->st));
  TRY(tlh_devbuf_ensure(&s->p_mlp, (size_t)S * FF * 4, s->st));
  TRY(tlh_devbuf_ensure(&s->p_y, (size_t)S * H * 4, s->st));
  TRY(tlh_devbuf_ensure(&s->p_q, (size_t)tlk_cdiv(4 * S, 16) * 16 * FF, s->st));   /* plane tiles of the widest input (K = FF) */
  TRY(tlh_devbuf_ensure(&s->p_qs, (size_t)tlk_cdiv(S, 16) * 16 * sizeof(float), s->st));
  TRY(tlh_devbuf_ensure(&s->p_fpart, tlk_flash_split_floats(S, NQ) * 4, s->st));
  const size_t cb = tlk_flash_split_counters(S, NQ) * sizeof(int);
  if (cb > s->p_fcnt.n) {
    TRY(tlh_devbuf_ensure(&s->p_fcnt, cb, s->st));
    HIP_TRY(hipMemsetAsync(s->p_fcnt.p, 0, s->p_fcnt.n, s->st));   /* ordered before the prefill kernels */
  }
  return 0;
}

/* host copy between the caller's (pageable) rows and the pinned staging
 * buffer, split over up to 8 threads: a single-threaded copy runs at about a
 * quarter of the PCIe rate, and it is what the runtime's own pageable path
 * does chunk by chunk */
typedef struct CopyPiece {
  char* dst;
  const char* src;
  size_t n;
} CopyPiece;

static void* copy_piece(void* arg) {
  const CopyPiece* p = (const CopyPiece*)arg;
  memcpy(p->dst, p->src, p->n);
  return NULL;
}

static void parallel_copy(void* dst, const void* src, size_t n) {
  const size_t kPiece = (size_t)1 << 20;
  const long hw = sysconf(_SC_NPROCESSORS_ONLN);
  size_t nt = 8;
  if ((size_t)(hw > 0 ? hw : 1) < nt) nt = (size_t)(hw > 0 ? hw : 1);
  if (n / kPiece < nt) nt = n / kPiece;
  if (nt <= 1) {
    memcpy(dst, src, n);
    return;
  }
  const size_t per = ((n + nt - 1) / nt + 63) & ~(size_t)63;
  pthread_t th[8];
  CopyPiece pc[8];
  bool started[8] = {false};
  for (size_t i = 1; i < nt && i * per < n; i++) {
    const size_t o = i * per;
    pc[i].dst = (char*)dst + o;
    pc[i].src = (const char*)src + o;
    pc[i].n = per < n - o ? per : n - o;
    started[i] = pthread_create(&th[i], NULL, copy_piece, &pc[i]) == 0;
    if (!started[i]) memcpy(pc[i].dst, pc[i].src, pc[i].n);
  }
  memcpy(dst, src, per < n ? per : n);
  for (size_t i = 1; i < nt; i++)
    if (started[i]) pthread_join(th[i], NULL);
}

/* one prefill call on host hidden rows: chunks of at most `chunk` tokens
 * (chunked mode: each attends to the whole cache), then the cache advances */
static int prefill_host(const ModelWeights* m, KVCache* c, float* hidden, DecoderScratch* s, int S,
                        const float* cos_tab, const float* sin_tab, const float* token_cos, const float* token_sin,
                        int chunk, bool chunked) {
  TRY(check_handles(m, c, s));
  REQ(hidden && S >= 1, "bad arguments");
  REQ(c->seq_len + S <= c->max_seq, "KV cache too small for the prefill");
  const float* cos_dev = NULL;
  const float* sin_dev = NULL;
  if (token_cos) {
    REQ(token_sin, "NULL token_sin");
    TRY(tlh_devbuf_ensure(&s->p_cos, (size_t)S * 64 * 4, s->st));
    TRY(tlh_devbuf_ensure(&s->p_sin, (size_t)S * 64 * 4, s->st));
    HIP_TRY(hipMemcpyAsync(s->p_cos.p, token_cos, (size_t)S * 64 * 4, hipMemcpyHostToDevice, s->st));
    HIP_TRY(hipMemcpyAsync(s->p_sin.p, token_sin, (size_t)S * 64 * 4, hipMemcpyHostToDevice, s->st));
    cos_dev = (const float*)s->p_cos.p;
    sin_dev = (const float*)s->p_sin.p;
  } else {
    RopeDev* r;
    TRY(rope_device(c, cos_tab, sin_tab, &r));
    cos_dev = r->cos;
    sin_dev = r->sin;
  }
  const int step = chunked ? (chunk > 1 ? chunk : 1) : S;
  TRY(ensure_prefill_buffers(s, step < S ? step : S));
  for (int t0 = 0; t0 < S; t0 += step) {
    const int n = step < S - t0 ? step : S - t0;
    const int base = c->seq_len;
    const size_t rb = (size_t)n * H * 4;
    TRY(tlh_pinned_ensure(&s->pin_rows, rb));
    parallel_copy(s->pin_rows.p, hidden + (size_t)t0 * H, rb);
    HIP_TRY(hipMemcpyAsync(s->p_h.p, s->pin_rows.p, rb, hipMemcpyHostToDevice, s->st));
    /* sequential positions: rows base + t of the tables; 3-D: rows t0 + t of the token tables */
    const size_t rrow = token_cos ? (size_t)t0 : (size_t)base;
    TRY(enqueue_prefill(m, c, s, n, cos_dev + rrow * 64, sin_dev + rrow * 64, base, chunked ? 0 : base,
                        chunked ? base : 0, s->st));
    HIP_TRY(hipMemcpyAsync(s->pin_rows.p, s->p_h.p, rb, hipMemcpyDeviceToHost, s->st));
    HIP_TRY(hipStreamSynchronize(s->st));
    parallel_copy(hidden + (size_t)t0 * H, s->pin_rows.p, rb);
    advance(c, n);
  }
  return 0;
}

/* one captured graph of what `enqueue(ctx)` launches on st */
static int capture(hipStream_t st, int (*enqueue)(void*), void* ctx, hipGraphExec_t* out) {
  HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  hipGraph_t g = NULL;
  if (enqueue(ctx) != 0) {
    (void)hipStreamEndCapture(st, &g);
    if (g) (void)hipGraphDestroy(g);
    return -1;
  }
  HIP_TRY(hipStreamEndCapture(st, &g));
  hipGraphExec_t exec = NULL;
  const hipError_t e = hipGraphInstantiate(&exec, g, NULL, NULL, 0);
  (void)hipGraphDestroy(g);
  HIP_TRY(e);
  *out = exec;
  return 0;
}

/* pinned staging of a scratch: decode state at 0, a hidden row at 64 */
#define STAGE_HIDDEN 64

static int rope_pos(const KVCache* c) { return c->rope_offset ? c->rope_offset : c->seq_len; }

/* decode state from the host counters: position, rotary position, counter */
static int write_state(KVCache* c, DecoderScratch* s, int counter) {
  HIP_TRY(hipStreamSynchronize(s->st));   /* the staging buffer is idle */
  int* h = (int*)s->pin.p;
  h[0] = c->seq_len;
  h[1] = rope_pos(c);
  h[2] = counter;
  h[3] = 0;
  HIP_TRY(hipMemcpyAsync(c->state, h, 4 * sizeof(int), hipMemcpyHostToDevice, s->st));
  return 0;
}

/* One layer's host arrays.  qkv_w / gate_up_w are the fused row
 * concatenations Q||K||V [4096 x 2048] and gate||up [12288 x 2048]
 * (decoder.py:290-302); when given they are the source of those rows, and
 * the separate q/k/v or gate/up arrays are not read. */
typedef struct LayerSources {
  const int8_t *q_w, *k_w, *v_w, *o_w, *gate_w, *up_w, *down_w, *qkv_w, *gate_up_w;
  const float *q_s, *k_s, *v_s, *o_s, *gate_s, *up_s, *down_s, *qkv_s, *gate_up_s;
  const float *input_ln, *post_attn_ln, *q_norm, *k_norm;
} LayerSources;

static int build_layer(const LayerSources* w, LayerDev* L) {
  hipStream_t st = NULL;
  if (w->qkv_w && w->qkv_s) {
    TRY(tlh_weights_from_codes(w->qkv_w, w->qkv_s, QKVD, H, false, st, &L->qkv));
  } else {
    /* Q||K||V rows (decoder.py:290-296): bit-identical to the separate GEMVs */
    int8_t* cw = (int8_t*)malloc((size_t)QKVD * H);
    float* cs = (float*)malloc((size_t)QKVD * 4);
    if (!cw || !cs) {
      free(cw);
      free(cs);
      return tlh_fail("out of host memory");
    }
    memcpy(cw, w->q_w, (size_t)H * H);
    memcpy(cw + (size_t)H * H, w->k_w, (size_t)KVD * H);
    memcpy(cw + (size_t)(H + KVD) * H, w->v_w, (size_t)KVD * H);
    memcpy(cs, w->q_s, H * 4);
    memcpy(cs + H, w->k_s, KVD * 4);
    memcpy(cs + H + KVD, w->v_s, KVD * 4);
    const int rc = tlh_weights_from_codes(cw, cs, QKVD, H, false, st, &L->qkv);
    free(cw);
    free(cs);
    TRY(rc);
  }
  TRY(tlh_weights_from_codes(w->o_w, w->o_s, H, H, false, st, &L->o));
  {
    /* gate and up interleaved per 16-row group: rows 16b..16b+7 are gate
     * rows 8b.., rows 16b+8.. the up rows 8b.. (EPI_SWIGLU) */
    const bool fused = w->gate_up_w && w->gate_up_s;
    const int8_t* gate_w = fused ? w->gate_up_w : w->gate_w;
    const int8_t* up_w = fused ? w->gate_up_w + (size_t)FF * H : w->up_w;
    const float* gate_s = fused ? w->gate_up_s : w->gate_s;
    const float* up_s = fused ? w->gate_up_s + FF : w->up_s;
    int8_t* gw = (int8_t*)malloc((size_t)2 * FF * H);
    float* gs = (float*)malloc((size_t)2 * FF * 4);
    if (!gw || !gs) {
      free(gw);
      free(gs);
      return tlh_fail("out of host memory");
    }
    for (int b = 0; b < FF / 8; b++) {
      memcpy(gw + (size_t)(16 * b) * H, gate_w + (size_t)(8 * b) * H, (size_t)8 * H);
      memcpy(gw + (size_t)(16 * b + 8) * H, up_w + (size_t)(8 * b) * H, (size_t)8 * H);
      memcpy(gs + 16 * b, gate_s + 8 * b, 8 * 4);
      memcpy(gs + 16 * b + 8, up_s + 8 * b, 8 * 4);
    }
    const int rc = tlh_weights_from_codes(gw, gs, 2 * FF, H, false, st, &L->gu);
    free(gw);
    free(gs);
    TRY(rc);
  }
  TRY(tlh_weights_from_codes(w->down_w, w->down_s, H, FF, false, st, &L->down));
  HIP_TRY(hipMalloc((void**)&L->norms, (size_t)(2 * H + 2 * HDIM) * 4));
  HIP_TRY(hipMemcpy(L->norms, w->input_ln, H * 4, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(L->norms + H, w->post_attn_ln, H * 4, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(L->norms + 2 * H, w->q_norm, HDIM * 4, hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(L->norms + 2 * H + HDIM, w->k_norm, HDIM * 4, hipMemcpyHostToDevice));
  return 0;
}

static int set_layer(ModelWeights* m, int l, const LayerSources* w) {
  REQ(m, "NULL model");
  REQ(l >= 0 && l < NL, "layer index out of range");
  int dev;
  TRY(tlh_current_device(&dev));
  REQ(m->dev == dev, "model lives on another device");
  REQ(w->o_w && w->o_s && w->down_w && w->down_s, "NULL weight pointer");
  REQ(w->input_ln && w->post_attn_ln && w->q_norm && w->k_norm, "NULL norm pointer");
  REQ((w->qkv_w && w->qkv_s) || (w->q_w && w->q_s && w->k_w && w->k_s && w->v_w && w->v_s), "NULL q/k/v pointer");
  REQ((w->gate_up_w && w->gate_up_s) || (w->gate_w && w->gate_s && w->up_w && w->up_s), "NULL gate/up pointer");
  LayerDev L;
  memset(&L, 0, sizeof L);
  if (build_layer(w, &L) != 0) {
    layer_release(&L);
    return -1;
  }
  layer_release(&m->layers[l]);
  m->layers[l] = L;
  m->version = tlh_next_uid();
  return 0;
}

/* ---- handles (decoder.c:320-366) ----------------------------------------- */
ModelWeights* decoder_model_alloc(void) {
  tlh_begin();
  int dev = -1;
  int rc = tlh_current_device(&dev);
  ModelWeights* m = NULL;
  if (rc == 0) {
    m = (ModelWeights*)calloc(1, sizeof *m);
    if (!m) rc = tlh_fail("out of host memory");
  }
  if (m) {
    m->dev = dev;
    m->version = tlh_next_uid();
  }
  tlh_finish("decoder_model_alloc", rc);
  return m;
}

void decoder_model_free(ModelWeights* m) {
  if (!m) return;
  for (int l = 0; l < NL; l++) layer_release(&m->layers[l]);
  free(m);
}

static void cache_free(KVCache* c) {
  if (c->k) (void)hipFree(c->k);
  if (c->v) (void)hipFree(c->v);
  if (c->state) (void)hipFree(c->state);
  RopeDev* r = c->rope;
  while (r) {
    RopeDev* next = r->next;
    if (r->cos) (void)hipFree(r->cos);
    if (r->sin) (void)hipFree(r->sin);
    free(r);
    r = next;
  }
  free(c);
}

static int cache_alloc_impl(int max_seq, KVCache** out) {
  REQ(max_seq >= 1, "max_seq must be >= 1");
  KVCache* p = (KVCache*)calloc(1, sizeof *p);
  REQ(p, "out of host memory");
  int rc = 0;
  TRY_GO(tlh_current_device(&p->dev), fail);
  p->max_seq = max_seq;
  p->uid = tlh_next_uid();
  const size_t bytes = (size_t)NL * layer_floats(p) * sizeof(float);
  HIP_GO(hipMalloc((void**)&p->k, bytes), fail);
  HIP_GO(hipMalloc((void**)&p->v, bytes), fail);
  HIP_GO(hipMalloc((void**)&p->state, 4 * sizeof(int)), fail);
  /* null stream, completed before return: the kernels run on other streams */
  HIP_GO(hipMemsetAsync(p->state, 0, 4 * sizeof(int), NULL), fail);
  HIP_GO(hipStreamSynchronize(NULL), fail);
  *out = p;
  return 0;
fail:
  cache_free(p);
  return rc;
}

KVCache* decoder_cache_alloc(int max_seq) {
  tlh_begin();
  KVCache* c = NULL;
  const int rc = cache_alloc_impl(max_seq, &c);
  tlh_finish("decoder_cache_alloc", rc);
  return rc == 0 ? c : NULL;
}

void decoder_cache_free(KVCache* c) {
  if (c) cache_free(c);
}

void decoder_cache_clear(KVCache* c) {
  if (c) {
    c->seq_len = 0;
    c->rope_offset = 0;
  }
}

void decoder_cache_set_rope_offset(KVCache* c, int offset) {
  if (c) c->rope_offset = offset;
}

static void scratch_free(DecoderScratch* s) {
  if (s->st) (void)hipStreamSynchronize(s->st);
  drop_graph(&s->layers_exec);
  drop_graph(&s->gen_exec);
  float* fp[] = {s->hidden, s->qkv, s->attn, s->mlp, s->pm, s->pl, s->po};
  for (size_t i = 0; i < sizeof fp / sizeof fp[0]; i++)
    if (fp[i]) (void)hipFree(fp[i]);
  if (s->count) (void)hipFree(s->count);
  DevBuf* bufs[] = {&s->p_h, &s->p_xn, &s->p_qkv, &s->p_att, &s->p_gu, &s->p_mlp, &s->p_y, &s->p_cos,
                    &s->p_sin, &s->p_q, &s->p_qs, &s->p_fpart, &s->p_fcnt, &s->keys, &s->tokens, &s->fnorm};
  for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) tlh_devbuf_free(bufs[i]);
  tlh_pinned_free(&s->pin);
  tlh_pinned_free(&s->pin_rows);
  if (s->st) (void)hipStreamDestroy(s->st);
  free(s);
}

static int scratch_alloc_impl(int max_seq, DecoderScratch** out) {
  REQ(max_seq >= 1, "max_seq must be >= 1");
  DecoderScratch* p = (DecoderScratch*)calloc(1, sizeof *p);
  REQ(p, "out of host memory");
  int rc = 0;
  TRY_GO(tlh_current_device(&p->dev), fail);
  p->max_seq = max_seq;
  p->C = tlk_attn_chunks(max_seq);
  HIP_GO(hipStreamCreateWithFlags(&p->st, hipStreamNonBlocking), fail);
  HIP_GO(hipMalloc((void**)&p->hidden, (size_t)H * 4), fail);
  HIP_GO(hipMalloc((void**)&p->qkv, (size_t)QKVD * 4), fail);
  HIP_GO(hipMalloc((void**)&p->mlp, (size_t)FF * 4), fail);
  HIP_GO(hipMalloc((void**)&p->attn, (size_t)H * 4), fail);
  HIP_GO(hipMalloc((void**)&p->pm, (size_t)NQ * p->C * 4), fail);
  HIP_GO(hipMalloc((void**)&p->pl, (size_t)NQ * p->C * 4), fail);
  HIP_GO(hipMalloc((void**)&p->po, (size_t)NQ * p->C * HDIM * 4), fail);
  HIP_GO(hipMalloc((void**)&p->count, (size_t)NKV * sizeof(int)), fail);
  HIP_GO(hipMemsetAsync(p->count, 0, (size_t)NKV * sizeof(int), p->st), fail);
  HIP_GO(hipStreamSynchronize(p->st), fail);
  TRY_GO(tlh_pinned_ensure(&p->pin, STAGE_HIDDEN + (size_t)H * 4), fail);
  *out = p;
  return 0;
fail:
  scratch_free(p);
  return rc;
}

DecoderScratch* decoder_scratch_alloc_fn(int max_seq) {
  tlh_begin();
  DecoderScratch* s = NULL;
  const int rc = scratch_alloc_impl(max_seq, &s);
  tlh_finish("decoder_scratch_alloc_fn", rc);
  return rc == 0 ? s : NULL;
}

void decoder_scratch_free_fn(DecoderScratch* s) {
  if (s) scratch_free(s);
}

/* ---- weights (decoder.c:368-423) ------------------------------------------- */
void decoder_set_layer_weights(ModelWeights* model, int layer_idx, const int8_t* q_w, const float* q_s,
                               const int8_t* k_w, const float* k_s, const int8_t* v_w, const float* v_s,
                               const int8_t* o_w, const float* o_s, const int8_t* gate_w, const float* gate_s,
                               const int8_t* up_w, const float* up_s, const int8_t* down_w, const float* down_s,
                               const float* input_ln, const float* post_attn_ln, const float* q_norm,
                               const float* k_norm) {
  tlh_begin();
  const LayerSources w = {q_w, k_w, v_w, o_w, gate_w, up_w, down_w, NULL, NULL,
                          q_s, k_s, v_s, o_s, gate_s, up_s, down_s, NULL, NULL,
                          input_ln, post_attn_ln, q_norm, k_norm};
  tlh_finish("decoder_set_layer_weights", set_layer(model, layer_idx, &w));
}

void decoder_set_layer_weights_v32(ModelWeights* model, int layer_idx, const int8_t* q_w, const float* q_s,
                                   const int8_t* k_w, const float* k_s, const int8_t* v_w, const float* v_s,
                                   const int8_t* o_w, const float* o_s, const int8_t* gate_w, const float* gate_s,
                                   const int8_t* up_w, const float* up_s, const int8_t* down_w, const float* down_s,
                                   const float* input_ln, const float* post_attn_ln, const float* q_norm,
                                   const float* k_norm, const int8_t* qkv_w, const float* qkv_s,
                                   const int8_t* gate_up_w, const float* gate_up_s) {
  tlh_begin();
  const LayerSources w = {q_w, k_w, v_w, o_w, gate_w, up_w, down_w, qkv_w, gate_up_w,
                          q_s, k_s, v_s, o_s, gate_s, up_s, down_s, qkv_s, gate_up_s,
                          input_ln, post_attn_ln, q_norm, k_norm};
  tlh_finish("decoder_set_layer_weights_v32", set_layer(model, layer_idx, &w));
}

/* ---- rope tables (decoder.c:494-503 -> ops.c:150-177) ------------------------ */
void decoder_precompute_rope(float* cos_tab, float* sin_tab, int max_seq, int head_dim, const int sections[3],
                             const float theta_bases[3]) {
  (void)sections;   /* sequential positions: every section has the same angle */
  tlh_begin();
  if (!(cos_tab && sin_tab && theta_bases && max_seq >= 1 && head_dim >= 2)) {
    tlh_finish("decoder_precompute_rope", tlh_fail("bad arguments"));
    return;
  }
  const int half = head_dim / 2;
  for (int pos = 0; pos < max_seq; pos++)
    for (int j = 0; j < half; j++) {
      const float inv_freq = 1.0f / powf(theta_bases[0], (float)(2 * j) / (float)head_dim);
      const float angle = (float)pos * inv_freq;
      cos_tab[(size_t)pos * half + j] = cosf(angle);
      sin_tab[(size_t)pos * half + j] = sinf(angle);
    }
}

/* ---- one decode step on a host hidden row (decoder.c:452-462) --------------- */
typedef struct LayersCtx {
  const ModelWeights* m;
  const KVCache* c;
  DecoderScratch* s;
  const RopeDev* r;
} LayersCtx;

static int enqueue_layers_cb(void* p) {
  const LayersCtx* x = (const LayersCtx*)p;
  return enqueue_layers(x->m, x->c, x->s, x->r, x->s->st);
}

static int decode_step_impl(const ModelWeights* model, KVCache* cache, float* hidden, DecoderScratch* s,
                            const float* cos_tab, const float* sin_tab) {
  TRY(check_handles(model, cache, s));
  REQ(hidden, "NULL hidden");
  REQ(cache->seq_len < cache->max_seq, "KV cache is full");
  REQ(rope_pos(cache) < cache->max_seq, "rotary position past the rope tables");
  RopeDev* r;
  TRY(rope_device(cache, cos_tab, sin_tab, &r));
  const uint64_t key[4] = {model->version, cache->uid, r->uid, (uint64_t)num_layers(model)};
  if (!s->layers_exec || memcmp(key, s->layers_key, sizeof key) != 0) {
    drop_graph(&s->layers_exec);
    LayersCtx ctx = {model, cache, s, r};
    TRY(capture(s->st, enqueue_layers_cb, &ctx, &s->layers_exec));
    memcpy(s->layers_key, key, sizeof key);
  }
  TRY(write_state(cache, s, 0));   /* also leaves the stream idle */
  char* stage = (char*)s->pin.p + STAGE_HIDDEN;
  memcpy(stage, hidden, (size_t)H * 4);
  HIP_TRY(hipMemcpyAsync(s->hidden, stage, (size_t)H * 4, hipMemcpyHostToDevice, s->st));
  HIP_TRY(hipGraphLaunch(s->layers_exec, s->st));
  HIP_TRY(hipMemcpyAsync(stage, s->hidden, (size_t)H * 4, hipMemcpyDeviceToHost, s->st));
  HIP_TRY(hipStreamSynchronize(s->st));
  memcpy(hidden, stage, (size_t)H * 4);
  advance(cache, 1);
  return 0;
}

void decoder_decode_step(const ModelWeights* model, KVCache* cache, float* hidden, DecoderScratch* scratch,
                         const float* cos_tab, const float* sin_tab) {
  tlh_begin();
  tlh_finish("decoder_decode_step", decode_step_impl(model, cache, hidden, scratch, cos_tab, sin_tab));
}

/* ---- prefill (decoder.c:437-507) -------------------------------------------- */
static int prefill_checked(const ModelWeights* model, KVCache* cache, float* hidden, DecoderScratch* scratch,
                           const float* cos_tab, const float* sin_tab, int seq_len, int chunk, bool chunked) {
  REQ(cache, "NULL cache");
  REQ(cache->seq_len + seq_len <= cache->max_seq, "rotary positions past the rope tables");
  return prefill_host(model, cache, hidden, scratch, seq_len, cos_tab, sin_tab, NULL, NULL, chunk, chunked);
}

void decoder_prefill_step(const ModelWeights* model, KVCache* cache, float* hidden, DecoderScratch* scratch,
                          const float* cos_tab, const float* sin_tab, int seq_len) {
  tlh_begin();
  tlh_finish("decoder_prefill_step",
             prefill_checked(model, cache, hidden, scratch, cos_tab, sin_tab, seq_len, 0, false));
}

void decoder_chunked_prefill_step(const ModelWeights* model, KVCache* cache, float* hidden, DecoderScratch* scratch,
                                  const float* cos_tab, const float* sin_tab, int total_seq_len, int chunk_size) {
  tlh_begin();
  const int rc = chunk_size >= 1 ? prefill_checked(model, cache, hidden, scratch, cos_tab, sin_tab, total_seq_len,
                                                   chunk_size, true)
                                 : tlh_fail("chunk_size must be >= 1");
  tlh_finish("decoder_chunked_prefill_step", rc);
}

void decoder_hybrid_chunked_prefill_step(const ModelWeights* model, KVCache* cache, float* hidden,
                                         DecoderScratch* scratch, const float* cos_tab, const float* sin_tab,
                                         int seq_len, int chunk_size) {
  (void)chunk_size;   /* the reference chunks only its GEMMs; the results are those of one pass */
  tlh_begin();
  tlh_finish("decoder_hybrid_chunked_prefill_step",
             prefill_checked(model, cache, hidden, scratch, cos_tab, sin_tab, seq_len, 0, false));
}

void decoder_prefill_step_3d(const ModelWeights* model, KVCache* cache, float* hidden, DecoderScratch* scratch,
                             const float* token_cos, const float* token_sin, int seq_len) {
  tlh_begin();
  const int rc = (token_cos && token_sin)
                     ? prefill_host(model, cache, hidden, scratch, seq_len, NULL, NULL, token_cos, token_sin, 0, false)
                     : tlh_fail("NULL token tables");
  tlh_finish("decoder_prefill_step_3d", rc);
}

/* mrope_build_cos_sin_3d (ops.c:188-223): dims j < 3 min(sections[1],
 * sections[2]) take the T / H / W position j % 3, the rest T */
void decoder_build_rope_3d(float* cos_out, float* sin_out, const int* pos_ids, int seq_len, int head_dim,
                           const int sections[3], const float theta_bases[3]) {
  tlh_begin();
  if (!(cos_out && sin_out && pos_ids && sections && theta_bases && seq_len >= 1 && head_dim >= 2)) {
    tlh_finish("decoder_build_rope_3d", tlh_fail("bad arguments"));
    return;
  }
  const int half = head_dim / 2;
  const int min_s = sections[1] < sections[2] ? sections[1] : sections[2];
  for (int t = 0; t < seq_len; t++)
    for (int j = 0; j < half; j++) {
      const int sect = j < 3 * min_s ? j % 3 : 0;
      const int pos = pos_ids[sect * seq_len + t];
      const float inv_freq = 1.0f / powf(theta_bases[0], (float)(2 * j) / (float)head_dim);
      const float angle = (float)pos * inv_freq;
      cos_out[(size_t)t * half + j] = cosf(angle);
      sin_out[(size_t)t * half + j] = sinf(angle);
    }
}

/* ==========================================================================
 * Part 2 extensions
 * ========================================================================== */
int tl_decoder_num_layers(const ModelWeights* model) { return model ? num_layers(model) : -1; }

static int read_cache_impl(const KVCache* cache, int layer, float* k, float* v) {
  REQ(cache && layer >= 0 && layer < NL, "bad arguments");
  int dev;
  TRY(tlh_current_device(&dev));
  REQ(cache->dev == dev, "cache lives on another device");
  const size_t n = layer_floats(cache);
  if (k) HIP_TRY(hipMemcpy(k, cache->k + (size_t)layer * n, n * 4, hipMemcpyDeviceToHost));
  if (v) HIP_TRY(hipMemcpy(v, cache->v + (size_t)layer * n, n * 4, hipMemcpyDeviceToHost));
  return 0;
}
int tl_decoder_read_cache(const KVCache* cache, int layer, float* k, float* v) {
  tlh_begin();
  return tlh_finish("tl_decoder_read_cache", read_cache_impl(cache, layer, k, v));
}

int tl_decoder_cache_len(const KVCache* cache) { return cache ? cache->seq_len : -1; }

int tl_prefill_set_fused_quant(int on) {
  tlh_begin();
  if (on != 0 && on != 1) return tlh_finish("tl_prefill_set_fused_quant", tlh_fail("on must be 0 or 1"));
  atomic_store_explicit(&g_prefill_fused_quant, on != 0, memory_order_relaxed);
  return 0;
}

int tl_decoder_set_prefill_w8a8(ModelWeights* model, int on) {
  tlh_begin();
  if (!model) return tlh_finish("tl_decoder_set_prefill_w8a8", tlh_fail("NULL model"));
  model->prefill_w8a8 = on != 0;
  return 0;
}

typedef struct GenCtx {
  LayersCtx layers;
  const tl_weights* lm_head;
  const float* fn;
  const float* embed;
  int blocks, max_tokens;
} GenCtx;

static int enqueue_generate_cb(void* p) {
  const GenCtx* g = (const GenCtx*)p;
  DecoderScratch* s = g->layers.s;
  TRY(enqueue_layers_cb(&((GenCtx*)p)->layers));
  GemvLaunch L = tlk_gemv_launch_init();
  L.x = s->hidden;
  L.wt = g->lm_head->tiles;
  L.ws = g->lm_head->scales;
  L.N = g->lm_head->rows;
  L.K = H;
  L.epi = EPI_ARGMAX;
  L.keys = (uint64_t*)s->keys.p;
  L.norm = NORM_NUMPY;
  L.norm_w = g->fn;
  HIP_TRY(tlk_launch_gemv_i8(&L, s->st));
  HIP_TRY(tlk_launch_step_end((const uint64_t*)s->keys.p, g->blocks, g->embed, H, s->hidden, g->layers.c->state,
                              (int32_t*)s->tokens.p, g->max_tokens, s->st));
  return 0;
}

static int generate_impl(const ModelWeights* model, KVCache* cache, DecoderScratch* s, const tl_weights* lm_head,
                         const float* final_norm, const float* embed, int first_token, int n_steps, int32_t* tokens,
                         const float* cos_tab, const float* sin_tab) {
  TRY(check_handles(model, cache, s));
  TRY(tlh_check_weights(lm_head));
  REQ(embed && tokens && n_steps >= 1, "bad arguments");
  REQ(lm_head->cols == H, "lm_head must have hidden-size columns");
  REQ(first_token >= 0 && first_token < lm_head->rows, "first_token out of range");
  REQ(cache->seq_len + n_steps <= cache->max_seq, "KV cache too small for n_steps");
  REQ(rope_pos(cache) + n_steps <= cache->max_seq, "rotary positions past the rope tables");
  RopeDev* r;
  TRY(rope_device(cache, cos_tab, sin_tab, &r));
  GemvPlan plan;
  tlk_gemv_plan(lm_head->rows, H, &plan);
  TRY(tlh_devbuf_ensure(&s->keys, (size_t)plan.blocks * sizeof(uint64_t), s->st));
  TRY(tlh_devbuf_ensure(&s->tokens, (size_t)n_steps * sizeof(int32_t), s->st));
  TRY(tlh_devbuf_ensure(&s->fnorm, (size_t)H * 4, s->st));
  const float* fn = NULL;
  if (final_norm) {
    HIP_TRY(hipMemcpyAsync(s->fnorm.p, final_norm, (size_t)H * 4, hipMemcpyHostToDevice, s->st));
    fn = (const float*)s->fnorm.p;
  }
  const int max_tokens = (int)(s->tokens.n / sizeof(int32_t));
  /* embed is the caller's device pointer: its contents are read at replay */
  const uint64_t key[9] = {model->version,
                           cache->uid,
                           r->uid,
                           lm_head->uid,
                           (uint64_t)(uintptr_t)fn,
                           (uint64_t)(uintptr_t)embed,
                           (uint64_t)(uintptr_t)s->tokens.p,
                           (uint64_t)(uintptr_t)s->keys.p,
                           (uint64_t)num_layers(model) * 1000003u + (uint64_t)max_tokens};
  if (!s->gen_exec || memcmp(key, s->gen_key, sizeof key) != 0) {
    drop_graph(&s->gen_exec);
    GenCtx g = {{model, cache, s, r}, lm_head, fn, embed, plan.blocks, max_tokens};
    TRY(capture(s->st, enqueue_generate_cb, &g, &s->gen_exec));
    memcpy(s->gen_key, key, sizeof key);
  }
  TRY(write_state(cache, s, 0));
  HIP_TRY(hipMemcpyAsync(s->hidden, embed + (size_t)first_token * H, (size_t)H * 4, hipMemcpyDeviceToDevice, s->st));
  for (int i = 0; i < n_steps; i++) HIP_TRY(hipGraphLaunch(s->gen_exec, s->st));
  HIP_TRY(hipMemcpyAsync(tokens, s->tokens.p, (size_t)n_steps * sizeof(int32_t), hipMemcpyDeviceToHost, s->st));
  HIP_TRY(hipStreamSynchronize(s->st));
  advance(cache, n_steps);
  return 0;
}

int tl_decoder_generate(const ModelWeights* model, KVCache* cache, DecoderScratch* scratch, const tl_weights* lm_head,
                        const float* final_norm, const float* embed, int first_token, int n_steps, int32_t* tokens,
                        const float* cos_tab, const float* sin_tab) {
  tlh_begin();
  return tlh_finish("tl_decoder_generate", generate_impl(model, cache, scratch, lm_head, final_norm, embed,
                                                         first_token, n_steps, tokens, cos_tab, sin_tab));
}

/* ---- attention test hooks ----------------------------------------------------- */
static int attn_decode_body(const float* qkv, const float* q_norm, const float* k_norm, const float* cos_tab,
                            const float* sin_tab, float* k_cache, float* v_cache, int max_seq, int pos, int rpos,
                            float* out, hipStream_t st, DevBuf* ws) {
  const int C = tlk_attn_chunks(max_seq);
  const size_t part = (size_t)NQ * C * (2 + HDIM) * sizeof(float);
  TRY(tlh_devbuf_ensure(ws, part + 64 + (size_t)NKV * sizeof(int), st));
  char* base = (char*)ws->p;
  int* state = (int*)(base + part);
  int* count = (int*)(base + part + 64);
  const int hs[4] = {pos, rpos, 0, 0};
  HIP_TRY(hipMemsetAsync(count, 0, (size_t)NKV * sizeof(int), st));
  HIP_TRY(hipMemcpyAsync(state, hs, sizeof hs, hipMemcpyHostToDevice, st));
  AttnDecodeArgs a = tlk_attn_decode_init();
  a.qkv = qkv;
  a.q_norm = q_norm;
  a.k_norm = k_norm;
  a.cos_tab = cos_tab;
  a.sin_tab = sin_tab;
  a.kc = k_cache;
  a.vc = v_cache;
  a.state = state;
  a.pm = (float*)base;
  a.pl = a.pm + (size_t)NQ * C;
  a.po = a.pl + (size_t)NQ * C;
  a.count = count;
  a.out = out;
  a.nq = NQ;
  a.nkv = NKV;
  a.max_seq = max_seq;
  a.T = tlk_attn_chunk_size(max_seq);
  a.C = C;
  a.scale = SCALE;
  a.eps = EPS;
  HIP_TRY(tlk_launch_attn_decode(&a, st));
  HIP_TRY(hipStreamSynchronize(st));
  return 0;
}

static int attn_decode_dev_impl(const float* qkv, const float* q_norm, const float* k_norm, const float* cos_tab,
                                const float* sin_tab, float* k_cache, float* v_cache, int max_seq, int pos, int rpos,
                                float* out, void* stream) {
  REQ(qkv && q_norm && k_norm && cos_tab && sin_tab && k_cache && v_cache && out, "NULL argument");
  REQ(max_seq >= 1 && pos >= 0 && pos < max_seq && rpos >= 0 && rpos < max_seq, "bad positions");
  hipStream_t st = (hipStream_t)stream;
  DevBuf ws = {0};
  const int rc = attn_decode_body(qkv, q_norm, k_norm, cos_tab, sin_tab, k_cache, v_cache, max_seq, pos, rpos, out,
                                  st, &ws);
  /* the stream drains before the work-space goes, also on errors */
  (void)hipStreamSynchronize(st);
  tlh_devbuf_free(&ws);
  return rc;
}

int tl_attn_decode_dev(const float* qkv, const float* q_norm, const float* k_norm, const float* cos_tab,
                       const float* sin_tab, float* k_cache, float* v_cache, int max_seq, int pos, int rope_pos,
                       float* out, void* stream) {
  tlh_begin();
  return tlh_finish("tl_attn_decode_dev", attn_decode_dev_impl(qkv, q_norm, k_norm, cos_tab, sin_tab, k_cache, v_cache,
                                                               max_seq, pos, rope_pos, out, stream));
}

static int attn_prefill_body(const float* qkv, const float* k_cache, const float* v_cache, float* out, int S,
                             int max_seq, int key0, int qoff, int split, hipStream_t st, DevBuf* part, DevBuf* cnt) {
  if (split) {
    TRY(tlh_devbuf_ensure(part, tlk_flash_split_floats(S, NQ) * 4, st));
    TRY(tlh_devbuf_ensure(cnt, tlk_flash_split_counters(S, NQ) * sizeof(int), st));
    HIP_TRY(hipMemsetAsync(cnt->p, 0, cnt->n, st));
  }
  HIP_TRY(tlk_launch_flash_prefill(qkv, k_cache, v_cache, out, S, NQ, max_seq, key0, qoff, SCALE, (float*)part->p,
                                   (int*)cnt->p, st));
  HIP_TRY(hipStreamSynchronize(st));
  return 0;
}

static int attn_prefill_dev_impl(const float* qkv, const float* k_cache, const float* v_cache, float* out, int S,
                                 int max_seq, int key0, int qoff, int split, void* stream) {
  REQ(qkv && k_cache && v_cache && out, "NULL argument");
  REQ(S >= 1 && key0 >= 0 && qoff >= 0 && key0 + qoff + S <= max_seq, "bad sizes");
  hipStream_t st = (hipStream_t)stream;
  DevBuf part = {0}, cnt = {0};
  const int rc = attn_prefill_body(qkv, k_cache, v_cache, out, S, max_seq, key0, qoff, split, st, &part, &cnt);
  /* the stream drains before the work-space goes, also on errors */
  (void)hipStreamSynchronize(st);
  tlh_devbuf_free(&part);
  tlh_devbuf_free(&cnt);
  return rc;
}

int tl_attn_prefill_dev(const float* qkv, const float* k_cache, const float* v_cache, float* out, int S, int max_seq,
                        int key0, int qoff, int split, void* stream) {
  tlh_begin();
  return tlh_finish("tl_attn_prefill_dev",
                    attn_prefill_dev_impl(qkv, k_cache, v_cache, out, S, max_seq, key0, qoff, split, stream));
}
