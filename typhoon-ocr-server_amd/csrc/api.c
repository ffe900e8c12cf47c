/* api.c -- C ABI of libtyphoon_linear.so (declared in include/typhoon_linear.h).
 *
 * Part 1 keeps the reference's host-pointer entry points
 * (kernel/w8a32_kernel.c:63-68, :355-363; kernel/w8a8_kernel.c:102-114,
 * :270-272; kernel/w8a16_kernel.c:44, :218-219): the arguments are borrowed
 * host memory, the call is synchronous and Y is complete on return.  Each call
 * stages X through pinned memory into HBM, runs the kernels on a library
 * stream, and copies Y back.  Quantized weights stay resident in HBM as 16x64
 * tiles: a registry keyed by (weight pointer, scale pointer, rows, cols,
 * device) and validated with a sampled content fingerprint uploads and packs
 * a weight matrix the first time it is used (the reference keeps the same
 * host arrays alive for the model's lifetime: decoder.py:215, :259).
 *
 * Part 2 exposes the same kernels on device pointers and caller streams.
 * Split-reduction work-space (partials + arrival counters, counters zero at
 * rest) is owned per (device, stream).
 *
 * The kernels are reached through their C ABI (tl_kernels.h, tlk_*). */
#include "host.h"

#include <pthread.h>
#include <stdarg.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define MAX_DEVICES 64

/* ==========================================================================
 * errors, ids, buffers
 * ========================================================================== */
static _Thread_local char t_msg[1024];   /* the innermost failure */
static _Thread_local char t_err[1280];   /* "entry point: message" */
static _Thread_local bool t_has_err = false;

int tlh_fail(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(t_msg, sizeof t_msg, fmt, ap);
  va_end(ap);
  return -1;
}

int tlh_fail_hip(const char* expr, hipError_t e) { return tlh_fail("%s -> %s", expr, hipGetErrorString(e)); }

void tlh_begin(void) {
  t_has_err = false;
  t_msg[0] = 0;
}

int tlh_finish(const char* fn, int rc) {
  if (rc != 0) {
    snprintf(t_err, sizeof t_err, "%s: %s", fn, t_msg[0] ? t_msg : "unknown error");
    t_has_err = true;
    fprintf(stderr, "[typhoon_linear] %s\n", t_err);
  }
  return rc;
}

int tlh_current_device(int* dev) {
  int d = -1;
  HIP_TRY(hipGetDevice(&d));
  *dev = d;
  return 0;
}

uint64_t tlh_next_uid(void) {
  static atomic_uint_fast64_t counter = 1;
  return (uint64_t)atomic_fetch_add_explicit(&counter, 1, memory_order_relaxed);
}

int tlh_devbuf_ensure(DevBuf* b, size_t bytes, hipStream_t st) {
  if (bytes <= b->n) return 0;
  if (b->p) {
    HIP_TRY(hipStreamSynchronize(st));
    HIP_TRY(hipFree(b->p));
    b->p = NULL;
    b->n = 0;
  }
  const size_t want = bytes < 256 ? 256 : bytes;
  HIP_TRY(hipMalloc(&b->p, want));
  b->n = want;
  return 0;
}

void tlh_devbuf_free(DevBuf* b) {
  if (b->p) (void)hipFree(b->p);
  b->p = NULL;
  b->n = 0;
}

int tlh_pinned_ensure(PinnedBuf* b, size_t bytes) {
  if (bytes <= b->n) return 0;
  if (b->p) {
    HIP_TRY(hipHostFree(b->p));
    b->p = b->dp = NULL;
    b->n = 0;
  }
  const size_t want = bytes < 4096 ? 4096 : bytes;
  HIP_TRY(hipHostMalloc(&b->p, want, hipHostMallocDefault));
  const hipError_t e = hipHostGetDevicePointer(&b->dp, b->p, 0);
  if (e != hipSuccess) {   /* never leave a buffer without its device mapping */
    (void)hipHostFree(b->p);
    b->p = b->dp = NULL;
    return tlh_fail_hip("hipHostGetDevicePointer", e);
  }
  b->n = want;
  return 0;
}

void tlh_pinned_free(PinnedBuf* b) {
  if (b->p) (void)hipHostFree(b->p);
  b->p = b->dp = NULL;
  b->n = 0;
}

static size_t min_sz(size_t a, size_t b) { return a < b ? a : b; }

/* ==========================================================================
 * weights
 * ========================================================================== */
int tlh_weights_alloc(int rows, int cols, tl_weights** out) {
  REQ(rows > 0 && cols > 0, "rows and cols must be positive");
  int dev;
  TRY(tlh_current_device(&dev));
  tl_weights* W = (tl_weights*)calloc(1, sizeof *W);
  REQ(W, "out of host memory");
  W->uid = tlh_next_uid();
  W->dev = dev;
  W->rows = rows;
  W->cols = cols;
  W->KB = tlk_cdiv(cols, 64);
  W->NG = tlk_cdiv(rows, 16);
  const size_t tb = (size_t)W->NG * W->KB * 1024;
  const size_t sb = (size_t)W->NG * 16 * sizeof(float);
  if (hipMalloc((void**)&W->tiles, tb) != hipSuccess) {
    free(W);
    return tlh_fail("out of device memory for weight tiles");
  }
  if (hipMalloc((void**)&W->scales, sb) != hipSuccess) {
    (void)hipFree(W->tiles);
    free(W);
    return tlh_fail("out of device memory for weight scales");
  }
  W->bytes = tb + sb;
  *out = W;
  return 0;
}

void tlh_weights_free(tl_weights* W) {
  if (!W) return;
  if (W->tiles) (void)hipFree(W->tiles);
  if (W->scales) (void)hipFree(W->scales);
  free(W);
}

int tlh_weights_from_codes(const int8_t* w, const float* s, int rows, int cols, bool on_device, hipStream_t st,
                           tl_weights** out) {
  tl_weights* W = NULL;
  TRY(tlh_weights_alloc(rows, cols, &W));
  int rc = 0;
  void* tmp = NULL;
  const size_t wb = (size_t)rows * cols;
  HIP_GO(hipMemsetAsync(W->scales, 0, (size_t)W->NG * 16 * sizeof(float), st), fail);
  HIP_GO(hipMemcpyAsync(W->scales, s, (size_t)rows * sizeof(float),
                        on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st),
         fail);
  if (on_device) {
    HIP_GO(tlk_launch_pack_tiles(w, rows, cols, W->tiles, st), fail);
    HIP_GO(hipStreamSynchronize(st), fail);
  } else {
    HIP_GO(hipMalloc(&tmp, wb), fail);
    hipError_t e = hipMemcpyAsync(tmp, w, wb, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = tlk_launch_pack_tiles((const int8_t*)tmp, rows, cols, W->tiles, st);
    const hipError_t e2 = hipStreamSynchronize(st);
    (void)hipFree(tmp);
    HIP_GO(e, fail);
    HIP_GO(e2, fail);
  }
  *out = W;
  return 0;
fail:
  (void)hipStreamSynchronize(st);
  tlh_weights_free(W);
  return rc;
}

int tlh_check_weights(const tl_weights* W) {
  REQ(W != NULL, "weights handle is NULL");
  int dev;
  TRY(tlh_current_device(&dev));
  REQ(W->dev == dev, "weights live on another device");
  return 0;
}

/* ==========================================================================
 * per (device, stream) work-space
 * ========================================================================== */
typedef struct Workspace {
  int dev;
  hipStream_t st;
  DevBuf part;       /* split partial sums */
  DevBuf cnt;        /* arrival counters (zero at rest) */
  size_t cnt_n;
  DevBuf act;        /* activation codes (tiles or padded rows) */
  DevBuf act_s;      /* activation scales */
  DevBuf xn;         /* normalised hidden row (lm_head argmax) */
  DevBuf keys;       /* per-work-group argmax keys */
  DevBuf planes;     /* W8A32 batches: int8 plane tiles of the fp32 rows and their exponents */
  pthread_mutex_t mu;   /* held by one operation from its first buffer use to its last launch */
  struct Workspace* next;
} Workspace;

static pthread_mutex_t g_ws_mu = PTHREAD_MUTEX_INITIALIZER;
static Workspace* g_ws = NULL;

/* The work-space of (dev, st), returned locked: threads that enqueue on the
 * same stream (the null stream, say) take turns, so one never grows or frees
 * a buffer that another has just bound into its launches.  The caller unlocks
 * it after its last launch. */
static int workspace_lock(int dev, hipStream_t st, Workspace** out) {
  pthread_mutex_lock(&g_ws_mu);
  Workspace* w = g_ws;
  while (w && !(w->dev == dev && w->st == st)) w = w->next;
  if (!w) {
    w = (Workspace*)calloc(1, sizeof *w);
    if (w) {
      w->dev = dev;
      w->st = st;
      pthread_mutex_init(&w->mu, NULL);
      w->next = g_ws;
      g_ws = w;
    }
  }
  pthread_mutex_unlock(&g_ws_mu);
  REQ(w, "out of host memory");
  pthread_mutex_lock(&w->mu);
  *out = w;
  return 0;
}

#define WS_CALL(dev, st, call)               \
  do {                                       \
    Workspace* ws_;                          \
    TRY(workspace_lock((dev), (st), &ws_));  \
    const int rc_ = call;                    \
    pthread_mutex_unlock(&ws_->mu);          \
    return rc_;                              \
  } while (0)

static int ensure_counters(Workspace* w, size_t n, hipStream_t st, uint32_t** out) {
  if (n > w->cnt_n) {
    const size_t want = n < 65536 ? 65536 : n;
    TRY(tlh_devbuf_ensure(&w->cnt, want * sizeof(uint32_t), st));
    HIP_TRY(hipMemsetAsync(w->cnt.p, 0, want * sizeof(uint32_t), st));
    HIP_TRY(hipStreamSynchronize(st));
    w->cnt_n = want;
  }
  *out = (uint32_t*)w->cnt.p;
  return 0;
}

/* ==========================================================================
 * host-weight registry
 * ========================================================================== */
/* A registry-owned matrix, shared: a call holds a reference until it returns,
 * so an eviction by another thread (LRU, tl_evict_weights, a changed array)
 * only drops the registry's reference. */
typedef struct WRef {
  tl_weights* W;
  atomic_int refs;
} WRef;

static WRef* wref_new(tl_weights* W) {
  WRef* r = (WRef*)malloc(sizeof *r);
  if (!r) return NULL;
  r->W = W;
  atomic_init(&r->refs, 1);
  return r;
}
static WRef* wref_take(WRef* r) {
  atomic_fetch_add_explicit(&r->refs, 1, memory_order_relaxed);
  return r;
}
static void wref_drop(WRef* r) {
  if (r && atomic_fetch_sub_explicit(&r->refs, 1, memory_order_acq_rel) == 1) {
    tlh_weights_free(r->W);
    free(r);
  }
}

typedef struct RegNode {
  const void* w;
  const void* s;
  int rows, cols, dev;
  WRef* ref;
  uint64_t fp, tick;
  struct RegNode* next;
} RegNode;

#define REG_BUCKETS 1024
static pthread_mutex_t g_reg_mu = PTHREAD_MUTEX_INITIALIZER;
static RegNode* g_reg[REG_BUCKETS];
static size_t g_reg_count = 0;
static uint64_t g_tick = 0;
static size_t g_reg_bytes = 0;

static uint64_t mix64(uint64_t h, uint64_t v) {
  h ^= v + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
  h ^= h >> 31;
  h *= 0xbf58476d1ce4e5b9ull;
  return h ^ (h >> 29);
}

/* HBM budget for cached weights (288 GB per GPU), or TL_REGISTRY_MAX_BYTES;
 * read once */
static size_t g_reg_cap = 0;
static pthread_once_t g_reg_cap_once = PTHREAD_ONCE_INIT;
static void read_registry_cap(void) {
  const char* e = getenv("TL_REGISTRY_MAX_BYTES");
  g_reg_cap = (e && *e) ? (size_t)strtoull(e, NULL, 10) : (size_t)96 << 30;
}
static size_t registry_cap(void) {
  pthread_once(&g_reg_cap_once, read_registry_cap);
  return g_reg_cap;
}

/* sampled content fingerprint: 64 eight-byte windows of W, 32 scales, shape */
static uint64_t fingerprint(const int8_t* w, const float* s, int rows, int cols) {
  uint64_t h = mix64((uint64_t)rows, (uint64_t)cols);
  const size_t n = (size_t)rows * cols;
  if (n >= 8) {
    for (int i = 0; i < 64; i++) {
      const size_t off = (size_t)(((unsigned __int128)(n - 8) * (unsigned)i) / 63);
      uint64_t v;
      memcpy(&v, w + off, 8);
      h = mix64(h, v);
    }
  } else {
    for (size_t i = 0; i < n; i++) h = mix64(h, (uint64_t)(uint8_t)w[i]);
  }
  for (int i = 0; i < 32; i++) {
    const size_t r = (size_t)(((unsigned long long)(rows - 1) * (unsigned)i) / 31);
    uint32_t v;
    memcpy(&v, s + r, 4);
    h = mix64(h, v);
  }
  return h;
}

static size_t reg_bucket(const void* w, const void* s, int rows, int cols, int dev) {
  uint64_t h = mix64((uint64_t)(uintptr_t)w, (uint64_t)(uintptr_t)s);
  h = mix64(h, ((uint64_t)(uint32_t)rows << 32) | (uint32_t)cols);
  h = mix64(h, (uint64_t)(uint32_t)dev);
  return (size_t)(h & (REG_BUCKETS - 1));
}

static RegNode** reg_find_locked(const void* w, const void* s, int rows, int cols, int dev) {
  RegNode** pp = &g_reg[reg_bucket(w, s, rows, cols, dev)];
  while (*pp) {
    const RegNode* n = *pp;
    if (n->w == w && n->s == s && n->rows == rows && n->cols == cols && n->dev == dev) return pp;
    pp = &(*pp)->next;
  }
  return NULL;
}

/* unlinks *pp and drops the registry's reference */
static void reg_erase_locked(RegNode** pp) {
  RegNode* n = *pp;
  *pp = n->next;
  g_reg_bytes -= n->ref->W->bytes;
  g_reg_count--;
  wref_drop(n->ref);
  free(n);
}

static void registry_evict_lru_locked(size_t need) {
  while (g_reg_count > 0 && g_reg_bytes + need > registry_cap()) {
    RegNode** victim = NULL;
    for (int b = 0; b < REG_BUCKETS; b++)
      for (RegNode** pp = &g_reg[b]; *pp; pp = &(*pp)->next)
        if (!victim || (*pp)->tick < (*victim)->tick) victim = pp;
    reg_erase_locked(victim);
  }
}

static int reg_insert_locked(const void* w, const void* s, int dev, WRef* ref, uint64_t fp) {
  RegNode* n = (RegNode*)calloc(1, sizeof *n);
  REQ(n, "out of host memory");
  const tl_weights* W = ref->W;
  n->w = w;
  n->s = s;
  n->rows = W->rows;
  n->cols = W->cols;
  n->dev = dev;
  n->ref = ref;
  n->fp = fp;
  n->tick = ++g_tick;
  RegNode** head = &g_reg[reg_bucket(w, s, W->rows, W->cols, dev)];
  n->next = *head;
  *head = n;
  g_reg_count++;
  g_reg_bytes += W->bytes;
  return 0;
}

/* the resident matrix of host arrays (w, s), uploaded and packed on first
 * use (or again when their contents changed); the caller drops *out.
 * A miss uploads without holding the registry lock, so calls whose weights
 * are resident go on meanwhile (a first lm_head upload moves 311 MB); two
 * threads that miss on the same arrays both upload, and the second to
 * insert takes the first one's entry and frees its own copy.  The LRU
 * eviction runs at the insert, so the budget can be exceeded by the matrices
 * in flight. */
static int registry_get(const int8_t* w, const float* s, int rows, int cols, hipStream_t st, WRef** out) {
  REQ(w && s, "weight and scale pointers must be non-NULL");
  int dev;
  TRY(tlh_current_device(&dev));
  const uint64_t fp = fingerprint(w, s, rows, cols);
  pthread_mutex_lock(&g_reg_mu);
  RegNode** pp = reg_find_locked(w, s, rows, cols, dev);
  if (pp && (*pp)->fp == fp) {
    (*pp)->tick = ++g_tick;
    *out = wref_take((*pp)->ref);
    pthread_mutex_unlock(&g_reg_mu);
    return 0;
  }
  pthread_mutex_unlock(&g_reg_mu);
  tl_weights* W = NULL;
  TRY(tlh_weights_from_codes(w, s, rows, cols, false, st, &W));
  WRef* ref = wref_new(W);
  if (!ref) {
    tlh_weights_free(W);
    return tlh_fail("out of host memory");
  }
  pthread_mutex_lock(&g_reg_mu);
  pp = reg_find_locked(w, s, rows, cols, dev);
  if (pp && (*pp)->fp == fp) {              /* another thread's upload of the same contents won */
    (*pp)->tick = ++g_tick;
    *out = wref_take((*pp)->ref);
    pthread_mutex_unlock(&g_reg_mu);
    wref_drop(ref);
    return 0;
  }
  if (pp) reg_erase_locked(pp);             /* contents changed in place: replace */
  registry_evict_lru_locked(W->bytes);
  if (reg_insert_locked(w, s, dev, ref, fp) != 0) {
    pthread_mutex_unlock(&g_reg_mu);
    wref_drop(ref);
    return -1;
  }
  *out = wref_take(ref);
  pthread_mutex_unlock(&g_reg_mu);
  return 0;
}

/* makes W (owned by the registry from here on) the entry of host arrays
 * (w, s) that hold its codes and scales; replaces an existing entry */
static int registry_put(const int8_t* w, const float* s, tl_weights* W) {
  const uint64_t fp = fingerprint(w, s, W->rows, W->cols);
  int rc = 0;
  pthread_mutex_lock(&g_reg_mu);
  RegNode** pp = reg_find_locked(w, s, W->rows, W->cols, W->dev);
  WRef* ref = NULL;
  if (pp) {
    if ((*pp)->ref->W == W) ref = wref_take((*pp)->ref);   /* re-adopting the same matrix */
    reg_erase_locked(pp);
  }
  if (!ref) {
    ref = wref_new(W);
    REQ_GO(ref, done, "out of host memory");
  }
  registry_evict_lru_locked(W->bytes);
  if (reg_insert_locked(w, s, W->dev, ref, fp) != 0) {
    wref_drop(ref);
    rc = -1;
  }
done:
  pthread_mutex_unlock(&g_reg_mu);
  return rc;
}

/* ==========================================================================
 * host-call contexts (Part 1): a call leases one for its duration (its own
 * stream, staging and pinned buffers), so calls from different threads run
 * concurrently; contexts return to a per-device pool, which holds as many as
 * calls ever overlapped
 * ========================================================================== */
typedef struct HostCtx {
  int dev;
  hipStream_t st;
  DevBuf x, y, bias, xs;
  PinnedBuf hin, hout, htok;
  struct HostCtx* next;
} HostCtx;

static pthread_mutex_t g_host_mu = PTHREAD_MUTEX_INITIALIZER;   /* guards the pool only */
static HostCtx* g_host_free[MAX_DEVICES];

static int host_lease(HostCtx** out) {
  int dev;
  TRY(tlh_current_device(&dev));
  REQ(dev >= 0 && dev < MAX_DEVICES, "device index out of range");
  pthread_mutex_lock(&g_host_mu);
  HostCtx* c = g_host_free[dev];
  if (c) g_host_free[dev] = c->next;
  pthread_mutex_unlock(&g_host_mu);
  if (!c) {
    c = (HostCtx*)calloc(1, sizeof *c);
    REQ(c, "out of host memory");
    c->dev = dev;
    if (hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking) != hipSuccess) {
      free(c);
      return tlh_fail("hipStreamCreateWithFlags failed");
    }
  }
  *out = c;
  return 0;
}

/* back to the pool, also after an error: its next user waits on its stream
 * before reusing a staging buffer */
static void host_release(HostCtx* c) {
  pthread_mutex_lock(&g_host_mu);
  c->next = g_host_free[c->dev];
  g_host_free[c->dev] = c;
  pthread_mutex_unlock(&g_host_mu);
}

static int h2d(HostCtx* c, DevBuf* d, const void* src, size_t bytes) {
  TRY(tlh_pinned_ensure(&c->hin, bytes));
  TRY(tlh_devbuf_ensure(d, bytes, c->st));
  HIP_TRY(hipStreamSynchronize(c->st));   /* hin may still be the source of an earlier copy */
  memcpy(c->hin.p, src, bytes);
  HIP_TRY(hipMemcpyAsync(d->p, c->hin.p, bytes, hipMemcpyHostToDevice, c->st));
  return 0;
}

static int d2h(HostCtx* c, void* dst, const void* src, size_t bytes) {
  TRY(tlh_pinned_ensure(&c->hout, bytes));
  HIP_TRY(hipMemcpyAsync(c->hout.p, src, bytes, hipMemcpyDeviceToHost, c->st));
  HIP_TRY(hipStreamSynchronize(c->st));
  memcpy(dst, c->hout.p, bytes);
  return 0;
}

static int check_shape(int batch, int M, int K) {
  REQ(batch >= 1, "batch must be >= 1");
  REQ(M >= 1, "M (output features) must be >= 1");
  REQ(K >= 1, "K (input features) must be >= 1");
  return 0;
}

/* ==========================================================================
 * device-level operations shared by Part 1 and Part 2
 * ========================================================================== */

/* precomputed codes for the GEMV: row-major, zero padded to KB*64 */
static int quantize_padded(Workspace* ws, const float* x, int K, hipStream_t st, uint8_t** codes, float** xs_dev) {
  const int kpad = tlk_cdiv(K, 64) * 64;
  TRY(tlh_devbuf_ensure(&ws->act, (size_t)kpad, st));
  TRY(tlh_devbuf_ensure(&ws->act_s, sizeof(float), st));
  HIP_TRY(tlk_launch_copy_pad_bytes(NULL, 0, ws->act.p, (size_t)kpad, st));   /* zero padding, a kernel node */
  HIP_TRY(tlk_launch_quantize_rows(x, (int8_t*)ws->act.p, (float*)ws->act_s.p, 1, K, false, st));
  *xs_dev = (float*)ws->act_s.p;
  *codes = (uint8_t*)ws->act.p;
  return 0;
}

/* 1 KiB of zeros per device: the int8 GEMM copies it in place of k-blocks
 * past K */
static pthread_mutex_t g_zero_mu = PTHREAD_MUTEX_INITIALIZER;
static uint8_t* g_zero[MAX_DEVICES];

static int zero_tile(const uint8_t** out) {
  int dev;
  TRY(tlh_current_device(&dev));
  REQ(dev >= 0 && dev < MAX_DEVICES, "device index out of range");
  int rc = 0;
  pthread_mutex_lock(&g_zero_mu);
  if (!g_zero[dev]) {
    void* p = NULL;
    HIP_GO(hipMalloc(&p, 1024), done);
    HIP_GO(hipMemset(p, 0, 1024), done);   /* blocks the host until done */
    HIP_GO(hipDeviceSynchronize(), done);
    g_zero[dev] = (uint8_t*)p;
  }
  *out = g_zero[dev];
done:
  pthread_mutex_unlock(&g_zero_mu);
  return rc;
}

static int run_gemm(Workspace* ws, GemmLaunch* L, hipStream_t st) {
  TRY(zero_tile(&L->zero_tile));
  size_t part_bytes = 0, counters = 0;
  tlk_gemm_needs(L, &part_bytes, &counters);
  if (part_bytes > 0) {
    TRY(tlh_devbuf_ensure(&ws->part, part_bytes, st));
    L->part = ws->part.p;
    TRY(ensure_counters(ws, counters, st, &L->cnt));
  }
  HIP_TRY(tlk_launch_gemm(L, st));
  return 0;
}

/* 1..8 rows with fp32 semantics as int8 digit planes (rows.hip); *done = false
 * when the shape or alignment is not one it takes, or the path is switched off */
/* tuning switches; atomic, since a setter may run while other threads call */
static atomic_bool g_rows_off = false;
static atomic_bool g_gemv_w8a16_off = false;   /* W8A16 batch 1 on the bf16 / fp16 MFMA kernel instead */
static atomic_int g_gemv_rows2 = 1;             /* W8A32 batch 2..4 on the GEMV: 0 never, 1 planner, 2 always */

/* W8A32 batch 2..4 on the GEMV's token-row mode (mode 1 the measured choice,
 * 2 wherever the kernel takes the shape).  Against the digit-row kernel
 * (rows.hip) and the planes GEMM (graph-replayed calls over rotating weights):
 * 2 tokens 2.97-7.11 against 3.92-8.04 us on every decoder shape, lm_head
 * 48.8 against 54.3 us; 3 / 4 tokens 3.92-8.20 against 4.37-9.57 us on every
 * decoder shape (down 7.40 / 7.48 against 9.50 / 9.57), while an lm_head-wide
 * weight (53.6 / 55.8 against 54.4 / 54.7 us) stays on the planes GEMM */
static bool gemv_rows_ok(const tl_weights* W, int batch, int mode) {
  const int xv = tlk_gemv_fused_xv(W->cols);
  if (xv == 0 || (batch > 2 && xv > 8)) return false;
  if (mode == 2 || batch == 2) return true;
  return W->NG < 2048;
}

static int run_rows(Workspace* ws, GemmLaunch* L, hipStream_t st, bool* done) {
  *done = false;
  if (atomic_load_explicit(&g_rows_off, memory_order_relaxed) || !tlk_rows_supported(L)) return 0;
  RowsPlan p;
  tlk_rows_plan(L->M, L->N, L->K, &p);
  if (p.split > 1) {
    TRY(tlh_devbuf_ensure(&ws->part, tlk_rows_workspace_bytes(L->M, L->N, L->K), st));
    L->part = ws->part.p;
    TRY(ensure_counters(ws, tlk_rows_counter_count(L->N), st, &L->cnt));
  }
  HIP_TRY(tlk_launch_rows(L, st));
  *done = true;
  return 0;
}

static int op_w8a32_ws(Workspace* ws, const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st) {
  if (batch == 1) {
    GemvLaunch L = tlk_gemv_launch_init();
    L.wt = W->tiles;
    L.ws = W->scales;
    L.bias = bias;
    L.y = Y;
    L.N = W->rows;
    L.K = W->cols;
    L.epi = EPI_W8A32;
    if (tlk_gemv_fused_xv(W->cols) > 0) {
      L.x = X;
    } else {
      uint8_t* xq;
      float* xs;
      TRY(quantize_padded(ws, X, W->cols, st, &xq, &xs));
      L.xq = xq;
      L.xs_in = xs;
    }
    HIP_TRY(tlk_launch_gemv_i8(&L, st));
    return 0;
  }
  GemmLaunch L = tlk_gemm_launch_init();
  L.amode = A_F32X3;
  L.A = X;
  L.lda = W->cols;
  L.Bt = W->tiles;
  L.ws = W->scales;
  L.bias = bias;
  L.Y = Y;
  L.ldy = W->rows;
  L.M = batch;
  L.N = W->rows;
  L.K = W->cols;
  L.ep = EP_SCALE;
  L.out = OUT_F32;
  /* 2..4 token rows: the batch-1 GEMV's weight stream with four int8 digit
   * rows per token (the arithmetic of the digit-row kernel below at one K
   * slice, so the same bits), every weight read once for all of them */
  const int rows_mode = atomic_load_explicit(&g_gemv_rows2, memory_order_relaxed);
  if (batch >= 2 && batch <= 4 && rows_mode != 0 && gemv_rows_ok(W, batch, rows_mode)) {
    GemvLaunch G = tlk_gemv_launch_init();
    G.x = X;
    G.wt = W->tiles;
    G.ws = W->scales;
    G.bias = bias;
    G.y = Y;
    G.N = W->rows;
    G.K = W->cols;
    G.epi = EPI_W8A32_ROWS;
    G.ntok = batch;
    HIP_TRY(tlk_launch_gemv_i8(&G, st));
    return 0;
  }
  /* 2..8 token rows over a weight of fewer than 32768 rows: int8 digit planes
   * of the fp32 rows, made inside the one launch (rows.hip; every work-group
   * splits its activation slice, which an lm_head-wide grid repeats too
   * often: 151936 rows at 2 tokens 60.1 us there against 57.0 us below, at 8
   * tokens 133 against 68 us) */
  /* ... except 5..8 rows with K past 2048 (more than 32 k-blocks), which the
   * digit-row kernel's LDS takes in several K slices and a merge: there the
   * planes below are faster (2048x6144 at 5 / 8 tokens 13.8 / 14.7 us against
   * 11.2 / 11.4 us), unless a slice count is forced for tuning */
  const bool rows_sliced = batch > 4 && tlk_cdiv(W->cols, 64) > 32 && tlk_rows_forced_split() == 0;
  if (batch <= 8 && W->NG < 2048 && !rows_sliced) {
    bool done;
    TRY(run_rows(ws, &L, st, &done));
    if (done) return 0;
  }
  if (W->cols <= 2048 && ((batch <= 16 && W->NG <= 768) || (batch <= 32 && W->NG <= 384))) {
    /* a few token rows over a weight of up to 12288 rows with a short K: the
     * small-M kernel splits the fp32 rows into three bf16 terms as it loads
     * them (one launch, where a separate plane split costs more than it
     * saves: 2048x2048 at 9 / 16 / 32 tokens 6.9 / 8.6 / 8.6 us; 6144x2048
     * at 24 / 32 tokens 10.8 / 11.4 us against 14.8 / 15.4 us on the planes,
     * 12288x2048 at 9 / 16 tokens 10.7 / 11.9 against 15.8 / 16.1).  Every
     * work-group reads all the token rows of its token group, which more
     * tokens over many weight rows or a long K make the cost: 12288x2048 at
     * 24 / 32 tokens 17.9 / 19.9 us here against 15.3 / 16.1 us on the
     * planes, 2048x4096 at 9 / 16 tokens 11.9 / 14.4 against 11.1 / 12.6 */
    return run_gemm(ws, &L, st);
  }
  /* fp32 rows as four int8 planes each (x = 2^e (q0 + q1/254 + q2/254^2 +
   * q3/254^3), about 2^-32 of the row's absmax), then one int8 MFMA GEMM over
   * the 4 batch code rows whose epilogue folds each token's planes (no int8
   * -> 16-bit widening of the weights, the VALU bound of the three-term bf16
   * path) */
  const int K = W->cols, M4 = 4 * batch;
  const size_t tb = (size_t)tlk_cdiv(M4, 16) * W->KB * 1024;
  const size_t xe_off = (tb + 255) & ~(size_t)255;
  TRY(tlh_devbuf_ensure(&ws->planes, xe_off + (size_t)batch * sizeof(int), st));
  uint8_t* tiles = (uint8_t*)ws->planes.p;
  int* xe = (int*)(tiles + xe_off);
  /* one work-group per row where the shape allows it (the same planes) */
  const bool by_rows = (K == 1024 || K == 2048 || K == 4096 || K == 6144) && (((uintptr_t)X) & 15) == 0;
  if (by_rows) HIP_TRY(tlk_launch_split_rows_planes(X, K, batch, K, tiles, xe, st));
  else HIP_TRY(tlk_launch_split_i8x4(X, K, batch, K, tiles, xe, st));
  GemmLaunch P = tlk_gemm_launch_init();
  P.amode = A_I8;
  P.A = tiles;
  P.Bt = W->tiles;
  P.ws = W->scales;
  P.xe = xe;
  P.xraw = X;       /* outputs of a row holding Inf / NaN are taken from it */
  P.ldxr = K;
  P.bias = bias;
  P.Y = Y;
  P.ldy = W->rows;
  P.M = M4;
  P.N = W->rows;
  P.K = K;
  P.out = OUT_F32_X4;
  return run_gemm(ws, &P, st);
}

static int op_w8a32(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st) {
  WS_CALL(W->dev, st, op_w8a32_ws(ws_, X, W, bias, Y, batch, st));
}

/* W8A8 on row-major device codes */
static int op_w8a8_codes_ws(Workspace* ws, const int8_t* xq, const float* xs, const tl_weights* W, const float* bias, void* Y, int out,
                         int batch, hipStream_t st) {
  const int K = W->cols, KB = W->KB;
  if (batch == 1 && out != OUT_I32) {
    /* codes must be zero padded to KB*64 for the GEMV */
    const int kpad = KB * 64;
    TRY(tlh_devbuf_ensure(&ws->act, (size_t)kpad, st));
    HIP_TRY(tlk_launch_copy_pad_bytes(xq, (size_t)K, ws->act.p, (size_t)kpad, st));
    GemvLaunch L = tlk_gemv_launch_init();
    L.xq = (const uint8_t*)ws->act.p;
    L.xs_in = xs;
    L.wt = W->tiles;
    L.ws = W->scales;
    L.bias = bias;
    L.y = (float*)Y;
    L.N = W->rows;
    L.K = K;
    L.epi = EPI_W8A8;
    HIP_TRY(tlk_launch_gemv_i8(&L, st));
    return 0;
  }
  const size_t tb = (size_t)tlk_cdiv(batch, 16) * KB * 1024;
  TRY(tlh_devbuf_ensure(&ws->act, tb, st));
  HIP_TRY(tlk_launch_pack_tiles(xq, batch, K, (uint8_t*)ws->act.p, st));
  GemmLaunch L = tlk_gemm_launch_init();
  L.amode = A_I8;
  L.A = ws->act.p;
  L.Bt = W->tiles;
  L.ws = W->scales;
  L.xs = xs;
  L.bias = bias;
  L.Y = Y;
  L.ldy = W->rows;
  L.M = batch;
  L.N = W->rows;
  L.K = K;
  L.out = out;
  return run_gemm(ws, &L, st);
}

static int op_w8a8_codes(const int8_t* xq, const float* xs, const tl_weights* W, const float* bias, void* Y, int out,
                         int batch, hipStream_t st) {
  WS_CALL(W->dev, st, op_w8a8_codes_ws(ws_, xq, xs, W, bias, Y, out, batch, st));
}

/* per-token int8 activations of fp32 X (the GEMV quantizes inside its
 * prologue at batch 1), int8 GEMM, fp32 out */
static int op_w8a8_f32_ws(Workspace* ws, const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st) {
  if (batch == 1) {
    GemvLaunch L = tlk_gemv_launch_init();
    L.wt = W->tiles;
    L.ws = W->scales;
    L.bias = bias;
    L.y = Y;
    L.N = W->rows;
    L.K = W->cols;
    L.epi = EPI_W8A8;
    if (tlk_gemv_fused_xv(W->cols) > 0) {
      L.x = X;
    } else {
      uint8_t* xq;
      float* xs;
      TRY(quantize_padded(ws, X, W->cols, st, &xq, &xs));
      L.xq = xq;
      L.xs_in = xs;
    }
    HIP_TRY(tlk_launch_gemv_i8(&L, st));
    return 0;
  }
  const int MG = tlk_cdiv(batch, 16);
  TRY(tlh_devbuf_ensure(&ws->act, (size_t)MG * W->KB * 1024, st));
  TRY(tlh_devbuf_ensure(&ws->act_s, (size_t)MG * 16 * sizeof(float), st));
  {
    const int K = W->cols;
    const bool by_rows = (K == 1024 || K == 2048 || K == 4096 || K == 6144) && (((uintptr_t)X) & 15) == 0;
    if (by_rows)
      HIP_TRY(tlk_launch_quantize_rows_by_row(X, batch, K, (uint8_t*)ws->act.p, (float*)ws->act_s.p, st));
    else
      HIP_TRY(tlk_launch_quantize_rows_tiled(X, batch, K, (uint8_t*)ws->act.p, (float*)ws->act_s.p, true, st));
  }
  GemmLaunch L = tlk_gemm_launch_init();
  L.amode = A_I8;
  L.A = ws->act.p;
  L.Bt = W->tiles;
  L.ws = W->scales;
  L.xs = (const float*)ws->act_s.p;
  L.bias = bias;
  L.Y = Y;
  L.ldy = W->rows;
  L.M = batch;
  L.N = W->rows;
  L.K = W->cols;
  L.out = OUT_F32;
  return run_gemm(ws, &L, st);
}

static int op_w8a8_f32(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st) {
  WS_CALL(W->dev, st, op_w8a8_f32_ws(ws_, X, W, bias, Y, batch, st));
}

static int op_w8a16_ws(Workspace* ws, const void* X, int x_type, const tl_weights* W, const float* bias, void* Y, int y_type, int batch,
                    hipStream_t st) {
  REQ(x_type == TL_BF16 || x_type == TL_F16, "x_type must be TL_BF16 or TL_F16");
  REQ(y_type == TL_F32 || y_type == TL_BF16 || y_type == TL_F16, "bad y_type");
  GemmLaunch L = tlk_gemm_launch_init();
  L.amode = (x_type == TL_BF16) ? A_BF16 : A_F16;
  L.A = X;
  L.lda = W->cols;
  L.Bt = W->tiles;
  L.ws = W->scales;
  L.bias = bias;
  L.Y = Y;
  L.ldy = W->rows;
  L.M = batch;
  L.N = W->rows;
  L.K = W->cols;
  /* batch==1 fuses the bias into one fma (kernel/w8a16_kernel.c:134); batch>1
   * adds it after the product (:193-200) */
  L.ep = (batch == 1) ? EP_SCALE_FMA : EP_SCALE;
  L.out = (y_type == TL_F32) ? OUT_F32 : (y_type == TL_BF16 ? OUT_BF16 : OUT_F16);
  if (batch == 1 && tlk_gemv_fused_xv(W->cols) > 0 && !atomic_load_explicit(&g_gemv_w8a16_off, memory_order_relaxed)) {
    /* one token: the GEMV's weight stream with x as four int8 digit rows
     * (fp32-accurate products, y = fma(sum, ws, bias) as the reference's
     * r * ws + b) */
    GemvLaunch G = tlk_gemv_launch_init();
    G.x = (const float*)X;
    G.x_type = x_type == TL_BF16 ? 1 : 2;
    G.wt = W->tiles;
    G.ws = W->scales;
    G.bias = bias;
    G.y = (float*)Y;
    G.N = W->rows;
    G.K = W->cols;
    G.epi = EPI_W8A16;
    G.out = L.out;
    HIP_TRY(tlk_launch_gemv_i8(&G, st));
    return 0;
  }
  return run_gemm(ws, &L, st);
}

static int op_w8a16(const void* X, int x_type, const tl_weights* W, const float* bias, void* Y, int y_type, int batch,
                    hipStream_t st) {
  WS_CALL(W->dev, st, op_w8a16_ws(ws_, X, x_type, W, bias, Y, y_type, batch, st));
}

int tlh_linear_w8a32(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st) {
  return op_w8a32(X, W, bias, Y, batch, st);
}

int tlh_linear_w8a8(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st) {
  return op_w8a8_f32(X, W, bias, Y, batch, st);
}

static int linear_w8a32_planes_ws(Workspace* ws, const uint8_t* tiles, const int* xe, const tl_weights* W, float* Y, int batch,
                            hipStream_t st) {
  GemmLaunch L = tlk_gemm_launch_init();
  L.amode = A_I8;
  L.A = tiles;
  L.Bt = W->tiles;
  L.ws = W->scales;
  L.xe = xe;
  L.Y = Y;
  L.ldy = W->rows;
  L.M = 4 * batch;
  L.N = W->rows;
  L.K = W->cols;
  L.out = OUT_F32_X4;
  return run_gemm(ws, &L, st);
}

int tlh_linear_w8a32_planes(const uint8_t* tiles, const int* xe, const tl_weights* W, float* Y, int batch,
                            hipStream_t st) {
  WS_CALL(W->dev, st, linear_w8a32_planes_ws(ws_, tiles, xe, W, Y, batch, st));
}

static int linear_w8a8_tiles_ws(Workspace* ws, const uint8_t* tiles, const float* xs, const tl_weights* W,
                                const float* bias, float* Y, int batch, hipStream_t st) {
  GemmLaunch L = tlk_gemm_launch_init();
  L.amode = A_I8;
  L.A = tiles;
  L.Bt = W->tiles;
  L.ws = W->scales;
  L.xs = xs;
  L.bias = bias;
  L.Y = Y;
  L.ldy = W->rows;
  L.M = batch;
  L.N = W->rows;
  L.K = W->cols;
  L.out = OUT_F32;
  return run_gemm(ws, &L, st);
}

int tlh_linear_w8a8_tiles(const uint8_t* tiles, const float* xs, const tl_weights* W, float* Y, int batch,
                          hipStream_t st) {
  WS_CALL(W->dev, st, linear_w8a8_tiles_ws(ws_, tiles, xs, W, NULL, Y, batch, st));
}

/* Quantizes rows of host fp32 on the GPU and returns codes and scales to the
 * host.  With `pack` (the weight quantizers) the same device codes are also
 * packed into HBM tiles as they are produced, and the packed matrix becomes
 * the registry entry of the returned host arrays: the load step quantizes and
 * packs in one pass, and the first linear call on those arrays uploads
 * nothing (the reference quantizes on the CPU at load, decoder.py:248-260,
 * then hands the arrays to the C decoder, decoder.c:393-423). */
static int host_quantize_body(HostCtx* c, const float* src, int8_t* dst, float* scales, int rows, int cols,
                              bool clamp127, tl_weights* W, int chunk) {
  if (W) HIP_TRY(hipMemsetAsync(W->scales, 0, (size_t)W->NG * 16 * sizeof(float), c->st));
  TRY(tlh_devbuf_ensure(&c->y, (size_t)chunk * cols, c->st));
  TRY(tlh_devbuf_ensure(&c->xs, (size_t)chunk * sizeof(float), c->st));
  for (int r0 = 0; r0 < rows; r0 += chunk) {
    const int nr = chunk < rows - r0 ? chunk : rows - r0;
    TRY(h2d(c, &c->x, src + (size_t)r0 * cols, (size_t)nr * cols * sizeof(float)));
    HIP_TRY(tlk_launch_quantize_rows((const float*)c->x.p, (int8_t*)c->y.p, (float*)c->xs.p, nr, cols, clamp127,
                                     c->st));
    if (W) {
      HIP_TRY(tlk_launch_pack_tiles_rows((const int8_t*)c->y.p, nr, cols, W->NG, r0 / 16, W->tiles, c->st));
      HIP_TRY(hipMemcpyAsync(W->scales + r0, c->xs.p, (size_t)nr * sizeof(float), hipMemcpyDeviceToDevice, c->st));
    }
    TRY(d2h(c, dst + (size_t)r0 * cols, c->y.p, (size_t)nr * cols));
    TRY(d2h(c, scales + r0, c->xs.p, (size_t)nr * sizeof(float)));
  }
  return 0;
}

static int host_quantize(const float* src, int8_t* dst, float* scales, int rows, int cols, bool clamp127, bool pack) {
  REQ(src && dst && scales, "NULL pointer");
  REQ(rows >= 1 && cols >= 1, "rows and cols must be >= 1");
  HostCtx* c;
  TRY(host_lease(&c));
  /* chunks of at most 64 MiB of fp32 input, whole 16-row groups when packing */
  const size_t ch = ((size_t)64 << 20) / ((size_t)cols * 4);   /* <= 16 Mi: fits an int */
  int chunk = ch < 1 ? 1 : (int)ch;
  if (pack) {
    chunk &= ~15;
    if (chunk < 16) chunk = 16;
  }
  if (chunk > rows) chunk = rows;
  tl_weights* W = NULL;
  int rc = 0;
  if (pack) TRY_GO(tlh_weights_alloc(rows, cols, &W), out);
  rc = host_quantize_body(c, src, dst, scales, rows, cols, clamp127, W, chunk);
  if (rc != 0 && W) {
    (void)hipStreamSynchronize(c->st);
    tlh_weights_free(W);
    W = NULL;
  }
out:
  host_release(c);
  if (rc == 0 && W) rc = registry_put(dst, scales, W);
  return rc;
}

/* ==========================================================================
 * packed-weight cache file
 * ========================================================================== */
/* A file is a sequence of self-describing records, one per matrix:
 *   RecHeader (64 bytes, little-endian)
 *   name      (name_len bytes, zero padded to a multiple of 64)
 *   tiles     (NG * KB * 1024 bytes: the HBM tile array as resident)
 *   scales    (NG * 16 * 4 bytes: fp32, zero padded)
 * The payload is copied between the file and HBM as it is, with no kernel.
 * `checksum` covers tiles then scales (CacheHash below); readers check the
 * magic, the version, that the sizes follow from rows and cols, and the sum. */
static const char kRecMagic[8] = {'T', 'L', 'W', 'C', 'R', 'E', 'C', '1'};
enum { kRecVersion = 1 };
typedef struct RecHeader {
  char magic[8];
  uint32_t version;
  uint32_t name_len;
  int32_t rows, cols, NG, KB;
  uint64_t tile_bytes, scale_bytes, checksum;
  uint64_t reserved;
} RecHeader;
_Static_assert(sizeof(RecHeader) == 64, "record header is 64 bytes");

static size_t pad64(size_t n) { return (n + 63) & ~(size_t)63; }

/* 64-bit streaming hash over 32-byte blocks (four independent multiply-xor
 * lanes, so it runs at memory speed); every chunk but the last is a multiple
 * of 32 bytes */
typedef struct CacheHash {
  uint64_t h[4];
  uint64_t n;
} CacheHash;

static void hash_init(CacheHash* c) {
  c->h[0] = 0x243f6a8885a308d3ull;
  c->h[1] = 0x13198a2e03707344ull;
  c->h[2] = 0xa4093822299f31d0ull;
  c->h[3] = 0x082efa98ec4e6c89ull;
  c->n = 0;
}
static uint64_t hash_step(uint64_t h, uint64_t v) {
  h ^= v;
  h *= 0x9e3779b97f4a7c15ull;
  return h ^ (h >> 32);
}
static void hash_add(CacheHash* c, const void* p, size_t bytes) {
  const uint8_t* b = (const uint8_t*)p;
  size_t i = 0;
  for (; i + 32 <= bytes; i += 32) {
    uint64_t v[4];
    memcpy(v, b + i, 32);
    c->h[0] = hash_step(c->h[0], v[0]);
    c->h[1] = hash_step(c->h[1], v[1]);
    c->h[2] = hash_step(c->h[2], v[2]);
    c->h[3] = hash_step(c->h[3], v[3]);
  }
  for (; i < bytes; i++) c->h[i & 3] = hash_step(c->h[i & 3], (uint64_t)b[i] | 0x100);
  c->n += bytes;
}
static uint64_t hash_value(const CacheHash* c) {
  return mix64(mix64(mix64(mix64(c->n, c->h[0]), c->h[1]), c->h[2]), c->h[3]);
}

#define CACHE_CHUNK ((size_t)64 << 20)

/* reads the next record header and name (name_out: at least 4096 bytes) at
 * the current position; *got = false at a clean end of file */
static int read_rec_header(FILE* f, RecHeader* h, char* name_out, bool* got) {
  const size_t n = fread(h, 1, sizeof *h, f);
  *got = false;
  if (n == 0 && feof(f)) return 0;
  REQ(n == sizeof *h, "truncated record header");
  REQ(memcmp(h->magic, kRecMagic, 8) == 0, "not a weight cache record (bad magic)");
  REQ(h->version == kRecVersion, "unsupported weight cache version");
  REQ(h->rows > 0 && h->cols > 0 && h->NG == tlk_cdiv(h->rows, 16) && h->KB == tlk_cdiv(h->cols, 64),
      "inconsistent record shape");
  REQ(h->tile_bytes == (uint64_t)h->NG * h->KB * 1024 && h->scale_bytes == (uint64_t)h->NG * 16 * 4,
      "inconsistent record sizes");
  REQ(h->name_len < 4096, "record name too long");
  char nb[4096 + 64];
  const size_t nl = pad64(h->name_len);
  REQ(fread(nb, 1, nl, f) == nl, "truncated record name");
  memcpy(name_out, nb, h->name_len);
  name_out[h->name_len] = 0;
  *got = true;
  return 0;
}

/* streams `bytes` from the file into device memory through pinned staging */
static int file_to_device(FILE* f, void* dst, size_t bytes, PinnedBuf* stage, CacheHash* hash, hipStream_t st) {
  TRY(tlh_pinned_ensure(stage, min_sz(bytes, CACHE_CHUNK)));
  for (size_t off = 0; off < bytes; off += CACHE_CHUNK) {
    const size_t n = min_sz(CACHE_CHUNK, bytes - off);
    HIP_TRY(hipStreamSynchronize(st));   /* staging idle */
    REQ(fread(stage->p, 1, n, f) == n, "truncated record payload");
    hash_add(hash, stage->p, n);
    HIP_TRY(hipMemcpyAsync((char*)dst + off, stage->p, n, hipMemcpyHostToDevice, st));
  }
  HIP_TRY(hipStreamSynchronize(st));
  return 0;
}

static int device_to_file(FILE* f, const void* src, size_t bytes, PinnedBuf* stage, CacheHash* hash,
                          hipStream_t st) {
  TRY(tlh_pinned_ensure(stage, min_sz(bytes, CACHE_CHUNK)));
  for (size_t off = 0; off < bytes; off += CACHE_CHUNK) {
    const size_t n = min_sz(CACHE_CHUNK, bytes - off);
    HIP_TRY(hipMemcpyAsync(stage->p, (const char*)src + off, n, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    if (hash) hash_add(hash, stage->p, n);
    if (f) REQ(fwrite(stage->p, 1, n, f) == n, "write failed");
  }
  return 0;
}

/* ==========================================================================
 * Part 1 -- reference entry points
 * ========================================================================== */
void w8a32_quantize(const float* w_fp32, int8_t* w_int8, float* scales, int rows, int cols) {
  tlh_begin();
  tlh_finish("w8a32_quantize", host_quantize(w_fp32, w_int8, scales, rows, cols, true, true));
}

void w8a8_quantize_weights(const float* w_fp32, int8_t* w_int8, float* w_scales, int rows, int cols) {
  tlh_begin();
  tlh_finish("w8a8_quantize_weights", host_quantize(w_fp32, w_int8, w_scales, rows, cols, true, true));
}

void w8a8_quantize_activations(const float* x_fp32, int8_t* x_int8, float* x_scales, int batch, int K) {
  tlh_begin();
  tlh_finish("w8a8_quantize_activations", host_quantize(x_fp32, x_int8, x_scales, batch, K, true, false));
}

void w8a16_quantize_weights(const float* w_fp32, int8_t* w_int8, float* scales, int rows, int cols) {
  tlh_begin();
  tlh_finish("w8a16_quantize_weights", host_quantize(w_fp32, w_int8, scales, rows, cols, true, true));
}

/* the bias of a host call on the device, or NULL */
static int stage_bias(HostCtx* c, const float* bias, int M, const float** out) {
  *out = NULL;
  if (!bias) return 0;
  TRY(tlh_devbuf_ensure(&c->bias, (size_t)M * sizeof(float), c->st));
  HIP_TRY(hipMemcpyAsync(c->bias.p, bias, (size_t)M * sizeof(float), hipMemcpyHostToDevice, c->st));
  *out = (const float*)c->bias.p;
  return 0;
}

static int w8a32_linear_body(HostCtx* c, const float* X, const int8_t* w_int8, const float* scales,
                             const float* bias, float* Y, int batch, int M, int K) {
  WRef* ref = NULL;
  TRY(registry_get(w_int8, scales, M, K, c->st, &ref));
  const tl_weights* W = ref->W;
  int rc = 0;
  const float* b;
  TRY_GO(stage_bias(c, bias, M, &b), out);
  if (batch == 1) {
    /* decode: x comes in through mapped pinned memory by a copy kernel and
     * the GEMV writes y straight into mapped pinned memory, so the call is
     * two kernels and one synchronisation (no DMA transfers) */
    const size_t xb = (size_t)K * sizeof(float), yb = (size_t)M * sizeof(float);
    TRY_GO(tlh_pinned_ensure(&c->hin, xb), out);
    TRY_GO(tlh_pinned_ensure(&c->hout, yb), out);
    TRY_GO(tlh_devbuf_ensure(&c->x, xb, c->st), out);
    HIP_GO(hipStreamSynchronize(c->st), out);   /* staging buffers idle */
    memcpy(c->hin.p, X, xb);
    HIP_GO(tlk_launch_copy_words(c->hin.dp, c->x.p, xb, c->st), out);
    TRY_GO(op_w8a32((const float*)c->x.p, W, b, (float*)c->hout.dp, 1, c->st), out);
    HIP_GO(hipStreamSynchronize(c->st), out);
    memcpy(Y, c->hout.p, yb);
    goto out;
  }
  TRY_GO(h2d(c, &c->x, X, (size_t)batch * K * sizeof(float)), out);
  TRY_GO(tlh_devbuf_ensure(&c->y, (size_t)batch * M * sizeof(float), c->st), out);
  TRY_GO(op_w8a32((const float*)c->x.p, W, b, (float*)c->y.p, batch, c->st), out);
  TRY_GO(d2h(c, Y, c->y.p, (size_t)batch * M * sizeof(float)), out);
out:
  wref_drop(ref);
  return rc;
}

void w8a32_linear(const float* X, const int8_t* w_int8, const float* scales, const float* bias, float* Y,
                  float* scratch, int batch, int M, int K) {
  (void)scratch;   /* unused, as in the reference (kernel/w8a32_kernel.c:364) */
  tlh_begin();
  int rc = check_shape(batch, M, K);
  if (rc == 0 && !(X && Y)) rc = tlh_fail("X and Y must be non-NULL");
  if (rc == 0) {
    HostCtx* c;
    rc = host_lease(&c);
    if (rc == 0) {
      rc = w8a32_linear_body(c, X, w_int8, scales, bias, Y, batch, M, K);
      host_release(c);
    }
  }
  tlh_finish("w8a32_linear", rc);
}

static int w8a8_linear_body(HostCtx* c, const int8_t* x_int8, const float* x_scales, const int8_t* w_int8,
                            const float* w_scales, const float* bias, float* Y, int batch, int M, int K) {
  WRef* ref = NULL;
  TRY(registry_get(w_int8, w_scales, M, K, c->st, &ref));
  const tl_weights* W = ref->W;
  int rc = 0;
  TRY_GO(h2d(c, &c->x, x_int8, (size_t)batch * K), out);
  TRY_GO(tlh_devbuf_ensure(&c->xs, (size_t)batch * sizeof(float), c->st), out);
  HIP_GO(hipMemcpyAsync(c->xs.p, x_scales, (size_t)batch * sizeof(float), hipMemcpyHostToDevice, c->st), out);
  const float* b;
  TRY_GO(stage_bias(c, bias, M, &b), out);
  TRY_GO(tlh_devbuf_ensure(&c->y, (size_t)batch * M * sizeof(float), c->st), out);
  TRY_GO(op_w8a8_codes((const int8_t*)c->x.p, (const float*)c->xs.p, W, b, c->y.p, OUT_F32, batch, c->st), out);
  TRY_GO(d2h(c, Y, c->y.p, (size_t)batch * M * sizeof(float)), out);
out:
  wref_drop(ref);
  return rc;
}

void w8a8_linear(const int8_t* x_int8, const float* x_scales, const int8_t* w_int8, const float* w_scales,
                 const float* bias, float* Y, int batch, int M, int K) {
  tlh_begin();
  int rc = check_shape(batch, M, K);
  if (rc == 0 && !(x_int8 && x_scales && Y)) rc = tlh_fail("x_int8, x_scales and Y must be non-NULL");
  if (rc == 0) {
    HostCtx* c;
    rc = host_lease(&c);
    if (rc == 0) {
      rc = w8a8_linear_body(c, x_int8, x_scales, w_int8, w_scales, bias, Y, batch, M, K);
      host_release(c);
    }
  }
  tlh_finish("w8a8_linear", rc);
}

static int w8a16_linear_body(HostCtx* c, const uint16_t* x_bf16_raw, const int8_t* w_int8, const float* w_scales,
                             const float* bias, float* Y, int batch, int M, int K) {
  WRef* ref = NULL;
  TRY(registry_get(w_int8, w_scales, M, K, c->st, &ref));
  const tl_weights* W = ref->W;
  int rc = 0;
  TRY_GO(h2d(c, &c->x, x_bf16_raw, (size_t)batch * K * sizeof(uint16_t)), out);
  const float* b;
  TRY_GO(stage_bias(c, bias, M, &b), out);
  TRY_GO(tlh_devbuf_ensure(&c->y, (size_t)batch * M * sizeof(float), c->st), out);
  TRY_GO(op_w8a16(c->x.p, TL_BF16, W, b, c->y.p, TL_F32, batch, c->st), out);
  TRY_GO(d2h(c, Y, c->y.p, (size_t)batch * M * sizeof(float)), out);
out:
  wref_drop(ref);
  return rc;
}

void w8a16_linear(const uint16_t* x_bf16_raw, const int8_t* w_int8, const float* w_scales, const float* bias,
                  float* Y, int batch, int M, int K) {
  tlh_begin();
  int rc = check_shape(batch, M, K);
  if (rc == 0 && !(x_bf16_raw && Y)) rc = tlh_fail("x and Y must be non-NULL");
  if (rc == 0) {
    HostCtx* c;
    rc = host_lease(&c);
    if (rc == 0) {
      rc = w8a16_linear_body(c, x_bf16_raw, w_int8, w_scales, bias, Y, batch, M, K);
      host_release(c);
    }
  }
  tlh_finish("w8a16_linear", rc);
}

/* ==========================================================================
 * Part 2 -- extensions
 * ========================================================================== */
const char* tl_last_error(void) { return t_has_err ? t_err : NULL; }
void tl_clear_error(void) { t_has_err = false; }
const char* tl_version(void) { return "typhoon_linear 0.1 gfx950"; }

int tl_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

static int gemv_set_plan_impl(int rows, int u) {
  REQ(rows == 0 || rows == 8 || rows == 16, "rows must be 0, 8 or 16");
  REQ(u == 0 || u == 2 || u == 4 || u == 6 || u == 8 || u == 12, "u must be 0, 2, 4, 6, 8 or 12");
  REQ(u == 0 || rows == 0 || (rows == 16 ? u != 6 : u != 12), "u = 6 needs rows 8, u = 12 rows 16");
  tlk_gemv_set_plan(rows, u);
  return 0;
}
int tl_gemv_set_plan(int rows, int u) {
  tlh_begin();
  return tlh_finish("tl_gemv_set_plan", gemv_set_plan_impl(rows, u));
}

static int rows_set_split_impl(int split) {
  REQ(split >= -1 && split <= 64, "split must be -1 (path off), 0 (planner) or 1..64");
  atomic_store_explicit(&g_rows_off, split < 0, memory_order_relaxed);
  tlk_rows_set_split(split > 0 ? split : 0);
  return 0;
}
int tl_rows_set_split(int split) {
  tlh_begin();
  return tlh_finish("tl_rows_set_split", rows_set_split_impl(split));
}

static int rows_set_groups_impl(int groups) {
  REQ(groups >= 0 && groups <= 3, "groups must be 0 (planner) or 1..3");
  tlk_rows_set_groups(groups);
  return 0;
}
int tl_rows_set_groups(int groups) {
  tlh_begin();
  return tlh_finish("tl_rows_set_groups", rows_set_groups_impl(groups));
}

static int w8a16_set_gemv_impl(int on) {
  REQ(on == 0 || on == 1, "on must be 0 or 1");
  atomic_store_explicit(&g_gemv_w8a16_off, on == 0, memory_order_relaxed);
  return 0;
}
int tl_w8a16_set_gemv(int on) {
  tlh_begin();
  return tlh_finish("tl_w8a16_set_gemv", w8a16_set_gemv_impl(on));
}

static int w8a32_set_gemv2_impl(int on) {
  REQ(on >= 0 && on <= 2, "on must be 0, 1 or 2");
  atomic_store_explicit(&g_gemv_rows2, on, memory_order_relaxed);
  return 0;
}
int tl_w8a32_set_gemv2(int on) {
  tlh_begin();
  return tlh_finish("tl_w8a32_set_gemv2", w8a32_set_gemv2_impl(on));
}

static int gemm_i8_set_cfg_impl(int cfg) {
  REQ(cfg >= -1 && cfg <= 7, "cfg must be -1 (planner) or 0..7");
  tlk_gemm_i8_set_cfg(cfg);
  return 0;
}
int tl_gemm_i8_set_cfg(int cfg) {
  tlh_begin();
  return tlh_finish("tl_gemm_i8_set_cfg", gemm_i8_set_cfg_impl(cfg));
}

static int gemm_i8_set_split_impl(int split) {
  REQ(split >= 0 && split <= 64, "split must be 0 (planner) or 1..64");
  tlk_gemm_i8_set_split(split);
  return 0;
}
int tl_gemm_i8_set_split(int split) {
  tlh_begin();
  return tlh_finish("tl_gemm_i8_set_split", gemm_i8_set_split_impl(split));
}

static int gemm_b16_set_plan_impl(int cfg, int split) {
  REQ(cfg >= -1 && cfg <= 8, "cfg must be -1 (planner), 0..2 or 4..8 (tiles) or 3 (small-M kernel)");
  REQ((split >= 0 && split <= 64) || (cfg == 3 && split >= 112 && split <= 444),
      "split must be 0 (planner) or 1..64 (with cfg 3: 0, or the shape code 100 R + 10 TG + U)");
  tlk_gemm_b16_set_plan(cfg, split);
  return 0;
}
int tl_gemm_b16_set_plan(int cfg, int split) {
  tlh_begin();
  return tlh_finish("tl_gemm_b16_set_plan", gemm_b16_set_plan_impl(cfg, split));
}

static int stream_read_impl(const void* p, size_t bytes, int grid, int u, uint32_t* sink, void* stream) {
  REQ(p && sink, "NULL pointer");
  REQ(bytes > 0 && bytes % 16 == 0 && (((uintptr_t)p) & 15) == 0,
      "bytes must be a positive multiple of 16 and p 16-byte aligned");
  REQ(grid >= 1 && grid <= 65536, "grid must be 1..65536");
  REQ(u == 4 || u == 8, "u must be 4 or 8");
  HIP_TRY(tlk_launch_stream_read(p, bytes, grid, u, sink, (hipStream_t)stream));
  return 0;
}
int tl_stream_read_dev(const void* p, size_t bytes, int grid, int u, uint32_t* sink, void* stream) {
  tlh_begin();
  return tlh_finish("tl_stream_read_dev", stream_read_impl(p, bytes, grid, u, sink, stream));
}

static int attn_set_chunk_impl(int positions) {
  REQ(positions == 0 || positions == 32 || positions == 64 || positions == 128, "positions must be 0, 32, 64 or 128");
  tlk_attn_set_chunk(positions);
  return 0;
}
int tl_attn_set_chunk(int positions) {
  tlh_begin();
  return tlh_finish("tl_attn_set_chunk", attn_set_chunk_impl(positions));
}

static int register_weights_impl(const int8_t* w_int8, const float* scales, int rows, int cols) {
  HostCtx* c;
  TRY(host_lease(&c));
  WRef* ref = NULL;
  const int rc = registry_get(w_int8, scales, rows, cols, c->st, &ref);
  host_release(c);
  if (ref) wref_drop(ref);
  return rc;
}
int tl_register_weights(const int8_t* w_int8, const float* scales, int rows, int cols) {
  tlh_begin();
  return tlh_finish("tl_register_weights", register_weights_impl(w_int8, scales, rows, cols));
}

int tl_evict_weights(const int8_t* w_int8) {
  tlh_begin();
  pthread_mutex_lock(&g_reg_mu);
  for (int b = 0; b < REG_BUCKETS; b++) {
    RegNode** pp = &g_reg[b];
    while (*pp) {
      if ((*pp)->w == (const void*)w_int8) reg_erase_locked(pp);
      else pp = &(*pp)->next;
    }
  }
  pthread_mutex_unlock(&g_reg_mu);
  return 0;
}

void tl_registry_clear(void) {
  pthread_mutex_lock(&g_reg_mu);
  for (int b = 0; b < REG_BUCKETS; b++)
    while (g_reg[b]) reg_erase_locked(&g_reg[b]);
  g_reg_bytes = 0;
  pthread_mutex_unlock(&g_reg_mu);
}

size_t tl_registry_bytes(void) {
  pthread_mutex_lock(&g_reg_mu);
  const size_t b = g_reg_bytes;
  pthread_mutex_unlock(&g_reg_mu);
  return b;
}

int tl_registry_entries(void) {
  pthread_mutex_lock(&g_reg_mu);
  const int n = (int)g_reg_count;
  pthread_mutex_unlock(&g_reg_mu);
  return n;
}

tl_weights* tl_weights_create(const int8_t* w_int8, const float* scales, int rows, int cols, int src_on_device) {
  tlh_begin();
  tl_weights* out = NULL;
  int rc = (w_int8 && scales) ? 0 : tlh_fail("NULL pointer");
  if (rc == 0) rc = tlh_weights_from_codes(w_int8, scales, rows, cols, src_on_device != 0, NULL, &out);
  tlh_finish("tl_weights_create", rc);
  return rc == 0 ? out : NULL;
}

static int weights_quantize_dev_impl(const float* w_fp32, int rows, int cols, int8_t* codes_out, float* scales_out,
                                     void* stream, tl_weights** out) {
  REQ(w_fp32, "NULL pointer");
  hipStream_t st = (hipStream_t)stream;
  tl_weights* W = NULL;
  TRY(tlh_weights_alloc(rows, cols, &W));
  hipError_t e = hipMemsetAsync(W->scales, 0, (size_t)W->NG * 16 * sizeof(float), st);
  if (e == hipSuccess) e = hipMemsetAsync(W->tiles, 0, (size_t)W->NG * W->KB * 1024, st);
  if (e == hipSuccess) e = tlk_launch_quantize_rows_tiled(w_fp32, rows, cols, W->tiles, W->scales, true, st);
  if (e == hipSuccess && codes_out) {
    float* s2 = scales_out;
    void* tmp = NULL;
    if (!s2) {
      e = hipMalloc(&tmp, (size_t)rows * sizeof(float));
      s2 = (float*)tmp;
    }
    if (e == hipSuccess) e = tlk_launch_quantize_rows(w_fp32, codes_out, s2, rows, cols, true, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (tmp) (void)hipFree(tmp);
  } else if (e == hipSuccess && scales_out) {
    e = hipMemcpyAsync(scales_out, W->scales, (size_t)rows * sizeof(float), hipMemcpyDeviceToDevice, st);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) {
    (void)hipStreamSynchronize(st);
    tlh_weights_free(W);
    return tlh_fail("quantize: %s", hipGetErrorString(e));
  }
  *out = W;
  return 0;
}
tl_weights* tl_weights_quantize_dev(const float* w_fp32, int rows, int cols, int8_t* codes_out, float* scales_out,
                                    void* stream) {
  tlh_begin();
  tl_weights* out = NULL;
  const int rc = weights_quantize_dev_impl(w_fp32, rows, cols, codes_out, scales_out, stream, &out);
  tlh_finish("tl_weights_quantize_dev", rc);
  return rc == 0 ? out : NULL;
}

void tl_weights_destroy(tl_weights* w) { tlh_weights_free(w); }
int tl_weights_rows(const tl_weights* w) { return w ? w->rows : -1; }
int tl_weights_cols(const tl_weights* w) { return w ? w->cols : -1; }
size_t tl_weights_bytes(const tl_weights* w) { return w ? w->bytes : 0; }

static int w8a32_linear_dev_impl(const float* X, const tl_weights* W, const float* bias, float* Y, int batch,
                                 void* stream) {
  TRY(tlh_check_weights(W));
  REQ(batch >= 1 && X && Y, "bad arguments");
  return op_w8a32(X, W, bias, Y, batch, (hipStream_t)stream);
}
int tl_w8a32_linear_dev(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, void* stream) {
  tlh_begin();
  return tlh_finish("tl_w8a32_linear_dev", w8a32_linear_dev_impl(X, W, bias, Y, batch, stream));
}

static int quantize_rows_dev_impl(const float* src, int8_t* codes, float* scales, int rows, int cols, int clamp127,
                                  void* stream) {
  REQ(src && codes && scales && rows >= 1 && cols >= 1, "bad arguments");
  HIP_TRY(tlk_launch_quantize_rows(src, codes, scales, rows, cols, clamp127 != 0, (hipStream_t)stream));
  return 0;
}
int tl_quantize_rows_dev(const float* src, int8_t* codes, float* scales, int rows, int cols, int clamp127,
                         void* stream) {
  tlh_begin();
  return tlh_finish("tl_quantize_rows_dev", quantize_rows_dev_impl(src, codes, scales, rows, cols, clamp127, stream));
}

static int w8a8_linear_dev_impl(const int8_t* x_int8, const float* x_scales, const tl_weights* W, const float* bias,
                                float* Y, int batch, void* stream) {
  TRY(tlh_check_weights(W));
  REQ(batch >= 1 && x_int8 && x_scales && Y, "bad arguments");
  return op_w8a8_codes(x_int8, x_scales, W, bias, Y, OUT_F32, batch, (hipStream_t)stream);
}
int tl_w8a8_linear_dev(const int8_t* x_int8, const float* x_scales, const tl_weights* W, const float* bias, float* Y,
                       int batch, void* stream) {
  tlh_begin();
  return tlh_finish("tl_w8a8_linear_dev", w8a8_linear_dev_impl(x_int8, x_scales, W, bias, Y, batch, stream));
}

static int w8a8_linear_f32_dev_impl(const float* X, const tl_weights* W, const float* bias, float* Y, int batch,
                                    void* stream) {
  TRY(tlh_check_weights(W));
  REQ(batch >= 1 && X && Y, "bad arguments");
  return op_w8a8_f32(X, W, bias, Y, batch, (hipStream_t)stream);
}
int tl_w8a8_linear_f32_dev(const float* X, const tl_weights* W, const float* bias, float* Y, int batch,
                           void* stream) {
  tlh_begin();
  return tlh_finish("tl_w8a8_linear_f32_dev", w8a8_linear_f32_dev_impl(X, W, bias, Y, batch, stream));
}

/* the two halves of tl_w8a8_linear_f32_dev at batch > 1 */
size_t tl_w8a8_tiles_bytes(int batch, int K) {
  if (batch < 1 || K < 1) return 0;
  return (size_t)tlk_cdiv(batch, 16) * 16 * (size_t)tlk_cdiv(K, 64) * 64;
}

static int w8a8_quantize_tiles_impl(const float* X, int batch, int K, uint8_t* x_tiles, float* x_scales,
                                    void* stream) {
  REQ(X && x_tiles && x_scales && batch >= 1 && K >= 1, "bad arguments");
  hipStream_t st = (hipStream_t)stream;
  const bool by_rows = (K == 1024 || K == 2048 || K == 4096 || K == 6144) && (((uintptr_t)X) & 15) == 0;
  if (by_rows) HIP_TRY(tlk_launch_quantize_rows_by_row(X, batch, K, x_tiles, x_scales, st));
  else HIP_TRY(tlk_launch_quantize_rows_tiled(X, batch, K, x_tiles, x_scales, true, st));
  return 0;
}
int tl_w8a8_quantize_tiles_dev(const float* X, int batch, int K, uint8_t* x_tiles, float* x_scales, void* stream) {
  tlh_begin();
  return tlh_finish("tl_w8a8_quantize_tiles_dev", w8a8_quantize_tiles_impl(X, batch, K, x_tiles, x_scales, stream));
}

static int w8a8_linear_tiles_impl(const uint8_t* x_tiles, const float* x_scales, const tl_weights* W,
                                  const float* bias, float* Y, int batch, void* stream) {
  TRY(tlh_check_weights(W));
  REQ(x_tiles && x_scales && Y && batch >= 1, "bad arguments");
  hipStream_t st = (hipStream_t)stream;
  WS_CALL(W->dev, st, linear_w8a8_tiles_ws(ws_, x_tiles, x_scales, W, bias, Y, batch, st));
}
int tl_w8a8_linear_tiles_dev(const uint8_t* x_tiles, const float* x_scales, const tl_weights* W, const float* bias,
                             float* Y, int batch, void* stream) {
  tlh_begin();
  return tlh_finish("tl_w8a8_linear_tiles_dev",
                    w8a8_linear_tiles_impl(x_tiles, x_scales, W, bias, Y, batch, stream));
}

static int w8a16_linear_dev_impl(const void* X, int x_type, const tl_weights* W, const float* bias, void* Y,
                                 int y_type, int batch, void* stream) {
  TRY(tlh_check_weights(W));
  REQ(batch >= 1 && X && Y, "bad arguments");
  return op_w8a16(X, x_type, W, bias, Y, y_type, batch, (hipStream_t)stream);
}
int tl_w8a16_linear_dev(const void* X, int x_type, const tl_weights* W, const float* bias, void* Y, int y_type,
                        int batch, void* stream) {
  tlh_begin();
  return tlh_finish("tl_w8a16_linear_dev", w8a16_linear_dev_impl(X, x_type, W, bias, Y, y_type, batch, stream));
}

static int w8a32_gemv_acc_dev_impl(const float* x, const tl_weights* W, int32_t* acc, float* x_scale, void* stream) {
  TRY(tlh_check_weights(W));
  REQ(x && acc, "bad arguments");
  REQ(tlk_gemv_fused_xv(W->cols) > 0, "K too large for the fused GEMV");
  GemvLaunch L = tlk_gemv_launch_init();
  L.x = x;
  L.wt = W->tiles;
  L.ws = W->scales;
  L.acc_out = acc;
  L.xs_out = x_scale;
  L.N = W->rows;
  L.K = W->cols;
  L.epi = EPI_ACC;
  HIP_TRY(tlk_launch_gemv_i8(&L, (hipStream_t)stream));
  return 0;
}
int tl_w8a32_gemv_acc_dev(const float* x, const tl_weights* W, int32_t* acc, float* x_scale, void* stream) {
  tlh_begin();
  return tlh_finish("tl_w8a32_gemv_acc_dev", w8a32_gemv_acc_dev_impl(x, W, acc, x_scale, stream));
}

static int rmsnorm_np_dev_impl(const float* h, const float* norm_w, float* out, int K, void* stream) {
  REQ(h && out, "h and out must be non-NULL");
  REQ(K >= 128 && K <= 16384 && (K & (K - 1)) == 0, "K must be a power of two in [128, 16384]");
  HIP_TRY(tlk_launch_rmsnorm_np(h, norm_w, out, K, 1e-6f, (hipStream_t)stream));
  return 0;
}
int tl_rmsnorm_np_dev(const float* h, const float* norm_w, float* out, int K, void* stream) {
  tlh_begin();
  return tlh_finish("tl_rmsnorm_np_dev", rmsnorm_np_dev_impl(h, norm_w, out, K, stream));
}

/* ---- greedy lm_head step: final RMSNorm, GEMV with argmax keys, key
 *      reduction (lmhead.hip) ------------------------------------------------ */
static size_t lm_head_argmax_keys(int N, int K) {
  GemvPlan p;
  tlk_gemv_plan(N, K, &p);
  return (size_t)p.blocks;
}

/* The greedy step's launches on caller-provided work-space: keys (one 8-byte
 * key per GEMV work-group, 16-byte aligned) and xn (K floats, used only when
 * the final RMSNorm cannot run inside the GEMV's prologue). */
static int lm_head_argmax_enqueue(const float* h, const float* norm_w, const tl_weights* W, float* logits,
                                  int32_t* token, float* max_logit, uint64_t* keys, float* xn, hipStream_t st) {
  const int K = W->cols;
  REQ(K >= 128 && K <= TLK_RMS_MAX_K && (K & (K - 1)) == 0, "K must be a power of two in [128, 16384]");
  GemvLaunch L = tlk_gemv_launch_init();
  if (tlk_gemv_fused_norm_ok(K, h, norm_w)) {
    /* every GEMV work-group normalises the row itself: one launch fewer */
    L.x = h;
    L.norm = NORM_NUMPY;
    L.norm_w = norm_w;
  } else {
    HIP_TRY(tlk_launch_rmsnorm_np(h, norm_w, xn, K, 1e-6f, st));
    L.x = xn;
  }
  L.wt = W->tiles;
  L.ws = W->scales;
  L.y = logits;
  L.keys = keys;
  L.N = W->rows;
  L.K = K;
  L.epi = EPI_ARGMAX;
  HIP_TRY(tlk_launch_gemv_i8(&L, st));
  HIP_TRY(tlk_launch_argmax_keys(keys, (int)lm_head_argmax_keys(W->rows, K), token, max_logit, st));
  return 0;
}

static int op_lm_head_argmax_ws(Workspace* ws, const float* h, const float* norm_w, const tl_weights* W, float* logits, int32_t* token,
                             float* max_logit, hipStream_t st) {
  TRY(tlh_devbuf_ensure(&ws->keys, lm_head_argmax_keys(W->rows, W->cols) * sizeof(uint64_t), st));
  TRY(tlh_devbuf_ensure(&ws->xn, (size_t)W->cols * sizeof(float), st));
  return lm_head_argmax_enqueue(h, norm_w, W, logits, token, max_logit, (uint64_t*)ws->keys.p, (float*)ws->xn.p, st);
}

static int op_lm_head_argmax(const float* h, const float* norm_w, const tl_weights* W, float* logits, int32_t* token,
                             float* max_logit, hipStream_t st) {
  WS_CALL(W->dev, st, op_lm_head_argmax_ws(ws_, h, norm_w, W, logits, token, max_logit, st));
}

static int lm_head_argmax_dev_impl(const float* h, const float* norm_w, const tl_weights* W, float* logits,
                                   int32_t* token, float* max_logit, void* stream) {
  TRY(tlh_check_weights(W));
  REQ(h && token, "h and token must be non-NULL");
  return op_lm_head_argmax(h, norm_w, W, logits, token, max_logit, (hipStream_t)stream);
}
int tl_lm_head_argmax_dev(const float* h, const float* norm_w, const tl_weights* W, float* logits, int32_t* token,
                          float* max_logit, void* stream) {
  tlh_begin();
  return tlh_finish("tl_lm_head_argmax_dev", lm_head_argmax_dev_impl(h, norm_w, W, logits, token, max_logit, stream));
}

/* tl_lm_head_argmax_noalloc_dev: the greedy step with its work-space in the
 * file-scope device array of lmhead.hip (tlk_noalloc_workspace), for callers
 * that cannot allocate; calls that overlap on one device share it and race */
static int lm_head_argmax_noalloc_impl(const float* h, const float* norm_w, const tl_weights* W, float* logits,
                                       int32_t* token, float* max_logit, void* stream) {
  TRY(tlh_check_weights(W));
  REQ(h && token, "h and token must be non-NULL");
  REQ(W->rows <= TLK_NA_MAX_ROWS, "lm_head has more rows than the no-allocation work-space holds (262144)");
  REQ(lm_head_argmax_keys(W->rows, W->cols) * sizeof(uint64_t) <= (size_t)TLK_NA_KEY_BYTES,
      "the GEMV plan needs more argmax keys than the no-allocation work-space holds");
  uint8_t* base = NULL;
  HIP_TRY(tlk_noalloc_workspace(W->dev, &base));
  return lm_head_argmax_enqueue(h, norm_w, W, logits, token, max_logit, (uint64_t*)base,
                                (float*)(base + TLK_NA_KEY_BYTES), (hipStream_t)stream);
}
int tl_lm_head_argmax_noalloc_dev(const float* h, const float* norm_w, const tl_weights* W, float* logits,
                                  int32_t* token, float* max_logit, void* stream) {
  tlh_begin();
  return tlh_finish("tl_lm_head_argmax_noalloc_dev",
                    lm_head_argmax_noalloc_impl(h, norm_w, W, logits, token, max_logit, stream));
}

static int lm_head_argmax_body(HostCtx* c, const float* h, const float* norm_w, const int8_t* w_int8,
                               const float* scales, int N, int K, float* logits, int32_t* token) {
  WRef* ref = NULL;
  TRY(registry_get(w_int8, scales, N, K, c->st, &ref));
  const tl_weights* W = ref->W;
  int rc = 0;
  /* h and the norm weights in one staging copy: [h | norm_w] */
  const size_t kb = (size_t)K * sizeof(float);
  const size_t inb = norm_w ? 2 * kb : kb;
  TRY_GO(tlh_pinned_ensure(&c->hin, inb), out);
  TRY_GO(tlh_pinned_ensure(&c->htok, 16), out);
  TRY_GO(tlh_devbuf_ensure(&c->x, inb, c->st), out);
  HIP_GO(hipStreamSynchronize(c->st), out);
  memcpy(c->hin.p, h, kb);
  if (norm_w) memcpy((char*)c->hin.p + kb, norm_w, kb);
  HIP_GO(tlk_launch_copy_words(c->hin.dp, c->x.p, inb, c->st), out);
  const float* hd = (const float*)c->x.p;
  const float* wd = norm_w ? hd + K : NULL;
  float* ld = NULL;
  if (logits) {
    TRY_GO(tlh_devbuf_ensure(&c->y, kb > (size_t)N * 4 ? kb : (size_t)N * 4, c->st), out);
    ld = (float*)c->y.p;
  }
  int32_t* td = (int32_t*)c->htok.dp;
  TRY_GO(op_lm_head_argmax(hd, wd, W, ld, td, NULL, c->st), out);
  if (logits) {
    TRY_GO(d2h(c, logits, ld, (size_t)N * sizeof(float)), out);
  } else {
    HIP_GO(hipStreamSynchronize(c->st), out);
  }
  *token = *(const int32_t*)c->htok.p;
out:
  wref_drop(ref);
  return rc;
}
int tl_lm_head_argmax(const float* h, const float* norm_w, const int8_t* w_int8, const float* scales, int N, int K,
                      float* logits, int32_t* token) {
  tlh_begin();
  int rc = check_shape(1, N, K);
  if (rc == 0 && !(h && token)) rc = tlh_fail("h and token must be non-NULL");
  if (rc == 0) {
    HostCtx* c;
    rc = host_lease(&c);
    if (rc == 0) {
      rc = lm_head_argmax_body(c, h, norm_w, w_int8, scales, N, K, logits, token);
      host_release(c);
    }
  }
  return tlh_finish("tl_lm_head_argmax", rc);
}

static int gemv_fused_dev_impl(const float* x, const tl_weights* W, const float* bias, float* y, int epi, int norm,
                               const float* norm_w, void* stream) {
  TRY(tlh_check_weights(W));
  REQ(x && y, "bad arguments");
  REQ(epi == EPI_W8A32 || epi == EPI_SWIGLU, "epi must be 0 (W8A32) or 4 (SwiGLU)");
  REQ(norm >= NORM_NONE && norm <= NORM_DECODER, "norm must be 0, 1 or 2");
  REQ(norm == NORM_NONE || tlk_gemv_fused_norm_ok(W->cols, x, norm_w ? norm_w : x),
      "a fused RMSNorm needs K = 1024 * 2^j <= 16384 and 16-byte aligned vectors");
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
  HIP_TRY(tlk_launch_gemv_i8(&L, (hipStream_t)stream));
  return 0;
}
int tl_gemv_fused_dev(const float* x, const tl_weights* W, const float* bias, float* y, int epi, int norm,
                      const float* norm_w, void* stream) {
  tlh_begin();
  return tlh_finish("tl_gemv_fused_dev", gemv_fused_dev_impl(x, W, bias, y, epi, norm, norm_w, stream));
}

static int w8a8_gemm_acc_dev_impl(const int8_t* x_int8, const tl_weights* W, int32_t* acc, int batch, void* stream) {
  TRY(tlh_check_weights(W));
  REQ(batch >= 1 && x_int8 && acc, "bad arguments");
  return op_w8a8_codes(x_int8, NULL, W, NULL, acc, OUT_I32, batch, (hipStream_t)stream);
}
int tl_w8a8_gemm_acc_dev(const int8_t* x_int8, const tl_weights* W, int32_t* acc, int batch, void* stream) {
  tlh_begin();
  return tlh_finish("tl_w8a8_gemm_acc_dev", w8a8_gemm_acc_dev_impl(x_int8, W, acc, batch, stream));
}

/* ---- packed-weight cache file, registry adoption, code export ------------- */
static int weights_save_impl(const tl_weights* W, const char* path, const char* name, int append) {
  TRY(tlh_check_weights(W));
  REQ(path && name, "NULL path or name");
  const size_t nl = strlen(name);
  REQ(nl < 4096, "record name too long");
  hipStream_t st = NULL;
  PinnedBuf stage = {0};
  FILE* f = NULL;
  int rc = 0;
  if (append) f = fopen(path, "r+b");
  if (!f) f = fopen(path, "wb");
  REQ_GO(f, out, "cannot open %s for writing", path);
  REQ_GO(fseek(f, 0, SEEK_END) == 0, out, "seek failed");
  const long pos = ftell(f);
  REQ_GO(pos >= 0, out, "ftell failed");
  /* header with the checksum filled in after the payload went out */
  RecHeader h;
  memset(&h, 0, sizeof h);
  memcpy(h.magic, kRecMagic, 8);
  h.version = kRecVersion;
  h.name_len = (uint32_t)nl;
  h.rows = W->rows;
  h.cols = W->cols;
  h.NG = W->NG;
  h.KB = W->KB;
  h.tile_bytes = (uint64_t)W->NG * W->KB * 1024;
  h.scale_bytes = (uint64_t)W->NG * 16 * 4;
  REQ_GO(fwrite(&h, 1, sizeof h, f) == sizeof h, out, "write failed");
  char nb[4096 + 64];
  memset(nb, 0, sizeof nb);
  memcpy(nb, name, nl);
  REQ_GO(fwrite(nb, 1, pad64(nl), f) == pad64(nl), out, "write failed");
  CacheHash hash;
  hash_init(&hash);
  TRY_GO(device_to_file(f, W->tiles, h.tile_bytes, &stage, &hash, st), out);
  TRY_GO(device_to_file(f, W->scales, h.scale_bytes, &stage, &hash, st), out);
  h.checksum = hash_value(&hash);
  REQ_GO(fseek(f, pos, SEEK_SET) == 0, out, "seek failed");
  REQ_GO(fwrite(&h, 1, sizeof h, f) == sizeof h, out, "write failed");
  REQ_GO(fflush(f) == 0, out, "write failed");
out:
  if (f) fclose(f);
  tlh_pinned_free(&stage);
  return rc;
}
int tl_weights_save(const tl_weights* W, const char* path, const char* name, int append) {
  tlh_begin();
  return tlh_finish("tl_weights_save", weights_save_impl(W, path, name, append));
}

static int weights_load_impl(const char* path, const char* name, tl_weights** out) {
  REQ(path && name, "NULL path or name");
  FILE* f = fopen(path, "rb");
  REQ(f, "cannot open %s", path);
  RecHeader h;
  char rn[4096];
  int rc = 0;
  PinnedBuf stage = {0};
  tl_weights* W = NULL;
  for (;;) {
    bool got;
    TRY_GO(read_rec_header(f, &h, rn, &got), done);
    REQ_GO(got, done, "no record named %s in %s", name, path);
    if (strcmp(rn, name) == 0) break;
    REQ_GO(fseek(f, (long)(h.tile_bytes + h.scale_bytes), SEEK_CUR) == 0, done, "seek failed");
  }
  TRY_GO(tlh_weights_alloc(h.rows, h.cols, &W), done);
  CacheHash hash;
  hash_init(&hash);
  TRY_GO(file_to_device(f, W->tiles, h.tile_bytes, &stage, &hash, NULL), done);
  TRY_GO(file_to_device(f, W->scales, h.scale_bytes, &stage, &hash, NULL), done);
  REQ_GO(hash_value(&hash) == h.checksum, done, "checksum mismatch in record %s", name);
  *out = W;
  W = NULL;
done:
  if (W) tlh_weights_free(W);
  tlh_pinned_free(&stage);
  fclose(f);
  return rc;
}
tl_weights* tl_weights_load(const char* path, const char* name) {
  tlh_begin();
  tl_weights* out = NULL;
  const int rc = weights_load_impl(path, name, &out);
  tlh_finish("tl_weights_load", rc);
  return rc == 0 ? out : NULL;
}

static int weights_cache_list_impl(const char* path, char* names, size_t names_len, int* count) {
  REQ(path, "NULL path");
  FILE* f = fopen(path, "rb");
  REQ(f, "cannot open %s", path);
  RecHeader h;
  char rn[4096];
  int rc = 0, n = 0;
  size_t used = 0;
  for (;;) {
    bool got;
    TRY_GO(read_rec_header(f, &h, rn, &got), done);
    if (!got) break;
    const size_t l = strlen(rn);
    if (names && names_len) {
      REQ_GO(used + l + 1 < names_len, done, "names buffer too small");
      memcpy(names + used, rn, l);
      names[used + l] = '\n';
    }
    used += l + 1;
    n++;
    REQ_GO(fseek(f, (long)(h.tile_bytes + h.scale_bytes), SEEK_CUR) == 0, done, "seek failed");
  }
  if (names && names_len) names[used] = 0;
  *count = n;
done:
  fclose(f);
  return rc;
}
int tl_weights_cache_list(const char* path, char* names, size_t names_len) {
  tlh_begin();
  int count = -1;
  const int rc = weights_cache_list_impl(path, names, names_len, &count);
  tlh_finish("tl_weights_cache_list", rc);
  return rc == 0 ? count : -1;
}

static int weights_export_impl(const tl_weights* W, int8_t* codes, float* scales, int dst_on_device) {
  TRY(tlh_check_weights(W));
  REQ(codes || scales, "nothing to export");
  hipStream_t st = NULL;
  const size_t cb = (size_t)W->rows * W->cols, sb = (size_t)W->rows * sizeof(float);
  if (dst_on_device) {
    if (codes) HIP_TRY(tlk_launch_unpack_tiles(W->tiles, W->rows, W->cols, codes, st));
    if (scales) HIP_TRY(hipMemcpyAsync(scales, W->scales, sb, hipMemcpyDeviceToDevice, st));
    HIP_TRY(hipStreamSynchronize(st));
    return 0;
  }
  int rc = 0;
  DevBuf tmp = {0};
  if (codes) {
    TRY_GO(tlh_devbuf_ensure(&tmp, cb, st), out);
    HIP_GO(tlk_launch_unpack_tiles(W->tiles, W->rows, W->cols, (int8_t*)tmp.p, st), out);
    HIP_GO(hipMemcpyAsync(codes, tmp.p, cb, hipMemcpyDeviceToHost, st), out);
    HIP_GO(hipStreamSynchronize(st), out);
  }
  if (scales) {
    HIP_GO(hipMemcpyAsync(scales, W->scales, sb, hipMemcpyDeviceToHost, st), out);
    HIP_GO(hipStreamSynchronize(st), out);
  }
out:
  if (tmp.p) (void)hipStreamSynchronize(st);
  tlh_devbuf_free(&tmp);
  return rc;
}
int tl_weights_export(const tl_weights* W, int8_t* codes, float* scales, int dst_on_device) {
  tlh_begin();
  return tlh_finish("tl_weights_export", weights_export_impl(W, codes, scales, dst_on_device));
}

static int registry_adopt_impl(const int8_t* w_int8, const float* scales, tl_weights* W) {
  TRY(tlh_check_weights(W));
  REQ(w_int8 && scales, "NULL pointer");
  return registry_put(w_int8, scales, W);
}
int tl_registry_adopt(const int8_t* w_int8, const float* scales, tl_weights* W) {
  tlh_begin();
  return tlh_finish("tl_registry_adopt", registry_adopt_impl(w_int8, scales, W));
}
