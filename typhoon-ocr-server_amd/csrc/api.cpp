// api.cpp -- C ABI of libtyphoon_linear.so (declared in include/typhoon_linear.h).
//
// Part 1 keeps the reference's host-pointer entry points
// (kernel/w8a32_kernel.c:63-68, :355-363; kernel/w8a8_kernel.c:102-114,
// :270-272; kernel/w8a16_kernel.c:44, :218-219): the arguments are borrowed
// host memory, the call is synchronous and Y is complete on return.  Each call
// stages X through pinned memory into HBM, runs the kernels on a library
// stream, and copies Y back.  Quantized weights stay resident in HBM as 16x64
// tiles: a registry keyed by (weight pointer, scale pointer, rows, cols,
// device) and validated with a sampled content fingerprint uploads and packs
// a weight matrix the first time it is used (the reference keeps the same
// host arrays alive for the model's lifetime: decoder.py:215, :259).
//
// Part 2 exposes the same kernels on device pointers and caller streams.
// Split-reduction work-space (partials + arrival counters, counters zero at
// rest) is owned per (device, stream).
#include "host.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

using namespace tl;


namespace tlhost {

thread_local std::string t_err;
thread_local bool t_has_err = false;

void record_error(const char* fn, const std::string& msg) {
  t_err = std::string(fn) + ": " + msg;
  t_has_err = true;
  std::fprintf(stderr, "[typhoon_linear] %s\n", t_err.c_str());
}

int current_device() {
  int d = -1;
  HIP_OK(hipGetDevice(&d));
  return d;
}

uint64_t next_uid() {
  static std::atomic<uint64_t> counter{1};
  return counter.fetch_add(1, std::memory_order_relaxed);
}

tl_weights* weights_alloc(int rows, int cols) {
  REQUIRE(rows > 0 && cols > 0, "rows and cols must be positive");
  tl_weights* W = new tl_weights();
  W->uid = next_uid();
  W->dev = current_device();
  W->rows = rows;
  W->cols = cols;
  W->KB = cdiv(cols, 64);
  W->NG = cdiv(rows, 16);
  const size_t tb = (size_t)W->NG * W->KB * 1024;
  const size_t sb = (size_t)W->NG * 16 * sizeof(float);
  if (hipMalloc(&W->tiles, tb) != hipSuccess) {
    delete W;
    throw Fail{"out of device memory for weight tiles"};
  }
  if (hipMalloc(&W->scales, sb) != hipSuccess) {
    (void)hipFree(W->tiles);
    delete W;
    throw Fail{"out of device memory for weight scales"};
  }
  W->bytes = tb + sb;
  return W;
}

void weights_free(tl_weights* W) {
  if (!W) return;
  if (W->tiles) (void)hipFree(W->tiles);
  if (W->scales) (void)hipFree(W->scales);
  delete W;
}

// pack row-major int8 (host or device) + scales into a new tl_weights
tl_weights* weights_from_codes(const int8_t* w, const float* s, int rows, int cols, bool on_device,
                               hipStream_t st) {
  tl_weights* W = weights_alloc(rows, cols);
  try {
    const size_t wb = (size_t)rows * cols;
    HIP_OK(hipMemsetAsync(W->scales, 0, (size_t)W->NG * 16 * sizeof(float), st));
    HIP_OK(hipMemcpyAsync(W->scales, s, (size_t)rows * sizeof(float),
                          on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st));
    if (on_device) {
      HIP_OK(launch_pack_tiles(w, rows, cols, W->tiles, st));
      HIP_OK(hipStreamSynchronize(st));
    } else {
      void* tmp = nullptr;
      HIP_OK(hipMalloc(&tmp, wb));
      hipError_t e = hipMemcpyAsync(tmp, w, wb, hipMemcpyHostToDevice, st);
      if (e == hipSuccess) e = launch_pack_tiles(static_cast<const int8_t*>(tmp), rows, cols, W->tiles, st);
      hipError_t e2 = hipStreamSynchronize(st);
      (void)hipFree(tmp);
      HIP_OK(e);
      HIP_OK(e2);
    }
  } catch (...) {
    weights_free(W);
    throw;
  }
  return W;
}

void check_weights(const tl_weights* W) {
  REQUIRE(W != nullptr, "weights handle is NULL");
  REQUIRE(W->dev == current_device(), "weights live on another device");
}

}  // namespace tlhost

using namespace tlhost;

namespace {

// --------------------------------------------------------------------------
// per (device, stream) work-space
// --------------------------------------------------------------------------
struct Workspace {
  DevBuf part;        // split partial sums
  DevBuf cnt;         // arrival counters (zero at rest)
  size_t cnt_n = 0;
  DevBuf act;         // activation codes (tiles or padded rows)
  DevBuf act_s;       // activation scales
  DevBuf xn;          // normalised hidden row (lm_head argmax)
  DevBuf keys;        // per-work-group argmax keys
  DevBuf planes;      // W8A32 batches: int8 plane tiles of the fp32 rows and their exponents
};

std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace*> g_ws;

Workspace& workspace(int dev, hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  auto key = std::make_pair(dev, st);
  auto it = g_ws.find(key);
  if (it != g_ws.end()) return *it->second;
  Workspace* w = new Workspace();
  g_ws[key] = w;
  return *w;
}

uint32_t* ensure_counters(Workspace& w, size_t n, hipStream_t st) {
  if (n > w.cnt_n) {
    size_t want = n < 65536 ? 65536 : n;
    w.cnt.ensure(want * sizeof(uint32_t), st);
    HIP_OK(hipMemsetAsync(w.cnt.p, 0, want * sizeof(uint32_t), st));
    HIP_OK(hipStreamSynchronize(st));
    w.cnt_n = want;
  }
  return static_cast<uint32_t*>(w.cnt.p);
}

// --------------------------------------------------------------------------
// host-weight registry
// --------------------------------------------------------------------------
struct RegKey {
  const void* w;
  const void* s;
  int rows, cols, dev;
  bool operator<(const RegKey& o) const {
    if (w != o.w) return w < o.w;
    if (s != o.s) return s < o.s;
    if (rows != o.rows) return rows < o.rows;
    if (cols != o.cols) return cols < o.cols;
    return dev < o.dev;
  }
};
// entries are shared: a call holds its weights until it returns, so an
// eviction by another thread (LRU, tl_evict_weights, a changed array)
// only drops the registry's reference
using WeightsRef = std::shared_ptr<tl_weights>;
inline WeightsRef own_weights(tl_weights* W) { return WeightsRef(W, weights_free); }

struct RegEntry {
  WeightsRef W;
  uint64_t fp = 0;
  uint64_t tick = 0;
};

std::mutex g_reg_mu;
std::map<RegKey, RegEntry> g_reg;
uint64_t g_tick = 0;
size_t g_reg_bytes = 0;

size_t registry_cap() {
  static size_t cap = [] {
    const char* e = std::getenv("TL_REGISTRY_MAX_BYTES");
    if (e && *e) return (size_t)std::strtoull(e, nullptr, 10);
    return (size_t)96 << 30;  // HBM budget for cached weights (288 GB per GPU)
  }();
  return cap;
}

inline uint64_t mix64(uint64_t h, uint64_t v) {
  h ^= v + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
  h ^= h >> 31;
  h *= 0xbf58476d1ce4e5b9ull;
  return h ^ (h >> 29);
}

// sampled content fingerprint: 64 eight-byte windows of W, 32 scales, shape
uint64_t fingerprint(const int8_t* w, const float* s, int rows, int cols) {
  uint64_t h = mix64((uint64_t)rows, (uint64_t)cols);
  const size_t n = (size_t)rows * cols;
  if (n >= 8) {
    for (int i = 0; i < 64; i++) {
      size_t off = (size_t)(((unsigned __int128)(n - 8) * (unsigned)i) / 63);
      uint64_t v;
      std::memcpy(&v, w + off, 8);
      h = mix64(h, v);
    }
  } else {
    for (size_t i = 0; i < n; i++) h = mix64(h, (uint64_t)(uint8_t)w[i]);
  }
  for (int i = 0; i < 32; i++) {
    size_t r = (size_t)(((unsigned long long)(rows - 1) * (unsigned)i) / 31);
    uint32_t v;
    std::memcpy(&v, s + r, 4);
    h = mix64(h, v);
  }
  return h;
}

void registry_evict_lru_locked(size_t need) {
  while (!g_reg.empty() && g_reg_bytes + need > registry_cap()) {
    auto victim = g_reg.begin();
    for (auto it = g_reg.begin(); it != g_reg.end(); ++it)
      if (it->second.tick < victim->second.tick) victim = it;
    g_reg_bytes -= victim->second.W->bytes;
    g_reg.erase(victim);
  }
}

WeightsRef registry_get(const int8_t* w, const float* s, int rows, int cols, hipStream_t st) {
  REQUIRE(w && s, "weight and scale pointers must be non-NULL");
  const int dev = current_device();
  const uint64_t fp = fingerprint(w, s, rows, cols);
  std::lock_guard<std::mutex> lk(g_reg_mu);
  RegKey key{w, s, rows, cols, dev};
  auto it = g_reg.find(key);
  if (it != g_reg.end()) {
    if (it->second.fp == fp) {
      it->second.tick = ++g_tick;
      return it->second.W;
    }
    g_reg_bytes -= it->second.W->bytes;  // contents changed in place: re-upload
    g_reg.erase(it);
  }
  const size_t need = (size_t)cdiv(rows, 16) * 16 * (size_t)cdiv(cols, 64) * 64 + (size_t)rows * 4;
  registry_evict_lru_locked(need);
  WeightsRef W = own_weights(weights_from_codes(w, s, rows, cols, false, st));
  g_reg[key] = RegEntry{W, fp, ++g_tick};
  g_reg_bytes += W->bytes;
  return W;
}

// makes W (owned by the registry from here on) the entry of host arrays
// (w, s) that hold its codes and scales; replaces an existing entry
void registry_put(const int8_t* w, const float* s, tl_weights* W) {
  const uint64_t fp = fingerprint(w, s, W->rows, W->cols);
  std::lock_guard<std::mutex> lk(g_reg_mu);
  RegKey key{w, s, W->rows, W->cols, W->dev};
  auto it = g_reg.find(key);
  WeightsRef ref;
  if (it != g_reg.end()) {
    g_reg_bytes -= it->second.W->bytes;
    if (it->second.W.get() == W) ref = it->second.W;   // re-adopting the same matrix
    g_reg.erase(it);
  }
  if (!ref) ref = own_weights(W);
  registry_evict_lru_locked(W->bytes);
  g_reg[key] = RegEntry{ref, fp, ++g_tick};
  g_reg_bytes += W->bytes;
}

// --------------------------------------------------------------------------
// host-call contexts (Part 1): a call leases one for its duration (its own
// stream, staging and pinned buffers), so calls from different threads run
// concurrently; contexts return to a per-device pool, which holds as many as
// calls ever overlapped
// --------------------------------------------------------------------------
struct HostCtx {
  hipStream_t st = nullptr;
  DevBuf x, y, bias, xs;
  PinnedBuf hin, hout, htok;
};
std::mutex g_host_mu;                             // guards the pool only
std::map<int, std::vector<HostCtx*>> g_host_free;

struct HostLease {
  int dev;
  HostCtx* c = nullptr;
  HostLease() : dev(current_device()) {
    {
      std::lock_guard<std::mutex> lk(g_host_mu);
      auto& pool = g_host_free[dev];
      if (!pool.empty()) {
        c = pool.back();
        pool.pop_back();
      }
    }
    if (!c) {
      auto* n = new HostCtx();
      if (hipStreamCreateWithFlags(&n->st, hipStreamNonBlocking) != hipSuccess) {
        delete n;
        throw Fail{"hipStreamCreateWithFlags failed"};
      }
      c = n;
    }
  }
  // back to the pool, also after an error: its next user waits on its stream
  // before reusing a staging buffer
  ~HostLease() {
    std::lock_guard<std::mutex> lk(g_host_mu);
    g_host_free[dev].push_back(c);
  }
  HostLease(const HostLease&) = delete;
  HostLease& operator=(const HostLease&) = delete;
};

void h2d(HostCtx& c, DevBuf& d, const void* src, size_t bytes) {
  c.hin.ensure(bytes);
  d.ensure(bytes, c.st);
  HIP_OK(hipStreamSynchronize(c.st));  // hin may still be the source of an earlier copy
  std::memcpy(c.hin.p, src, bytes);
  HIP_OK(hipMemcpyAsync(d.p, c.hin.p, bytes, hipMemcpyHostToDevice, c.st));
}

void d2h(HostCtx& c, void* dst, const void* src, size_t bytes) {
  c.hout.ensure(bytes);
  HIP_OK(hipMemcpyAsync(c.hout.p, src, bytes, hipMemcpyDeviceToHost, c.st));
  HIP_OK(hipStreamSynchronize(c.st));
  std::memcpy(dst, c.hout.p, bytes);
}

void check_shape(int batch, int M, int K) {
  REQUIRE(batch >= 1, "batch must be >= 1");
  REQUIRE(M >= 1, "M (output features) must be >= 1");
  REQUIRE(K >= 1, "K (input features) must be >= 1");
}

// --------------------------------------------------------------------------
// device-level operations shared by Part 1 and Part 2
// --------------------------------------------------------------------------

// precomputed codes for the GEMV: row-major, zero padded to KB*64
uint8_t* quantize_padded(Workspace& ws, const float* x, int K, float** xs_dev, hipStream_t st) {
  const int kpad = cdiv(K, 64) * 64;
  ws.act.ensure((size_t)kpad, st);
  ws.act_s.ensure(sizeof(float), st);
  HIP_OK(hipMemsetAsync(ws.act.p, 0, (size_t)kpad, st));
  HIP_OK(launch_quantize_rows(x, static_cast<int8_t*>(ws.act.p), static_cast<float*>(ws.act_s.p), 1, K,
                              false, st));
  *xs_dev = static_cast<float*>(ws.act_s.p);
  return static_cast<uint8_t*>(ws.act.p);
}

void run_gemv(Workspace&, GemvLaunch& L, hipStream_t st) { HIP_OK(launch_gemv_i8(L, st)); }

// 1 KiB of zeros per device: the int8 GEMM copies it in place of k-blocks
// past K
std::mutex g_zero_mu;
std::map<int, uint8_t*> g_zero;

const uint8_t* zero_tile(int dev) {
  std::lock_guard<std::mutex> lk(g_zero_mu);
  auto it = g_zero.find(dev);
  if (it != g_zero.end()) return it->second;
  void* p = nullptr;
  HIP_OK(hipMalloc(&p, 1024));
  HIP_OK(hipMemset(p, 0, 1024));
  HIP_OK(hipDeviceSynchronize());
  g_zero[dev] = static_cast<uint8_t*>(p);
  return static_cast<uint8_t*>(p);
}

void run_gemm(Workspace& ws, GemmLaunch& L, hipStream_t st) {
  L.zero_tile = zero_tile(current_device());
  GemmPlan p = gemm_plan(L.amode, L.M, L.N, L.K);
  if (p.split > 1) {
    ws.part.ensure(gemm_workspace_bytes(L.amode, L.M, L.N, L.K), st);
    L.part = ws.part.p;
    L.cnt = ensure_counters(ws, gemm_counter_count(L.amode, L.M, L.N, L.K), st);
  }
  HIP_OK(launch_gemm(L, st));
}

// 1..8 rows with fp32 semantics as int8 digit planes (rows.hip); false when
// the shape or alignment is not one it takes, or the path is switched off
bool g_rows_off = false;
bool g_gemv_w8a16_off = false;   // tuning: W8A16 batch 1 on the bf16 / fp16 MFMA kernel instead

bool run_rows(Workspace& ws, GemmLaunch& L, hipStream_t st) {
  if (g_rows_off || !rows_supported(L)) return false;
  const RowsPlan p = rows_plan(L.M, L.N, L.K);
  if (p.split > 1) {
    ws.part.ensure(rows_workspace_bytes(L.M, L.N, L.K), st);
    L.part = ws.part.p;
    L.cnt = ensure_counters(ws, rows_counter_count(L.N), st);
  }
  HIP_OK(launch_rows(L, st));
  return true;
}

void op_w8a32(const float* X, const tl_weights* W, const float* bias, float* Y, int batch,
              hipStream_t st) {
  Workspace& ws = workspace(W->dev, st);
  if (batch == 1) {
    GemvLaunch L;
    L.wt = W->tiles;
    L.ws = W->scales;
    L.bias = bias;
    L.y = Y;
    L.N = W->rows;
    L.K = W->cols;
    L.epi = EPI_W8A32;
    if (gemv_fused_xv(W->cols) > 0) {
      L.x = X;
    } else {
      float* xs = nullptr;
      L.xq = quantize_padded(ws, X, W->cols, &xs, st);
      L.xs_in = xs;
    }
    run_gemv(ws, L, st);
    return;
  }
  GemmLaunch L;
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
  // 2..8 token rows over a weight of fewer than 32768 rows: int8 digit planes
  // of the fp32 rows, made inside the one launch (rows.hip; every work-group
  // splits its activation slice, which an lm_head-wide grid repeats too
  // often: 151936 rows at 2 tokens 60.1 us there against 57.0 us below, at 8
  // tokens 133 against 68 us)
  if (batch <= 8 && W->NG < 2048 && run_rows(ws, L, st)) return;
  if ((batch <= 16 && W->NG < 2048) || (batch <= 32 && W->NG <= 256)) {
    // a few token rows over a narrow weight: the small-M kernel splits the
    // fp32 rows into three bf16 terms as it loads them (one launch; a
    // separate plane split costs more than it saves at these sizes: at
    // N <= 4096, 24-32 tokens 13.7-15.1 us here against 16.6-17.0 us on the
    // planes, which win from 48 tokens)
    run_gemm(ws, L, st);
  } else {
    // fp32 rows as four int8 planes each (x = 2^e (q0 + q1/254 + q2/254^2 +
    // q3/254^3), about 2^-32 of the row's absmax), then one int8 MFMA GEMM
    // over the 4 batch code rows whose epilogue folds each token's planes
    // (no int8 -> 16-bit widening of the weights, the VALU bound of the
    // three-term bf16 path)
    const int K = W->cols, M4 = 4 * batch;
    const size_t tb = (size_t)cdiv(M4, 16) * W->KB * 1024;
    const size_t xe_off = (tb + 255) & ~(size_t)255;
    ws.planes.ensure(xe_off + (size_t)batch * sizeof(int), st);
    uint8_t* tiles = static_cast<uint8_t*>(ws.planes.p);
    int* xe = reinterpret_cast<int*>(tiles + xe_off);
    HIP_OK(launch_split_i8x4(X, K, batch, K, tiles, xe, st));
    GemmLaunch P;
    P.amode = A_I8;
    P.A = tiles;
    P.Bt = W->tiles;
    P.ws = W->scales;
    P.xe = xe;
    P.bias = bias;
    P.Y = Y;
    P.ldy = W->rows;
    P.M = M4;
    P.N = W->rows;
    P.K = K;
    P.out = OUT_F32_X4;
    run_gemm(ws, P, st);
  }
}

// W8A8 on row-major device codes
void op_w8a8_codes(const int8_t* xq, const float* xs, const tl_weights* W, const float* bias,
                   void* Y, int out, int batch, hipStream_t st) {
  Workspace& ws = workspace(W->dev, st);
  const int K = W->cols, KB = W->KB;
  if (batch == 1 && out != OUT_I32) {
    // codes must be zero padded to KB*64 for the GEMV
    const int kpad = KB * 64;
    ws.act.ensure((size_t)kpad, st);
    if (kpad != K) HIP_OK(hipMemsetAsync(ws.act.p, 0, (size_t)kpad, st));
    HIP_OK(hipMemcpyAsync(ws.act.p, xq, (size_t)K, hipMemcpyDeviceToDevice, st));
    GemvLaunch L;
    L.xq = static_cast<const uint8_t*>(ws.act.p);
    L.xs_in = xs;
    L.wt = W->tiles;
    L.ws = W->scales;
    L.bias = bias;
    L.y = static_cast<float*>(Y);
    L.N = W->rows;
    L.K = K;
    L.epi = EPI_W8A8;
    run_gemv(ws, L, st);
    return;
  }
  const size_t tb = (size_t)cdiv(batch, 16) * KB * 1024;
  ws.act.ensure(tb, st);
  HIP_OK(launch_pack_tiles(xq, batch, K, static_cast<uint8_t*>(ws.act.p), st));
  GemmLaunch L;
  L.amode = A_I8;
  L.A = ws.act.p;
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
  run_gemm(ws, L, st);
}

void op_w8a16(const void* X, int x_type, const tl_weights* W, const float* bias, void* Y,
              int y_type, int batch, hipStream_t st) {
  REQUIRE(x_type == TL_BF16 || x_type == TL_F16, "x_type must be TL_BF16 or TL_F16");
  REQUIRE(y_type == TL_F32 || y_type == TL_BF16 || y_type == TL_F16, "bad y_type");
  Workspace& ws = workspace(W->dev, st);
  GemmLaunch L;
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
  // batch==1 fuses the bias into one fma (kernel/w8a16_kernel.c:134); batch>1
  // adds it after the product (:193-200)
  L.ep = (batch == 1) ? EP_SCALE_FMA : EP_SCALE;
  L.out = (y_type == TL_F32) ? OUT_F32 : (y_type == TL_BF16 ? OUT_BF16 : OUT_F16);
  if (batch == 1 && gemv_fused_xv(W->cols) > 0 && !g_gemv_w8a16_off) {
    // one token: the GEMV's weight stream with x as four int8 digit rows
    // (fp32-accurate products, y = fma(sum, ws, bias) as the reference's
    // r * ws + b)
    GemvLaunch G;
    G.x = static_cast<const float*>(X);
    G.x_type = x_type == TL_BF16 ? 1 : 2;
    G.wt = W->tiles;
    G.ws = W->scales;
    G.bias = bias;
    G.y = static_cast<float*>(Y);
    G.N = W->rows;
    G.K = W->cols;
    G.epi = EPI_W8A16;
    G.out = L.out;
    run_gemv(ws, G, st);
    return;
  }
  run_gemm(ws, L, st);
}

// Quantizes rows of host fp32 on the GPU and returns codes and scales to the
// host.  With `pack` (the weight quantizers) the same device codes are also
// packed into HBM tiles as they are produced, and the packed matrix becomes
// the registry entry of the returned host arrays: the load step quantizes and
// packs in one pass, and the first linear call on those arrays uploads
// nothing (the reference quantizes on the CPU at load, decoder.py:248-260,
// then hands the arrays to the C decoder, decoder.c:393-423).
void host_quantize(const char* fn, const float* src, int8_t* dst, float* scales, int rows,
                   int cols, bool clamp127, bool pack) {
  (void)fn;
  REQUIRE(src && dst && scales, "NULL pointer");
  REQUIRE(rows >= 1 && cols >= 1, "rows and cols must be >= 1");
  HostLease lease;
  HostCtx& c = *lease.c;
  // chunks of at most 64 MiB of fp32 input, whole 16-row groups when packing
  int chunk = (int)std::max<size_t>(1, ((size_t)64 << 20) / ((size_t)cols * 4));
  if (pack) chunk = std::max(16, chunk & ~15);
  if (chunk > rows) chunk = rows;
  tl_weights* W = nullptr;
  if (pack) {
    W = weights_alloc(rows, cols);
  }
  try {
    if (W) HIP_OK(hipMemsetAsync(W->scales, 0, (size_t)W->NG * 16 * sizeof(float), c.st));
    c.y.ensure((size_t)chunk * cols, c.st);
    c.xs.ensure((size_t)chunk * sizeof(float), c.st);
    for (int r0 = 0; r0 < rows; r0 += chunk) {
      const int nr = std::min(chunk, rows - r0);
      h2d(c, c.x, src + (size_t)r0 * cols, (size_t)nr * cols * sizeof(float));
      HIP_OK(launch_quantize_rows(static_cast<const float*>(c.x.p), static_cast<int8_t*>(c.y.p),
                                  static_cast<float*>(c.xs.p), nr, cols, clamp127, c.st));
      if (W) {
        HIP_OK(launch_pack_tiles_rows(static_cast<const int8_t*>(c.y.p), nr, cols, W->NG, r0 / 16, W->tiles,
                                      c.st));
        HIP_OK(hipMemcpyAsync(W->scales + r0, c.xs.p, (size_t)nr * sizeof(float), hipMemcpyDeviceToDevice,
                              c.st));
      }
      d2h(c, dst + (size_t)r0 * cols, c.y.p, (size_t)nr * cols);
      d2h(c, scales + r0, c.xs.p, (size_t)nr * sizeof(float));
    }
  } catch (...) {
    if (W) {
      (void)hipStreamSynchronize(c.st);
      weights_free(W);
    }
    throw;
  }
  if (W) registry_put(dst, scales, W);
}

// --------------------------------------------------------------------------
// packed-weight cache file
// --------------------------------------------------------------------------
// A file is a sequence of self-describing records, one per matrix:
//   RecHeader (64 bytes, little-endian)
//   name      (name_len bytes, zero padded to a multiple of 64)
//   tiles     (NG * KB * 1024 bytes: the HBM tile array as resident)
//   scales    (NG * 16 * 4 bytes: fp32, zero padded)
// The payload is copied between the file and HBM as it is, with no kernel.
// `checksum` covers tiles then scales (cache_hash below); readers check the
// magic, the version, that the sizes follow from rows and cols, and the sum.
constexpr char kRecMagic[8] = {'T', 'L', 'W', 'C', 'R', 'E', 'C', '1'};
constexpr uint32_t kRecVersion = 1;
struct RecHeader {
  char magic[8];
  uint32_t version;
  uint32_t name_len;
  int32_t rows, cols, NG, KB;
  uint64_t tile_bytes, scale_bytes, checksum;
  uint64_t reserved;
};
static_assert(sizeof(RecHeader) == 64, "record header is 64 bytes");

size_t pad64(size_t n) { return (n + 63) & ~(size_t)63; }

// 64-bit streaming hash over 32-byte blocks (four independent multiply-xor
// lanes, so it runs at memory speed); every chunk but the last is a multiple
// of 32 bytes
struct CacheHash {
  uint64_t h[4] = {0x243f6a8885a308d3ull, 0x13198a2e03707344ull, 0xa4093822299f31d0ull,
                   0x082efa98ec4e6c89ull};
  uint64_t n = 0;
  static uint64_t step(uint64_t h, uint64_t v) {
    h ^= v;
    h *= 0x9e3779b97f4a7c15ull;
    return h ^ (h >> 32);
  }
  void add(const void* p, size_t bytes) {
    const uint8_t* b = static_cast<const uint8_t*>(p);
    size_t i = 0;
    for (; i + 32 <= bytes; i += 32) {
      uint64_t v[4];
      std::memcpy(v, b + i, 32);
      h[0] = step(h[0], v[0]);
      h[1] = step(h[1], v[1]);
      h[2] = step(h[2], v[2]);
      h[3] = step(h[3], v[3]);
    }
    for (; i < bytes; i++) h[i & 3] = step(h[i & 3], (uint64_t)b[i] | 0x100);
    n += bytes;
  }
  uint64_t value() const { return mix64(mix64(mix64(mix64(n, h[0]), h[1]), h[2]), h[3]); }
};

struct File {
  std::FILE* f = nullptr;
  ~File() {
    if (f) std::fclose(f);
  }
};

constexpr size_t kCacheChunk = (size_t)64 << 20;

// reads the next record header (and name) at the current position; false at
// a clean end of file
bool read_rec_header(std::FILE* f, RecHeader& h, std::string& name) {
  const size_t got = std::fread(&h, 1, sizeof h, f);
  if (got == 0 && std::feof(f)) return false;
  REQUIRE(got == sizeof h, "truncated record header");
  REQUIRE(std::memcmp(h.magic, kRecMagic, 8) == 0, "not a weight cache record (bad magic)");
  REQUIRE(h.version == kRecVersion, "unsupported weight cache version");
  REQUIRE(h.rows > 0 && h.cols > 0 && h.NG == cdiv(h.rows, 16) && h.KB == cdiv(h.cols, 64),
          "inconsistent record shape");
  REQUIRE(h.tile_bytes == (uint64_t)h.NG * h.KB * 1024 && h.scale_bytes == (uint64_t)h.NG * 16 * 4,
          "inconsistent record sizes");
  REQUIRE(h.name_len < 4096, "record name too long");
  std::vector<char> nb(pad64(h.name_len));
  REQUIRE(std::fread(nb.data(), 1, nb.size(), f) == nb.size(), "truncated record name");
  name.assign(nb.data(), h.name_len);
  return true;
}

// streams `bytes` from the file into device memory through pinned staging
void file_to_device(std::FILE* f, void* dst, size_t bytes, PinnedBuf& stage, CacheHash& hash,
                    hipStream_t st) {
  stage.ensure(std::min(bytes, kCacheChunk));
  for (size_t off = 0; off < bytes; off += kCacheChunk) {
    const size_t n = std::min(kCacheChunk, bytes - off);
    HIP_OK(hipStreamSynchronize(st));  // staging idle
    REQUIRE(std::fread(stage.p, 1, n, f) == n, "truncated record payload");
    hash.add(stage.p, n);
    HIP_OK(hipMemcpyAsync(static_cast<char*>(dst) + off, stage.p, n, hipMemcpyHostToDevice, st));
  }
  HIP_OK(hipStreamSynchronize(st));
}

void device_to_file(std::FILE* f, const void* src, size_t bytes, PinnedBuf& stage, CacheHash* hash,
                    hipStream_t st) {
  stage.ensure(std::min(bytes, kCacheChunk));
  for (size_t off = 0; off < bytes; off += kCacheChunk) {
    const size_t n = std::min(kCacheChunk, bytes - off);
    HIP_OK(hipMemcpyAsync(stage.p, static_cast<const char*>(src) + off, n, hipMemcpyDeviceToHost, st));
    HIP_OK(hipStreamSynchronize(st));
    if (hash) hash->add(stage.p, n);
    if (f) REQUIRE(std::fwrite(stage.p, 1, n, f) == n, "write failed");
  }
}

}  // namespace

namespace tlhost {
void linear_w8a32(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st) {
  op_w8a32(X, W, bias, Y, batch, st);
}
void linear_w8a8(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st) {
  if (tl_w8a8_linear_f32_dev(X, W, bias, Y, batch, st) != 0) throw Fail{t_err};
}
void linear_w8a32_planes(const uint8_t* tiles, const int* xe, const tl_weights* W, float* Y, int batch,
                         hipStream_t st) {
  Workspace& ws = workspace(W->dev, st);
  GemmLaunch L;
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
  run_gemm(ws, L, st);
}
void linear_w8a8_tiles(const uint8_t* tiles, const float* xs, const tl_weights* W, float* Y, int batch,
                       hipStream_t st) {
  Workspace& ws = workspace(W->dev, st);
  GemmLaunch L;
  L.amode = A_I8;
  L.A = tiles;
  L.Bt = W->tiles;
  L.ws = W->scales;
  L.xs = xs;
  L.Y = Y;
  L.ldy = W->rows;
  L.M = batch;
  L.N = W->rows;
  L.K = W->cols;
  L.out = OUT_F32;
  run_gemm(ws, L, st);
}
}  // namespace tlhost

// ==========================================================================
// Part 1 -- reference entry points
// ==========================================================================
extern "C" {

void w8a32_quantize(const float* w_fp32, int8_t* w_int8, float* scales, int rows, int cols) {
  guarded("w8a32_quantize", [&] { host_quantize("w8a32_quantize", w_fp32, w_int8, scales, rows, cols, true, true); });
}

void w8a8_quantize_weights(const float* w_fp32, int8_t* w_int8, float* w_scales, int rows, int cols) {
  guarded("w8a8_quantize_weights",
          [&] { host_quantize("w8a8_quantize_weights", w_fp32, w_int8, w_scales, rows, cols, true, true); });
}

void w8a8_quantize_activations(const float* x_fp32, int8_t* x_int8, float* x_scales, int batch, int K) {
  guarded("w8a8_quantize_activations",
          [&] { host_quantize("w8a8_quantize_activations", x_fp32, x_int8, x_scales, batch, K, true, false); });
}

void w8a16_quantize_weights(const float* w_fp32, int8_t* w_int8, float* scales, int rows, int cols) {
  guarded("w8a16_quantize_weights",
          [&] { host_quantize("w8a16_quantize_weights", w_fp32, w_int8, scales, rows, cols, true, true); });
}

void w8a32_linear(const float* X, const int8_t* w_int8, const float* scales, const float* bias,
                  float* Y, float* scratch, int batch, int M, int K) {
  (void)scratch;  // unused, as in the reference (kernel/w8a32_kernel.c:364)
  guarded("w8a32_linear", [&] {
    check_shape(batch, M, K);
    REQUIRE(X && Y, "X and Y must be non-NULL");
    HostLease lease;
    HostCtx& c = *lease.c;
    const WeightsRef Wr = registry_get(w_int8, scales, M, K, c.st);
    const tl_weights* W = Wr.get();
    const float* b = nullptr;
    if (bias) {
      c.bias.ensure((size_t)M * sizeof(float), c.st);
      HIP_OK(hipMemcpyAsync(c.bias.p, bias, (size_t)M * sizeof(float), hipMemcpyHostToDevice, c.st));
      b = static_cast<const float*>(c.bias.p);
    }
    if (batch == 1) {
      // decode: x comes in through mapped pinned memory by a copy kernel and
      // the GEMV writes y straight into mapped pinned memory, so the call is
      // two kernels and one synchronisation (no DMA transfers)
      const size_t xb = (size_t)K * sizeof(float), yb = (size_t)M * sizeof(float);
      c.hin.ensure(xb);
      c.hout.ensure(yb);
      c.x.ensure(xb, c.st);
      HIP_OK(hipStreamSynchronize(c.st));  // staging buffers idle
      std::memcpy(c.hin.p, X, xb);
      HIP_OK(launch_copy_words(c.hin.dp, c.x.p, xb, c.st));
      op_w8a32(static_cast<const float*>(c.x.p), W, b, static_cast<float*>(c.hout.dp), 1, c.st);
      HIP_OK(hipStreamSynchronize(c.st));
      std::memcpy(Y, c.hout.p, yb);
      return;
    }
    h2d(c, c.x, X, (size_t)batch * K * sizeof(float));
    c.y.ensure((size_t)batch * M * sizeof(float), c.st);
    op_w8a32(static_cast<const float*>(c.x.p), W, b, static_cast<float*>(c.y.p), batch, c.st);
    d2h(c, Y, c.y.p, (size_t)batch * M * sizeof(float));
  });
}

void w8a8_linear(const int8_t* x_int8, const float* x_scales, const int8_t* w_int8,
                 const float* w_scales, const float* bias, float* Y, int batch, int M, int K) {
  guarded("w8a8_linear", [&] {
    check_shape(batch, M, K);
    REQUIRE(x_int8 && x_scales && Y, "x_int8, x_scales and Y must be non-NULL");
    HostLease lease;
    HostCtx& c = *lease.c;
    const WeightsRef Wr = registry_get(w_int8, w_scales, M, K, c.st);
    const tl_weights* W = Wr.get();
    h2d(c, c.x, x_int8, (size_t)batch * K);
    c.xs.ensure((size_t)batch * sizeof(float), c.st);
    HIP_OK(hipMemcpyAsync(c.xs.p, x_scales, (size_t)batch * sizeof(float), hipMemcpyHostToDevice, c.st));
    const float* b = nullptr;
    if (bias) {
      c.bias.ensure((size_t)M * sizeof(float), c.st);
      HIP_OK(hipMemcpyAsync(c.bias.p, bias, (size_t)M * sizeof(float), hipMemcpyHostToDevice, c.st));
      b = static_cast<const float*>(c.bias.p);
    }
    c.y.ensure((size_t)batch * M * sizeof(float), c.st);
    op_w8a8_codes(static_cast<const int8_t*>(c.x.p), static_cast<const float*>(c.xs.p), W, b, c.y.p,
                  OUT_F32, batch, c.st);
    d2h(c, Y, c.y.p, (size_t)batch * M * sizeof(float));
  });
}

void w8a16_linear(const uint16_t* x_bf16_raw, const int8_t* w_int8, const float* w_scales,
                  const float* bias, float* Y, int batch, int M, int K) {
  guarded("w8a16_linear", [&] {
    check_shape(batch, M, K);
    REQUIRE(x_bf16_raw && Y, "x and Y must be non-NULL");
    HostLease lease;
    HostCtx& c = *lease.c;
    const WeightsRef Wr = registry_get(w_int8, w_scales, M, K, c.st);
    const tl_weights* W = Wr.get();
    h2d(c, c.x, x_bf16_raw, (size_t)batch * K * sizeof(uint16_t));
    const float* b = nullptr;
    if (bias) {
      c.bias.ensure((size_t)M * sizeof(float), c.st);
      HIP_OK(hipMemcpyAsync(c.bias.p, bias, (size_t)M * sizeof(float), hipMemcpyHostToDevice, c.st));
      b = static_cast<const float*>(c.bias.p);
    }
    c.y.ensure((size_t)batch * M * sizeof(float), c.st);
    op_w8a16(c.x.p, TL_BF16, W, b, c.y.p, TL_F32, batch, c.st);
    d2h(c, Y, c.y.p, (size_t)batch * M * sizeof(float));
  });
}

// ==========================================================================
// Part 2 -- extensions
// ==========================================================================
const char* tl_last_error(void) { return t_has_err ? t_err.c_str() : nullptr; }
void tl_clear_error(void) { t_has_err = false; }
const char* tl_version(void) { return "typhoon_linear 0.1 gfx950"; }

int tl_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int tl_gemv_set_plan(int rows, int u) {
  return guarded("tl_gemv_set_plan", [&] {
    REQUIRE(rows == 0 || rows == 8 || rows == 16, "rows must be 0, 8 or 16");
    REQUIRE(u == 0 || u == 2 || u == 4 || u == 6 || u == 8 || u == 12, "u must be 0, 2, 4, 6, 8 or 12");
    REQUIRE(u == 0 || rows == 0 || (rows == 16 ? u != 6 : u != 12), "u = 6 needs rows 8, u = 12 rows 16");
    gemv_set_plan(rows, u);
  });
}

int tl_rows_set_split(int split) {
  return guarded("tl_rows_set_split", [&] {
    REQUIRE(split >= -1 && split <= 64, "split must be -1 (path off), 0 (planner) or 1..64");
    g_rows_off = split < 0;
    rows_set_split(split > 0 ? split : 0);
  });
}

int tl_rows_set_groups(int groups) {
  return guarded("tl_rows_set_groups", [&] {
    REQUIRE(groups >= 0 && groups <= 3, "groups must be 0 (planner) or 1..3");
    rows_set_groups(groups);
  });
}

int tl_w8a16_set_gemv(int on) {
  return guarded("tl_w8a16_set_gemv", [&] {
    REQUIRE(on == 0 || on == 1, "on must be 0 or 1");
    g_gemv_w8a16_off = on == 0;
  });
}

int tl_gemm_i8_set_cfg(int cfg) {
  return guarded("tl_gemm_i8_set_cfg", [&] {
    REQUIRE(cfg >= -1 && cfg <= 7, "cfg must be -1 (planner) or 0..7");
    gemm_i8_set_cfg(cfg);
  });
}

int tl_stream_read_dev(const void* p, size_t bytes, int grid, int u, uint32_t* sink, void* stream) {
  return guarded("tl_stream_read_dev", [&] {
    REQUIRE(p && sink, "NULL pointer");
    REQUIRE(bytes > 0 && bytes % 16 == 0 && (((uintptr_t)p) & 15) == 0,
            "bytes must be a positive multiple of 16 and p 16-byte aligned");
    REQUIRE(grid >= 1 && grid <= 65536, "grid must be 1..65536");
    REQUIRE(u == 4 || u == 8, "u must be 4 or 8");
    HIP_OK(launch_stream_read(p, bytes, grid, u, sink, static_cast<hipStream_t>(stream)));
  });
}

int tl_attn_set_chunk(int positions) {
  return guarded("tl_attn_set_chunk", [&] {
    REQUIRE(positions == 0 || positions == 32 || positions == 64 || positions == 128,
            "positions must be 0, 32, 64 or 128");
    attn_set_chunk(positions);
  });
}

int tl_register_weights(const int8_t* w_int8, const float* scales, int rows, int cols) {
  return guarded("tl_register_weights", [&] {
    HostLease lease;
    (void)registry_get(w_int8, scales, rows, cols, lease.c->st);
  });
}

int tl_evict_weights(const int8_t* w_int8) {
  return guarded("tl_evict_weights", [&] {
    std::lock_guard<std::mutex> lk(g_reg_mu);
    for (auto it = g_reg.begin(); it != g_reg.end();) {
      if (it->first.w == (const void*)w_int8) {
        g_reg_bytes -= it->second.W->bytes;
        it = g_reg.erase(it);
      } else {
        ++it;
      }
    }
  });
}

void tl_registry_clear(void) {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  g_reg.clear();
  g_reg_bytes = 0;
}

size_t tl_registry_bytes(void) {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  return g_reg_bytes;
}

int tl_registry_entries(void) {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  return (int)g_reg.size();
}

tl_weights* tl_weights_create(const int8_t* w_int8, const float* scales, int rows, int cols,
                              int src_on_device) {
  tl_weights* out = nullptr;
  guarded("tl_weights_create", [&] {
    REQUIRE(w_int8 && scales, "NULL pointer");
    hipStream_t st = nullptr;
    out = weights_from_codes(w_int8, scales, rows, cols, src_on_device != 0, st);
  });
  return out;
}

tl_weights* tl_weights_quantize_dev(const float* w_fp32, int rows, int cols, int8_t* codes_out,
                                    float* scales_out, void* stream) {
  tl_weights* out = nullptr;
  guarded("tl_weights_quantize_dev", [&] {
    REQUIRE(w_fp32, "NULL pointer");
    hipStream_t st = static_cast<hipStream_t>(stream);
    tl_weights* W = weights_alloc(rows, cols);
    hipError_t e = hipMemsetAsync(W->scales, 0, (size_t)W->NG * 16 * sizeof(float), st);
    if (e == hipSuccess) e = hipMemsetAsync(W->tiles, 0, (size_t)W->NG * W->KB * 1024, st);
    if (e == hipSuccess) e = launch_quantize_rows_tiled(w_fp32, rows, cols, W->tiles, W->scales, true, st);
    if (e == hipSuccess && codes_out) {
      float* s2 = scales_out;
      DevBuf tmp;
      if (!s2) {
        tmp.ensure((size_t)rows * sizeof(float), st);
        s2 = static_cast<float*>(tmp.p);
      }
      e = launch_quantize_rows(w_fp32, codes_out, s2, rows, cols, true, st);
      if (e == hipSuccess) e = hipStreamSynchronize(st);
      if (tmp.p) (void)hipFree(tmp.p);
    } else if (e == hipSuccess && scales_out) {
      e = hipMemcpyAsync(scales_out, W->scales, (size_t)rows * sizeof(float), hipMemcpyDeviceToDevice, st);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
      weights_free(W);
      throw Fail{std::string("quantize: ") + hipGetErrorString(e)};
    }
    out = W;
  });
  return out;
}

void tl_weights_destroy(tl_weights* w) { weights_free(w); }
int tl_weights_rows(const tl_weights* w) { return w ? w->rows : -1; }
int tl_weights_cols(const tl_weights* w) { return w ? w->cols : -1; }
size_t tl_weights_bytes(const tl_weights* w) { return w ? w->bytes : 0; }

int tl_w8a32_linear_dev(const float* X, const tl_weights* W, const float* bias, float* Y, int batch,
                        void* stream) {
  return guarded("tl_w8a32_linear_dev", [&] {
    check_weights(W);
    REQUIRE(batch >= 1 && X && Y, "bad arguments");
    op_w8a32(X, W, bias, Y, batch, static_cast<hipStream_t>(stream));
  });
}

int tl_quantize_rows_dev(const float* src, int8_t* codes, float* scales, int rows, int cols,
                         int clamp127, void* stream) {
  return guarded("tl_quantize_rows_dev", [&] {
    REQUIRE(src && codes && scales && rows >= 1 && cols >= 1, "bad arguments");
    HIP_OK(launch_quantize_rows(src, codes, scales, rows, cols, clamp127 != 0,
                                static_cast<hipStream_t>(stream)));
  });
}

int tl_w8a8_linear_dev(const int8_t* x_int8, const float* x_scales, const tl_weights* W,
                       const float* bias, float* Y, int batch, void* stream) {
  return guarded("tl_w8a8_linear_dev", [&] {
    check_weights(W);
    REQUIRE(batch >= 1 && x_int8 && x_scales && Y, "bad arguments");
    op_w8a8_codes(x_int8, x_scales, W, bias, Y, OUT_F32, batch, static_cast<hipStream_t>(stream));
  });
}

int tl_w8a8_linear_f32_dev(const float* X, const tl_weights* W, const float* bias, float* Y, int batch,
                           void* stream) {
  return guarded("tl_w8a8_linear_f32_dev", [&] {
    check_weights(W);
    REQUIRE(batch >= 1 && X && Y, "bad arguments");
    hipStream_t st = static_cast<hipStream_t>(stream);
    Workspace& ws = workspace(W->dev, st);
    if (batch == 1) {
      GemvLaunch L;
      L.wt = W->tiles;
      L.ws = W->scales;
      L.bias = bias;
      L.y = Y;
      L.N = W->rows;
      L.K = W->cols;
      L.epi = EPI_W8A8;
      if (gemv_fused_xv(W->cols) > 0) {
        L.x = X;
      } else {
        float* xs = nullptr;
        L.xq = quantize_padded(ws, X, W->cols, &xs, st);
        L.xs_in = xs;
      }
      run_gemv(ws, L, st);
      return;
    }
    const int MG = cdiv(batch, 16);
    ws.act.ensure((size_t)MG * W->KB * 1024, st);
    ws.act_s.ensure((size_t)MG * 16 * sizeof(float), st);
    HIP_OK(launch_quantize_rows_tiled(X, batch, W->cols, static_cast<uint8_t*>(ws.act.p),
                                      static_cast<float*>(ws.act_s.p), true, st));
    GemmLaunch L;
    L.amode = A_I8;
    L.A = ws.act.p;
    L.Bt = W->tiles;
    L.ws = W->scales;
    L.xs = static_cast<const float*>(ws.act_s.p);
    L.bias = bias;
    L.Y = Y;
    L.ldy = W->rows;
    L.M = batch;
    L.N = W->rows;
    L.K = W->cols;
    L.out = OUT_F32;
    run_gemm(ws, L, st);
  });
}

int tl_w8a16_linear_dev(const void* X, int x_type, const tl_weights* W, const float* bias, void* Y,
                        int y_type, int batch, void* stream) {
  return guarded("tl_w8a16_linear_dev", [&] {
    check_weights(W);
    REQUIRE(batch >= 1 && X && Y, "bad arguments");
    op_w8a16(X, x_type, W, bias, Y, y_type, batch, static_cast<hipStream_t>(stream));
  });
}

int tl_w8a32_gemv_acc_dev(const float* x, const tl_weights* W, int32_t* acc, float* x_scale,
                          void* stream) {
  return guarded("tl_w8a32_gemv_acc_dev", [&] {
    check_weights(W);
    REQUIRE(x && acc, "bad arguments");
    REQUIRE(gemv_fused_xv(W->cols) > 0, "K too large for the fused GEMV");
    hipStream_t st = static_cast<hipStream_t>(stream);
    Workspace& ws = workspace(W->dev, st);
    GemvLaunch L;
    L.x = x;
    L.wt = W->tiles;
    L.ws = W->scales;
    L.acc_out = acc;
    L.xs_out = x_scale;
    L.N = W->rows;
    L.K = W->cols;
    L.epi = EPI_ACC;
    run_gemv(ws, L, st);
  });
}

int tl_rmsnorm_np_dev(const float* h, const float* norm_w, float* out, int K, void* stream) {
  return guarded("tl_rmsnorm_np_dev", [&] {
    REQUIRE(h && out, "h and out must be non-NULL");
    REQUIRE(K >= 128 && K <= 16384 && (K & (K - 1)) == 0, "K must be a power of two in [128, 16384]");
    HIP_OK(launch_rmsnorm_np(h, norm_w, out, K, 1e-6f, static_cast<hipStream_t>(stream)));
  });
}

// final RMSNorm, lm_head GEMV with per-work-group argmax keys, key reduction
void op_lm_head_argmax(const float* h, const float* norm_w, const tl_weights* W, float* logits,
                       int32_t* token, float* max_logit, hipStream_t st) {
  Workspace& ws = workspace(W->dev, st);
  ws.keys.ensure(lm_head_argmax_keys(W->rows, W->cols) * sizeof(uint64_t), st);
  ws.xn.ensure((size_t)W->cols * sizeof(float), st);
  lm_head_argmax_enqueue(h, norm_w, W, logits, token, max_logit, static_cast<uint64_t*>(ws.keys.p),
                         static_cast<float*>(ws.xn.p), st);
}

int tl_lm_head_argmax_dev(const float* h, const float* norm_w, const tl_weights* W, float* logits,
                          int32_t* token, float* max_logit, void* stream) {
  return guarded("tl_lm_head_argmax_dev", [&] {
    check_weights(W);
    REQUIRE(h && token, "h and token must be non-NULL");
    op_lm_head_argmax(h, norm_w, W, logits, token, max_logit, static_cast<hipStream_t>(stream));
  });
}

int tl_lm_head_argmax(const float* h, const float* norm_w, const int8_t* w_int8, const float* scales,
                      int N, int K, float* logits, int32_t* token) {
  return guarded("tl_lm_head_argmax", [&] {
    check_shape(1, N, K);
    REQUIRE(h && token, "h and token must be non-NULL");
    HostLease lease;
    HostCtx& c = *lease.c;
    const WeightsRef Wr = registry_get(w_int8, scales, N, K, c.st);
    const tl_weights* W = Wr.get();
    // h and the norm weights in one staging copy: [h | norm_w]
    const size_t kb = (size_t)K * sizeof(float);
    const size_t inb = norm_w ? 2 * kb : kb;
    c.hin.ensure(inb);
    c.htok.ensure(16);
    c.x.ensure(inb, c.st);
    HIP_OK(hipStreamSynchronize(c.st));
    std::memcpy(c.hin.p, h, kb);
    if (norm_w) std::memcpy(static_cast<char*>(c.hin.p) + kb, norm_w, kb);
    HIP_OK(launch_copy_words(c.hin.dp, c.x.p, inb, c.st));
    const float* hd = static_cast<const float*>(c.x.p);
    const float* wd = norm_w ? hd + K : nullptr;
    float* ld = nullptr;
    if (logits) {
      c.y.ensure(kb > (size_t)N * 4 ? kb : (size_t)N * 4, c.st);
      ld = static_cast<float*>(c.y.p);
    }
    int32_t* td = static_cast<int32_t*>(c.htok.dp);
    op_lm_head_argmax(hd, wd, W, ld, td, nullptr, c.st);
    if (logits) {
      d2h(c, logits, ld, (size_t)N * sizeof(float));
    } else {
      HIP_OK(hipStreamSynchronize(c.st));
    }
    *token = *static_cast<const int32_t*>(c.htok.p);
  });
}

int tl_gemv_fused_dev(const float* x, const tl_weights* W, const float* bias, float* y, int epi, int norm,
                      const float* norm_w, void* stream) {
  return guarded("tl_gemv_fused_dev", [&] {
    check_weights(W);
    REQUIRE(x && y, "bad arguments");
    REQUIRE(epi == EPI_W8A32 || epi == EPI_SWIGLU, "epi must be 0 (W8A32) or 4 (SwiGLU)");
    REQUIRE(norm >= NORM_NONE && norm <= NORM_DECODER, "norm must be 0, 1 or 2");
    REQUIRE(norm == NORM_NONE || gemv_fused_norm_ok(W->cols, x, norm_w ? norm_w : x),
            "a fused RMSNorm needs K = 1024 * 2^j <= 16384 and 16-byte aligned vectors");
    GemvLaunch L;
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
    HIP_OK(launch_gemv_i8(L, static_cast<hipStream_t>(stream)));
  });
}

int tl_w8a8_gemm_acc_dev(const int8_t* x_int8, const tl_weights* W, int32_t* acc, int batch,
                         void* stream) {
  return guarded("tl_w8a8_gemm_acc_dev", [&] {
    check_weights(W);
    REQUIRE(batch >= 1 && x_int8 && acc, "bad arguments");
    op_w8a8_codes(x_int8, nullptr, W, nullptr, acc, OUT_I32, batch, static_cast<hipStream_t>(stream));
  });
}

// --------------------------------------------------------------------------
// packed-weight cache file, registry adoption, code export
// --------------------------------------------------------------------------
int tl_weights_save(const tl_weights* W, const char* path, const char* name, int append) {
  return guarded("tl_weights_save", [&] {
    check_weights(W);
    REQUIRE(path && name, "NULL path or name");
    const size_t nl = std::strlen(name);
    REQUIRE(nl < 4096, "record name too long");
    hipStream_t st = nullptr;
    PinnedBuf stage;
    struct Free {
      PinnedBuf& b;
      ~Free() {
        if (b.p) (void)hipHostFree(b.p);
      }
    } free_stage{stage};
    File file;
    if (append) file.f = std::fopen(path, "r+b");
    if (!file.f) file.f = std::fopen(path, "wb");
    REQUIRE(file.f, std::string("cannot open ") + path + " for writing");
    REQUIRE(std::fseek(file.f, 0, SEEK_END) == 0, "seek failed");
    const long pos = std::ftell(file.f);
    REQUIRE(pos >= 0, "ftell failed");
    // header with the checksum filled in after the payload went out
    RecHeader h{};
    std::memcpy(h.magic, kRecMagic, 8);
    h.version = kRecVersion;
    h.name_len = (uint32_t)nl;
    h.rows = W->rows;
    h.cols = W->cols;
    h.NG = W->NG;
    h.KB = W->KB;
    h.tile_bytes = (uint64_t)W->NG * W->KB * 1024;
    h.scale_bytes = (uint64_t)W->NG * 16 * 4;
    REQUIRE(std::fwrite(&h, 1, sizeof h, file.f) == sizeof h, "write failed");
    std::vector<char> nb(pad64(nl), 0);
    std::memcpy(nb.data(), name, nl);
    REQUIRE(std::fwrite(nb.data(), 1, nb.size(), file.f) == nb.size(), "write failed");
    CacheHash hash;
    device_to_file(file.f, W->tiles, h.tile_bytes, stage, &hash, st);
    device_to_file(file.f, W->scales, h.scale_bytes, stage, &hash, st);
    h.checksum = hash.value();
    REQUIRE(std::fseek(file.f, pos, SEEK_SET) == 0, "seek failed");
    REQUIRE(std::fwrite(&h, 1, sizeof h, file.f) == sizeof h, "write failed");
    REQUIRE(std::fflush(file.f) == 0, "write failed");
  });
}

tl_weights* tl_weights_load(const char* path, const char* name) {
  tl_weights* out = nullptr;
  guarded("tl_weights_load", [&] {
    REQUIRE(path && name, "NULL path or name");
    File file;
    file.f = std::fopen(path, "rb");
    REQUIRE(file.f, std::string("cannot open ") + path);
    RecHeader h;
    std::string rn;
    for (;;) {
      REQUIRE(read_rec_header(file.f, h, rn), std::string("no record named ") + name + " in " + path);
      if (rn == name) break;
      REQUIRE(std::fseek(file.f, (long)(h.tile_bytes + h.scale_bytes), SEEK_CUR) == 0, "seek failed");
    }
    tl_weights* W = weights_alloc(h.rows, h.cols);
    PinnedBuf stage;
    try {
      hipStream_t st = nullptr;
      CacheHash hash;
      file_to_device(file.f, W->tiles, h.tile_bytes, stage, hash, st);
      file_to_device(file.f, W->scales, h.scale_bytes, stage, hash, st);
      REQUIRE(hash.value() == h.checksum, std::string("checksum mismatch in record ") + name);
    } catch (...) {
      if (stage.p) (void)hipHostFree(stage.p);
      weights_free(W);
      throw;
    }
    if (stage.p) (void)hipHostFree(stage.p);
    out = W;
  });
  return out;
}

int tl_weights_cache_list(const char* path, char* names, size_t names_len) {
  int count = -1;
  guarded("tl_weights_cache_list", [&] {
    REQUIRE(path, "NULL path");
    File file;
    file.f = std::fopen(path, "rb");
    REQUIRE(file.f, std::string("cannot open ") + path);
    RecHeader h;
    std::string rn, all;
    int n = 0;
    while (read_rec_header(file.f, h, rn)) {
      all += rn;
      all += '\n';
      n++;
      REQUIRE(std::fseek(file.f, (long)(h.tile_bytes + h.scale_bytes), SEEK_CUR) == 0, "seek failed");
    }
    if (names && names_len) {
      REQUIRE(all.size() < names_len, "names buffer too small");
      std::memcpy(names, all.c_str(), all.size() + 1);
    }
    count = n;
  });
  return count;
}

int tl_weights_export(const tl_weights* W, int8_t* codes, float* scales, int dst_on_device) {
  return guarded("tl_weights_export", [&] {
    check_weights(W);
    REQUIRE(codes || scales, "nothing to export");
    hipStream_t st = nullptr;
    const size_t cb = (size_t)W->rows * W->cols, sb = (size_t)W->rows * sizeof(float);
    if (dst_on_device) {
      if (codes) HIP_OK(launch_unpack_tiles(W->tiles, W->rows, W->cols, codes, st));
      if (scales) HIP_OK(hipMemcpyAsync(scales, W->scales, sb, hipMemcpyDeviceToDevice, st));
      HIP_OK(hipStreamSynchronize(st));
      return;
    }
    if (codes) {
      DevBuf tmp;
      struct Free {
        DevBuf& b;
        ~Free() {
          if (b.p) (void)hipFree(b.p);
        }
      } free_tmp{tmp};
      tmp.ensure(cb, st);
      HIP_OK(launch_unpack_tiles(W->tiles, W->rows, W->cols, static_cast<int8_t*>(tmp.p), st));
      HIP_OK(hipMemcpyAsync(codes, tmp.p, cb, hipMemcpyDeviceToHost, st));
      HIP_OK(hipStreamSynchronize(st));
    }
    if (scales) {
      HIP_OK(hipMemcpyAsync(scales, W->scales, sb, hipMemcpyDeviceToHost, st));
      HIP_OK(hipStreamSynchronize(st));
    }
  });
}

int tl_registry_adopt(const int8_t* w_int8, const float* scales, tl_weights* W) {
  return guarded("tl_registry_adopt", [&] {
    check_weights(W);
    REQUIRE(w_int8 && scales, "NULL pointer");
    registry_put(w_int8, scales, W);
  });
}

}  // extern "C"
