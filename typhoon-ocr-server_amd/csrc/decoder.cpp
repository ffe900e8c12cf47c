// decoder.cpp -- the reference's decoder C ABI (kernel/decoder.h,
// kernel/decoder.c:300-526) with the decode loop resident on the GPU.
//
// Handles keep the reference's names and roles, as opaque types:
//   ModelWeights    per layer: fused Q||K||V, O, gate/up interleaved per
//                   16-row group (for the SwiGLU epilogue), down, as HBM tiles,
//                   plus the four norm vectors (decoder_set_layer_weights*)
//   KVCache         K and V [layer][kv head][max_seq][128] fp32 in HBM, the
//                   reference's seq_len / rope_offset counters, and the
//                   device copy of the decode state (position, rotary position,
//                   token counter) that the kernels read
//   DecoderScratch  activation buffers, attention partials, a stream and the
//                   captured step graphs
//
// One layer of a decode step is five launches (decoder.c:33-157):
//   1. QKV GEMV, input RMSNorm in its prologue                  -> qkv
//   2. attention: QK RMSNorm, M-RoPE, KV append, chunk partials, and the
//      merge in the last work-group of each kv head             -> attn
//   3. O GEMV + residual (the residual is the GEMV bias, in place) -> hidden
//   4. gate/up GEMV, post-attention RMSNorm prologue, SwiGLU epilogue -> mlp
//   5. down GEMV + residual                                     -> hidden
// The layer loop is captured once into a HIP graph per (model, cache, rope
// tables) and replayed; the decode state is written before each replay.
// tl_decoder_generate adds the lm_head (numpy final RMSNorm + argmax keys)
// and step_end (token, next embedding row, position advance) to the graph, so
// consecutive greedy steps are graph replays with no host round trip.
//
// Calls on one scratch must not overlap (the reference's are synchronous too).
#include "host.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

using namespace tl;
using namespace tlhost;

namespace {
constexpr int H = 2048, KVD = 1024, FF = 6144, NQ = 16, NKV = 8, HDIM = 128, NL = 28;
constexpr int QKVD = H + 2 * KVD;
constexpr float EPS = 1e-6f;
constexpr float SCALE = 0.08838834764831843f;   // 1/sqrt(128), decoder.c:28

struct LayerDev {
  tl_weights* qkv = nullptr;
  tl_weights* o = nullptr;
  tl_weights* gu = nullptr;     // gate/up interleaved per 16-row group
  tl_weights* down = nullptr;
  float* norms = nullptr;       // input_ln [H] | post_attn_ln [H] | q_norm [128] | k_norm [128]
  void release() {
    weights_free(qkv);
    weights_free(o);
    weights_free(gu);
    weights_free(down);
    if (norms) (void)hipFree(norms);
    *this = LayerDev();
  }
};

struct RopeDev {
  float* cos = nullptr;
  float* sin = nullptr;
  uint64_t fp = 0;
  uint64_t uid = 0;             // process-unique (next_uid), drawn at allocation
};

uint64_t mix(uint64_t h, uint64_t v) {
  h ^= v + 0x9e3779b97f4a7c15ull + (h << 6) + (h >> 2);
  h *= 0xbf58476d1ce4e5b9ull;
  return h ^ (h >> 31);
}

// sampled fingerprint of a rope table pair (rows x 64 floats each)
uint64_t rope_fp(const float* c, const float* s, int rows) {
  uint64_t h = (uint64_t)rows;
  const size_t n = (size_t)rows * 64;
  for (int i = 0; i < 64; i++) {
    const size_t k = (size_t)(((unsigned __int128)(n - 1) * (unsigned)i) / 63);
    uint32_t a, b;
    std::memcpy(&a, c + k, 4);
    std::memcpy(&b, s + k, 4);
    h = mix(mix(h, a), b);
  }
  return h;
}
}  // namespace

struct ModelWeights {
  int dev = -1;
  LayerDev layers[NL];
  uint64_t version = next_uid();   // process-unique, redrawn whenever a layer changes
  bool prefill_w8a8 = false;    // prefill linears on per-token int8 activations
  int num_layers() const {
    int n = 0;
    while (n < NL && layers[n].qkv) n++;
    return n;
  }
};

struct KVCache {
  int dev = -1;
  int max_seq = 0;
  int seq_len = 0, rope_offset = 0;     // kv_cache.h fields
  float* k = nullptr;
  float* v = nullptr;
  int* state = nullptr;                 // device: position, rotary position, token counter
  uint64_t uid = next_uid();            // process-unique, never reused
  std::map<std::pair<const float*, const float*>, RopeDev> rope;   // device copies of host tables
  size_t layer_floats() const { return (size_t)NKV * max_seq * HDIM; }
};

struct DecoderScratch {
  int dev = -1;
  int max_seq = 0;
  hipStream_t st = nullptr;
  float *hidden = nullptr, *qkv = nullptr, *attn = nullptr, *mlp = nullptr;
  float *pm = nullptr, *pl = nullptr, *po = nullptr;   // attention chunk partials [NQ][C](x128)
  int* count = nullptr;                 // attention arrival counters [NKV], zero between launches
  int C = 0;
  DevBuf keys, tokens, fnorm;
  PinnedBuf pin;
  PinnedBuf pin_rows;                   // prefill hidden rows on their way to / from HBM
  // prefill activations (token-major, grown to the longest prefill)
  DevBuf p_h, p_xn, p_qkv, p_att, p_gu, p_mlp, p_y, p_cos, p_sin;
  DevBuf p_q, p_qs;                     // int8 activation tiles, per-token scales (W8A8) or exponents (planes)
  DevBuf p_fpart, p_fcnt;               // prefill attention's split-key partials and counters (zero between launches)
  // captured graphs and what they were captured for: process-unique ids of
  // the handles whose device memory they bake in (a freed handle's successor
  // can reuse its host address, never its id) and the device pointers the
  // scratch itself owns
  hipGraphExec_t layers_exec = nullptr;
  uint64_t layers_key[4] = {};
  hipGraphExec_t gen_exec = nullptr;
  uint64_t gen_key[9] = {};
};

namespace {

void drop_graph(hipGraphExec_t& g) {
  if (g) (void)hipGraphExecDestroy(g);
  g = nullptr;
}

const RopeDev& rope_device(KVCache* c, const float* cos_tab, const float* sin_tab) {
  REQUIRE(cos_tab && sin_tab, "rope tables must be non-NULL");
  const uint64_t fp = rope_fp(cos_tab, sin_tab, c->max_seq);
  RopeDev& r = c->rope[{cos_tab, sin_tab}];
  if (!r.cos) {
    HIP_OK(hipMalloc(&r.cos, (size_t)c->max_seq * 64 * 4));
    HIP_OK(hipMalloc(&r.sin, (size_t)c->max_seq * 64 * 4));
    r.uid = next_uid();
  }
  if (r.fp != fp) {
    HIP_OK(hipMemcpy(r.cos, cos_tab, (size_t)c->max_seq * 64 * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(r.sin, sin_tab, (size_t)c->max_seq * 64 * 4, hipMemcpyHostToDevice));
    r.fp = fp;
  }
  return r;
}

void check_handles(const ModelWeights* m, const KVCache* c, const DecoderScratch* s) {
  REQUIRE(m && c && s, "NULL handle");
  const int d = current_device();
  REQUIRE(m->dev == d && c->dev == d && s->dev == d, "handles live on another device");
  REQUIRE(s->max_seq >= c->max_seq, "scratch max_seq is smaller than the cache's");
  REQUIRE(m->num_layers() > 0, "no layer weights set");
}

void gemv(const tl_weights* W, const float* x, float* y, const float* bias, int epi, int norm,
          const float* norm_w, hipStream_t st) {
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
  L.norm_eps = EPS;
  HIP_OK(launch_gemv_i8(L, st));
}

// the six launches of each layer (see the file comment)
void enqueue_layers(const ModelWeights* m, const KVCache* c, DecoderScratch* s, const RopeDev& r,
                    hipStream_t st) {
  const int nl = m->num_layers();
  for (int l = 0; l < nl; l++) {
    const LayerDev& L = m->layers[l];
    gemv(L.qkv, s->hidden, s->qkv, nullptr, EPI_W8A32, NORM_DECODER, L.norms, st);
    AttnDecodeArgs a;
    a.qkv = s->qkv;
    a.q_norm = L.norms + 2 * H;
    a.k_norm = L.norms + 2 * H + HDIM;
    a.cos_tab = r.cos;
    a.sin_tab = r.sin;
    a.kc = c->k + (size_t)l * c->layer_floats();
    a.vc = c->v + (size_t)l * c->layer_floats();
    a.state = c->state;
    a.pm = s->pm;
    a.pl = s->pl;
    a.po = s->po;
    a.count = s->count;
    a.out = s->attn;
    a.nq = NQ;
    a.nkv = NKV;
    a.max_seq = c->max_seq;
    a.T = attn_chunk_size(c->max_seq);
    a.C = attn_chunks(c->max_seq);
    a.scale = SCALE;
    a.eps = EPS;
    HIP_OK(launch_attn_decode(a, st));
    gemv(L.o, s->attn, s->hidden, s->hidden, EPI_W8A32, NORM_NONE, nullptr, st);
    gemv(L.gu, s->hidden, s->mlp, nullptr, EPI_SWIGLU, NORM_DECODER, L.norms + H, st);
    gemv(L.down, s->mlp, s->hidden, s->hidden, EPI_W8A32, NORM_NONE, nullptr, st);
  }
}

void advance(KVCache* c, int n);

// prefill with the activation quantization / plane split fused into the
// RMSNorm and SwiGLU kernels (default), or each linear's own launch
// (tl_prefill_set_fused_quant)
bool g_prefill_fused_quant = true;

// Prefill of S tokens through every layer (decoder.c:33-157 with seq_len > 1):
// token t is rotated with rows t of cos_rows / sin_rows, its K/V go to cache
// row row0 + t, and it attends cache rows key0 .. key0 + qoff + t.
void enqueue_prefill(const ModelWeights* m, KVCache* c, DecoderScratch* s, int S, const float* cos_rows,
                     const float* sin_rows, int row0, int key0, int qoff, hipStream_t st) {
  float* Hd = static_cast<float*>(s->p_h.p);
  float* Xn = static_cast<float*>(s->p_xn.p);
  float* QKV = static_cast<float*>(s->p_qkv.p);
  float* ATT = static_cast<float*>(s->p_att.p);
  float* GU = static_cast<float*>(s->p_gu.p);
  float* MLP = static_cast<float*>(s->p_mlp.p);
  float* Y = static_cast<float*>(s->p_y.p);
  const long long n = (long long)S * H;
  // w8a32_linear at batch S (decoder.c), or W8A8 with per-token activation
  // codes.  The layer's two RMSNorms and the SwiGLU write their output rows
  // directly as the GEMM's activations (the fp32 rows are never stored): the
  // W8A8 codes and scales, or, for w8a32_linear's fp32 semantics, the four
  // int8 planes and exponents it splits a batch of more than 32 rows into
  // (S <= 32 keeps the fp32 rows: w8a32_linear takes other kernels there).
  // Only the attention output goes through its linear's own quantization.
  auto linear = m->prefill_w8a8 ? linear_w8a8 : linear_w8a32;
  const bool fused_q = g_prefill_fused_quant && (m->prefill_w8a8 || S > 32);
  uint8_t* Aq = static_cast<uint8_t*>(s->p_q.p);
  float* As = m->prefill_w8a8 ? static_cast<float*>(s->p_qs.p) : nullptr;
  int* Ae = m->prefill_w8a8 ? nullptr : static_cast<int*>(s->p_qs.p);
  auto linear_q = [&](const tl_weights* W, float* out) {
    if (m->prefill_w8a8) linear_w8a8_tiles(Aq, As, W, out, S, st);
    else linear_w8a32_planes(Aq, Ae, W, out, S, st);
  };
  for (int l = 0; l < m->num_layers(); l++) {
    const LayerDev& L = m->layers[l];
    float* kc = c->k + (size_t)l * c->layer_floats();
    float* vc = c->v + (size_t)l * c->layer_floats();
    if (fused_q) {
      HIP_OK(launch_rmsnorm_rows_q(Hd, L.norms, Aq, As, Ae, S, H, EPS, st));
      linear_q(L.qkv, QKV);
    } else {
      HIP_OK(launch_rmsnorm_rows(Hd, L.norms, Xn, S, H, EPS, st));
      linear(Xn, L.qkv, nullptr, QKV, S, st);
    }
    HIP_OK(launch_prefill_qk(QKV, L.norms + 2 * H, L.norms + 2 * H + HDIM, cos_rows, sin_rows, kc, vc, c->max_seq,
                             row0, S, NKV, EPS, st));
    HIP_OK(launch_flash_prefill(QKV, kc, vc, ATT, S, NQ, c->max_seq, key0, qoff, SCALE,
                                static_cast<float*>(s->p_fpart.p), static_cast<int*>(s->p_fcnt.p), st));
    linear(ATT, L.o, nullptr, Y, S, st);
    HIP_OK(launch_residual_add(Y, Hd, n, st));
    if (fused_q) {
      HIP_OK(launch_rmsnorm_rows_q(Hd, L.norms + H, Aq, As, Ae, S, H, EPS, st));
      linear_q(L.gu, GU);
      HIP_OK(launch_swiglu_rows_q(GU, Aq, As, Ae, S, FF, st));
      linear_q(L.down, Y);
    } else {
      HIP_OK(launch_rmsnorm_rows(Hd, L.norms + H, Xn, S, H, EPS, st));
      linear(Xn, L.gu, nullptr, GU, S, st);
      HIP_OK(launch_swiglu_rows(GU, MLP, S, FF, st));
      linear(MLP, L.down, nullptr, Y, S, st);
    }
    HIP_OK(launch_residual_add(Y, Hd, n, st));
  }
}

void ensure_prefill_buffers(DecoderScratch* s, int S) {
  s->p_h.ensure((size_t)S * H * 4, s->st);
  s->p_xn.ensure((size_t)S * H * 4, s->st);
  s->p_qkv.ensure((size_t)S * QKVD * 4, s->st);
  s->p_att.ensure((size_t)S * H * 4, s->st);
  s->p_gu.ensure((size_t)S * 2 * FF * 4, s->st);
  s->p_mlp.ensure((size_t)S * FF * 4, s->st);
  s->p_y.ensure((size_t)S * H * 4, s->st);
  s->p_q.ensure((size_t)cdiv(4 * S, 16) * 16 * FF, s->st);    // plane tiles of the widest input (K = FF)
  s->p_qs.ensure((size_t)cdiv(S, 16) * 16 * sizeof(float), s->st);
  s->p_fpart.ensure(flash_split_floats(S, NQ) * 4, s->st);
  const size_t cb = flash_split_counters(S, NQ) * sizeof(int);
  if (cb > s->p_fcnt.n) {
    s->p_fcnt.ensure(cb, s->st);
    HIP_OK(hipMemsetAsync(s->p_fcnt.p, 0, s->p_fcnt.n, s->st));   // ordered before the prefill kernels
  }
}

// host copy between the caller's (pageable) rows and the pinned staging
// buffer, split over up to 8 threads: a single-threaded copy runs at about a
// quarter of the PCIe rate, and it is what the runtime's own pageable path
// does chunk by chunk
void parallel_copy(void* dst, const void* src, size_t n) {
  constexpr size_t kPiece = (size_t)1 << 20;
  const unsigned hw = std::thread::hardware_concurrency();
  const size_t nt = std::min<size_t>({8, hw ? hw : 1, n / kPiece});
  if (nt <= 1) {
    std::memcpy(dst, src, n);
    return;
  }
  const size_t per = ((n + nt - 1) / nt + 63) & ~(size_t)63;
  std::vector<std::thread> th;
  for (size_t i = 1; i < nt && i * per < n; i++) {
    const size_t o = i * per;
    th.emplace_back([=] { std::memcpy(static_cast<char*>(dst) + o, static_cast<const char*>(src) + o, std::min(per, n - o)); });
  }
  std::memcpy(dst, src, std::min(per, n));
  for (auto& t : th) t.join();
}

// one prefill call on host hidden rows: chunks of at most `chunk` tokens
// (chunked mode: each attends to the whole cache), then the cache advances
void prefill_host(const ModelWeights* m, KVCache* c, float* hidden, DecoderScratch* s, int S, const float* cos_tab,
                  const float* sin_tab, const float* token_cos, const float* token_sin, int chunk, bool chunked) {
  check_handles(m, c, s);
  REQUIRE(hidden && S >= 1, "bad arguments");
  REQUIRE(c->seq_len + S <= c->max_seq, "KV cache too small for the prefill");
  const float* cos_dev = nullptr;
  const float* sin_dev = nullptr;
  if (token_cos) {
    REQUIRE(token_sin, "NULL token_sin");
    s->p_cos.ensure((size_t)S * 64 * 4, s->st);
    s->p_sin.ensure((size_t)S * 64 * 4, s->st);
    HIP_OK(hipMemcpyAsync(s->p_cos.p, token_cos, (size_t)S * 64 * 4, hipMemcpyHostToDevice, s->st));
    HIP_OK(hipMemcpyAsync(s->p_sin.p, token_sin, (size_t)S * 64 * 4, hipMemcpyHostToDevice, s->st));
    cos_dev = static_cast<const float*>(s->p_cos.p);
    sin_dev = static_cast<const float*>(s->p_sin.p);
  } else {
    const RopeDev& r = rope_device(c, cos_tab, sin_tab);
    cos_dev = r.cos;
    sin_dev = r.sin;
  }
  const int step = chunked ? std::max(1, chunk) : S;
  ensure_prefill_buffers(s, std::min(step, S));
  for (int t0 = 0; t0 < S; t0 += step) {
    const int n = std::min(step, S - t0);
    const int base = c->seq_len;
    const size_t rb = (size_t)n * H * 4;
    s->pin_rows.ensure(rb);
    parallel_copy(s->pin_rows.p, hidden + (size_t)t0 * H, rb);
    HIP_OK(hipMemcpyAsync(s->p_h.p, s->pin_rows.p, rb, hipMemcpyHostToDevice, s->st));
    // sequential positions: rows base + t of the tables; 3-D: rows t0 + t of the token tables
    const size_t rrow = token_cos ? (size_t)t0 : (size_t)base;
    enqueue_prefill(m, c, s, n, cos_dev + rrow * 64, sin_dev + rrow * 64, base, chunked ? 0 : base,
                    chunked ? base : 0, s->st);
    HIP_OK(hipMemcpyAsync(s->pin_rows.p, s->p_h.p, rb, hipMemcpyDeviceToHost, s->st));
    HIP_OK(hipStreamSynchronize(s->st));
    parallel_copy(hidden + (size_t)t0 * H, s->pin_rows.p, rb);
    advance(c, n);
  }
}

template <class F>
hipGraphExec_t capture(hipStream_t st, F&& enqueue) {
  HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  hipGraph_t g = nullptr;
  try {
    enqueue();
  } catch (...) {
    (void)hipStreamEndCapture(st, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  HIP_OK(hipStreamEndCapture(st, &g));
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  HIP_OK(e);
  return exec;
}

// pinned staging of a scratch: decode state at 0, a hidden row at 64
constexpr size_t kStageHidden = 64;

int rope_pos(const KVCache* c) { return c->rope_offset ? c->rope_offset : c->seq_len; }

// decode state from the host counters: position, rotary position, counter
void write_state(KVCache* c, DecoderScratch* s, int counter) {
  HIP_OK(hipStreamSynchronize(s->st));   // the staging buffer is idle
  int* h = static_cast<int*>(s->pin.p);
  h[0] = c->seq_len;
  h[1] = rope_pos(c);
  h[2] = counter;
  h[3] = 0;
  HIP_OK(hipMemcpyAsync(c->state, h, 4 * sizeof(int), hipMemcpyHostToDevice, s->st));
}

void advance(KVCache* c, int n) {   // kv_cache_advance (kernel/kv_cache.c:108-112)
  c->seq_len += n;
  if (c->rope_offset > 0) c->rope_offset += n;
}

void set_layer(ModelWeights* m, int l, const int8_t* q_w, const float* q_s, const int8_t* k_w, const float* k_s,
               const int8_t* v_w, const float* v_s, const int8_t* o_w, const float* o_s, const int8_t* gate_w,
               const float* gate_s, const int8_t* up_w, const float* up_s, const int8_t* down_w,
               const float* down_s, const float* input_ln, const float* post_attn_ln, const float* q_norm,
               const float* k_norm, const int8_t* qkv_w, const float* qkv_s) {
  REQUIRE(m, "NULL model");
  REQUIRE(l >= 0 && l < NL, "layer index out of range");
  REQUIRE(m->dev == current_device(), "model lives on another device");
  REQUIRE(o_w && o_s && gate_w && gate_s && up_w && up_s && down_w && down_s, "NULL weight pointer");
  REQUIRE(input_ln && post_attn_ln && q_norm && k_norm, "NULL norm pointer");
  REQUIRE((qkv_w && qkv_s) || (q_w && q_s && k_w && k_s && v_w && v_s), "NULL q/k/v pointer");
  LayerDev L;
  try {
    hipStream_t st = nullptr;
    if (qkv_w && qkv_s) {
      L.qkv = weights_from_codes(qkv_w, qkv_s, QKVD, H, false, st);
    } else {
      // Q||K||V rows (decoder.py:290-296): bit-identical to the separate GEMVs
      std::vector<int8_t> w((size_t)QKVD * H);
      std::vector<float> s(QKVD);
      std::memcpy(w.data(), q_w, (size_t)H * H);
      std::memcpy(w.data() + (size_t)H * H, k_w, (size_t)KVD * H);
      std::memcpy(w.data() + (size_t)(H + KVD) * H, v_w, (size_t)KVD * H);
      std::memcpy(s.data(), q_s, H * 4);
      std::memcpy(s.data() + H, k_s, KVD * 4);
      std::memcpy(s.data() + H + KVD, v_s, KVD * 4);
      L.qkv = weights_from_codes(w.data(), s.data(), QKVD, H, false, st);
    }
    L.o = weights_from_codes(o_w, o_s, H, H, false, st);
    {
      // gate and up interleaved per 16-row group: rows 16b..16b+7 are gate
      // rows 8b.., rows 16b+8.. the up rows 8b.. (EPI_SWIGLU)
      std::vector<int8_t> w((size_t)2 * FF * H);
      std::vector<float> s(2 * FF);
      for (int b = 0; b < FF / 8; b++) {
        std::memcpy(w.data() + (size_t)(16 * b) * H, gate_w + (size_t)(8 * b) * H, (size_t)8 * H);
        std::memcpy(w.data() + (size_t)(16 * b + 8) * H, up_w + (size_t)(8 * b) * H, (size_t)8 * H);
        std::memcpy(s.data() + 16 * b, gate_s + 8 * b, 8 * 4);
        std::memcpy(s.data() + 16 * b + 8, up_s + 8 * b, 8 * 4);
      }
      L.gu = weights_from_codes(w.data(), s.data(), 2 * FF, H, false, st);
    }
    L.down = weights_from_codes(down_w, down_s, H, FF, false, st);
    HIP_OK(hipMalloc(&L.norms, (size_t)(2 * H + 2 * HDIM) * 4));
    HIP_OK(hipMemcpy(L.norms, input_ln, H * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(L.norms + H, post_attn_ln, H * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(L.norms + 2 * H, q_norm, HDIM * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(L.norms + 2 * H + HDIM, k_norm, HDIM * 4, hipMemcpyHostToDevice));
  } catch (...) {
    L.release();
    throw;
  }
  m->layers[l].release();
  m->layers[l] = L;
  m->version = next_uid();
}

}  // namespace

extern "C" {

// ---- handles (decoder.c:320-366) -----------------------------------------
ModelWeights* decoder_model_alloc(void) {
  ModelWeights* m = nullptr;
  guarded("decoder_model_alloc", [&] {
    m = new ModelWeights();
    m->dev = current_device();
  });
  return m;
}

void decoder_model_free(ModelWeights* m) {
  if (!m) return;
  for (auto& L : m->layers) L.release();
  delete m;
}

KVCache* decoder_cache_alloc(int max_seq) {
  KVCache* c = nullptr;
  guarded("decoder_cache_alloc", [&] {
    REQUIRE(max_seq >= 1, "max_seq must be >= 1");
    std::unique_ptr<KVCache> p(new KVCache());
    p->dev = current_device();
    p->max_seq = max_seq;
    const size_t bytes = (size_t)NL * p->layer_floats() * sizeof(float);
    HIP_OK(hipMalloc(&p->k, bytes));
    HIP_OK(hipMalloc(&p->v, bytes));
    HIP_OK(hipMalloc(&p->state, 4 * sizeof(int)));
    // null stream, completed before return: the kernels run on other streams
    HIP_OK(hipMemsetAsync(p->state, 0, 4 * sizeof(int), nullptr));
    HIP_OK(hipStreamSynchronize(nullptr));
    c = p.release();
  });
  return c;
}

void decoder_cache_free(KVCache* c) {
  if (!c) return;
  if (c->k) (void)hipFree(c->k);
  if (c->v) (void)hipFree(c->v);
  if (c->state) (void)hipFree(c->state);
  for (auto& kv : c->rope) {
    if (kv.second.cos) (void)hipFree(kv.second.cos);
    if (kv.second.sin) (void)hipFree(kv.second.sin);
  }
  delete c;
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

DecoderScratch* decoder_scratch_alloc_fn(int max_seq) {
  DecoderScratch* s = nullptr;
  guarded("decoder_scratch_alloc_fn", [&] {
    REQUIRE(max_seq >= 1, "max_seq must be >= 1");
    std::unique_ptr<DecoderScratch> p(new DecoderScratch());
    p->dev = current_device();
    p->max_seq = max_seq;
    p->C = attn_chunks(max_seq);
    HIP_OK(hipStreamCreateWithFlags(&p->st, hipStreamNonBlocking));
    HIP_OK(hipMalloc(&p->hidden, (size_t)H * 4));
    HIP_OK(hipMalloc(&p->qkv, (size_t)QKVD * 4));
    HIP_OK(hipMalloc(&p->mlp, (size_t)FF * 4));
    HIP_OK(hipMalloc(&p->attn, (size_t)H * 4));
    HIP_OK(hipMalloc(&p->pm, (size_t)NQ * p->C * 4));
    HIP_OK(hipMalloc(&p->pl, (size_t)NQ * p->C * 4));
    HIP_OK(hipMalloc(&p->po, (size_t)NQ * p->C * HDIM * 4));
    HIP_OK(hipMalloc(&p->count, (size_t)NKV * sizeof(int)));
    HIP_OK(hipMemsetAsync(p->count, 0, (size_t)NKV * sizeof(int), p->st));
    HIP_OK(hipStreamSynchronize(p->st));
    p->pin.ensure(kStageHidden + (size_t)H * 4);
    s = p.release();
  });
  return s;
}

void decoder_scratch_free_fn(DecoderScratch* s) {
  if (!s) return;
  if (s->st) (void)hipStreamSynchronize(s->st);
  drop_graph(s->layers_exec);
  drop_graph(s->gen_exec);
  for (float* p : {s->hidden, s->qkv, s->attn, s->mlp})
    if (p) (void)hipFree(p);
  for (float* p : {s->pm, s->pl, s->po})
    if (p) (void)hipFree(p);
  if (s->count) (void)hipFree(s->count);
  for (DevBuf* b : {&s->p_h, &s->p_xn, &s->p_qkv, &s->p_att, &s->p_gu, &s->p_mlp, &s->p_y, &s->p_cos, &s->p_sin,
                    &s->p_q, &s->p_qs,
                    &s->p_fpart, &s->p_fcnt})
    if (b->p) (void)hipFree(b->p);
  if (s->keys.p) (void)hipFree(s->keys.p);
  if (s->tokens.p) (void)hipFree(s->tokens.p);
  if (s->fnorm.p) (void)hipFree(s->fnorm.p);
  if (s->pin.p) (void)hipHostFree(s->pin.p);
  if (s->pin_rows.p) (void)hipHostFree(s->pin_rows.p);
  if (s->st) (void)hipStreamDestroy(s->st);
  delete s;
}

// ---- weights (decoder.c:368-423) -------------------------------------------
void decoder_set_layer_weights(ModelWeights* model, int layer_idx, const int8_t* q_w, const float* q_s,
                               const int8_t* k_w, const float* k_s, const int8_t* v_w, const float* v_s,
                               const int8_t* o_w, const float* o_s, const int8_t* gate_w, const float* gate_s,
                               const int8_t* up_w, const float* up_s, const int8_t* down_w, const float* down_s,
                               const float* input_ln, const float* post_attn_ln, const float* q_norm,
                               const float* k_norm) {
  guarded("decoder_set_layer_weights", [&] {
    set_layer(model, layer_idx, q_w, q_s, k_w, k_s, v_w, v_s, o_w, o_s, gate_w, gate_s, up_w, up_s, down_w,
              down_s, input_ln, post_attn_ln, q_norm, k_norm, nullptr, nullptr);
  });
}

void decoder_set_layer_weights_v32(ModelWeights* model, int layer_idx, const int8_t* q_w, const float* q_s,
                                   const int8_t* k_w, const float* k_s, const int8_t* v_w, const float* v_s,
                                   const int8_t* o_w, const float* o_s, const int8_t* gate_w,
                                   const float* gate_s, const int8_t* up_w, const float* up_s,
                                   const int8_t* down_w, const float* down_s, const float* input_ln,
                                   const float* post_attn_ln, const float* q_norm, const float* k_norm,
                                   const int8_t* qkv_w, const float* qkv_s, const int8_t* gate_up_w,
                                   const float* gate_up_s) {
  (void)gate_up_w;   // gate and up are re-laid out from the separate matrices
  (void)gate_up_s;
  guarded("decoder_set_layer_weights_v32", [&] {
    set_layer(model, layer_idx, q_w, q_s, k_w, k_s, v_w, v_s, o_w, o_s, gate_w, gate_s, up_w, up_s, down_w,
              down_s, input_ln, post_attn_ln, q_norm, k_norm, qkv_w, qkv_s);
  });
}

// ---- rope tables (decoder.c:494-503 -> ops.c:150-177) ------------------------
void decoder_precompute_rope(float* cos_tab, float* sin_tab, int max_seq, int head_dim, const int sections[3],
                             const float theta_bases[3]) {
  (void)sections;   // sequential positions: every section has the same angle
  guarded("decoder_precompute_rope", [&] {
    REQUIRE(cos_tab && sin_tab && theta_bases && max_seq >= 1 && head_dim >= 2, "bad arguments");
    const int half = head_dim / 2;
    for (int pos = 0; pos < max_seq; pos++)
      for (int j = 0; j < half; j++) {
        const float inv_freq = 1.0f / powf(theta_bases[0], (float)(2 * j) / (float)head_dim);
        const float angle = (float)pos * inv_freq;
        cos_tab[(size_t)pos * half + j] = cosf(angle);
        sin_tab[(size_t)pos * half + j] = sinf(angle);
      }
  });
}

// ---- one decode step on a host hidden row (decoder.c:452-462) ---------------
void decoder_decode_step(const ModelWeights* model, KVCache* cache, float* hidden, DecoderScratch* scratch,
                         const float* cos_tab, const float* sin_tab) {
  guarded("decoder_decode_step", [&] {
    check_handles(model, cache, scratch);
    REQUIRE(hidden, "NULL hidden");
    REQUIRE(cache->seq_len < cache->max_seq, "KV cache is full");
    REQUIRE(rope_pos(cache) < cache->max_seq, "rotary position past the rope tables");
    DecoderScratch* s = scratch;
    const RopeDev& r = rope_device(cache, cos_tab, sin_tab);
    const uint64_t key[4] = {model->version, cache->uid, r.uid, (uint64_t)model->num_layers()};
    if (!s->layers_exec || std::memcmp(key, s->layers_key, sizeof key)) {
      drop_graph(s->layers_exec);
      s->layers_exec = capture(s->st, [&] { enqueue_layers(model, cache, s, r, s->st); });
      std::memcpy(s->layers_key, key, sizeof key);
    }
    write_state(cache, s, 0);   // also leaves the stream idle
    char* stage = static_cast<char*>(s->pin.p) + kStageHidden;
    std::memcpy(stage, hidden, (size_t)H * 4);
    HIP_OK(hipMemcpyAsync(s->hidden, stage, (size_t)H * 4, hipMemcpyHostToDevice, s->st));
    HIP_OK(hipGraphLaunch(s->layers_exec, s->st));
    HIP_OK(hipMemcpyAsync(stage, s->hidden, (size_t)H * 4, hipMemcpyDeviceToHost, s->st));
    HIP_OK(hipStreamSynchronize(s->st));
    std::memcpy(hidden, stage, (size_t)H * 4);
    advance(cache, 1);
  });
}

// ---- prefill (decoder.c:437-507) --------------------------------------------
void decoder_prefill_step(const ModelWeights* model, KVCache* cache, float* hidden, DecoderScratch* scratch,
                          const float* cos_tab, const float* sin_tab, int seq_len) {
  guarded("decoder_prefill_step", [&] {
    REQUIRE(cache, "NULL cache");
    REQUIRE(cache->seq_len + seq_len <= cache->max_seq, "rotary positions past the rope tables");
    prefill_host(model, cache, hidden, scratch, seq_len, cos_tab, sin_tab, nullptr, nullptr, 0, false);
  });
}

void decoder_chunked_prefill_step(const ModelWeights* model, KVCache* cache, float* hidden, DecoderScratch* scratch,
                                  const float* cos_tab, const float* sin_tab, int total_seq_len, int chunk_size) {
  guarded("decoder_chunked_prefill_step", [&] {
    REQUIRE(cache, "NULL cache");
    REQUIRE(chunk_size >= 1, "chunk_size must be >= 1");
    REQUIRE(cache->seq_len + total_seq_len <= cache->max_seq, "rotary positions past the rope tables");
    prefill_host(model, cache, hidden, scratch, total_seq_len, cos_tab, sin_tab, nullptr, nullptr, chunk_size, true);
  });
}

void decoder_hybrid_chunked_prefill_step(const ModelWeights* model, KVCache* cache, float* hidden,
                                         DecoderScratch* scratch, const float* cos_tab, const float* sin_tab,
                                         int seq_len, int chunk_size) {
  (void)chunk_size;   // the reference chunks only its GEMMs; the results are those of one pass
  guarded("decoder_hybrid_chunked_prefill_step", [&] {
    REQUIRE(cache, "NULL cache");
    REQUIRE(cache->seq_len + seq_len <= cache->max_seq, "rotary positions past the rope tables");
    prefill_host(model, cache, hidden, scratch, seq_len, cos_tab, sin_tab, nullptr, nullptr, 0, false);
  });
}

void decoder_prefill_step_3d(const ModelWeights* model, KVCache* cache, float* hidden, DecoderScratch* scratch,
                             const float* token_cos, const float* token_sin, int seq_len) {
  guarded("decoder_prefill_step_3d", [&] {
    REQUIRE(token_cos && token_sin, "NULL token tables");
    prefill_host(model, cache, hidden, scratch, seq_len, nullptr, nullptr, token_cos, token_sin, 0, false);
  });
}

// mrope_build_cos_sin_3d (ops.c:188-223): dims j < 3 min(sections[1],
// sections[2]) take the T / H / W position j % 3, the rest T
void decoder_build_rope_3d(float* cos_out, float* sin_out, const int* pos_ids, int seq_len, int head_dim,
                           const int sections[3], const float theta_bases[3]) {
  guarded("decoder_build_rope_3d", [&] {
    REQUIRE(cos_out && sin_out && pos_ids && sections && theta_bases && seq_len >= 1 && head_dim >= 2,
            "bad arguments");
    const int half = head_dim / 2;
    const int min_s = std::min(sections[1], sections[2]);
    for (int t = 0; t < seq_len; t++)
      for (int j = 0; j < half; j++) {
        const int sect = j < 3 * min_s ? j % 3 : 0;
        const int pos = pos_ids[sect * seq_len + t];
        const float inv_freq = 1.0f / powf(theta_bases[0], (float)(2 * j) / (float)head_dim);
        const float angle = (float)pos * inv_freq;
        cos_out[(size_t)t * half + j] = cosf(angle);
        sin_out[(size_t)t * half + j] = sinf(angle);
      }
  });
}

// ==========================================================================
// Part 2 extensions
// ==========================================================================
int tl_decoder_num_layers(const ModelWeights* model) { return model ? model->num_layers() : -1; }


int tl_decoder_read_cache(const KVCache* cache, int layer, float* k, float* v) {
  return guarded("tl_decoder_read_cache", [&] {
    REQUIRE(cache && layer >= 0 && layer < NL, "bad arguments");
    REQUIRE(cache->dev == current_device(), "cache lives on another device");
    const size_t n = cache->layer_floats();
    if (k) HIP_OK(hipMemcpy(k, cache->k + (size_t)layer * n, n * 4, hipMemcpyDeviceToHost));
    if (v) HIP_OK(hipMemcpy(v, cache->v + (size_t)layer * n, n * 4, hipMemcpyDeviceToHost));
  });
}

int tl_decoder_cache_len(const KVCache* cache) { return cache ? cache->seq_len : -1; }

int tl_prefill_set_fused_quant(int on) {
  return guarded("tl_prefill_set_fused_quant", [&] {
    REQUIRE(on == 0 || on == 1, "on must be 0 or 1");
    g_prefill_fused_quant = on != 0;
  });
}

int tl_decoder_set_prefill_w8a8(ModelWeights* model, int on) {
  return guarded("tl_decoder_set_prefill_w8a8", [&] {
    REQUIRE(model, "NULL model");
    model->prefill_w8a8 = on != 0;
  });
}

int tl_decoder_generate(const ModelWeights* model, KVCache* cache, DecoderScratch* scratch,
                        const tl_weights* lm_head, const float* final_norm, const float* embed, int first_token,
                        int n_steps, int32_t* tokens, const float* cos_tab, const float* sin_tab) {
  return guarded("tl_decoder_generate", [&] {
    check_handles(model, cache, scratch);
    check_weights(lm_head);
    REQUIRE(embed && tokens && n_steps >= 1, "bad arguments");
    REQUIRE(lm_head->cols == H, "lm_head must have hidden-size columns");
    REQUIRE(first_token >= 0 && first_token < lm_head->rows, "first_token out of range");
    REQUIRE(cache->seq_len + n_steps <= cache->max_seq, "KV cache too small for n_steps");
    REQUIRE(rope_pos(cache) + n_steps <= cache->max_seq, "rotary positions past the rope tables");
    DecoderScratch* s = scratch;
    const RopeDev& r = rope_device(cache, cos_tab, sin_tab);
    const GemvPlan plan = gemv_plan(lm_head->rows, H);
    s->keys.ensure((size_t)plan.blocks * sizeof(uint64_t), s->st);
    s->tokens.ensure((size_t)n_steps * sizeof(int32_t), s->st);
    s->fnorm.ensure((size_t)H * 4, s->st);
    const float* fn = nullptr;
    if (final_norm) {
      HIP_OK(hipMemcpyAsync(s->fnorm.p, final_norm, (size_t)H * 4, hipMemcpyHostToDevice, s->st));
      fn = static_cast<const float*>(s->fnorm.p);
    }
    const int max_tokens = (int)(s->tokens.n / sizeof(int32_t));
    // embed is the caller's device pointer: its contents are read at replay
    const uint64_t key[9] = {model->version,
                             cache->uid,
                             r.uid,
                             lm_head->uid,
                             (uint64_t)(uintptr_t)fn,
                             (uint64_t)(uintptr_t)embed,
                             (uint64_t)(uintptr_t)s->tokens.p,
                             (uint64_t)(uintptr_t)s->keys.p,
                             (uint64_t)model->num_layers() * 1000003u + (uint64_t)max_tokens};
    if (!s->gen_exec || std::memcmp(key, s->gen_key, sizeof key)) {
      drop_graph(s->gen_exec);
      s->gen_exec = capture(s->st, [&] {
        enqueue_layers(model, cache, s, r, s->st);
        GemvLaunch L;
        L.x = s->hidden;
        L.wt = lm_head->tiles;
        L.ws = lm_head->scales;
        L.N = lm_head->rows;
        L.K = H;
        L.epi = EPI_ARGMAX;
        L.keys = static_cast<uint64_t*>(s->keys.p);
        L.norm = NORM_NUMPY;
        L.norm_w = fn;
        HIP_OK(launch_gemv_i8(L, s->st));
        HIP_OK(launch_step_end(static_cast<const uint64_t*>(s->keys.p), plan.blocks, embed, H, s->hidden,
                               cache->state, static_cast<int32_t*>(s->tokens.p), max_tokens, s->st));
      });
      std::memcpy(s->gen_key, key, sizeof key);
    }
    write_state(cache, s, 0);
    HIP_OK(hipMemcpyAsync(s->hidden, embed + (size_t)first_token * H, (size_t)H * 4, hipMemcpyDeviceToDevice,
                          s->st));
    for (int i = 0; i < n_steps; i++) HIP_OK(hipGraphLaunch(s->gen_exec, s->st));
    HIP_OK(hipMemcpyAsync(tokens, s->tokens.p, (size_t)n_steps * sizeof(int32_t), hipMemcpyDeviceToHost, s->st));
    HIP_OK(hipStreamSynchronize(s->st));
    advance(cache, n_steps);
  });
}

// ---- attention test hooks -----------------------------------------------------
int tl_attn_decode_dev(const float* qkv, const float* q_norm, const float* k_norm, const float* cos_tab,
                       const float* sin_tab, float* k_cache, float* v_cache, int max_seq, int pos, int rope_pos,
                       float* out, void* stream) {
  return guarded("tl_attn_decode_dev", [&] {
    REQUIRE(qkv && q_norm && k_norm && cos_tab && sin_tab && k_cache && v_cache && out, "NULL argument");
    REQUIRE(max_seq >= 1 && pos >= 0 && pos < max_seq && rope_pos >= 0 && rope_pos < max_seq, "bad positions");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int C = attn_chunks(max_seq);
    DevBuf ws;
    const size_t part = (size_t)NQ * C * (2 + HDIM) * sizeof(float);
    ws.ensure(part + 64 + (size_t)NKV * sizeof(int), st);
    struct Free {   // the stream drains before the work-space goes, also on errors
      DevBuf& b;
      hipStream_t st;
      ~Free() {
        (void)hipStreamSynchronize(st);
        if (b.p) (void)hipFree(b.p);
      }
    } guard{ws, st};
    char* base = static_cast<char*>(ws.p);
    int* state = reinterpret_cast<int*>(base + part);
    int* count = reinterpret_cast<int*>(base + part + 64);
    const int hs[4] = {pos, rope_pos, 0, 0};
    HIP_OK(hipMemsetAsync(count, 0, (size_t)NKV * sizeof(int), st));
    HIP_OK(hipMemcpyAsync(state, hs, sizeof hs, hipMemcpyHostToDevice, st));
    AttnDecodeArgs a;
    a.qkv = qkv;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.cos_tab = cos_tab;
    a.sin_tab = sin_tab;
    a.kc = k_cache;
    a.vc = v_cache;
    a.state = state;
    a.pm = reinterpret_cast<float*>(base);
    a.pl = a.pm + (size_t)NQ * C;
    a.po = a.pl + (size_t)NQ * C;
    a.count = count;
    a.out = out;
    a.nq = NQ;
    a.nkv = NKV;
    a.max_seq = max_seq;
    a.T = attn_chunk_size(max_seq);
    a.C = C;
    a.scale = SCALE;
    a.eps = EPS;
    HIP_OK(launch_attn_decode(a, st));
    HIP_OK(hipStreamSynchronize(st));
  });
}

int tl_attn_prefill_dev(const float* qkv, const float* k_cache, const float* v_cache, float* out, int S,
                        int max_seq, int key0, int qoff, int split, void* stream) {
  return guarded("tl_attn_prefill_dev", [&] {
    REQUIRE(qkv && k_cache && v_cache && out, "NULL argument");
    REQUIRE(S >= 1 && key0 >= 0 && qoff >= 0 && key0 + qoff + S <= max_seq, "bad sizes");
    hipStream_t st = static_cast<hipStream_t>(stream);
    DevBuf part, cnt;
    struct Free {   // the stream drains before the work-space goes, also on errors
      DevBuf& a;
      DevBuf& b;
      hipStream_t st;
      ~Free() {
        (void)hipStreamSynchronize(st);
        if (a.p) (void)hipFree(a.p);
        if (b.p) (void)hipFree(b.p);
      }
    } guard{part, cnt, st};
    if (split) {
      part.ensure(flash_split_floats(S, NQ) * 4, st);
      cnt.ensure(flash_split_counters(S, NQ) * sizeof(int), st);
      HIP_OK(hipMemsetAsync(cnt.p, 0, cnt.n, st));
    }
    HIP_OK(launch_flash_prefill(qkv, k_cache, v_cache, out, S, NQ, max_seq, key0, qoff, SCALE,
                                static_cast<float*>(part.p), static_cast<int*>(cnt.p), st));
    HIP_OK(hipStreamSynchronize(st));
  });
}

}  // extern "C"
