// lmhead.hip -- the steps around the lm_head GEMV of a greedy decode step.
//
// Reference: decoder.py:443-464 (_get_logits + the greedy branch of _sample):
//   h      = last hidden row (float32 [K])
//   rms    = np.sqrt(np.mean(h * h) + 1e-6)          (numpy, float32)
//   x      = (h / rms) * final_norm_w                (float32)
//   logits = w8a32_linear(x, lm_head, batch=1)
//   token  = argmax(logits)                          (first index of the max)
//
// rmsnorm_np_kernel reproduces numpy's float32 arithmetic exactly: np.mean of
// a contiguous float32 vector is numpy's pairwise sum (blocks of 128 summed
// with 8 interleaved accumulators, ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), and
// the halves of longer ranges added recursively) divided by K in float32;
// the epsilon is added in float32 (a Python float meets a float32 scalar).
// For K = 128 * 2^j every leaf is a full 128-block and the recursion is a
// balanced binary tree over the blocks, which is what is built here.  (The
// argmax keys must be 16-byte aligned: they are read two per load.)
//
// The GEMV's EPI_ARGMAX epilogue leaves one key per work-group (tl_common.h
// argmax_key); argmax_keys_kernel reduces them to the token.
#include "host.h"
#include "tl_common.h"
#include "tl_kernels.h"

#include <mutex>

namespace tl {

constexpr int kRmsMaxK = 16384;

// One work-group.  Thread p = 8b + j owns accumulator j of block b: its 16
// terms x[128b + 8i + j]^2 are loaded at once and added in order i = 0..15.
// The 8 accumulators of a block are 8 consecutive lanes, and the 8 blocks of
// a wave are 8 consecutive lane groups, so xor butterflies over lanes 1, 2, 4
// (within a block) and 8, 16, 32 (across blocks) are exactly numpy's
// combination order (IEEE addition commutes); groups of 8 blocks meet in a
// balanced tree in LDS.  Lanes past the last block add +0, which changes no
// sum of squares.
__global__ __launch_bounds__(256) void rmsnorm_np_kernel(const float* __restrict__ h,
                                                         const float* __restrict__ w,
                                                         float* __restrict__ out, int K, float eps) {
  __shared__ float s_grp[kRmsMaxK / 1024];   // one partial per 8 blocks
  __shared__ float s_rms;
  const int nb = K >> 7;
  const int ngrp = nb >= 8 ? nb >> 3 : 1;
  for (int base = 0; base < 8 * (ngrp * 8); base += 256) {
    const int p = base + threadIdx.x;
    const int b = p >> 3, j = p & 7;
    float r = 0.0f;
    if (b < nb) {
      const float* src = h + 128 * b + j;
      float v[16];
#pragma unroll
      for (int i = 0; i < 16; i++) v[i] = src[8 * i];
      r = __fmul_rn(v[0], v[0]);
#pragma unroll
      for (int i = 1; i < 16; i++) r = __fadd_rn(r, __fmul_rn(v[i], v[i]));
    }
    r = wave_sum(r);   // numpy's xor-butterfly order, through DPP (see final_rmsnorm in gemv.hip)
    if ((threadIdx.x & 63) == 0 && (p >> 6) < ngrp) s_grp[p >> 6] = r;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    // balanced tree over the groups of 8 blocks (a power of two of them)
    for (int wdt = 1; wdt < ngrp; wdt <<= 1)
      for (int i = 0; i < ngrp; i += 2 * wdt) s_grp[i] = __fadd_rn(s_grp[i], s_grp[i + wdt]);
    const float mean = __fdiv_rn(s_grp[0], (float)K);
    // sqrtf is correctly rounded here (the default correctly rounded fp32
    // divide/sqrt); __fsqrt_rn measured 15% of results one ulp off
    s_rms = sqrtf(__fadd_rn(mean, eps));
  }
  __syncthreads();
  const float rms = s_rms;
  for (int i = threadIdx.x; i < K; i += 256) {
    const float v = __fdiv_rn(h[i], rms);
    out[i] = w ? __fmul_rn(v, w[i]) : v;
  }
}

// one work-group: the largest key, decoded to (index, value); keys are read
// two per 16-byte load, several loads in flight per thread
__global__ __launch_bounds__(1024) void argmax_keys_kernel(const uint64_t* __restrict__ keys, int n,
                                                           int32_t* __restrict__ token, float* __restrict__ value) {
  __shared__ uint64_t s_k[16];
  uint64_t k = 0;
  const int n2 = n >> 1;
  const ulonglong2* k2 = reinterpret_cast<const ulonglong2*>(keys);
  for (int i0 = threadIdx.x; i0 < n2; i0 += 1024 * 8) {
    ulonglong2 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = i0 + 1024 * u;
      v[u] = i < n2 ? k2[i] : make_ulonglong2(0, 0);
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      k = v[u].x > k ? v[u].x : k;
      k = v[u].y > k ? v[u].y : k;
    }
  }
  if ((n & 1) && threadIdx.x == 0) k = keys[n - 1] > k ? keys[n - 1] : k;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t t = __shfl_xor(k, o, 64);
    k = t > k ? t : k;
  }
  if ((threadIdx.x & 63) == 0) s_k[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 16; i++) k = s_k[i] > k ? s_k[i] : k;
    *token = argmax_key_index(k);
    if (value) *value = argmax_key_value(k);
  }
}

hipError_t launch_rmsnorm_np(const float* h, const float* w, float* out, int K, float eps, hipStream_t st) {
  if (K < 128 || K > kRmsMaxK || (K & (K - 1)) != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rmsnorm_np_kernel, dim3(1), dim3(256), 0, st, h, w, out, K, eps);
  return hipGetLastError();
}

hipError_t launch_argmax_keys(const uint64_t* keys, int n, int32_t* token, float* value, hipStream_t st) {
  if (n < 1 || !token) return hipErrorInvalidValue;
  hipLaunchKernelGGL(argmax_keys_kernel, dim3(1), dim3(1024), 0, st, keys, n, token, value);
  return hipGetLastError();
}

}  // namespace tl

namespace tlhost {
using namespace tl;

size_t lm_head_argmax_keys(int N, int K) { return (size_t)gemv_plan(N, K).blocks; }

// The greedy step's launches on caller-provided work-space: keys (one 8-byte
// key per GEMV work-group, 16-byte aligned) and xn (K floats, used only when
// the final RMSNorm cannot run inside the GEMV's prologue).
void lm_head_argmax_enqueue(const float* h, const float* norm_w, const tl_weights* W, float* logits,
                            int32_t* token, float* max_logit, uint64_t* keys, float* xn, hipStream_t st) {
  const int K = W->cols;
  REQUIRE(K >= 128 && K <= kRmsMaxK && (K & (K - 1)) == 0, "K must be a power of two in [128, 16384]");
  GemvLaunch L;
  if (gemv_fused_norm_ok(K, h, norm_w)) {
    // every GEMV work-group normalises the row itself: one launch fewer
    L.x = h;
    L.norm = NORM_NUMPY;
    L.norm_w = norm_w;
  } else {
    HIP_OK(launch_rmsnorm_np(h, norm_w, xn, K, 1e-6f, st));
    L.x = xn;
  }
  L.wt = W->tiles;
  L.ws = W->scales;
  L.y = logits;
  L.keys = keys;
  L.N = W->rows;
  L.K = K;
  L.epi = EPI_ARGMAX;
  HIP_OK(launch_gemv_i8(L, st));
  HIP_OK(launch_argmax_keys(keys, (int)lm_head_argmax_keys(W->rows, K), token, max_logit, st));
}

}  // namespace tlhost

// --------------------------------------------------------------------------
// tl_lm_head_argmax_noalloc_dev: the greedy step with its work-space in a
// file-scope device array, for callers that cannot allocate (HIP graph
// capture, serving loops).  The array holds the argmax keys of up to
// kNaMaxRows lm_head rows (16-row work-groups) and one normalised row of
// kRmsMaxK floats.  Every device the library runs on keeps its own copy
// until the process ends; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (the array's name is a
// host-side stand-in, not a device address).  Nothing in it needs to start
// at zero: each call writes every key and element it reads.  Calls that
// overlap on one device share the array and race.
// --------------------------------------------------------------------------
namespace {
constexpr int kNaMaxRows = 262144;
constexpr size_t kNaKeyBytes = (size_t)kNaMaxRows / 16 * sizeof(uint64_t);   // 128 KiB
constexpr size_t kNaBytes = kNaKeyBytes + (size_t)tl::kRmsMaxK * sizeof(float);   // + 64 KiB
constexpr int kNaMaxDevices = 64;
}  // namespace

static __device__ __align__(256) uint8_t scratch[kNaBytes];

namespace {
using tlhost::Fail;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kNaMaxDevices] = {};

// the device address of `scratch` on the current device, looked up once per device
uint8_t* scratch_on(int dev) {
  REQUIRE(dev >= 0 && dev < kNaMaxDevices, "device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    HIP_OK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    REQUIRE(p != nullptr, "hipGetSymbolAddress returned NULL for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  return static_cast<uint8_t*>(g_scratch_ptr[dev]);
}
}  // namespace

extern "C" int tl_lm_head_argmax_noalloc_dev(const float* h, const float* norm_w, const tl_weights* W,
                                             float* logits, int32_t* token, float* max_logit, void* stream) {
  using namespace tlhost;
  return guarded("tl_lm_head_argmax_noalloc_dev", [&] {
    check_weights(W);
    REQUIRE(h && token, "h and token must be non-NULL");
    REQUIRE(W->rows <= kNaMaxRows, "lm_head has more rows than the no-allocation work-space holds (262144)");
    REQUIRE(lm_head_argmax_keys(W->rows, W->cols) * sizeof(uint64_t) <= kNaKeyBytes,
            "the GEMV plan needs more argmax keys than the no-allocation work-space holds");
    uint8_t* base = scratch_on(W->dev);
    lm_head_argmax_enqueue(h, norm_w, W, logits, token, max_logit, reinterpret_cast<uint64_t*>(base),
                           reinterpret_cast<float*>(base + kNaKeyBytes), static_cast<hipStream_t>(stream));
  });
}
