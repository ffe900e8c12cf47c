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
#include "tl_common.h"
#include "tl_kernels.h"

#include <mutex>

namespace tl {

constexpr int kRmsMaxK = TLK_RMS_MAX_K;

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

// --------------------------------------------------------------------------
// The no-allocation work-space of tl_lm_head_argmax_noalloc_dev (api.c): a
// file-scope device array for callers that cannot allocate (HIP graph
// capture, serving loops).  It holds the argmax keys of up to
// TLK_NA_MAX_ROWS lm_head rows (16-row work-groups) and one normalised row of
// kRmsMaxK floats.  Every device the library runs on keeps its own copy until
// the process ends; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (the array's name is a
// host-side stand-in, not a device address), looked up once per device here.
// Nothing in it needs to start at zero: each call writes every key and
// element it reads.  Calls that overlap on one device share the array and
// race.
// --------------------------------------------------------------------------
namespace {
constexpr size_t kNaBytes = (size_t)TLK_NA_KEY_BYTES + (size_t)tl::kRmsMaxK * sizeof(float);   // 192 KiB
constexpr int kNaMaxDevices = 64;
static_assert((size_t)TLK_NA_KEY_BYTES == (size_t)TLK_NA_MAX_ROWS / 16 * sizeof(uint64_t), "key bytes");
}  // namespace

static __device__ __align__(256) uint8_t scratch[kNaBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kNaMaxDevices] = {};
}  // namespace

extern "C" {
hipError_t tlk_launch_rmsnorm_np(const float* h, const float* w, float* out, int K, float eps, hipStream_t st) {
  return tl::launch_rmsnorm_np(h, w, out, K, eps, st);
}
hipError_t tlk_launch_argmax_keys(const uint64_t* keys, int n, int32_t* token, float* value, hipStream_t st) {
  return tl::launch_argmax_keys(keys, n, token, value, st);
}
// the device address of `scratch` on device `dev` (current), looked up once
hipError_t tlk_noalloc_workspace(int dev, uint8_t** base) {
  if (dev < 0 || dev >= kNaMaxDevices || !base) return hipErrorInvalidValue;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *base = static_cast<uint8_t*>(g_scratch_ptr[dev]);
  return hipSuccess;
}
}  // extern "C"
