// host.h -- host-side plumbing shared by the C-ABI sources (api.cpp,
// decoder.cpp): the device weight handle, error capture, device buffers and
// weight packing.  Internal to the library.
#pragma once
#include "../../include/typhoon_linear.h"
#include "tl_kernels.h"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <exception>
#include <string>

struct tl_weights {
  int dev = -1;
  int rows = 0, cols = 0;
  int KB = 0, NG = 0;
  uint8_t* tiles = nullptr;   // NG * KB * 1024 bytes
  float* scales = nullptr;    // NG * 16 floats, zero padded
  size_t bytes = 0;
  uint64_t uid = 0;           // process-unique, never reused (graph cache keys)
};

namespace tlhost {

// --------------------------------------------------------------------------
// errors
// --------------------------------------------------------------------------
extern thread_local std::string t_err;
extern thread_local bool t_has_err;

struct Fail {
  std::string msg;
};

void record_error(const char* fn, const std::string& msg);

#define HIP_OK(expr)                                                                     \
  do {                                                                                   \
    hipError_t _e = (expr);                                                              \
    if (_e != hipSuccess) throw Fail{std::string(#expr) + " -> " + hipGetErrorString(_e)}; \
  } while (0)
#define REQUIRE(cond, msg) \
  do {                     \
    if (!(cond)) throw Fail{msg}; \
  } while (0)

template <class F>
int guarded(const char* fn, F&& f) {
  t_has_err = false;
  try {
    f();
    return 0;
  } catch (const Fail& e) {
    record_error(fn, e.msg);
  } catch (const std::exception& e) {
    record_error(fn, e.what());
  } catch (...) {
    record_error(fn, "unknown error");
  }
  return -1;
}

int current_device();

// process-unique id, never reused: captured graphs are keyed on these rather
// than on host addresses, which a freed handle's successor can reuse
uint64_t next_uid();

// --------------------------------------------------------------------------
// buffers
// --------------------------------------------------------------------------
struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
  // grows to at least `bytes`; `st` is synchronized before an old buffer is freed
  void ensure(size_t bytes, hipStream_t st) {
    if (bytes <= n) return;
    if (p) {
      HIP_OK(hipStreamSynchronize(st));
      HIP_OK(hipFree(p));
      p = nullptr;
      n = 0;
    }
    size_t want = bytes < 256 ? 256 : bytes;
    HIP_OK(hipMalloc(&p, want));
    n = want;
  }
};

// pinned host staging, mapped into the device address space (dp)
struct PinnedBuf {
  void* p = nullptr;
  void* dp = nullptr;
  size_t n = 0;
  void ensure(size_t bytes) {
    if (bytes <= n) return;
    if (p) {
      HIP_OK(hipHostFree(p));
      p = dp = nullptr;
      n = 0;
    }
    size_t want = bytes < 4096 ? 4096 : bytes;
    HIP_OK(hipHostMalloc(&p, want, hipHostMallocDefault));
    n = want;
    HIP_OK(hipHostGetDevicePointer(&dp, p, 0));
  }
};

// --------------------------------------------------------------------------
// weights (api.cpp)
// --------------------------------------------------------------------------
tl_weights* weights_alloc(int rows, int cols);
void weights_free(tl_weights* W);
// pack row-major int8 (host or device) + scales into a new tl_weights
tl_weights* weights_from_codes(const int8_t* w, const float* s, int rows, int cols, bool on_device,
                               hipStream_t st);
void check_weights(const tl_weights* W);
// w8a32_linear semantics on device pointers (batch 1: GEMV; batch > 1: the
// fp32-accurate GEMM), stream-ordered
void linear_w8a32(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st);
// per-token int8 activations of fp32 X, int8 GEMM, fp32 out (tl_w8a8_linear_f32_dev)
void linear_w8a8(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st);
// the W8A8 GEMM on activations already quantized into int8 tiles (row groups
// of 16 tokens, ceil(K / 64) k-blocks) with their per-token scales
void linear_w8a8_tiles(const uint8_t* tiles, const float* xs, const tl_weights* W, float* Y, int batch,
                       hipStream_t st);
// the fp32-semantics GEMM (w8a32_linear at batch > 32) on activations already
// split into four int8 planes per token (code rows 4t + p) with their exponents
void linear_w8a32_planes(const uint8_t* tiles, const int* xe, const tl_weights* W, float* Y, int batch,
                         hipStream_t st);
// greedy lm_head step (lmhead.hip): final RMSNorm, GEMV with argmax keys, key
// reduction; keys: lm_head_argmax_keys(N, K) entries, xn: K floats
size_t lm_head_argmax_keys(int N, int K);
void lm_head_argmax_enqueue(const float* h, const float* norm_w, const tl_weights* W, float* logits,
                            int32_t* token, float* max_logit, uint64_t* keys, float* xn, hipStream_t st);

}  // namespace tlhost
