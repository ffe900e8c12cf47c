/* host.h -- plumbing shared by the C host layer (api.c, decoder_host.c): the
 * device weight handle, error capture, device and pinned buffers, and the
 * device-pointer linear operations the decoder calls.  Internal to the
 * library.
 *
 * Errors: every internal function returns 0 on success and -1 on failure,
 * after recording a message in a thread-local buffer (tlh_fail*); an entry
 * point clears the state on entry (tlh_begin) and on failure prefixes the
 * message with its own name (tlh_finish), which tl_last_error then returns. */
#pragma once
#include "../../include/typhoon_linear.h"
#include "tl_kernels.h"

#include <hip/hip_runtime_api.h>
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

struct tl_weights {
  int dev;
  int rows, cols;
  int KB, NG;
  uint8_t* tiles;   /* NG * KB * 1024 bytes */
  float* scales;    /* NG * 16 floats, zero padded */
  size_t bytes;
  uint64_t uid;     /* process-unique, never reused (graph cache keys) */
};

/* ---- errors --------------------------------------------------------------- */
int tlh_fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int tlh_fail_hip(const char* expr, hipError_t e);
void tlh_begin(void);
int tlh_finish(const char* fn, int rc);

#define HIP_TRY(expr)                                       \
  do {                                                      \
    hipError_t e_ = (expr);                                 \
    if (e_ != hipSuccess) return tlh_fail_hip(#expr, e_);   \
  } while (0)
#define REQ(cond, ...)                          \
  do {                                          \
    if (!(cond)) return tlh_fail(__VA_ARGS__);  \
  } while (0)
#define TRY(expr)                 \
  do {                            \
    if ((expr) != 0) return -1;   \
  } while (0)
/* the same with a jump to a cleanup label; `rc` must be an int in scope */
#define HIP_GO(expr, label)                  \
  do {                                       \
    hipError_t e_ = (expr);                  \
    if (e_ != hipSuccess) {                  \
      rc = tlh_fail_hip(#expr, e_);          \
      goto label;                            \
    }                                        \
  } while (0)
#define REQ_GO(cond, label, ...)       \
  do {                                 \
    if (!(cond)) {                     \
      rc = tlh_fail(__VA_ARGS__);      \
      goto label;                      \
    }                                  \
  } while (0)
#define TRY_GO(expr, label)   \
  do {                        \
    if ((expr) != 0) {        \
      rc = -1;                \
      goto label;             \
    }                         \
  } while (0)

int tlh_current_device(int* dev);
/* process-unique id, never reused: captured graphs are keyed on these rather
 * than on host addresses, which a freed handle's successor can reuse */
uint64_t tlh_next_uid(void);

/* ---- buffers -------------------------------------------------------------- */
typedef struct DevBuf {
  void* p;
  size_t n;
} DevBuf;
/* grows to at least `bytes`; `st` is synchronized before an old buffer is freed */
int tlh_devbuf_ensure(DevBuf* b, size_t bytes, hipStream_t st);
void tlh_devbuf_free(DevBuf* b);

/* pinned host staging, mapped into the device address space (dp) */
typedef struct PinnedBuf {
  void* p;
  void* dp;
  size_t n;
} PinnedBuf;
int tlh_pinned_ensure(PinnedBuf* b, size_t bytes);
void tlh_pinned_free(PinnedBuf* b);

/* ---- weights and linear operations (api.c) -------------------------------- */
int tlh_weights_alloc(int rows, int cols, tl_weights** out);
void tlh_weights_free(tl_weights* W);
/* pack row-major int8 (host or device) + scales into a new tl_weights */
int tlh_weights_from_codes(const int8_t* w, const float* s, int rows, int cols, bool on_device, hipStream_t st,
                           tl_weights** out);
int tlh_check_weights(const tl_weights* W);
/* w8a32_linear semantics on device pointers (batch 1: GEMV; batch > 1: the
 * fp32-accurate GEMM), stream-ordered */
int tlh_linear_w8a32(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st);
/* per-token int8 activations of fp32 X, int8 GEMM, fp32 out */
int tlh_linear_w8a8(const float* X, const tl_weights* W, const float* bias, float* Y, int batch, hipStream_t st);
/* the W8A8 GEMM on activations already quantized into int8 tiles (row groups
 * of 16 tokens, ceil(K / 64) k-blocks) with their per-token scales */
int tlh_linear_w8a8_tiles(const uint8_t* tiles, const float* xs, const tl_weights* W, float* Y, int batch,
                          hipStream_t st);
/* the fp32-semantics GEMM (w8a32_linear at batch > 32) on activations already
 * split into four int8 planes per token (code rows 4t + p) with their exponents */
int tlh_linear_w8a32_planes(const uint8_t* tiles, const int* xe, const tl_weights* W, float* Y, int batch,
                            hipStream_t st);
