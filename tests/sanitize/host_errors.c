/* host_errors.c -- drives the C host layer (api.c, decoder_host.c) through
 * its argument checks and error paths on a machine without a GPU, built with
 * -fsanitize=address,undefined by tests/test_host_sanitizers.py.  Every call
 * here must fail cleanly (an error code or NULL, a message in tl_last_error)
 * and leave no memory error, leak or undefined behaviour behind; the same
 * calls also run from several threads at once (the messages are per thread).
 *
 * argv[1..]: packed-weight cache files written by tests/wcache_format.py:
 *   argv[1] a valid file holding records named in argv[2] (newline-joined),
 *   argv[3..] damaged files that every reader call must reject. */
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/typhoon_linear.h"

static int failures = 0;

#define EXPECT(cond, what)                                  \
  do {                                                      \
    if (!(cond)) {                                          \
      fprintf(stderr, "FAILED: %s (line %d)\n", what, __LINE__); \
      failures++;                                           \
    }                                                       \
  } while (0)

/* the last error of this thread names the entry point and holds `part` */
static void expect_error(const char* fn, const char* part) {
  const char* e = tl_last_error();
  if (!e || !strstr(e, fn) || (part && !strstr(e, part))) {
    fprintf(stderr, "FAILED: expected an error from %s containing '%s', got '%s'\n", fn, part ? part : "",
            e ? e : "(none)");
    failures++;
  }
}

static void argument_checks(void) {
  float x[16] = {0}, y[16] = {0}, s[16] = {1};
  int8_t w[256] = {0};
  tl_clear_error();
  w8a32_linear(x, w, s, NULL, y, NULL, 0, 16, 16);
  expect_error("w8a32_linear", "batch");
  w8a32_linear(NULL, w, s, NULL, y, NULL, 1, 16, 16);
  expect_error("w8a32_linear", "non-NULL");
  w8a8_linear(NULL, NULL, w, s, NULL, y, 1, 16, 16);
  expect_error("w8a8_linear", "non-NULL");
  w8a16_linear(NULL, w, s, NULL, y, 1, 0, 16);
  expect_error("w8a16_linear", "M (output features)");
  w8a32_quantize(NULL, w, s, 16, 16);
  expect_error("w8a32_quantize", "NULL");
  w8a8_quantize_activations(x, w, s, 0, 16);
  expect_error("w8a8_quantize_activations", "rows and cols");
  EXPECT(tl_weights_create(NULL, s, 16, 16, 0) == NULL, "tl_weights_create NULL");
  expect_error("tl_weights_create", "NULL");
  EXPECT(tl_weights_quantize_dev(NULL, 16, 16, NULL, NULL, NULL) == NULL, "tl_weights_quantize_dev NULL");
  expect_error("tl_weights_quantize_dev", "NULL");
  EXPECT(tl_w8a32_linear_dev(x, NULL, NULL, y, 1, NULL) != 0, "tl_w8a32_linear_dev NULL weights");
  expect_error("tl_w8a32_linear_dev", "NULL");
  EXPECT(tl_gemv_set_plan(7, 0) != 0, "tl_gemv_set_plan rows");
  expect_error("tl_gemv_set_plan", "rows");
  EXPECT(tl_rows_set_split(99) != 0, "tl_rows_set_split range");
  expect_error("tl_rows_set_split", "split");
  EXPECT(tl_rows_set_groups(4) != 0, "tl_rows_set_groups range");
  EXPECT(tl_w8a16_set_gemv(2) != 0, "tl_w8a16_set_gemv range");
  EXPECT(tl_gemm_i8_set_cfg(99) != 0, "tl_gemm_i8_set_cfg range");
  EXPECT(tl_attn_set_chunk(48) != 0, "tl_attn_set_chunk range");
  EXPECT(tl_stream_read_dev(NULL, 16, 1, 4, NULL, NULL) != 0, "tl_stream_read_dev NULL");
  EXPECT(tl_rmsnorm_np_dev(x, NULL, y, 100, NULL) != 0, "tl_rmsnorm_np_dev K");
  expect_error("tl_rmsnorm_np_dev", "power of two");
  EXPECT(tl_lm_head_argmax(NULL, NULL, w, s, 16, 16, NULL, NULL) != 0, "tl_lm_head_argmax NULL");
  EXPECT(tl_weights_export(NULL, w, s, 0) != 0, "tl_weights_export NULL");
  EXPECT(tl_weights_save(NULL, "/nonexistent/x", "m", 0) != 0, "tl_weights_save NULL");
  EXPECT(tl_registry_adopt(w, s, NULL) != 0, "tl_registry_adopt NULL");
  EXPECT(tl_registry_entries() == 0 && tl_registry_bytes() == 0, "empty registry");
  EXPECT(tl_evict_weights(w) == 0, "tl_evict_weights on an empty registry");
  tl_registry_clear();
  /* tuning switches that take valid values succeed without a device */
  EXPECT(tl_rows_set_split(0) == 0 && tl_rows_set_groups(0) == 0 && tl_w8a16_set_gemv(1) == 0, "valid tuning");
  EXPECT(tl_prefill_set_fused_quant(2) != 0, "tl_prefill_set_fused_quant range");
  EXPECT(tl_prefill_set_fused_quant(1) == 0, "tl_prefill_set_fused_quant valid");
  /* decoder entry points on NULL handles */
  decoder_decode_step(NULL, NULL, y, NULL, NULL, NULL);
  expect_error("decoder_decode_step", "NULL");
  decoder_prefill_step(NULL, NULL, y, NULL, NULL, NULL, 4);
  expect_error("decoder_prefill_step", "NULL cache");
  decoder_chunked_prefill_step(NULL, NULL, y, NULL, NULL, NULL, 4, 0);
  expect_error("decoder_chunked_prefill_step", "chunk_size");
  decoder_prefill_step_3d(NULL, NULL, y, NULL, NULL, NULL, 4);
  expect_error("decoder_prefill_step_3d", "NULL token tables");
  decoder_set_layer_weights(NULL, 0, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL,
                            NULL, NULL, NULL, NULL, NULL);
  expect_error("decoder_set_layer_weights", "NULL model");
  EXPECT(decoder_cache_alloc(0) == NULL, "decoder_cache_alloc(0)");
  expect_error("decoder_cache_alloc", "max_seq");
  EXPECT(decoder_scratch_alloc_fn(-1) == NULL, "decoder_scratch_alloc_fn(-1)");
  expect_error("decoder_scratch_alloc_fn", "max_seq");
  EXPECT(tl_decoder_generate(NULL, NULL, NULL, NULL, NULL, NULL, 0, 1, NULL, NULL, NULL) != 0, "generate NULL");
  EXPECT(tl_decoder_read_cache(NULL, 0, y, y) != 0, "read_cache NULL");
  EXPECT(tl_decoder_num_layers(NULL) == -1 && tl_decoder_cache_len(NULL) == -1, "NULL handle queries");
  EXPECT(tl_decoder_set_prefill_w8a8(NULL, 1) != 0, "set_prefill_w8a8 NULL");
  decoder_model_free(NULL);
  decoder_cache_free(NULL);
  decoder_scratch_free_fn(NULL);
  tl_weights_destroy(NULL);
  float ct[4 * 64], st[4 * 64];
  const int sections[3] = {16, 24, 24};
  const float theta[3] = {5e6f, 5e6f, 5e6f};
  decoder_precompute_rope(ct, st, 4, 128, sections, theta);   /* host-only: succeeds */
  const int pos[3 * 4] = {0, 1, 2, 3, 0, 1, 1, 2, 0, 2, 1, 3};
  decoder_build_rope_3d(ct, st, pos, 4, 128, sections, theta);
  decoder_build_rope_3d(NULL, st, pos, 4, 128, sections, theta);
  expect_error("decoder_build_rope_3d", "bad arguments");
}

static void cache_files(int argc, char** argv) {
  if (argc < 3) return;
  char names[4096];
  const int n = tl_weights_cache_list(argv[1], names, sizeof names);
  EXPECT(n >= 1, "valid cache file lists its records");
  if (n >= 1) EXPECT(strcmp(names, argv[2]) == 0, "listed names");
  char small[4];
  EXPECT(tl_weights_cache_list(argv[1], small, sizeof small) == -1, "names buffer too small");
  expect_error("tl_weights_cache_list", "too small");
  EXPECT(tl_weights_load(argv[1], "no such record") == NULL, "missing record");
  expect_error("tl_weights_load", "no record named");
  EXPECT(tl_weights_load("/nonexistent/file.tlw", "a") == NULL, "missing file");
  expect_error("tl_weights_load", "cannot open");
  for (int i = 3; i < argc; i++) {
    EXPECT(tl_weights_cache_list(argv[i], NULL, 0) == -1, "damaged file rejected by the list");
    EXPECT(tl_weights_load(argv[i], "m") == NULL, "damaged file rejected by the loader");
  }
}

typedef struct {
  int argc;
  char** argv;
} Args;

static void* worker(void* p) {
  const Args* a = (const Args*)p;
  for (int r = 0; r < 20; r++) {
    argument_checks();
    cache_files(a->argc, a->argv);
  }
  return NULL;
}

int main(int argc, char** argv) {
  printf("%s, %d device(s)\n", tl_version(), tl_device_count());
  argument_checks();
  cache_files(argc, argv);
  Args a = {argc, argv};
  pthread_t th[4];
  for (int i = 0; i < 4; i++) pthread_create(&th[i], NULL, worker, &a);
  for (int i = 0; i < 4; i++) pthread_join(th[i], NULL);
  printf("%d failures\n", failures);
  return failures ? 1 : 0;
}
