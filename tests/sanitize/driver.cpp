// driver.cpp — host-only exerciser of libglypr_hip's GGUF parser and C-ABI
// argument validation.  tests/test_sanitize.py builds it, with the library's
// host sources, under AddressSanitizer and UndefinedBehaviorSanitizer and runs
// it on valid, truncated and corrupt files.  Nothing here touches a GPU: every
// call below returns during parsing or validation.
//
//   driver FILE...      open each GGUF file; on success walk every getter
//   driver --validate   call each entry point with invalid arguments
#include <stdio.h>
#include <string.h>

#include "glypr_hip.h"

namespace {

const char* const kKeys[] = {"general.architecture", "general.alignment", "a.u32", "a.i32",
                             "a.neg", "a.u64", "a.f32", "a.f64", "a.bool", "a.arr", "a.strs",
                             "gemma-embedding2.block_count",
                             "gemma-embedding2.attention.head_count_kv",
                             "gemma-embedding2.attention.sliding_window_pattern", "absent"};

void walk(const glypr_gguf* g) {
  uint32_t v = 0, a = 0;
  glypr_gguf_version(g, &v, &a);
  int64_t n = 0;
  glypr_gguf_tensor_count(g, &n);
  for (int64_t i = -1; i <= n; i++) {   // one below and one past the range too
    const char* name = nullptr;
    const void* data = nullptr;
    int type = 0, nd = 0;
    int64_t ne[4], nbytes = 0;
    if (glypr_gguf_tensor_info(g, i, &name, &type, &nd, ne, &data, &nbytes) != GLYPR_OK)
      continue;
    int64_t idx = -1;
    glypr_gguf_find_tensor(g, name, &idx);
    // touch the mapped bytes the parser vouched for
    unsigned sum = 0;
    for (int64_t b = 0; data && b < nbytes; b++) sum += ((const unsigned char*)data)[b];
    printf("tensor %s type %d dims %d bytes %lld sum %u\n", name, type, nd, (long long)nbytes,
           sum);
  }
  for (const char* k : kKeys) {
    uint64_t u = 0;
    double f = 0;
    const char* s = nullptr;
    int et = 0;
    int64_t len = 0;
    glypr_gguf_get_u64(g, k, &u);
    glypr_gguf_get_f64(g, k, &f);
    glypr_gguf_get_str(g, k, &s);
    if (glypr_gguf_get_array(g, k, &et, &len) == GLYPR_OK)
      for (int64_t i = -1; i <= len && i < 4096; i++) glypr_gguf_get_array_u64(g, k, i, &u);
  }
}

int validate() {
  glypr_q8w* w = nullptr;
  glypr_hip_ctx* ctx = nullptr;
  glypr_model* m = nullptr;
  void* fake = (void*)0x1000;
  int bad = 0;
  auto expect = [&](int got, int want, const char* what) {
    if (got != want) {
      printf("validation %s: got %d, want %d (%s)\n", what, got, want, glypr_hip_last_error());
      bad++;
    }
  };
  expect(glypr_hip_q8_0_weight_create(nullptr, (const uint8_t*)fake, 1, 33, &w), GLYPR_ERR_SHAPE,
         "weight k % 32");
  expect(glypr_hip_q8_0_weight_create(nullptr, nullptr, 1, 32, &w), GLYPR_ERR_INVALID_ARG,
         "weight null blocks");
  expect(glypr_hip_q8_0_matmul(nullptr, nullptr, nullptr, nullptr, -1, 0, nullptr),
         GLYPR_ERR_SHAPE, "matmul m < 0");
  expect(glypr_hip_q8_0_matmul(nullptr, (const glypr_q8w*)fake, (const float*)0x1004,
                               (float*)fake, 4, 0, nullptr),
         GLYPR_ERR_ALIGNMENT, "matmul misaligned");
  expect(glypr_hip_mlp(nullptr, nullptr, nullptr, nullptr, nullptr, 4, 0, nullptr),
         GLYPR_ERR_INVALID_ARG, "mlp null");
  expect(glypr_hip_ctx_reserve(nullptr, 0), GLYPR_ERR_SHAPE, "reserve 0");
  expect(glypr_hip_ctx_reserve(nullptr, 1 << 20), GLYPR_ERR_INVALID_ARG, "reserve null ctx");
  expect(glypr_hip_attention(nullptr, (const float*)fake, (const float*)fake, (const float*)fake,
                             1e-6f, (const float*)fake, (const float*)fake, 512, 5, 1, 256, 0,
                             (float*)fake, nullptr),
         GLYPR_ERR_UNSUPPORTED, "attention 5:1");
  glypr_model_config c;
  memset(&c, 0, sizeof(c));
  c.hidden = 768; c.ffn = 1152; c.n_heads = 3; c.n_kv_heads = 1; c.head_dim = 256;
  c.n_layers = 24; c.vocab = 262144; c.sliding_window = 512; c.eps = 1e-6f;
  c.rope_theta_sliding = 1e4; c.rope_theta_full = 1e6;
  expect(glypr_hip_model_create(nullptr, &c, &m), GLYPR_ERR_INVALID_ARG, "model null ctx");
  c.n_heads = 5;
  expect(glypr_hip_model_create(nullptr, &c, &m), GLYPR_ERR_UNSUPPORTED, "model 5:1");
  c.n_heads = 3;
  c.hidden = 100;
  expect(glypr_hip_model_create(nullptr, &c, &m), GLYPR_ERR_SHAPE, "model hidden % 32");
  expect(glypr_hip_quantize_binary(nullptr, (const float*)fake, 1, 63, (uint64_t*)fake, nullptr),
         GLYPR_ERR_SHAPE, "binary dim % 64");
  expect(glypr_hip_int8_dot(nullptr, (const int8_t*)fake, 1, (const int8_t*)fake, 1, 65537,
                            (int32_t*)fake, nullptr),
         GLYPR_ERR_SHAPE, "int8 dim");
  expect(glypr_hip_q8_0_embed_gather(nullptr, (const glypr_q8w*)fake, (const uint32_t*)fake, -1,
                                     1.0f, (float*)fake, nullptr),
         GLYPR_ERR_SHAPE, "gather n < 0");
  expect(glypr_hip_model_load_gguf(nullptr, "/nonexistent.gguf", &m), GLYPR_ERR_INVALID_ARG,
         "load null ctx");
  expect(glypr_gguf_open(nullptr, nullptr), GLYPR_ERR_INVALID_ARG, "open null");
  (void)ctx;
  printf("validation failures %d\n", bad);
  return bad == 0 ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc == 2 && strcmp(argv[1], "--validate") == 0) return validate();
  for (int i = 1; i < argc; i++) {
    glypr_gguf* g = nullptr;
    const int rc = glypr_gguf_open(argv[i], &g);
    printf("open %s -> %d %s\n", argv[i], rc, rc == GLYPR_OK ? "" : glypr_hip_last_error());
    if (g) {
      walk(g);
      glypr_gguf_close(g);
    }
  }
  return 0;
}
