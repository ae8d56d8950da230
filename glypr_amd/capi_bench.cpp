// capi_bench.cpp — the C2/C3 layer-projection workload through the C ABI
// alone (no Python, no torch): the program to put under rocprofv3 when the
// counters of one projection kernel are wanted, and an example of driving
// libglypr_hip.so from C++.
//
// One step is the C2/C3 layer's seven Q8_0 projections as the library fuses
// them (qkv as one concatenated weight, gate|up as one):
//   glypr_hip_rmsnorm_q8_0_matmul  x -> RMSNorm -> qkv   768 -> 1280
//   glypr_hip_q8_0_matmul          attn -> o             768 -> 768
//   glypr_hip_rmsnorm_mlp          x -> RMSNorm -> gate|up + GeGLU -> down
// on synthetic Q8_0 weights (BASELINE's N(0, 0.02) quantized as
// BlockQ8_0::from_float does: d = amax / 127 as f16) and N(0, 1) activations.
//
//   capi_bench [--m 16384] [--variant int8|fma|bf16] [--steps 20] [--warmup 3]
//              [--copy-probe MB]
//   capi_bench --model [--t 512] [--variant int8|fma] [--steps 20] [--warmup 3]
//              [--copy-probe MB]
//
// Prints one JSON line: ms per step and TOPS (2 * m * 7-projection MACs).
// --model instead runs config 4: glypr_hip_model_embed of one t-token
// sequence through the 24-layer backbone (hidden 768, 3 q / 1 kv heads of
// 256, FFN 1152, the 262144 x 768 Q8_0 token table, MRL-256), synthetic
// weights as above and norm weights 1 + N(0, 0.1) (q/k norms x 0.25); its
// --variant (INT8_EXACT unless given) goes to glypr_hip_model_set_variant.
// --copy-probe MB ends the run with one device-to-device copy of MB MiB: the
// known-size launch that calibrates rocprofv3's FETCH_SIZE / WRITE_SIZE.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <random>
#include <vector>

#include "glypr_hip.h"

namespace {

constexpr int64_t H = 768, NQ = 768, NKV = 256, F = 1152;

void die(const char* what, int rc) {
  fprintf(stderr, "%s failed (%d): %s\n", what, rc, glypr_hip_last_error());
  exit(1);
}
#define CK(call)                      \
  do {                                \
    int rc_ = (call);                 \
    if (rc_ != 0) die(#call, rc_);    \
  } while (0)
#define HK(call)                                                              \
  do {                                                                        \
    hipError_t e_ = (call);                                                   \
    if (e_ != hipSuccess) {                                                   \
      fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));       \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

uint16_t f32_to_f16(float f) {
  // round to nearest even; the scales here are normal f16 values
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  int32_t e = (int32_t)((u >> 23) & 0xFF) - 127 + 15;
  uint32_t m = u & 0x7FFFFFu;
  if (e <= 0) return (uint16_t)sign;   // never reached for these scales
  uint32_t r = (uint32_t)(e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
  return (uint16_t)(sign | r);
}

// GGUF Q8_0 blocks [n][k/32][34 B] of N(0, sigma) values quantized as
// BlockQ8_0::from_float: d = amax / 127 (stored as f16), q = round(x / d).
std::vector<uint8_t> q8_0_weight(std::mt19937_64& rng, int64_t n, int64_t k, float sigma) {
  std::normal_distribution<float> nd(0.0f, sigma);
  std::vector<uint8_t> out((size_t)(n * (k / 32) * 34));
  float x[32];
  for (int64_t b = 0; b < n * (k / 32); b++) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
      x[i] = nd(rng);
      amax = fmaxf(amax, fabsf(x[i]));
    }
    const float d = amax / 127.0f;
    const uint16_t dh = f32_to_f16(d);
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t* blk = out.data() + b * 34;
    memcpy(blk, &dh, 2);
    for (int i = 0; i < 32; i++) {
      const float q = roundf(x[i] * id);
      blk[2 + i] = (uint8_t)(int8_t)(q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q));
    }
  }
  return out;
}

std::vector<float> host_normal(std::mt19937_64& rng, int64_t n, float mean, float sigma,
                              float scale = 1.0f) {
  std::normal_distribution<float> nd(mean, sigma);
  std::vector<float> h((size_t)n);
  for (auto& v : h) v = nd(rng) * scale;
  return h;
}

// Config 4 through glypr_hip_model_*: ms per embedding.
int run_model(int64_t t, int steps, int warmup, int variant) {
  constexpr int64_t L = 24, V = 262144, HD = 256;
  glypr_hip_ctx* ctx = nullptr;
  CK(glypr_hip_ctx_create(0, &ctx));
  glypr_model_config cfg{};
  cfg.hidden = H;
  cfg.ffn = F;
  cfg.n_heads = 3;
  cfg.n_kv_heads = 1;
  cfg.head_dim = HD;
  cfg.n_layers = L;
  cfg.vocab = V;
  cfg.sliding_window = 512;
  cfg.eps = 1e-6f;
  cfg.rope_theta_sliding = 10000.0;
  cfg.rope_theta_full = 1e6;
  glypr_model* m = nullptr;
  CK(glypr_hip_model_create(ctx, &cfg, &m));
  std::mt19937_64 rng(7);
  auto set_q8 = [&](const char* name, int64_t n, int64_t k) {
    const std::vector<uint8_t> b = q8_0_weight(rng, n, k, 0.02f);
    CK(glypr_hip_model_set_tensor(m, name, b.data(), n, k, 1));
  };
  auto set_f32 = [&](const char* name, int64_t n, float scale) {
    const std::vector<float> w = host_normal(rng, n, 1.0f, 0.1f, scale);
    CK(glypr_hip_model_set_tensor(m, name, w.data(), 1, n, 0));
  };
  set_q8("token_embd.weight", V, H);
  set_f32("output_norm.weight", H, 1.0f);
  char name[96];
  const struct { const char* n; int64_t rows, cols; } proj[] = {
      {"attn_q", NQ, H}, {"attn_k", NKV, H}, {"attn_v", NKV, H}, {"attn_output", H, NQ},
      {"ffn_gate", F, H}, {"ffn_up", F, H}, {"ffn_down", H, F}};
  const struct { const char* n; int64_t dim; float scale; } norms[] = {
      {"attn_norm", H, 1.0f}, {"post_attention_norm", H, 1.0f}, {"ffn_norm", H, 1.0f},
      {"post_ffw_norm", H, 1.0f}, {"attn_q_norm", HD, 0.25f}, {"attn_k_norm", HD, 0.25f}};
  for (int64_t i = 0; i < L; i++) {
    for (const auto& p : proj) {
      snprintf(name, sizeof name, "blk.%lld.%s.weight", (long long)i, p.n);
      set_q8(name, p.rows, p.cols);
    }
    for (const auto& nw : norms) {
      snprintf(name, sizeof name, "blk.%lld.%s.weight", (long long)i, nw.n);
      set_f32(name, nw.dim, nw.scale);
    }
  }
  CK(glypr_hip_model_finalize(m));
  CK(glypr_hip_model_set_variant(m, variant));
  std::vector<uint32_t> ids((size_t)t);
  std::uniform_int_distribution<uint32_t> ud(0, (uint32_t)V - 1);
  for (auto& v : ids) v = ud(rng);
  float* out = nullptr;
  HK(hipMalloc(&out, 256 * 4));
  hipStream_t s;
  HK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  for (int i = 0; i < warmup; i++) CK(glypr_hip_model_embed(m, ids.data(), t, 256, out, nullptr, s));
  HK(hipStreamSynchronize(s));
  hipEvent_t e0, e1;
  HK(hipEventCreate(&e0));
  HK(hipEventCreate(&e1));
  HK(hipEventRecord(e0, s));
  const auto h0 = std::chrono::steady_clock::now();
  for (int i = 0; i < steps; i++) CK(glypr_hip_model_embed(m, ids.data(), t, 256, out, nullptr, s));
  // host time to enqueue the steps: close to the GPU time when the launches,
  // not the kernels, set the pace
  const double host_ms =
      std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - h0).count();
  HK(hipEventRecord(e1, s));
  HK(hipEventSynchronize(e1));
  float ms = 0.0f;
  HK(hipEventElapsedTime(&ms, e0, e1));
  printf("{\"workload\": \"c4-embed\", \"variant\": %d, \"t\": %lld, \"layers\": %lld, "
         "\"steps\": %d, "
         "\"ms_per_embedding\": %.4f, \"embeddings_per_s\": %.2f, "
         "\"host_enqueue_ms_per_embedding\": %.4f}\n",
         variant, (long long)t, (long long)L, steps, ms / steps, 1000.0 * steps / ms,
         host_ms / steps);
  fflush(stdout);
  HK(hipFree(out));
  HK(hipStreamDestroy(s));
  CK(glypr_hip_model_destroy(m));
  CK(glypr_hip_ctx_destroy(ctx));
  return 0;
}

void copy_probe(int64_t probe_mb) {
  if (probe_mb <= 0) return;
  const size_t bytes = (size_t)probe_mb << 20;
  void *a = nullptr, *b = nullptr;
  HK(hipMalloc(&a, bytes));
  HK(hipMalloc(&b, bytes));
  HK(hipMemset(a, 1, bytes));
  HK(hipMemcpy(b, a, bytes, hipMemcpyDeviceToDevice));
  HK(hipDeviceSynchronize());
  HK(hipFree(a));
  HK(hipFree(b));
  printf("{\"copy_probe_bytes\": %zu}\n", bytes);
}

float* device_normal(std::mt19937_64& rng, int64_t n, float mean, float sigma) {
  std::normal_distribution<float> nd(mean, sigma);
  std::vector<float> h((size_t)n);
  for (auto& v : h) v = nd(rng);
  float* d = nullptr;
  HK(hipMalloc(&d, (size_t)n * 4));
  HK(hipMemcpy(d, h.data(), (size_t)n * 4, hipMemcpyHostToDevice));
  return d;
}

}  // namespace

int main(int argc, char** argv) {
  int64_t m = 16384;
  int variant = -1, steps = 20, warmup = 3;
  int64_t probe_mb = 0, t = 512;
  bool model = false;
  for (int i = 1; i < argc; i++) {
    if (!strcmp(argv[i], "--m") && i + 1 < argc) m = atoll(argv[++i]);
    else if (!strcmp(argv[i], "--model")) model = true;
    else if (!strcmp(argv[i], "--t") && i + 1 < argc) t = atoll(argv[++i]);
    else if (!strcmp(argv[i], "--variant") && i + 1 < argc) {
      ++i;
      variant = !strcmp(argv[i], "int8")   ? GLYPR_Q8_INT8_EXACT
                : !strcmp(argv[i], "fma")  ? GLYPR_Q8_INT8_FMA
                : !strcmp(argv[i], "bf16") ? GLYPR_Q8_BF16_DEQUANT
                                           : -2;
    } else if (!strcmp(argv[i], "--steps") && i + 1 < argc) steps = atoi(argv[++i]);
    else if (!strcmp(argv[i], "--warmup") && i + 1 < argc) warmup = atoi(argv[++i]);
    else if (!strcmp(argv[i], "--copy-probe") && i + 1 < argc) probe_mb = atoll(argv[++i]);
    else {
      fprintf(stderr,
              "usage: %s [--m M] [--variant int8|fma|bf16] [--steps K] [--warmup W] "
              "[--copy-probe MB]\n       %s --model [--t T] [--variant int8|fma] [--steps K] "
              "[--warmup W] [--copy-probe MB]\n", argv[0], argv[0]);
      return 2;
    }
  }
  if (m <= 0 || t <= 0 || t > 8192 || steps <= 0 || warmup < 0 || probe_mb < 0 ||
      probe_mb > 4096) {
    fprintf(stderr, "m, steps must be > 0, t in [1, 8192], warmup >= 0, copy-probe in "
                    "[0, 4096]\n");
    return 2;
  }
  if (variant == -2 || (model && variant == GLYPR_Q8_BF16_DEQUANT)) {
    fprintf(stderr, "--variant: int8, fma or (without --model) bf16\n");
    return 2;
  }
  if (model) {
    const int rc = run_model(t, steps, warmup, variant < 0 ? GLYPR_Q8_INT8_EXACT : variant);
    copy_probe(probe_mb);
    return rc;
  }
  if (variant < 0) variant = GLYPR_Q8_BF16_DEQUANT;
  glypr_hip_ctx* ctx = nullptr;
  CK(glypr_hip_ctx_create(0, &ctx));
  CK(glypr_hip_ctx_reserve(ctx, m));
  std::mt19937_64 rng(12345);
  const struct { const char* name; int64_t n, k; } shapes[] = {
      {"q", NQ, H}, {"k", NKV, H}, {"v", NKV, H}, {"o", H, NQ},
      {"gate", F, H}, {"up", F, H}, {"down", H, F}};
  glypr_q8w* w[7] = {};
  for (int i = 0; i < 7; i++) {
    const std::vector<uint8_t> b = q8_0_weight(rng, shapes[i].n, shapes[i].k, 0.02f);
    CK(glypr_hip_q8_0_weight_create(ctx, b.data(), shapes[i].n, shapes[i].k, &w[i]));
  }
  glypr_q8w *qkv = nullptr, *gate_up = nullptr;
  const glypr_q8w* p3[3] = {w[0], w[1], w[2]};
  const glypr_q8w* p2[2] = {w[4], w[5]};
  CK(glypr_hip_q8_0_weight_concat(ctx, p3, 3, &qkv, nullptr));
  CK(glypr_hip_q8_0_weight_concat(ctx, p2, 2, &gate_up, nullptr));
  float* x = device_normal(rng, m * H, 0.0f, 1.0f);
  float* attn = device_normal(rng, m * NQ, 0.0f, 1.0f);
  float* n1 = device_normal(rng, H, 1.0f, 0.1f);
  float* n2 = device_normal(rng, H, 1.0f, 0.1f);
  float *y_qkv = nullptr, *y_o = nullptr, *y_mlp = nullptr;
  HK(hipMalloc(&y_qkv, (size_t)(m * (NQ + 2 * NKV)) * 4));
  HK(hipMalloc(&y_o, (size_t)(m * H) * 4));
  HK(hipMalloc(&y_mlp, (size_t)(m * H) * 4));
  hipStream_t s;
  HK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  auto step = [&]() {
    CK(glypr_hip_rmsnorm_q8_0_matmul(ctx, qkv, x, n1, 1e-6f, y_qkv, m, variant, s));
    CK(glypr_hip_q8_0_matmul(ctx, w[3], attn, y_o, m, variant, s));
    CK(glypr_hip_rmsnorm_mlp(ctx, gate_up, w[6], x, n2, 1e-6f, y_mlp, m, variant, s));
  };
  for (int i = 0; i < warmup; i++) step();
  HK(hipStreamSynchronize(s));
  hipEvent_t e0, e1;
  HK(hipEventCreate(&e0));
  HK(hipEventCreate(&e1));
  HK(hipEventRecord(e0, s));
  for (int i = 0; i < steps; i++) step();
  HK(hipEventRecord(e1, s));
  HK(hipEventSynchronize(e1));
  float ms = 0.0f;
  HK(hipEventElapsedTime(&ms, e0, e1));
  const double per = ms / steps;
  const double macs = (double)m * (double)(H * (NQ + 2 * NKV) + NQ * H + H * 2 * F + F * H);
  printf("{\"workload\": \"c3-layer-projections\", \"m\": %lld, \"variant\": \"%s\", "
         "\"steps\": %d, \"ms_per_step\": %.4f, \"tops\": %.2f}\n",
         (long long)m,
         variant == GLYPR_Q8_INT8_EXACT ? "int8" : variant == GLYPR_Q8_INT8_FMA ? "fma" : "bf16",
         steps, per,
         2.0 * macs / (per / 1e3) / 1e12);
  fflush(stdout);
  copy_probe(probe_mb);
  for (auto* p : w) CK(glypr_hip_q8_0_weight_destroy(p));
  CK(glypr_hip_q8_0_weight_destroy(qkv));
  CK(glypr_hip_q8_0_weight_destroy(gate_up));
  for (float* p : {x, attn, n1, n2, y_qkv, y_o, y_mlp}) HK(hipFree(p));
  HK(hipStreamDestroy(s));
  CK(glypr_hip_ctx_destroy(ctx));
  return 0;
}
