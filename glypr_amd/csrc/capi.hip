// capi.hip — the C ABI (include/glypr_hip.h): argument validation, weight
// handles, workspace management and kernel dispatch.
//
// Validation order in every entry point: scalar arguments (sizes, variant),
// then pointers (null, 16-byte alignment), then context/device.  Nothing is
// launched or allocated before all three pass, so every error path can be
// exercised on a machine without a GPU.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <new>
#include <vector>

#include "host_common.hpp"
#include "internal.hpp"

namespace glypr {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

int hip_error(hipError_t e, const char* what) {
  if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
    return set_error(GLYPR_ERR_OOM, "%s: %s", what, hipGetErrorString(e));
  return set_error(GLYPR_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

namespace {

// Workspace bytes matmul_impl needs for [m, k] activations in `variant`
// (0 when the prologue-fused GEMM runs and needs none).
size_t matmul_ws_bytes(int64_t m, int64_t n, int64_t k, bool norm, int variant) {
  if (variant != GLYPR_Q8_BF16_DEQUANT)
    return gemm_i8_pro_ok(m, n, k, norm) ? 0 : q8_act_bytes(m, k);
  return align_up((size_t)(m * k) * 2, 256);
}

// Shared body of the plain, RMSNorm-prologue and no-allocation matmuls: the
// activation operand goes to `ws`, which holds matmul_ws_bytes.
int matmul_impl(glypr_hip_ctx* ctx, const glypr_q8w* w, const float* x, const float* norm_w,
                float eps, bool norm, float* y, int64_t m, int variant, void* ws,
                hipStream_t s) {
  const int64_t n = w->n, k = w->k;
  if (variant != GLYPR_Q8_BF16_DEQUANT) {
    const bool fma2 = variant == GLYPR_Q8_INT8_FMA;
    if (gemm_i8_pro_ok(m, n, k, norm)) {
      LAUNCH(GLYPR_K_GEMM_I8_PRO, s,
             launch_gemm_i8_pro(x, norm_w, eps, norm, w->qs(), w->dw(), y, m, n, k, n, s, fma2),
             "gemm_i8_pro launch");
      return GLYPR_OK;
    }
    Carve c(ws);
    int8_t* xq = c.take<int8_t>((size_t)(m * k));
    float* dx = c.take<float>((size_t)(m * (k / 32)));
    if (norm)
      LAUNCH(GLYPR_K_RMSNORM_QUANT, s, launch_rmsnorm_quant(x, norm_w, eps, m, k, xq, dx, s),
             "rmsnorm_quant launch");
    else
      LAUNCH(GLYPR_K_QUANTIZE, s, launch_quantize_planar(x, m, k, xq, dx, s), "quantize launch");
    LAUNCH(GLYPR_K_GEMM_I8, s, launch_gemm_i8(xq, dx, w->qs(), w->dw(), y, m, n, k, n, s, fma2),
           "gemm_i8 launch");
    return GLYPR_OK;
  }
  Carve c(ws);
  uint16_t* xb = c.take<uint16_t>((size_t)(m * k));
  if (norm)
    LAUNCH(GLYPR_K_RMSNORM_BF16, s, launch_rmsnorm_bf16(x, norm_w, eps, m, k, xb, s),
           "rmsnorm_bf16 launch");
  else
    LAUNCH(GLYPR_K_TO_BF16, s, launch_to_bf16(x, m * k, xb, s), "to_bf16 launch");
  LAUNCH(GLYPR_K_GEMM_BF16, s, launch_gemm_bf16(xb, w->qs(), w->dw(), y, m, n, k, n, s),
         "gemm_bf16 launch");
  return GLYPR_OK;
}

// matmul_impl on the context's workspace, grown first if needed.
int matmul_ws(glypr_hip_ctx* ctx, const glypr_q8w* w, const float* x, const float* norm_w,
              float eps, bool norm, float* y, int64_t m, int variant, hipStream_t s) {
  const size_t need = matmul_ws_bytes(m, w->n, w->k, norm, variant);
  if (need) RET_IF(ensure_ws(ctx, need));
  return matmul_impl(ctx, w, x, norm_w, eps, norm, y, m, variant, ctx->ws, s);
}

int mlp_impl(glypr_hip_ctx* ctx, const glypr_q8w* gu, const glypr_q8w* down, const float* x,
             const float* norm_w, float eps, bool norm, float* y, int64_t m, int variant,
             hipStream_t s) {
  const int64_t H = gu->k, F = down->k;
  if (variant != GLYPR_Q8_BF16_DEQUANT) {
    const bool fma2 = variant == GLYPR_Q8_INT8_FMA;
    RET_IF(ensure_ws(ctx, q8_act_bytes(m, H) + q8_act_bytes(m, F)));
    Carve c(ctx->ws);
    int8_t* xq = c.take<int8_t>((size_t)(m * H));
    float* dx = c.take<float>((size_t)(m * (H / 32)));
    int8_t* hq = c.take<int8_t>((size_t)(m * F));
    float* dh = c.take<float>((size_t)(m * (F / 32)));
    if (norm)
      LAUNCH(GLYPR_K_RMSNORM_QUANT, s, launch_rmsnorm_quant(x, norm_w, eps, m, H, xq, dx, s),
             "rmsnorm_quant launch");
    else
      LAUNCH(GLYPR_K_QUANTIZE, s, launch_quantize_planar(x, m, H, xq, dx, s), "quantize launch");
    LAUNCH(GLYPR_K_GEMM_I8_GEGLU, s,
           launch_gemm_i8_geglu(xq, dx, gu->qs(), gu->dw(), hq, dh, m, F, H, s, fma2),
           "gate/up GeGLU launch");
    LAUNCH(GLYPR_K_GEMM_I8, s,
           launch_gemm_i8(hq, dh, down->qs(), down->dw(), y, m, H, F, H, s, fma2),
           "down launch");
    return GLYPR_OK;
  }
  RET_IF(ensure_ws(ctx, align_up((size_t)(m * H) * 2, 256) + align_up((size_t)(m * F) * 2, 256)));
  Carve c(ctx->ws);
  uint16_t* xb = c.take<uint16_t>((size_t)(m * H));
  uint16_t* hb = c.take<uint16_t>((size_t)(m * F));
  if (norm)
    LAUNCH(GLYPR_K_RMSNORM_BF16, s, launch_rmsnorm_bf16(x, norm_w, eps, m, H, xb, s),
           "rmsnorm_bf16 launch");
  else
    LAUNCH(GLYPR_K_TO_BF16, s, launch_to_bf16(x, m * H, xb, s), "to_bf16 launch");
  LAUNCH(GLYPR_K_GEMM_BF16_GEGLU, s, launch_gemm_bf16_geglu(xb, gu->qs(), gu->dw(), hb, m, F, H, s),
         "bf16 gate/up GeGLU launch");
  LAUNCH(GLYPR_K_GEMM_BF16, s, launch_gemm_bf16(hb, down->qs(), down->dw(), y, m, H, F, H, s),
         "bf16 down launch");
  return GLYPR_OK;
}

int check_mlp_args(const glypr_q8w* gu, const glypr_q8w* down, const float* x, float* y,
                   int64_t m, int variant) {
  GLYPR_CHECK(m >= 0, GLYPR_ERR_SHAPE, "m = %lld is negative", (long long)m);
  RET_IF(check_variant(variant));
  GLYPR_CHECK(gu != nullptr && down != nullptr, GLYPR_ERR_INVALID_ARG, "weight handle is NULL");
  GLYPR_CHECK(m == 0 || (x != nullptr && y != nullptr), GLYPR_ERR_INVALID_ARG, "x or y is NULL");
  GLYPR_CHECK(aligned16(x) && aligned16(y), GLYPR_ERR_ALIGNMENT,
              "x and y must be 16-byte aligned");
  GLYPR_CHECK(gu->n == 2 * down->k, GLYPR_ERR_SHAPE,
              "gate_up has %lld rows, expected 2 x down.in_dim = %lld", (long long)gu->n,
              (long long)(2 * down->k));
  GLYPR_CHECK(down->n == gu->k, GLYPR_ERR_SHAPE,
              "down.out_dim %lld != gate_up.in_dim %lld", (long long)down->n, (long long)gu->k);
  return GLYPR_OK;
}

}  // namespace
}  // namespace glypr

using namespace glypr;

extern "C" {

const char* glypr_hip_last_error(void) { return g_err; }

int glypr_hip_abi_version(void) { return GLYPR_HIP_ABI_VERSION; }

int glypr_hip_ctx_create(int device, glypr_hip_ctx** out) {
  clear_error();
  GLYPR_CHECK(out != nullptr, GLYPR_ERR_INVALID_ARG, "out is NULL");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  GLYPR_CHECK(e == hipSuccess && count > 0, GLYPR_ERR_DEVICE, "no HIP device available (%s)",
              e == hipSuccess ? "count 0" : hipGetErrorString(e));
  GLYPR_CHECK(device >= 0 && device < count, GLYPR_ERR_DEVICE, "device %d out of range [0,%d)",
              device, count);
  DeviceScope ds(device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  hipDeviceProp_t prop;
  GLYPR_TRY_HIP(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  // this device's no-allocation scratch array (scratch.hip), with the device
  // current; if it cannot be resolved only glypr_hip_q8_0_matmul_noalloc fails
  void* scratch_ptr = nullptr;
  hipError_t se = resolve_scratch(&scratch_ptr);
  if (se == hipSuccess) se = scratch_guard_init(device);
  if (se != hipSuccess) scratch_ptr = nullptr;
  glypr_hip_ctx* ctx = new (std::nothrow) glypr_hip_ctx();
  GLYPR_CHECK(ctx != nullptr, GLYPR_ERR_OOM, "host allocation failed");
  ctx->device = device;
  ctx->cu_count = prop.multiProcessorCount;
  ctx->scratch = scratch_ptr;
  ctx->scratch_err = se;
  *out = ctx;
  return GLYPR_OK;
}

int glypr_hip_ctx_destroy(glypr_hip_ctx* ctx) {
  clear_error();
  if (!ctx) return GLYPR_OK;
  {
    DeviceScope ds(ctx->device);
    (void)hipDeviceSynchronize();
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->ids) (void)hipFree(ctx->ids);
    if (ctx->mask) (void)hipFree(ctx->mask);
    for (auto& kv : ctx->bcos)
      if (kv.second.dev) (void)hipFree(kv.second.dev);
    for (auto& r : ctx->prof) {
      (void)hipEventDestroy(r.start);
      (void)hipEventDestroy(r.stop);
    }
    for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
  }
  delete ctx;
  return GLYPR_OK;
}

int glypr_hip_sync(glypr_hip_ctx* ctx, glypr_stream stream) {
  clear_error();
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  GLYPR_TRY_HIP(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
  return GLYPR_OK;
}

int glypr_hip_ctx_reserve(glypr_hip_ctx* ctx, int64_t rows) {
  clear_error();
  GLYPR_CHECK(rows > 0, GLYPR_ERR_SHAPE, "reserve rows %lld must be positive", (long long)rows);
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  ctx->reserve_rows = rows;
  return reserve_for_weight(ctx, ctx->max_k);
}

int glypr_hip_q8_0_weight_create(glypr_hip_ctx* ctx, const uint8_t* gguf_blocks, int64_t n,
                                 int64_t k, glypr_q8w** out) {
  clear_error();
  GLYPR_CHECK(n > 0 && k > 0, GLYPR_ERR_SHAPE, "weight shape (%lld, %lld) must be positive",
              (long long)n, (long long)k);
  GLYPR_CHECK(k % 32 == 0, GLYPR_ERR_SHAPE, "in_dim %lld is not a multiple of 32",
              (long long)k);
  GLYPR_CHECK(gguf_blocks != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG,
              "gguf_blocks or out is NULL");
  *out = nullptr;
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  const size_t nblk = (size_t)(n * (k / 32));
  Q8Buffer* buf = new (std::nothrow) Q8Buffer();
  GLYPR_CHECK(buf != nullptr, GLYPR_ERR_OOM, "host allocation failed");
  buf->rows = n;
  buf->k = k;
  buf->device = ctx->device;
  uint8_t* tmp = nullptr;
  hipError_t e = hipMalloc((void**)&buf->qs, (size_t)(n * k));
  if (e == hipSuccess) e = hipMalloc((void**)&buf->dw, nblk * sizeof(float));
  if (e == hipSuccess) e = hipMalloc((void**)&tmp, nblk * 34);
  if (e == hipSuccess) e = hipMemcpy(tmp, gguf_blocks, nblk * 34, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_repack(tmp, buf->qs, buf->dw, n, k, nullptr);
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  if (tmp) (void)hipFree(tmp);
  if (e != hipSuccess) {
    if (buf->qs) (void)hipFree(buf->qs);
    if (buf->dw) (void)hipFree(buf->dw);
    delete buf;
    return hip_error(e, "weight upload/repack");
  }
  glypr_q8w* w = new (std::nothrow) glypr_q8w{buf, 0, n, k};
  if (!w) {
    (void)hipFree(buf->qs);
    (void)hipFree(buf->dw);
    delete buf;
    return set_error(GLYPR_ERR_OOM, "host allocation failed");
  }
  {
    std::lock_guard<std::mutex> lk(ctx->mu);
    const int rc = reserve_for_weight(ctx, k);
    if (rc != GLYPR_OK) {
      glypr_hip_q8_0_weight_destroy(w);
      return rc;
    }
  }
  *out = w;
  return GLYPR_OK;
}

int glypr_hip_q8_0_weight_concat(glypr_hip_ctx* ctx, const glypr_q8w* const* parts, int count,
                                 glypr_q8w** fused, glypr_q8w** views) {
  clear_error();
  GLYPR_CHECK(count >= 2, GLYPR_ERR_SHAPE, "concat needs at least 2 parts, got %d", count);
  GLYPR_CHECK(parts != nullptr && fused != nullptr, GLYPR_ERR_INVALID_ARG,
              "parts or fused is NULL");
  *fused = nullptr;
  int64_t rows = 0, k = -1;
  for (int i = 0; i < count; i++) {
    GLYPR_CHECK(parts[i] != nullptr, GLYPR_ERR_INVALID_ARG, "parts[%d] is NULL", i);
    if (k < 0) k = parts[i]->k;
    GLYPR_CHECK(parts[i]->k == k, GLYPR_ERR_SHAPE, "parts[%d] in_dim %lld != %lld", i,
                (long long)parts[i]->k, (long long)k);
    rows += parts[i]->n;
  }
  RET_IF(check_ctx(ctx));
  for (int i = 0; i < count; i++) RET_IF(check_weight_device(ctx, parts[i], "part"));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  Q8Buffer* buf = new (std::nothrow) Q8Buffer();
  GLYPR_CHECK(buf != nullptr, GLYPR_ERR_OOM, "host allocation failed");
  buf->rows = rows;
  buf->k = k;
  buf->device = ctx->device;
  const int64_t nb = k / 32;
  hipError_t e = hipMalloc((void**)&buf->qs, (size_t)(rows * k));
  if (e == hipSuccess) e = hipMalloc((void**)&buf->dw, (size_t)(rows * nb) * sizeof(float));
  int64_t off = 0;
  for (int i = 0; i < count && e == hipSuccess; i++) {
    e = hipMemcpy(buf->qs + off * k, parts[i]->qs(), (size_t)(parts[i]->n * k),
                  hipMemcpyDeviceToDevice);
    if (e == hipSuccess)
      e = hipMemcpy(buf->dw + off * nb, parts[i]->dw(), (size_t)(parts[i]->n * nb) * sizeof(float),
                    hipMemcpyDeviceToDevice);
    off += parts[i]->n;
  }
  if (e != hipSuccess) {
    if (buf->qs) (void)hipFree(buf->qs);
    if (buf->dw) (void)hipFree(buf->dw);
    delete buf;
    return hip_error(e, "concat copy");
  }
  {
    std::lock_guard<std::mutex> lk(ctx->mu);
    const int rc = reserve_for_weight(ctx, k);
    if (rc != GLYPR_OK) {
      (void)hipFree(buf->qs);
      (void)hipFree(buf->dw);
      delete buf;
      return rc;
    }
  }
  glypr_q8w* f = new glypr_q8w{buf, 0, rows, k};
  if (views) {
    int64_t r0 = 0;
    for (int i = 0; i < count; i++) {
      buf->refs.fetch_add(1);
      views[i] = new glypr_q8w{buf, r0, parts[i]->n, k};
      r0 += parts[i]->n;
    }
  }
  *fused = f;
  return GLYPR_OK;
}

int glypr_hip_q8_0_weight_view(const glypr_q8w* w, int64_t row0, int64_t rows, glypr_q8w** out) {
  clear_error();
  GLYPR_CHECK(w != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG, "w or out is NULL");
  GLYPR_CHECK(row0 >= 0 && rows > 0 && row0 + rows <= w->n, GLYPR_ERR_SHAPE,
              "view [%lld, %lld) outside %lld rows", (long long)row0, (long long)(row0 + rows),
              (long long)w->n);
  w->buf->refs.fetch_add(1);
  *out = new glypr_q8w{w->buf, w->row0 + row0, rows, w->k};
  return GLYPR_OK;
}

int glypr_hip_q8_0_weight_destroy(glypr_q8w* w) {
  clear_error();
  if (!w) return GLYPR_OK;
  Q8Buffer* buf = w->buf;
  delete w;
  if (buf->refs.fetch_sub(1) == 1) {
    DeviceScope ds(buf->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(buf->qs);
    (void)hipFree(buf->dw);
    delete buf;
  }
  return GLYPR_OK;
}

int glypr_hip_q8_0_weight_shape(const glypr_q8w* w, int64_t* n, int64_t* k) {
  clear_error();
  GLYPR_CHECK(w != nullptr, GLYPR_ERR_INVALID_ARG, "w is NULL");
  if (n) *n = w->n;
  if (k) *k = w->k;
  return GLYPR_OK;
}

int glypr_hip_q8_0_dequantize(glypr_hip_ctx* ctx, const glypr_q8w* w, float* out,
                              glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(w != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG, "w or out is NULL");
  GLYPR_CHECK(aligned16(out), GLYPR_ERR_ALIGNMENT, "out must be 16-byte aligned");
  RET_IF(check_ctx(ctx));
  RET_IF(check_weight_device(ctx, w, "w"));
  DeviceScope ds(ctx->device);
  LAUNCH(GLYPR_K_DEQUANT, (hipStream_t)stream,
         launch_dequant(w->qs(), w->dw(), w->n, w->k, out, (hipStream_t)stream),
         "dequantize launch");
  return GLYPR_OK;
}

int glypr_hip_bf16_weight_create(glypr_hip_ctx* ctx, const uint16_t* bf16_rows, int64_t n,
                                 int64_t k, glypr_bf16w** out) {
  clear_error();
  GLYPR_CHECK(out != nullptr && bf16_rows != nullptr, GLYPR_ERR_INVALID_ARG,
              "bf16_rows or out is NULL");
  *out = nullptr;
  GLYPR_CHECK(n > 0 && k > 0, GLYPR_ERR_SHAPE, "weight shape (%lld, %lld) must be positive",
              (long long)n, (long long)k);
  GLYPR_CHECK(k % 64 == 0, GLYPR_ERR_UNSUPPORTED,
              "in_dim %lld: dense bf16 weights need a multiple of 64", (long long)k);
  GLYPR_CHECK(2 * n * k < (int64_t(1) << 31), GLYPR_ERR_SHAPE, "weight of %lld x %lld too large",
              (long long)n, (long long)k);
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  glypr_bf16w* w = new (std::nothrow) glypr_bf16w();
  GLYPR_CHECK(w != nullptr, GLYPR_ERR_OOM, "host allocation failed");
  w->n = n;
  w->k = k;
  w->device = ctx->device;
  hipError_t e = hipMalloc((void**)&w->p, (size_t)(n * k) * 2);
  if (e == hipSuccess) e = hipMemcpy(w->p, bf16_rows, (size_t)(n * k) * 2, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    if (w->p) (void)hipFree(w->p);
    delete w;
    return hip_error(e, "bf16 weight upload");
  }
  {
    std::lock_guard<std::mutex> lk(ctx->mu);
    const int rc = reserve_for_weight(ctx, k);
    if (rc != GLYPR_OK) {
      glypr_hip_bf16_weight_destroy(w);
      return rc;
    }
  }
  *out = w;
  return GLYPR_OK;
}

int glypr_hip_bf16_weight_destroy(glypr_bf16w* w) {
  clear_error();
  if (!w) return GLYPR_OK;
  {
    DeviceScope ds(w->device);
    if (w->p) (void)hipFree(w->p);
  }
  delete w;
  return GLYPR_OK;
}

int glypr_hip_bf16_matmul(glypr_hip_ctx* ctx, const glypr_bf16w* w, const float* x, float* y,
                          int64_t m, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(m >= 0, GLYPR_ERR_SHAPE, "m = %lld is negative", (long long)m);
  GLYPR_CHECK(w != nullptr, GLYPR_ERR_INVALID_ARG, "w is NULL");
  GLYPR_CHECK(m == 0 || (x != nullptr && y != nullptr), GLYPR_ERR_INVALID_ARG, "x or y is NULL");
  GLYPR_CHECK(aligned16(x) && aligned16(y), GLYPR_ERR_ALIGNMENT, "x and y must be 16-byte aligned");
  GLYPR_CHECK(2 * m * w->k < (int64_t(1) << 31), GLYPR_ERR_SHAPE, "m = %lld too large",
              (long long)m);
  RET_IF(check_ctx(ctx));
  GLYPR_CHECK(w->device == ctx->device, GLYPR_ERR_DEVICE,
              "w lives on device %d, context is device %d", w->device, ctx->device);
  if (m == 0) return GLYPR_OK;
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  hipStream_t s = (hipStream_t)stream;
  RET_IF(ensure_ws(ctx, align_up((size_t)(m * w->k) * 2, 256)));
  uint16_t* xb = reinterpret_cast<uint16_t*>(ctx->ws);
  LAUNCH(GLYPR_K_TO_BF16, s, launch_to_bf16(x, m * w->k, xb, s), "to_bf16 launch");
  LAUNCH(GLYPR_K_GEMM_BF16W, s, launch_gemm_bf16w(xb, w->p, y, m, w->n, w->k, w->n, s),
         "gemm_bf16w launch");
  return GLYPR_OK;
}

int glypr_hip_q8_0_quantize(glypr_hip_ctx* ctx, const float* x, int64_t m, int64_t k,
                            uint8_t* out_blocks, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(m >= 0 && k > 0, GLYPR_ERR_SHAPE, "shape (%lld, %lld) invalid", (long long)m,
              (long long)k);
  GLYPR_CHECK(k % 32 == 0, GLYPR_ERR_SHAPE, "k %lld is not a multiple of 32", (long long)k);
  GLYPR_CHECK(x != nullptr && out_blocks != nullptr, GLYPR_ERR_INVALID_ARG,
              "x or out_blocks is NULL");
  GLYPR_CHECK(aligned16(x) && ((uintptr_t)out_blocks & 1u) == 0, GLYPR_ERR_ALIGNMENT,
              "x must be 16-byte and out_blocks 2-byte aligned");
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  LAUNCH(GLYPR_K_QUANTIZE, (hipStream_t)stream,
         launch_quantize_gguf(x, m, k, out_blocks, (hipStream_t)stream), "quantize launch");
  return GLYPR_OK;
}

int glypr_hip_q8_0_matmul(glypr_hip_ctx* ctx, const glypr_q8w* w, const float* x, float* y,
                          int64_t m, int variant, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(m >= 0, GLYPR_ERR_SHAPE, "m = %lld is negative", (long long)m);
  RET_IF(check_variant(variant));
  GLYPR_CHECK(w != nullptr, GLYPR_ERR_INVALID_ARG, "w is NULL");
  GLYPR_CHECK(m == 0 || (x != nullptr && y != nullptr), GLYPR_ERR_INVALID_ARG, "x or y is NULL");
  GLYPR_CHECK(aligned16(x) && aligned16(y), GLYPR_ERR_ALIGNMENT,
              "x and y must be 16-byte aligned");
  RET_IF(check_ctx(ctx));
  RET_IF(check_weight_device(ctx, w, "w"));
  if (m == 0) return GLYPR_OK;
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  return matmul_ws(ctx, w, x, nullptr, 0.0f, false, y, m, variant, (hipStream_t)stream);
}

int glypr_hip_q8_0_matmul_noalloc(glypr_hip_ctx* ctx, const glypr_q8w* w, const float* x,
                                  float* y, int64_t m, int variant, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(m >= 0, GLYPR_ERR_SHAPE, "m = %lld is negative", (long long)m);
  RET_IF(check_variant(variant));
  GLYPR_CHECK(w != nullptr, GLYPR_ERR_INVALID_ARG, "w is NULL");
  // every operand form takes at least m * k bytes: bound m before the byte
  // count is formed, so that it cannot wrap
  GLYPR_CHECK(m <= (int64_t)(GLYPR_NOALLOC_SCRATCH_BYTES / (size_t)w->k), GLYPR_ERR_SHAPE,
              "m = %lld, k = %lld exceeds the no-allocation matmul's %zu bytes of activation "
              "scratch",
              (long long)m, (long long)w->k, (size_t)GLYPR_NOALLOC_SCRATCH_BYTES);
  const size_t need = matmul_ws_bytes(m, w->n, w->k, false, variant);
  GLYPR_CHECK(need <= GLYPR_NOALLOC_SCRATCH_BYTES, GLYPR_ERR_SHAPE,
              "m = %lld, k = %lld needs %zu bytes of activation scratch; the no-allocation "
              "matmul has %zu",
              (long long)m, (long long)w->k, need, (size_t)GLYPR_NOALLOC_SCRATCH_BYTES);
  GLYPR_CHECK(m == 0 || (x != nullptr && y != nullptr), GLYPR_ERR_INVALID_ARG, "x or y is NULL");
  GLYPR_CHECK(aligned16(x) && aligned16(y), GLYPR_ERR_ALIGNMENT,
              "x and y must be 16-byte aligned");
  RET_IF(check_ctx(ctx));
  RET_IF(check_weight_device(ctx, w, "w"));
  GLYPR_CHECK(ctx->scratch != nullptr, GLYPR_ERR_DEVICE,
              "no scratch address for device %d (hipGetSymbolAddress: %s)", ctx->device,
              hipGetErrorString(ctx->scratch_err));
  if (m == 0) return GLYPR_OK;
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  ScratchGuard* g = scratch_guard(ctx->device);
  GLYPR_CHECK(g != nullptr, GLYPR_ERR_DEVICE, "no scratch guard for device %d", ctx->device);
  const hipStream_t s = (hipStream_t)stream;
  std::lock_guard<std::mutex> gl(g->mu);
  // a stream under graph capture runs later, at replay: nothing to check now
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const bool eager = hipStreamIsCapturing(s, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone;
  if (!eager) (void)hipGetLastError();
  if (eager && g->armed && g->last != s) {
    const hipError_t q = hipEventQuery(g->done);
    if (q == hipErrorNotReady) {
      (void)hipGetLastError();
      return set_error(GLYPR_ERR_BUSY,
                       "the no-allocation scratch of device %d is in use by a pending call on "
                       "another stream",
                       ctx->device);
    }
    if (q != hipSuccess) return hip_error(q, "hipEventQuery (scratch guard)");
  }
  std::lock_guard<std::mutex> lk(ctx->mu);
  ctx->no_events = true;
  const int rc = matmul_impl(ctx, w, x, nullptr, 0.0f, false, y, m, variant, ctx->scratch, s);
  ctx->no_events = false;
  if (rc == GLYPR_OK && eager) {
    GLYPR_TRY_HIP(hipEventRecord(g->done, s), "hipEventRecord (scratch guard)");
    g->last = s;
    g->armed = true;
  }
  return rc;
}

int glypr_hip_rmsnorm(glypr_hip_ctx* ctx, const float* x, const float* weight, float eps,
                      float* y, int64_t rows, int64_t dim, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(rows >= 0 && dim > 0, GLYPR_ERR_SHAPE, "shape (%lld, %lld) invalid",
              (long long)rows, (long long)dim);
  GLYPR_CHECK(rows == 0 || (x != nullptr && y != nullptr), GLYPR_ERR_INVALID_ARG, "x or y is NULL");
  RET_IF(check_ctx(ctx));
  if (rows == 0) return GLYPR_OK;
  DeviceScope ds(ctx->device);
  LAUNCH(GLYPR_K_RMSNORM, (hipStream_t)stream,
         launch_rmsnorm(x, weight, eps, y, rows, dim, (hipStream_t)stream), "rmsnorm launch");
  return GLYPR_OK;
}

int glypr_hip_rmsnorm_q8_0_matmul(glypr_hip_ctx* ctx, const glypr_q8w* w, const float* x,
                                  const float* norm_weight, float eps, float* y, int64_t m,
                                  int variant, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(m >= 0, GLYPR_ERR_SHAPE, "m = %lld is negative", (long long)m);
  RET_IF(check_variant(variant));
  GLYPR_CHECK(w != nullptr, GLYPR_ERR_INVALID_ARG, "w is NULL");
  GLYPR_CHECK(m == 0 || (x != nullptr && y != nullptr), GLYPR_ERR_INVALID_ARG, "x or y is NULL");
  GLYPR_CHECK(aligned16(x) && aligned16(y) && aligned16(norm_weight), GLYPR_ERR_ALIGNMENT,
              "x, y and norm_weight must be 16-byte aligned");
  RET_IF(check_ctx(ctx));
  RET_IF(check_weight_device(ctx, w, "w"));
  if (m == 0) return GLYPR_OK;
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  return matmul_ws(ctx, w, x, norm_weight, eps, true, y, m, variant, (hipStream_t)stream);
}

int glypr_hip_geglu(glypr_hip_ctx* ctx, const float* gate, const float* up, float* out,
                    int64_t n, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(n >= 0, GLYPR_ERR_SHAPE, "n = %lld is negative", (long long)n);
  GLYPR_CHECK(gate != nullptr && up != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG,
              "gate, up or out is NULL");
  RET_IF(check_ctx(ctx));
  if (n == 0) return GLYPR_OK;
  DeviceScope ds(ctx->device);
  LAUNCH(GLYPR_K_GEGLU, (hipStream_t)stream, launch_geglu(gate, up, out, n, (hipStream_t)stream),
         "geglu launch");
  return GLYPR_OK;
}

int glypr_hip_mlp(glypr_hip_ctx* ctx, const glypr_q8w* gate_up, const glypr_q8w* down,
                  const float* x, float* y, int64_t m, int variant, glypr_stream stream) {
  clear_error();
  RET_IF(check_mlp_args(gate_up, down, x, y, m, variant));
  RET_IF(check_ctx(ctx));
  RET_IF(check_weight_device(ctx, gate_up, "gate_up"));
  RET_IF(check_weight_device(ctx, down, "down"));
  if (m == 0) return GLYPR_OK;
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  return mlp_impl(ctx, gate_up, down, x, nullptr, 0.0f, false, y, m, variant,
                  (hipStream_t)stream);
}

int glypr_hip_rmsnorm_mlp(glypr_hip_ctx* ctx, const glypr_q8w* gate_up, const glypr_q8w* down,
                          const float* x, const float* norm_weight, float eps, float* y,
                          int64_t m, int variant, glypr_stream stream) {
  clear_error();
  RET_IF(check_mlp_args(gate_up, down, x, y, m, variant));
  GLYPR_CHECK(aligned16(norm_weight), GLYPR_ERR_ALIGNMENT, "norm_weight must be 16-byte aligned");
  RET_IF(check_ctx(ctx));
  RET_IF(check_weight_device(ctx, gate_up, "gate_up"));
  RET_IF(check_weight_device(ctx, down, "down"));
  if (m == 0) return GLYPR_OK;
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  return mlp_impl(ctx, gate_up, down, x, norm_weight, eps, true, y, m, variant,
                  (hipStream_t)stream);
}

int glypr_hip_q8_0_embed_gather(glypr_hip_ctx* ctx, const glypr_q8w* table, const uint32_t* ids,
                                int64_t n_ids, float scale, float* out, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(n_ids >= 0, GLYPR_ERR_SHAPE, "n_ids = %lld is negative", (long long)n_ids);
  GLYPR_CHECK(table != nullptr, GLYPR_ERR_INVALID_ARG, "table is NULL");
  GLYPR_CHECK((ids != nullptr || n_ids == 0) && out != nullptr, GLYPR_ERR_INVALID_ARG,
              "ids or out is NULL");
  GLYPR_CHECK(aligned16(out), GLYPR_ERR_ALIGNMENT, "out must be 16-byte aligned");
  for (int64_t i = 0; i < n_ids; i++)
    GLYPR_CHECK((int64_t)ids[i] < table->n, GLYPR_ERR_RANGE,
                "token id %u at position %lld is out of range for vocab %lld", ids[i],
                (long long)i, (long long)table->n);
  RET_IF(check_ctx(ctx));
  RET_IF(check_weight_device(ctx, table, "table"));
  if (n_ids == 0) return GLYPR_OK;
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  if (gather_host_ids_ok(table->k, n_ids)) {   // the ids travel in the kernel arguments
    LAUNCH(GLYPR_K_GATHER, (hipStream_t)stream,
           launch_gather_host_ids(table->qs(), table->dw(), table->k, ids, n_ids, scale, out,
                                  (hipStream_t)stream),
           "gather launch");
    return GLYPR_OK;
  }
  RET_IF(ensure_staging(ctx->ids, ctx->ids_cap, (size_t)n_ids));
  GLYPR_TRY_HIP(hipMemcpyAsync(ctx->ids, ids, (size_t)n_ids * 4, hipMemcpyHostToDevice,
                               (hipStream_t)stream),
                "ids upload");
  LAUNCH(GLYPR_K_GATHER, (hipStream_t)stream,
         launch_gather(table->qs(), table->dw(), table->k, ctx->ids, n_ids, scale, out,
                       (hipStream_t)stream),
         "gather launch");
  return GLYPR_OK;
}

int glypr_hip_pool_normalize(glypr_hip_ctx* ctx, const float* tokens, const uint8_t* mask,
                             int64_t t, int64_t d, int64_t trunc, float* out,
                             glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(t > 0 && d > 0 && trunc >= 0, GLYPR_ERR_SHAPE, "shape (t=%lld, d=%lld, trunc=%lld)",
              (long long)t, (long long)d, (long long)trunc);
  GLYPR_CHECK(tokens != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG,
              "tokens or out is NULL");
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  RET_IF(ensure_ws(ctx, pool_scratch_floats(t, d) * sizeof(float)));
  const uint8_t* dmask = nullptr;
  if (mask) {
    RET_IF(ensure_staging(ctx->mask, ctx->mask_cap, (size_t)t));
    GLYPR_TRY_HIP(hipMemcpyAsync(ctx->mask, mask, (size_t)t, hipMemcpyHostToDevice,
                                 (hipStream_t)stream),
                  "mask upload");
    dmask = ctx->mask;
  }
  LAUNCH(GLYPR_K_POOL, (hipStream_t)stream,
         launch_pool(tokens, dmask, t, d, trunc, out, (float*)ctx->ws, (hipStream_t)stream),
         "pool launch");
  return GLYPR_OK;
}

// ---- output-vector codecs (util.rs:52-197) -------------------------------

int glypr_hip_quantize_binary(glypr_hip_ctx* ctx, const float* x, int64_t n, int64_t dim,
                              uint64_t* out, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(n >= 0 && dim > 0, GLYPR_ERR_SHAPE, "shape (n=%lld, dim=%lld)", (long long)n,
              (long long)dim);
  GLYPR_CHECK(dim % 64 == 0, GLYPR_ERR_SHAPE,
              "binary quantization requires dim to be a multiple of 64, got %lld",
              (long long)dim);
  GLYPR_CHECK(x != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG, "x or out is NULL");
  GLYPR_CHECK(aligned16(x) && aligned16(out), GLYPR_ERR_ALIGNMENT,
              "x and out must be 16-byte aligned");
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  LAUNCH(GLYPR_K_VEC_ENCODE, (hipStream_t)stream,
         launch_quantize_binary(x, n, dim, out, (hipStream_t)stream), "quantize_binary launch");
  return GLYPR_OK;
}

int glypr_hip_quantize_int8(glypr_hip_ctx* ctx, const float* x, int64_t count, int8_t* out,
                            glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(count >= 0, GLYPR_ERR_SHAPE, "count %lld", (long long)count);
  GLYPR_CHECK(x != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG, "x or out is NULL");
  GLYPR_CHECK(aligned16(x) && aligned16(out), GLYPR_ERR_ALIGNMENT,
              "x and out must be 16-byte aligned");
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  LAUNCH(GLYPR_K_VEC_ENCODE, (hipStream_t)stream,
         launch_quantize_int8(x, count, out, (hipStream_t)stream), "quantize_int8 launch");
  return GLYPR_OK;
}

static int check_pairs(int64_t na, int64_t nb, int64_t len, const void* a, const void* b,
                       const void* out) {
  GLYPR_CHECK(na >= 0 && nb >= 0 && len >= 0, GLYPR_ERR_SHAPE, "shape (na=%lld, nb=%lld, %lld)",
              (long long)na, (long long)nb, (long long)len);
  GLYPR_CHECK(a != nullptr && b != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG,
              "a, b or out is NULL");
  GLYPR_CHECK(aligned16(a) && aligned16(b) && aligned16(out), GLYPR_ERR_ALIGNMENT,
              "a, b and out must be 16-byte aligned");
  return GLYPR_OK;
}

int glypr_hip_hamming(glypr_hip_ctx* ctx, const uint64_t* a, int64_t na, const uint64_t* b,
                      int64_t nb, int64_t words, uint32_t* out, glypr_stream stream) {
  clear_error();
  RET_IF(check_pairs(na, nb, words, a, b, out));
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  LAUNCH(GLYPR_K_VEC_SEARCH, (hipStream_t)stream,
         launch_hamming(a, na, b, nb, words, out, (hipStream_t)stream), "hamming launch");
  return GLYPR_OK;
}

int glypr_hip_binary_cosine(glypr_hip_ctx* ctx, const uint64_t* a, int64_t na,
                            const uint64_t* b, int64_t nb, int64_t words, float* out,
                            glypr_stream stream) {
  clear_error();
  RET_IF(check_pairs(na, nb, words, a, b, out));
  GLYPR_CHECK(words <= (int64_t(1) << 20), GLYPR_ERR_SHAPE, "words %lld > 2^20",
              (long long)words);
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  const int64_t dim = words * 64;
  auto it = ctx->bcos.find(dim);
  if (it == ctx->bcos.end()) {
    // binary_cosine_similarity evaluates (PI * (h as f32 / dim as f32)).cos() in
    // f32 with the platform libm; h is an integer in [0, dim], so the table is
    // that exact expression per h.  dim 0 -> 1.0 (the reference's early return).
    // One table per dim, written once by an upload ordered on this stream.
    glypr_hip_ctx::CosTable tab;
    tab.host.resize((size_t)dim + 1);
    const float pi = 3.14159265358979323846f;
    for (int64_t h = 0; h <= dim; h++)
      tab.host[(size_t)h] = dim == 0 ? 1.0f : cosf(pi * ((float)h / (float)dim));
    GLYPR_TRY_HIP(hipMalloc((void**)&tab.dev, tab.host.size() * sizeof(float)),
                  "binary cosine table: hipMalloc");
    it = ctx->bcos.emplace(dim, std::move(tab)).first;
    GLYPR_TRY_HIP(hipMemcpyAsync(it->second.dev, it->second.host.data(),
                                 it->second.host.size() * sizeof(float), hipMemcpyHostToDevice,
                                 (hipStream_t)stream),
                  "binary cosine table upload");
  }
  LAUNCH(GLYPR_K_VEC_SEARCH, (hipStream_t)stream,
         launch_binary_cosine(a, na, b, nb, words, it->second.dev, out, (hipStream_t)stream),
         "binary_cosine launch");
  return GLYPR_OK;
}

int glypr_hip_int8_dot(glypr_hip_ctx* ctx, const int8_t* a, int64_t na, const int8_t* b,
                       int64_t nb, int64_t dim, int32_t* out, glypr_stream stream) {
  clear_error();
  RET_IF(check_pairs(na, nb, dim, a, b, out));
  GLYPR_CHECK(dim <= 65536, GLYPR_ERR_SHAPE, "dim %lld > 65536 (i32 sums must not wrap)",
              (long long)dim);
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  LAUNCH(GLYPR_K_VEC_SEARCH, (hipStream_t)stream,
         launch_int8_dot(a, na, b, nb, dim, out, (hipStream_t)stream), "int8_dot launch");
  return GLYPR_OK;
}

int glypr_hip_int8_cosine(glypr_hip_ctx* ctx, const int8_t* a, int64_t na, const int8_t* b,
                          int64_t nb, int64_t dim, float* out, glypr_stream stream) {
  clear_error();
  RET_IF(check_pairs(na, nb, dim, a, b, out));
  GLYPR_CHECK(dim <= 65536, GLYPR_ERR_SHAPE, "dim %lld > 65536 (i32 sums must not wrap)",
              (long long)dim);
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  RET_IF(ensure_ws(ctx, (size_t)na * sizeof(int32_t)));
  LAUNCH(GLYPR_K_VEC_SEARCH, (hipStream_t)stream,
         launch_int8_cosine(a, na, b, nb, dim, (int32_t*)ctx->ws, out, (hipStream_t)stream),
         "int8_cosine launch");
  return GLYPR_OK;
}

// Not part of the public header: the INT8_EXACT GEMM route (GEMM_ROUTE_*) for a
// shape, and whether the prologue-fused kernel takes it, so host tests can pin
// the routing without a GPU.
int glypr_internal_gemm_i8_route(int64_t m, int64_t n, int64_t k, int prologue) {
  if (prologue == 1 || prologue == 2) return gemm_i8_pro_ok(m, n, k, prologue == 2) ? 4 : -1;
  return gemm_i8_route(m, n, k);
}

static const char* const kKernelNames[GLYPR_K_COUNT] = {
    "quantize",   "rmsnorm_quant",  "gemm_i8", "gemm_i8_geglu", "to_bf16", "rmsnorm_bf16",
    "gemm_bf16",  "gemm_bf16_geglu", "rmsnorm", "geglu",         "gather",  "dequant",
    "pool",       "qkv_post",       "attention", "residual_norm", "vec_encode", "vec_search",
    "gemm_i8_pro", "gemm_bf16w",   "gemm_i8_qkv"};

const char* glypr_hip_kernel_name(int id) {
  return (id >= 0 && id < GLYPR_K_COUNT) ? kKernelNames[id] : "";
}

static int drain_profile(glypr_hip_ctx* ctx) {
  int rc = GLYPR_OK;
  for (auto& r : ctx->prof) {
    float ms = 0.0f;
    hipError_t e = hipEventSynchronize(r.stop);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.start, r.stop);
    if (e != hipSuccess && rc == GLYPR_OK) rc = hip_error(e, "profile event");
    ctx->prof_ms[r.kernel] += ms;
    ctx->prof_n[r.kernel] += 1;
    ctx->event_pool.push_back(r.start);
    ctx->event_pool.push_back(r.stop);
  }
  ctx->prof.clear();
  return rc;
}

int glypr_hip_profile_enable(glypr_hip_ctx* ctx, int enable) {
  clear_error();
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  std::lock_guard<std::mutex> lk(ctx->mu);
  int rc = drain_profile(ctx);
  for (int i = 0; i < GLYPR_K_COUNT; i++) {
    ctx->prof_ms[i] = 0.0;
    ctx->prof_n[i] = 0;
  }
  ctx->profiling = enable != 0;
  return rc;
}

int glypr_hip_profile_read(glypr_hip_ctx* ctx, double* total_ms, int64_t* launches) {
  clear_error();
  GLYPR_CHECK(total_ms != nullptr && launches != nullptr, GLYPR_ERR_INVALID_ARG,
              "total_ms or launches is NULL");
  RET_IF(check_ctx(ctx));
  DeviceScope ds(ctx->device);
  std::lock_guard<std::mutex> lk(ctx->mu);
  int rc = drain_profile(ctx);
  for (int i = 0; i < GLYPR_K_COUNT; i++) {
    total_ms[i] = ctx->prof_ms[i];
    launches[i] = ctx->prof_n[i];
  }
  return rc;
}

}  // extern "C"
