// host_common.hpp — host-side helpers shared by the C ABI and the model
// driver: error macros, device scoping, workspace growth, per-kernel timing.
#pragma once

#include <hip/hip_runtime.h>

#include "internal.hpp"

namespace glypr {

void clear_error();  // capi.hip

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

#define GLYPR_TRY_HIP(expr, what)              \
  do {                                         \
    hipError_t e_ = (expr);                    \
    if (e_ != hipSuccess) return hip_error(e_, what); \
  } while (0)

#define GLYPR_CHECK(cond, code, ...)                     \
  do {                                                   \
    if (!(cond)) return set_error(code, __VA_ARGS__);    \
  } while (0)

#define RET_IF(x)              \
  do {                         \
    int rc_ = (x);             \
    if (rc_ != GLYPR_OK) return rc_; \
  } while (0)

// Make ctx->device current for the duration of a call.
struct DeviceScope {
  int prev = -1;
  bool changed = false;
  hipError_t err = hipSuccess;
  explicit DeviceScope(int dev) {
    err = hipGetDevice(&prev);
    if (err == hipSuccess && prev != dev) {
      err = hipSetDevice(dev);
      changed = err == hipSuccess;
    }
  }
  ~DeviceScope() {
    if (changed) (void)hipSetDevice(prev);
  }
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Grow the context workspace to at least `bytes`.  Growth waits for the device
// so no queued kernel still reads the old buffer.
inline int ensure_ws(glypr_hip_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->ws_cap) return GLYPR_OK;
  size_t cap = align_up(bytes + bytes / 4, 1 << 21);
  if (ctx->ws) {
    GLYPR_TRY_HIP(hipDeviceSynchronize(), "workspace growth: hipDeviceSynchronize");
    GLYPR_TRY_HIP(hipFree(ctx->ws), "workspace growth: hipFree");
    ctx->ws = nullptr;
    ctx->ws_cap = 0;
  }
  GLYPR_TRY_HIP(hipMalloc(&ctx->ws, cap), "workspace: hipMalloc");
  ctx->ws_cap = cap;
  return GLYPR_OK;
}

inline size_t q8_act_bytes(int64_t m, int64_t k);

// Workspace that any entry point needs for `rows` rows of a weight with in_dim
// k: two activation operands (the MLP's x and h; each the larger of the Q8_0
// planar form and the bf16 form) of up to k columns.
inline size_t ws_bytes_for(int64_t rows, int64_t k) {
  const size_t q8 = q8_act_bytes(rows, k);
  const size_t bf = align_up((size_t)(rows * k) * 2, 256);
  return 2 * (q8 > bf ? q8 : bf);
}

// A weight with in_dim k was created: size the workspace for it at the
// context's reserve rows, so calls within the reserve allocate nothing.
template <typename T>
inline int ensure_staging(T*& ptr, size_t& cap, size_t count);

inline int reserve_for_weight(glypr_hip_ctx* ctx, int64_t k) {
  if (k > ctx->max_k) ctx->max_k = k;
  RET_IF(ensure_staging(ctx->ids, ctx->ids_cap, (size_t)ctx->reserve_rows));
  RET_IF(ensure_staging(ctx->mask, ctx->mask_cap, (size_t)ctx->reserve_rows));
  return ensure_ws(ctx, ws_bytes_for(ctx->reserve_rows, ctx->max_k));
}

template <typename T>
inline int ensure_staging(T*& ptr, size_t& cap, size_t count) {
  if (count <= cap) return GLYPR_OK;
  size_t n = align_up(count, 4096);
  if (ptr) {
    GLYPR_TRY_HIP(hipDeviceSynchronize(), "staging growth: hipDeviceSynchronize");
    GLYPR_TRY_HIP(hipFree(ptr), "staging growth: hipFree");
    ptr = nullptr;
    cap = 0;
  }
  GLYPR_TRY_HIP(hipMalloc((void**)&ptr, n * sizeof(T)), "staging: hipMalloc");
  cap = n;
  return GLYPR_OK;
}

// Bump allocator over the workspace.
struct Carve {
  char* base;
  size_t off = 0;
  explicit Carve(void* b) : base((char*)b) {}
  template <typename T>
  T* take(size_t count) {
    off = align_up(off, 256);
    T* p = (T*)(base + off);
    off += count * sizeof(T);
    return p;
  }
};

inline size_t q8_act_bytes(int64_t m, int64_t k) {
  return align_up((size_t)(m * k), 256) + align_up((size_t)(m * (k / 32)) * 4, 256);
}

inline int check_ctx(glypr_hip_ctx* ctx) {
  GLYPR_CHECK(ctx != nullptr, GLYPR_ERR_INVALID_ARG, "ctx is NULL");
  return GLYPR_OK;
}

inline int check_weight_device(const glypr_hip_ctx* ctx, const glypr_q8w* w, const char* name) {
  GLYPR_CHECK(w->buf->device == ctx->device, GLYPR_ERR_DEVICE,
              "%s lives on device %d, context is device %d", name, w->buf->device, ctx->device);
  return GLYPR_OK;
}

inline int check_variant(int variant) {
  GLYPR_CHECK(variant == GLYPR_Q8_INT8_EXACT || variant == GLYPR_Q8_BF16_DEQUANT ||
                  variant == GLYPR_Q8_INT8_FMA,
              GLYPR_ERR_UNSUPPORTED, "unknown Q8_0 variant %d", variant);
  return GLYPR_OK;
}


inline hipEvent_t get_event(glypr_hip_ctx* ctx) {
  if (!ctx->event_pool.empty()) {
    hipEvent_t e = ctx->event_pool.back();
    ctx->event_pool.pop_back();
    return e;
  }
  // No system-scope release: a timing marker must not add an L2 write-back
  // between the kernels it brackets.
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return e;
}

// While profiling is on, brackets one kernel launch with events on its stream.
struct ProfScope {
  glypr_hip_ctx* ctx;
  int kernel;
  hipStream_t s;
  hipEvent_t a = nullptr, b = nullptr;
  ProfScope(glypr_hip_ctx* c, int k, hipStream_t st) : ctx(c), kernel(k), s(st) {
    if (!ctx->profiling || ctx->no_events) return;   // events may be created on demand
    a = get_event(ctx);
    b = get_event(ctx);
    if (a && b) (void)hipEventRecord(a, s);
  }
  ~ProfScope() {
    if (a && b) {
      (void)hipEventRecord(b, s);
      ctx->prof.push_back({kernel, a, b});
    }
  }
};

#define LAUNCH(kid, s, expr, what)                       \
  do {                                                   \
    ProfScope ps_(ctx, kid, s);                          \
    hipError_t e_ = (expr);                              \
    if (e_ != hipSuccess) return hip_error(e_, what);    \
  } while (0)


}  // namespace glypr
