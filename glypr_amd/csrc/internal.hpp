// internal.hpp — host-side structures and kernel launchers of libglypr_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

#include "glypr_hip.h"

// Device-resident Q8_0 weight, repacked once at load:
//   qs: int8 [rows][k]      (16-byte aligned rows; k % 32 == 0)
//   dw: f32  [rows][k/32]   (f32 of the GGUF f16 scale: exact)
struct Q8Buffer {
  int8_t* qs = nullptr;
  float* dw = nullptr;
  int64_t rows = 0, k = 0;
  int device = 0;
  std::atomic<int> refs{1};
};

struct glypr_q8w {
  Q8Buffer* buf;
  int64_t row0;  // first row of this view inside buf
  int64_t n, k;  // out_dim, in_dim
  const int8_t* qs() const { return buf->qs + row0 * k; }
  const float* dw() const { return buf->dw + row0 * (k / 32); }
};

struct glypr_bf16w {
  uint16_t* p = nullptr;  // [n][k] bf16
  int64_t n = 0, k = 0;
  int device = 0;
};

struct ProfRec {
  int kernel;
  hipEvent_t start, stop;
};

struct glypr_hip_ctx {
  int device = 0;
  bool profiling = false;
  std::vector<ProfRec> prof;          // recorded, not yet read
  std::vector<hipEvent_t> event_pool; // reusable events
  double prof_ms[GLYPR_K_COUNT] = {};
  int64_t prof_n[GLYPR_K_COUNT] = {};
  int cu_count = 0;
  std::mutex mu;
  void* ws = nullptr;       // activation workspace (quantized operands)
  size_t ws_cap = 0;
  uint32_t* ids = nullptr;  // token-id staging for the gather
  size_t ids_cap = 0;
  uint8_t* mask = nullptr;  // pooling-mask staging
  size_t mask_cap = 0;
  // Binary-cosine tables cos(pi * h / dim), h = 0 .. dim, one per dim, never
  // rewritten: the host copy stays alive until the stream-ordered upload has
  // read it, and a kernel queued earlier never sees its table change.
  struct CosTable {
    float* dev = nullptr;
    std::vector<float> host;
  };
  std::map<int64_t, CosTable> bcos;
  int64_t reserve_rows = 8320;  // rows the workspace is sized for (lib.rs:47)
  // device address of this device's no-allocation scratch array (capi.hip),
  // resolved once at context creation
  void* scratch = nullptr;
  hipError_t scratch_err = hipSuccess;
  bool no_events = false;       // a no-allocation call is running: no profile events
  int64_t max_k = 0;            // largest in_dim of a weight created on the context
};

namespace glypr {

// ---- scratch.hip ----
// This device's address of the no-allocation scratch array (the device must be
// current); on failure *ptr is NULL and the HIP error is returned.
hipError_t resolve_scratch(void** ptr);
// The device's record of its last no-allocation call: the stream it ran on
// and an event recorded after it (created by scratch_guard_init, with the
// device current, when the first context on the device is made).
struct ScratchGuard {
  std::mutex mu;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool armed = false;   // done holds a recorded call
};
hipError_t scratch_guard_init(int device);
ScratchGuard* scratch_guard(int device);   // null before scratch_guard_init

// error.cpp-style helpers (defined in capi.hip)
int set_error(int code, const char* fmt, ...);
int hip_error(hipError_t e, const char* what);

// ---- k_codec.hip ----
hipError_t launch_repack(const uint8_t* gguf, int8_t* qs, float* dw, int64_t rows, int64_t k,
                         hipStream_t s);
hipError_t launch_dequant(const int8_t* qs, const float* dw, int64_t rows, int64_t k, float* out,
                          hipStream_t s);
hipError_t launch_gather(const int8_t* qs, const float* dw, int64_t k, const uint32_t* ids,
                         int64_t n_ids, float scale, float* out, hipStream_t s);
// The same gather with the ids read from host memory at launch (they travel in
// the kernel arguments, so the ids need no device copy): rows of width k with
// k % 32 == 0 and k <= 1024, at most GATHER_ARG_IDS ids.
constexpr int GATHER_ARG_IDS = 768;
// Ids carried by value in the kernel arguments (up to GATHER_ARG_IDS of
// them, 3 KB): the launch needs no device copy of the ids, so the caller's
// host array is read when the launch is enqueued and nothing waits on it.
struct GatherIds {
  uint32_t v[GATHER_ARG_IDS];
  __device__ uint32_t operator[](int64_t i) const { return v[i]; }
};
bool gather_host_ids_ok(int64_t k, int64_t n_ids);
hipError_t launch_gather_host_ids(const int8_t* qs, const float* dw, int64_t k,
                                  const uint32_t* host_ids, int64_t n_ids, float scale, float* out,
                                  hipStream_t s);
hipError_t launch_quantize_planar(const float* x, int64_t m, int64_t k, int8_t* xq, float* dx,
                                  hipStream_t s);
hipError_t launch_quantize_gguf(const float* x, int64_t m, int64_t k, uint8_t* out,
                                hipStream_t s);
hipError_t launch_to_bf16(const float* x, int64_t n, uint16_t* out, hipStream_t s);

// ---- k_norm.hip ----
hipError_t launch_rmsnorm(const float* x, const float* w, float eps, float* y, int64_t rows,
                          int64_t dim, hipStream_t s);
hipError_t launch_rmsnorm_quant(const float* x, const float* w, float eps, int64_t rows,
                                int64_t dim, int8_t* xq, float* dx, hipStream_t s);
// The token gather x scale (launch_gather's arithmetic) and the first input
// RMSNorm + Q8_0 (launch_rmsnorm_quant's) in one launch: writes the gathered
// rows to h and their normalised Q8_0 to xq / dx.  Ids from host memory
// (host_ids, at most GATHER_ARG_IDS) or device memory (dev_ids).  Only for
// gather_norm_ok shapes.
bool gather_norm_ok(int64_t rows, int64_t dim);
hipError_t launch_gather_norm(const int8_t* qs, const float* dw, int64_t dim,
                              const uint32_t* host_ids, const uint32_t* dev_ids, int64_t rows,
                              float scale, const float* w, float eps, float* h, int8_t* xq,
                              float* dx, hipStream_t s);
hipError_t launch_rmsnorm_bf16(const float* x, const float* w, float eps, int64_t rows,
                               int64_t dim, uint16_t* xb, hipStream_t s);
hipError_t launch_geglu(const float* g, const float* u, float* out, int64_t n, hipStream_t s);
// scratch: pool_scratch_floats(t, d) floats
size_t pool_scratch_floats(int64_t t, int64_t d);
hipError_t launch_pool(const float* tok, const uint8_t* mask, int64_t t, int64_t d, int64_t trunc,
                       float* out, float* scratch, hipStream_t s);
// Several sequences at 64-aligned row offsets of tok [rows][d] (rows % 64 ==
// 0): seg is the per-row segment table (launch_qkv_post), seqs {offset,
// length} per sequence; out [n_seqs][trunc or d].  mixed: the lengths differ,
// so each mean divides by its count (the reference's masked batch pooling).
size_t pool_segments_scratch_floats(int64_t rows, int64_t n_seqs, int64_t d);
hipError_t launch_pool_segments(const float* tok, int64_t rows, const int32_t* seg,
                                const int32_t* seqs, int64_t n_seqs, int64_t d, int64_t trunc,
                                float* out, float* scratch, hipStream_t s, bool mixed);

// h = h + rmsnorm(x; w_post); if xq: (xq, dx) = Q8_0(rmsnorm(h; w_next)).  dim % 32 == 0.
// scalar (device, nullable): h = (h + RMSNorm(x)) * scalar.  plain_q: xq/dx
// receive Q8_0 of h itself instead of Q8_0 of RMSNorm(h; w_next).
// xb (nullable, instead of xq): bf16 of RMSNorm(h; w_next), the next dense-bf16
// GEMM's operand.  yf (nullable, instead of xq and xb): f32 RMSNorm(h; w_next),
// the model's final norm.
hipError_t launch_residual_norm(const float* x, const float* w_post, float* h, const float* w_next,
                                float eps, int64_t rows, int64_t dim, int8_t* xq, float* dx,
                                hipStream_t s, const float* scalar = nullptr,
                                bool plain_q = false, uint16_t* xb = nullptr,
                                float* yf = nullptr);
// x = x * mul + 0 (f32), in place
hipError_t launch_affine(float* x, int64_t n, float mul, hipStream_t s);
// Q8_0 of geglu(g, u): g [rows][dim], u row r at u + r * u_stride
hipError_t launch_geglu_quant(const float* g, const float* u, int64_t u_stride, int64_t rows,
                              int64_t dim, int8_t* hq, float* dh, hipStream_t s);

// ---- k_attn.hip, attn_plan.cpp ----
// Attention operands are padded to Tp = attn_padded_len(T) tokens.
constexpr int64_t ATTN_TP_ALIGN = 64;
// The partitioned kernels: keys per K/V tile; sequences up to ATTN_SMALL_T
// use 16-query blocks (more blocks to spread), longer ones 64-query blocks
// (each K/V tile serves 4x the queries; head_dim 256).
constexpr int ATTN_AK = 32;
constexpr int64_t ATTN_SMALL_T = 1024;
// Key partitions: enough (query block, partition) items for one round of
// workgroups (256 CUs), at most half the key tiles per partition and at most
// 64 partitions (the combine holds one partition per lane).
constexpr int64_t ATTN_BLOCKS = 256;
// From this many padded rows (a batch of sequences) head_dim 256 takes
// 64-query blocks.
constexpr int64_t ATTN_QS4_ROWS = 4096;
// Queries per block / 16 for the longest sequence T over `rows` padded rows.
int attn_qs(int64_t T, int64_t rows, int64_t hd);
// Key tiles per partition (returned) and the partition count (*kparts) for
// the longest sequence Tseg (its key range sets the tile count) over `rows`
// padded rows (they set the query blocks).
int attn_kb_per_part(int64_t Tseg, int64_t rows, int64_t hd, int64_t nq, int64_t nkv,
                     int64_t window, int* kparts);
inline int64_t attn_padded_len(int64_t t) { return (t + ATTN_TP_ALIGN - 1) / ATTN_TP_ALIGN * ATTN_TP_ALIGN; }
// q16 [nq][Tp][hd], k16 [nkv][Tp][hd], vt16 [nkv][hd][Tp] (f16).  hd == 256.
// seg (nullable, device int32 pairs [Tp][2]): row t holds position t - seg[t][0]
// of a sequence of seg[t][1] tokens starting at row seg[t][0] (sequences at
// 64-aligned row offsets); rows past a sequence's length are padding.
// Without it the rows are one sequence of T tokens.
hipError_t launch_qkv_post(const float* qkv, int64_t T, int64_t Tp, int64_t nq, int64_t nkv,
                           int64_t hd, const float* qnw, const float* knw, float eps,
                           const float* cos_t, const float* sin_t, uint16_t* q16, uint16_t* k16,
                           uint16_t* vt16, hipStream_t s, const int32_t* seg = nullptr);
// T: the (longest) sequence length; rows: the padded row count when several
// sequences share the buffers (0: attn_padded_len(T)).
size_t attention_scratch_floats(int64_t T, int64_t nq, int64_t nkv, int64_t hd, int64_t window,
                                int64_t rows = 0);
// The largest attention_scratch_floats over every longest-sequence length
// up to max_t (multiples of 32, and max_t) and every padded row count from
// attn_padded_len of it up to cap_rows (a multiple of 64).
size_t attention_scratch_bound(int64_t max_t, int64_t cap_rows, int64_t nq, int64_t nkv,
                               int64_t hd, int64_t window);
// Whether launch_attention runs this geometry: head_dim 256 or 512, nq / nkv
// in 1..4, at most 64 key partitions at T and attention_rows_ok (T <= 0: any
// length).
bool attention_supported(int64_t T, int64_t nq, int64_t nkv, int64_t hd, int64_t window);
// Whether `rows` padded rows of head dim hd keep every per-lane byte offset
// of the attention kernels (2 hd Tp) below 2^31.
bool attention_rows_ok(int64_t rows, int64_t hd);
// ctx (f32 [T][nq*hd]), (cq, dc) (Q8_0 planar) and cb (bf16 [T][nq*hd]) may
// each be null.
// seg / seg_max: the segment table of launch_qkv_post and the longest sequence;
// each query block attends to its own sequence's keys only.
hipError_t launch_attention(const uint16_t* q16, const uint16_t* k16, const uint16_t* vt16,
                            float* scratch, float* ctx, int8_t* cq, float* dc, int64_t T,
                            int64_t Tp, int64_t nq, int64_t nkv, int64_t hd, int64_t window,
                            hipStream_t s, uint16_t* cb = nullptr, const int32_t* seg = nullptr,
                            int64_t seg_max = 0);

// ---- k_gemm_i8.hip ----
// Which INT8_EXACT kernel runs an [M x Nrows x K] GEMM (plain or GeGLU):
// the LDS-ring small-M kernel, the 128 x 128 large-M kernel (both with 32-bit
// operand offsets) or the register-staged kernel (int64 offsets, any shape).
enum { GEMM_ROUTE_SMALL = 0, GEMM_ROUTE_BIG = 1, GEMM_ROUTE_REG128 = 2, GEMM_ROUTE_REG64 = 3 };
int gemm_i8_route(int64_t M, int64_t Nrows, int64_t K);
// y[m,n] = sum_b ((float)S_b * dw[n,b]) * dx[m,b], sequential over b (exact).
// fma2 (GLYPR_Q8_INT8_FMA): each block's term is added as
// fma(round(S_b * dw[n,b]), dx[m,b], acc), one rounding fewer per block.
hipError_t launch_gemm_i8(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                          float* y, int64_t M, int64_t N, int64_t K, int64_t ldc,
                          hipStream_t s, bool fma2 = false);
// Gate/up GEMM ([gate; up] rows, 2F x K) with GeGLU + Q8_0 quantization epilogue:
// hq int8 [M][F], dh f32 [M][F/32].
hipError_t launch_gemm_i8_geglu(const int8_t* xq, const float* dx, const int8_t* wq,
                                const float* dw, int8_t* hq, float* dh, int64_t M, int64_t F,
                                int64_t K, hipStream_t s, bool fma2 = false);

// The q|k|v projection (INT8_EXACT, or INT8_FMA with fma2; Q8_0 activations)
// with qkv_post's work as its epilogue: writes the attention operands q / k / vt (f16, rows padded
// to Tp, invalid rows zero) straight from the GEMM.  head_dim 256, K a
// multiple of 128; 16-row blocks for Tp <= 2048 with K in {512, 768, 1024,
// 1152}, 128-row blocks otherwise.
bool gemm_i8_qkv_ok(int64_t T, int64_t Tp, int64_t K, int64_t hd);
hipError_t launch_gemm_i8_qkv(const int8_t* xq, const float* dx, const int8_t* wq,
                              const float* dw, int64_t T, int64_t Tp, int64_t K, int64_t nq,
                              int64_t nkv, int64_t hd, const float* qnw, const float* knw,
                              float eps, const float* cos_t, const float* sin_t, uint16_t* q16,
                              uint16_t* k16, uint16_t* vt16, const int32_t* seg, hipStream_t s,
                              bool fma2 = false);

// The int8 GEMM with the activation prologue fused: x is f32 [M][K],
// quantized to Q8_0 inside the GEMM (norm: of RMSNorm(x; nw, eps), nw
// nullable), bit-identical to launch_quantize_planar / launch_rmsnorm_quant
// followed by launch_gemm_i8.  gemm_i8_pro_ok says where it is the faster
// route (small M).
bool gemm_i8_pro_ok(int64_t M, int64_t N, int64_t K, bool norm);
hipError_t launch_gemm_i8_pro(const float* x, const float* nw, float eps, bool norm,
                              const int8_t* wq, const float* dw, float* y, int64_t M, int64_t N,
                              int64_t K, int64_t ldc, hipStream_t s, bool fma2 = false);

// ---- k_gemm_bf16.hip, dense bf16 weights ----
// y = xb . wb^T (xb bf16 [M][K], wb bf16 [N][K]), f32 out; the GeGLU form takes
// wb = [gate; up] (2F rows) and writes h bf16 [M][F].  K % 64 == 0.
bool gemm_bf16w_ok(int64_t M, int64_t Nrows, int64_t K);
hipError_t launch_gemm_bf16w(const uint16_t* xb, const uint16_t* wb, float* y, int64_t M,
                             int64_t N, int64_t K, int64_t ldc, hipStream_t s);
hipError_t launch_gemm_bf16w_geglu(const uint16_t* xb, const uint16_t* wb, uint16_t* hb,
                                   int64_t M, int64_t F, int64_t K, hipStream_t s);
// The dense-bf16 q|k|v projection with qkv_post's work as its epilogue (f16
// q / k / vt, rows padded to Tp, invalid rows zero); head_dim 256, K % 64 == 0,
// Tp >= 2048 (where it beats the two launches).
bool gemm_bf16w_qkv_ok(int64_t T, int64_t Tp, int64_t K, int64_t hd);
hipError_t launch_gemm_bf16w_qkv(const uint16_t* xb, const uint16_t* wb, int64_t T, int64_t Tp,
                                 int64_t K, int64_t nq, int64_t nkv, int64_t hd, const float* qnw,
                                 const float* knw, float eps, const float* cos_t,
                                 const float* sin_t, uint16_t* q16, uint16_t* k16, uint16_t* vt16,
                                 const int32_t* seg, hipStream_t s);

// ---- k_vec.hip ----
hipError_t launch_quantize_binary(const float* x, int64_t n, int64_t dim, uint64_t* out,
                                  hipStream_t s);
hipError_t launch_quantize_int8(const float* x, int64_t count, int8_t* out, hipStream_t s);
hipError_t launch_hamming(const uint64_t* a, int64_t na, const uint64_t* b, int64_t nb,
                          int64_t words, uint32_t* out, hipStream_t s);
// table: cos(pi * h / (64 words)) for h = 0 .. 64 words (f32, device)
hipError_t launch_binary_cosine(const uint64_t* a, int64_t na, const uint64_t* b, int64_t nb,
                                int64_t words, const float* table, float* out, hipStream_t s);
hipError_t launch_int8_dot(const int8_t* a, int64_t na, const int8_t* b, int64_t nb, int64_t dim,
                           int32_t* out, hipStream_t s);
// norms: scratch of na int32 (the queries' squared norms)
hipError_t launch_int8_cosine(const int8_t* a, int64_t na, const int8_t* b, int64_t nb,
                              int64_t dim, int32_t* norms, float* out, hipStream_t s);

// ---- k_gemm_bf16.hip ----
hipError_t launch_gemm_bf16(const uint16_t* xb, const int8_t* wq, const float* dw, float* y,
                            int64_t M, int64_t N, int64_t K, int64_t ldc, hipStream_t s);
hipError_t launch_gemm_bf16_geglu(const uint16_t* xb, const int8_t* wq, const float* dw,
                                  uint16_t* hb, int64_t M, int64_t F, int64_t K, hipStream_t s);

}  // namespace glypr
