// k_norm.hip — RMSNorm (alone and as the GEMM prologue that emits Q8_0 or
// bf16 activations), elementwise GeGLU, and mean-pool/L2/MRL.
//
// RMSNorm reproduces simd_rmsnorm_row_f32 (cpu_simd/rmsnorm.rs:6-47) as pulp
// runs it on x86-64-v3 bit for bit: eight f32 lane accumulators, lane j
// chaining acc_j = fma(x[8c+j], x[8c+j], acc_j) over c in order, the AVX2
// horizontal sum ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)), a scalar x*x tail,
// inv = 1/sqrt(sum/d + eps), y = (x*inv)*w.  On the GPU a row is owned by an
// aligned group of 8 lanes, lane j running chain j, so a wave normalises 8
// rows at once.
#include "device_common.hpp"
#include "internal.hpp"

#include <cstring>

namespace glypr {

// Fallback for dims that are not a multiple of 4 or exceed 2048: eight lanes
// per row run the chains straight from global memory.
__global__ void __launch_bounds__(256) rmsnorm_generic_kernel(const float* x, const float* w,
                                                              float eps, float* y, int64_t rows,
                                                              int dim) {
  int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  int j = threadIdx.x & 7;
  bool valid = row < rows;
  const float* xr = x + row * dim;
  float acc = 0.0f;
  const int head = dim & ~7;
  if (valid)
    for (int c = j; c < head; c += 8) acc = fmaf(xr[c], xr[c], acc);
  float s = acc + __shfl_down(acc, 4, 8);
  float t = s + __shfl_down(s, 2, 8);
  float sum = t + __shfl_down(t, 1, 8);
  sum = __shfl(sum, 0, 8);
  if (!valid) return;
  for (int c = head; c < dim; c++) sum += xr[c] * xr[c];
  float inv = 1.0f / sqrtf(sum / (float)dim + eps);
  float* yr = y + row * dim;
  for (int c = j; c < dim; c += 8) yr[c] = w ? (xr[c] * inv) * w[c] : xr[c] * inv;
}

static hipError_t launch_rmsnorm_generic(const float* x, const float* w, float eps, float* y,
                                         int64_t rows, int64_t dim, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  rmsnorm_generic_kernel<<<(unsigned)((rows + 31) / 32), 256, 0, s>>>(x, w, eps, y, rows,
                                                                      (int)dim);
  return hipGetLastError();
}

// One row per wave.  The row is read once, coalesced (lane l holds float4 #l,
// #l+64, ... : with 8 lanes per 32-block that is exactly the quantizer's
// layout), and also written to LDS so that lanes 0..7 can run the reference's
// eight sequential FMA chains (lane j: elements j, j+8, j+16, ...) from LDS.
// The chains are the only serial part; quantization then uses all 64 lanes.
// A block holds 1, 2 or 4 row waves: about one block per CU when rows are few,
// 4 per block for long row counts.  Up to 2048 rows of at most 1024 values
// (dim % 32 == 0) the split kernels below take the row over NV waves
// instead.
constexpr int NORM_WAVES_MAX = 4;
inline int norm_waves(int64_t rows) { return rows <= 256 ? 1 : rows <= 512 ? 2 : 4; }

enum NormOut { OUT_F32 = 0, OUT_Q8 = 1, OUT_BF16 = 2 };

__device__ __forceinline__ uint32_t bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) r = (u >> 16) | 0x40u;
  return r;
}

// Chain-major row staging for the reference-order sum of squares (dim % 32
// == 0): element e of a row is stored at lrow[(e % 8) * S + e / 8] with
// S = dim / 8 + 4, so chain lane j reads its elements x[j], x[j+8], ... as
// consecutive ds_read_b128 and runs its FMA chain from registers.  Even and odd
// lanes of a row write 4 S apart (16 banks), so the staging stores do not
// conflict either.
__device__ __forceinline__ int chain_stride(int dim) { return dim / 8 + 4; }
__device__ __forceinline__ void stage_chains(float* lrow, int S, int c4, const v4f& v) {
  const int j0 = 4 * (c4 & 1), idx = c4 >> 1;
#pragma unroll
  for (int k = 0; k < 4; k++) lrow[(j0 + k) * S + idx] = v[k];
}
// 1/rms of a chain-major staged row (dim % 32 == 0, dim <= 256 NV) in the
// reference's order.  Lanes 0..7 run the chains with every ds_read_b128 of
// the chain issued before its first FMA: chunks past dim / 32 are read
// clamped and replaced by zeros.  The horizontal sum runs through DPP and
// lane 0's total is broadcast with readlane.
template <int NV, bool FULL>
__device__ __forceinline__ float chain_row_inv(const float* lrow, int dim, int lane, float eps) {
  // FULL: every chunk of the chain in one batch; else batches of up to 12
  // chunks (48 registers)
  constexpr int NC = 8 * NV, BATCH = FULL ? NC : (NC < 12 ? NC : 12);
  float sum = 0.0f;
  if (lane < 8) {
    const v4f* src = reinterpret_cast<const v4f*>(lrow + lane * chain_stride(dim));
    const int n = dim / 32;
    float acc = 0.0f;
#pragma unroll
    for (int b0 = 0; b0 < NC; b0 += BATCH) {
      constexpr int LAST = NC % BATCH == 0 ? BATCH : NC % BATCH;
      const int nb = b0 + BATCH <= NC ? BATCH : LAST;   // chunks of this batch
      v4f e[BATCH];
#pragma unroll
      for (int t = 0; t < BATCH; t++)
        if (t < nb) e[t] = src[b0 + t < n ? b0 + t : n - 1];
      __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the chain
      if (n == NC) {   // uniform: dim = 256 NV, every chunk is the row's
#pragma unroll
        for (int t = 0; t < BATCH; t++) {
          if (t >= nb) break;
          acc = fmaf(e[t][0], e[t][0], acc);
          acc = fmaf(e[t][1], e[t][1], acc);
          acc = fmaf(e[t][2], e[t][2], acc);
          acc = fmaf(e[t][3], e[t][3], acc);
        }
      } else {
        // chunks past n become zeros: fma(0, 0, acc) = acc exactly (acc >= +0)
#pragma unroll
        for (int t = 0; t < BATCH; t++) {
          if (t >= nb) break;
          const v4f z = b0 + t < n ? e[t] : v4f{0.0f, 0.0f, 0.0f, 0.0f};
          acc = fmaf(z[0], z[0], acc);
          acc = fmaf(z[1], z[1], acc);
          acc = fmaf(z[2], z[2], acc);
          acc = fmaf(z[3], z[3], acc);
        }
      }
    }
    sum = hsum8_avx2(acc);
  }
  sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sum), 0));
  return 1.0f / sqrtf(sum / (float)dim + eps);
}

// NV = float4s per lane = ceil(dim / 256).  dim % 4 == 0 (dim % 32 == 0 for Q8).
template <int NV, int MODE, bool CHAIN>
__global__ void __launch_bounds__(64 * NORM_WAVES_MAX)
rmsnorm_row_kernel(const float* x, const float* __restrict__ w, float eps, int64_t rows, int dim,
                   float* y, int8_t* __restrict__ xq, float* __restrict__ dx,
                   uint16_t* __restrict__ xb) {
  extern __shared__ float lds_rows[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
  if (row >= rows) return;  // whole wave exits together
  float* lrow = lds_rows + wave * (dim + 32);
  const float* xr = x + row * dim;
  const int n4 = dim >> 2;

  // row and weights are loaded together: one memory latency, not two
  v4f v[NV], wv[NV];
#pragma unroll
  for (int i = 0; i < NV; i++) {
    int c4 = lane + 64 * i;
    v[i] = c4 < n4 ? *reinterpret_cast<const v4f*>(xr + 4 * c4) : v4f{0, 0, 0, 0};
    wv[i] = (w && c4 < n4) ? *reinterpret_cast<const v4f*>(w + 4 * c4) : v4f{1, 1, 1, 1};
  }
  float inv;
  if constexpr (CHAIN) {
    const int S = chain_stride(dim);
#pragma unroll
    for (int i = 0; i < NV; i++) {
      int c4 = lane + 64 * i;
      if (c4 < n4) stage_chains(lrow, S, c4, v[i]);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    inv = chain_row_inv<NV, false>(lrow, dim, lane, eps);
  } else {
#pragma unroll
    for (int i = 0; i < NV; i++) {
      int c4 = lane + 64 * i;
      if (c4 < n4) *reinterpret_cast<v4f*>(lrow + 4 * c4) = v[i];
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    // Reference-order sum of squares on lanes 0..7.
    float sum = 0.0f;
    const int head = dim & ~7;
    if (lane < 8) {
      float acc = 0.0f;
#pragma unroll 16
      for (int c = lane; c < head; c += 8) {
        float e = lrow[c];
        acc = fmaf(e, e, acc);
      }
      float s = acc + __shfl_down(acc, 4, 8);
      float t = s + __shfl_down(s, 2, 8);
      sum = t + __shfl_down(t, 1, 8);
      for (int c = head; c < dim; c++) sum += lrow[c] * lrow[c];
    }
    sum = __shfl(sum, 0);
    inv = 1.0f / sqrtf(sum / (float)dim + eps);
  }

  v4f yv[NV];
#pragma unroll
  for (int i = 0; i < NV; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) yv[i][e] = w ? (v[i][e] * inv) * wv[i][e] : v[i][e] * inv;
  if constexpr (MODE == OUT_F32) {
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int c4 = lane + 64 * i;
      if (c4 < n4) *reinterpret_cast<v4f*>(y + row * dim + 4 * c4) = yv[i];
    }
  } else if constexpr (MODE == OUT_BF16) {
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int c4 = lane + 64 * i;
      if (c4 < n4) {
        uint32_t* dst = reinterpret_cast<uint32_t*>(xb + row * dim + 4 * c4);
        dst[0] = bf16_rne(yv[i][0]) | (bf16_rne(yv[i][1]) << 16);
        dst[1] = bf16_rne(yv[i][2]) | (bf16_rne(yv[i][3]) << 16);
      }
    }
  } else {
    // 8 consecutive lanes hold one 32-block (dim % 32 == 0 keeps blocks
    // whole); every chunk's scale first, then the stores.
    QScale sc[NV];
    uint32_t packed[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
      float a = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; e++) a = fmaxf(a, fabsf(yv[i][e]));
      sc[i] = q8_scale(max8(a));
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
      packed[i] = 0;
#pragma unroll
      for (int e = 0; e < 4; e++)
        packed[i] |= ((uint32_t)(quant_round(yv[i][e] * sc[i].id) & 0xFF)) << (8 * e);
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int c4 = lane + 64 * i;
      if (c4 < n4) {
        *reinterpret_cast<uint32_t*>(xq + row * dim + 4 * c4) = packed[i];
        if ((lane & 7) == 0) dx[row * (dim / QK) + (c4 >> 3)] = sc[i].dq;
      }
    }
  }
}

// Few rows (dim % 32 == 0, dim <= 1024): one row per block of NV waves,
// wave v holding float4 64 v + lane, as residual_norm_split_kernel (below);
// every wave's chain lanes run the row's chains from the block's LDS copy.
// Same arithmetic per element as rmsnorm_row_kernel.  x may equal y.
template <int NV, int MODE>
__global__ void __launch_bounds__(256)
rmsnorm_split_kernel(const float* x, const float* __restrict__ w, float eps, int dim, float* y,
                     int8_t* __restrict__ xq, float* __restrict__ dx, uint16_t* __restrict__ xb) {
  __shared__ __attribute__((aligned(16))) float lrow[NV * 256 + 32];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  const int n4 = dim >> 2;
  const int c4 = lane + 64 * wv;
  const bool ok = c4 < n4;
  const v4f v = ok ? *reinterpret_cast<const v4f*>(x + row * dim + 4 * c4) : v4f{0, 0, 0, 0};
  const v4f ww = (w && ok) ? *reinterpret_cast<const v4f*>(w + 4 * c4) : v4f{1, 1, 1, 1};
  if (ok) stage_chains(lrow, chain_stride(dim), c4, v);
  __syncthreads();
  const float inv = chain_row_inv<NV, true>(lrow, dim, lane, eps);
  v4f yv;
#pragma unroll
  for (int e = 0; e < 4; e++) yv[e] = w ? (v[e] * inv) * ww[e] : v[e] * inv;
  if constexpr (MODE == OUT_F32) {
    if (ok) *reinterpret_cast<v4f*>(y + row * dim + 4 * c4) = yv;
  } else if constexpr (MODE == OUT_BF16) {
    if (ok) {
      uint32_t* dst = reinterpret_cast<uint32_t*>(xb + row * dim + 4 * c4);
      dst[0] = bf16_rne(yv[0]) | (bf16_rne(yv[1]) << 16);
      dst[1] = bf16_rne(yv[2]) | (bf16_rne(yv[3]) << 16);
    }
  } else {
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) a = fmaxf(a, fabsf(yv[e]));
    const QScale sc = q8_scale(max8(a));
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; e++)
      packed |= ((uint32_t)(quant_round(yv[e] * sc.id) & 0xFF)) << (8 * e);
    if (ok) {
      *reinterpret_cast<uint32_t*>(xq + row * dim + 4 * c4) = packed;
      if ((lane & 7) == 0) dx[row * (dim / QK) + (c4 >> 3)] = sc.dq;
    }
  }
}

// Rows up to which the row norms run one row per block of NV waves.
inline bool norm_split(int64_t rows, int64_t dim) {
  return rows <= 2048 && dim % 32 == 0 && dim <= 1024;
}

template <int MODE>
static hipError_t launch_norm(const float* x, const float* w, float eps, int64_t rows, int64_t dim,
                              float* y, int8_t* xq, float* dx, uint16_t* xb, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  if (norm_split(rows, dim)) {
    switch ((dim + 255) / 256) {
#define NORM_SPLIT_CASE(N)                                                                    \
  case N:                                                                                     \
    rmsnorm_split_kernel<N, MODE><<<(unsigned)rows, 64 * N, 0, s>>>(x, w, eps, (int)dim, y,   \
                                                                     xq, dx, xb);             \
    break;
      NORM_SPLIT_CASE(1)
      NORM_SPLIT_CASE(2)
      NORM_SPLIT_CASE(3)
      NORM_SPLIT_CASE(4)
#undef NORM_SPLIT_CASE
      default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const int nw = norm_waves(rows);
  const unsigned grid = (unsigned)((rows + nw - 1) / nw);
  const size_t lds = (size_t)nw * (dim + 32) * sizeof(float);
  const int nv = (int)((dim + 255) / 256);
  const bool chain = dim % 32 == 0;
  switch (nv) {
#define NORM_CASE(N, NK)                                                                      \
  case N:                                                                                     \
    if (chain)                                                                                \
      rmsnorm_row_kernel<NK, MODE, true><<<grid, 64 * nw, lds, s>>>(                          \
          x, w, eps, rows, (int)dim, y, xq, dx, xb);                                          \
    else                                                                                      \
      rmsnorm_row_kernel<NK, MODE, false><<<grid, 64 * nw, lds, s>>>(                         \
          x, w, eps, rows, (int)dim, y, xq, dx, xb);                                          \
    break;
    NORM_CASE(1, 1)
    NORM_CASE(2, 2)
    NORM_CASE(3, 3)
    NORM_CASE(4, 4)
    NORM_CASE(5, 5)
    NORM_CASE(6, 6)
    NORM_CASE(7, 8)
    NORM_CASE(8, 8)
#undef NORM_CASE
    default:
      return hipErrorInvalidValue;  // dim > 2048: callers validate this
  }
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, float eps, float* y, int64_t rows,
                          int64_t dim, hipStream_t s) {
  if (dim % 4 != 0 || dim > 2048) return launch_rmsnorm_generic(x, w, eps, y, rows, dim, s);
  return launch_norm<OUT_F32>(x, w, eps, rows, dim, y, nullptr, nullptr, nullptr, s);
}

hipError_t launch_rmsnorm_quant(const float* x, const float* w, float eps, int64_t rows,
                                int64_t dim, int8_t* xq, float* dx, hipStream_t s) {
  return launch_norm<OUT_Q8>(x, w, eps, rows, dim, nullptr, xq, dx, nullptr, s);
}

hipError_t launch_rmsnorm_bf16(const float* x, const float* w, float eps, int64_t rows,
                               int64_t dim, uint16_t* xb, hipStream_t s) {
  return launch_norm<OUT_BF16>(x, w, eps, rows, dim, nullptr, nullptr, nullptr, xb, s);
}

// The model's first boundary for few rows: Embedding::forward x embed_scale
// (model.rs:254-255, 507-508) and layer 0's input RMSNorm + Q8_0 in one
// launch, one row per block of NV waves as rmsnorm_split_kernel.  Lane
// (wave v, lane l) dequantizes float4 64 v + l of table row ids[row] with
// gather_rows_kernel's arithmetic ((float)q * d, then * scale + 0), writes it
// to h and stages it for the reference-order chains; the rest is
// rmsnorm_split_kernel<NV, OUT_Q8>.  Bit-identical to the two launches.
template <int NV, class Ids>
__global__ void __launch_bounds__(256)
gather_norm_split_kernel(const int8_t* __restrict__ qs, const float* __restrict__ dw, Ids ids,
                         float scale, const float* __restrict__ w, float eps, int dim,
                         float* __restrict__ h, int8_t* __restrict__ xq, float* __restrict__ dx) {
  __shared__ __attribute__((aligned(16))) float lrow[NV * 256 + 32];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  const int n4 = dim >> 2;
  const int c4 = lane + 64 * wv;
  const bool ok = c4 < n4;
  const int64_t src = (int64_t)ids[row];
  const int q = ok ? *reinterpret_cast<const int*>(qs + src * dim + 4 * c4) : 0;
  const float d = ok ? dw[src * (dim / QK) + (c4 >> 3)] : 0.0f;
  const v4f ww = (w && ok) ? *reinterpret_cast<const v4f*>(w + 4 * c4) : v4f{1, 1, 1, 1};
  v4f v;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float y = (float)(int8_t)((q >> (8 * e)) & 0xFF) * d;
    v[e] = y * scale + 0.0f;
  }
  if (ok) {
    *reinterpret_cast<v4f*>(h + row * dim + 4 * c4) = v;
    stage_chains(lrow, chain_stride(dim), c4, v);
  }
  __syncthreads();
  const float inv = chain_row_inv<NV, true>(lrow, dim, lane, eps);
  v4f yv;
  float a = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    yv[e] = w ? (v[e] * inv) * ww[e] : v[e] * inv;
    a = fmaxf(a, fabsf(yv[e]));
  }
  const QScale sc = q8_scale(max8(a));
  uint32_t packed = 0;
#pragma unroll
  for (int e = 0; e < 4; e++)
    packed |= ((uint32_t)(quant_round(yv[e] * sc.id) & 0xFF)) << (8 * e);
  if (ok) {
    *reinterpret_cast<uint32_t*>(xq + row * dim + 4 * c4) = packed;
    if ((lane & 7) == 0) dx[row * (dim / QK) + (c4 >> 3)] = sc.dq;
  }
}

bool gather_norm_ok(int64_t rows, int64_t dim) { return rows > 0 && norm_split(rows, dim); }

hipError_t launch_gather_norm(const int8_t* qs, const float* dw, int64_t dim,
                              const uint32_t* host_ids, const uint32_t* dev_ids, int64_t rows,
                              float scale, const float* w, float eps, float* h, int8_t* xq,
                              float* dx, hipStream_t s) {
  if (!gather_norm_ok(rows, dim) || (host_ids && rows > GATHER_ARG_IDS) ||
      (!host_ids && !dev_ids))
    return hipErrorInvalidValue;
  GatherIds arg;
  if (host_ids) memcpy(arg.v, host_ids, (size_t)rows * 4);
  switch ((dim + 255) / 256) {
#define GATHER_NORM_CASE(N)                                                                    \
  case N:                                                                                      \
    if (host_ids)                                                                              \
      gather_norm_split_kernel<N, GatherIds><<<(unsigned)rows, 64 * N, 0, s>>>(                \
          qs, dw, arg, scale, w, eps, (int)dim, h, xq, dx);                                    \
    else                                                                                       \
      gather_norm_split_kernel<N, const uint32_t*><<<(unsigned)rows, 64 * N, 0, s>>>(          \
          qs, dw, dev_ids, scale, w, eps, (int)dim, h, xq, dx);                                \
    break;
    GATHER_NORM_CASE(1)
    GATHER_NORM_CASE(2)
    GATHER_NORM_CASE(3)
    GATHER_NORM_CASE(4)
#undef GATHER_NORM_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Layer boundary: RMSNorm::forward_residual_add (norm.rs:65-95),
//   h = h + rmsnorm(x; w_post),
// optionally followed by the next sublayer's RMSNorm prologue on the new h,
// emitting Q8_0 activations (xq, dx) for the next GEMM.  Both norms use the
// reference reduction order, so h and the quantized activations are
// bit-identical to the CPU path.  One row per wave.
// ---------------------------------------------------------------------------
// NEXT: 0 = only h; 1 = also Q8_0 of RMSNorm(h; w_next); 2 = also Q8_0 of h
// itself (the input of a projection that has no norm in front); 3 = bf16 of
// RMSNorm(h; w_next) (dense-bf16 weights).  scalar (device, nullable):
// forward_residual_add's layer_scalar, h = (h + n) * s.
template <int NV, int NEXT>
__global__ void __launch_bounds__(64 * NORM_WAVES_MAX)
residual_norm_kernel(const float* __restrict__ x, const float* __restrict__ w_post,
                     float* __restrict__ h, const float* __restrict__ w_next,
                     const float* __restrict__ scalar, float eps, int64_t rows, int dim,
                     int8_t* __restrict__ xq, float* __restrict__ dx, uint16_t* __restrict__ xb) {
  constexpr bool QNEXT = NEXT != 0;
  constexpr bool CHAIN2 = NEXT == 1 || NEXT == 3;
  extern __shared__ float lds_rows[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
  if (row >= rows) return;
  float* lrow = lds_rows + wave * (dim + 32);
  const int n4 = dim >> 2;
  const int S = chain_stride(dim);
  // every input is loaded up front: one memory latency for the row
  v4f v[NV], hv[NV], wp[NV], wn[NV];
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int c4 = lane + 64 * i;
    const bool ok = c4 < n4;
    v[i] = ok ? *reinterpret_cast<const v4f*>(x + row * dim + 4 * c4) : v4f{0, 0, 0, 0};
    hv[i] = ok ? *reinterpret_cast<const v4f*>(h + row * dim + 4 * c4) : v4f{0, 0, 0, 0};
    wp[i] = ok ? *reinterpret_cast<const v4f*>(w_post + 4 * c4) : v4f{0, 0, 0, 0};
    wn[i] = (QNEXT && w_next && ok) ? *reinterpret_cast<const v4f*>(w_next + 4 * c4)
                                    : v4f{1, 1, 1, 1};
  }
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int c4 = lane + 64 * i;
    if (c4 < n4) stage_chains(lrow, S, c4, v[i]);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  const float inv = chain_row_inv<NV, false>(lrow, dim, lane, eps);
  __builtin_amdgcn_wave_barrier();
  const float sv = scalar ? *scalar : 1.0f;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    int c4 = lane + 64 * i;
    if (c4 < n4) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float sum = hv[i][e] + (v[i][e] * inv) * wp[i][e];
        v[i][e] = scalar ? sum * sv : sum;
      }
      *reinterpret_cast<v4f*>(h + row * dim + 4 * c4) = v[i];
      if (CHAIN2) stage_chains(lrow, S, c4, v[i]);
    }
  }
  if constexpr (QNEXT) {
    float inv2 = 1.0f;
    if constexpr (CHAIN2) {
      // the staging writes must land; the h stores need not
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
      inv2 = chain_row_inv<NV, false>(lrow, dim, lane, eps);
    }
    // all NV chunks' scales first (independent chains the scheduler can
    // interleave), then the stores
    v4f yv[NV];
    float am[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
      am[i] = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        if (NEXT == 2) yv[i][e] = v[i][e];
        else yv[i][e] = w_next ? (v[i][e] * inv2) * wn[i][e] : v[i][e] * inv2;
        am[i] = fmaxf(am[i], fabsf(yv[i][e]));
      }
    }
    if constexpr (NEXT == 3) {
#pragma unroll
      for (int i = 0; i < NV; i++) {
        const int c4 = lane + 64 * i;
        if (c4 < n4) {
          uint32_t* dst = reinterpret_cast<uint32_t*>(xb + row * dim + 4 * c4);
          dst[0] = bf16_rne(yv[i][0]) | (bf16_rne(yv[i][1]) << 16);
          dst[1] = bf16_rne(yv[i][2]) | (bf16_rne(yv[i][3]) << 16);
        }
      }
    } else {
      QScale sc[NV];
      uint32_t packed[NV];
#pragma unroll
      for (int i = 0; i < NV; i++) sc[i] = q8_scale(max8(am[i]));
#pragma unroll
      for (int i = 0; i < NV; i++) {
        packed[i] = 0;
#pragma unroll
        for (int e = 0; e < 4; e++)
          packed[i] |= ((uint32_t)(quant_round(yv[i][e] * sc[i].id) & 0xFF)) << (8 * e);
      }
#pragma unroll
      for (int i = 0; i < NV; i++) {
        const int c4 = lane + 64 * i;
        if (c4 < n4) {
          *reinterpret_cast<uint32_t*>(xq + row * dim + 4 * c4) = packed[i];
          if ((lane & 7) == 0) dx[row * (dim / QK) + (c4 >> 3)] = sc[i].dq;
        }
      }
    }
  }
}

// The same layer boundary for few rows: one row per block of NV waves, wave
// v holding float4 64 v + lane of the row (one per lane, where
// residual_norm_kernel's single wave holds NV).  The chain lanes 0..7 of
// every wave run the row's two reference-order chains from the block's
// shared LDS copy (each wave gets inv itself, so no broadcast), and the
// elementwise work, the quantization and the stores are split NV ways: at
// 512 x 768 the row's waves fill 1536 SIMD slots instead of 512.  Each
// chain reads its own staging buffer, so the second staging needs no
// barrier in front of it.  Same arithmetic per element as
// residual_norm_kernel, so the outputs are bit-identical.
template <int NV, int NEXT>
__global__ void __launch_bounds__(256)
residual_norm_split_kernel(const float* __restrict__ x, const float* __restrict__ w_post,
                           float* __restrict__ h, const float* __restrict__ w_next,
                           const float* __restrict__ scalar, float eps, int dim,
                           int8_t* __restrict__ xq, float* __restrict__ dx,
                           uint16_t* __restrict__ xb, float* __restrict__ yf) {
  constexpr bool QNEXT = NEXT != 0;
  constexpr bool CHAIN2 = NEXT == 1 || NEXT == 3 || NEXT == 4;
  // chain-major staging reaches index 7 S + dim / 8 = dim + 28
  __shared__ __attribute__((aligned(16))) float lrow[CHAIN2 ? 2 : 1][NV * 256 + 32];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  const int n4 = dim >> 2;
  const int S = chain_stride(dim);
  const int c4 = lane + 64 * wv;
  const bool ok = c4 < n4;
  const v4f v = ok ? *reinterpret_cast<const v4f*>(x + row * dim + 4 * c4) : v4f{0, 0, 0, 0};
  const v4f hv = ok ? *reinterpret_cast<const v4f*>(h + row * dim + 4 * c4) : v4f{0, 0, 0, 0};
  const v4f wp = ok ? *reinterpret_cast<const v4f*>(w_post + 4 * c4) : v4f{0, 0, 0, 0};
  const v4f wn = (QNEXT && w_next && ok) ? *reinterpret_cast<const v4f*>(w_next + 4 * c4)
                                         : v4f{1, 1, 1, 1};
  if (ok) stage_chains(lrow[0], S, c4, v);
  __syncthreads();
  const float inv = chain_row_inv<NV, true>(lrow[0], dim, lane, eps);
  const float sv = scalar ? *scalar : 1.0f;
  v4f nh;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float sum = hv[e] + (v[e] * inv) * wp[e];
    nh[e] = scalar ? sum * sv : sum;
  }
  if (ok) {
    *reinterpret_cast<v4f*>(h + row * dim + 4 * c4) = nh;
    if (CHAIN2) stage_chains(lrow[CHAIN2 ? 1 : 0], S, c4, nh);
  }
  if constexpr (QNEXT) {
    float inv2 = 1.0f;
    if constexpr (CHAIN2) {
      __syncthreads();
      inv2 = chain_row_inv<NV, true>(lrow[1], dim, lane, eps);
    }
    v4f yv;
    float am = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      if (NEXT == 2) yv[e] = nh[e];
      else yv[e] = w_next ? (nh[e] * inv2) * wn[e] : nh[e] * inv2;
      am = fmaxf(am, fabsf(yv[e]));
    }
    if constexpr (NEXT == 4) {
      if (ok) *reinterpret_cast<v4f*>(yf + row * dim + 4 * c4) = yv;
    } else if constexpr (NEXT == 3) {
      if (ok) {
        uint32_t* dst = reinterpret_cast<uint32_t*>(xb + row * dim + 4 * c4);
        dst[0] = bf16_rne(yv[0]) | (bf16_rne(yv[1]) << 16);
        dst[1] = bf16_rne(yv[2]) | (bf16_rne(yv[3]) << 16);
      }
    } else {
      const QScale sc = q8_scale(max8(am));
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 4; e++)
        packed |= ((uint32_t)(quant_round(yv[e] * sc.id) & 0xFF)) << (8 * e);
      if (ok) {
        *reinterpret_cast<uint32_t*>(xq + row * dim + 4 * c4) = packed;
        if ((lane & 7) == 0) dx[row * (dim / QK) + (c4 >> 3)] = sc.dq;
      }
    }
  }
}


hipError_t launch_residual_norm(const float* x, const float* w_post, float* h, const float* w_next,
                                float eps, int64_t rows, int64_t dim, int8_t* xq, float* dx,
                                hipStream_t s, const float* scalar, bool plain_q, uint16_t* xb,
                                float* yf) {
  if (rows == 0) return hipSuccess;
  if (dim % 32 != 0 || dim > 1024) return hipErrorInvalidValue;
  if (yf && !norm_split(rows, dim)) {
    // the final norm as its own launch
    const hipError_t e = launch_residual_norm(x, w_post, h, nullptr, eps, rows, dim, nullptr,
                                              nullptr, s, scalar);
    return e != hipSuccess ? e : launch_rmsnorm(h, w_next, eps, yf, rows, dim, s);
  }
  if (norm_split(rows, dim)) {
    const int nv = (int)((dim + 255) / 256);
    const int mode =
        yf != nullptr ? 4 : xb != nullptr ? 3 : xq == nullptr ? 0 : (plain_q ? 2 : 1);
#define RES_SPLIT(N, MODE)                                                                     \
  residual_norm_split_kernel<N, MODE><<<(unsigned)rows, 64 * N, 0, s>>>(                       \
      x, w_post, h, w_next, scalar, eps, (int)dim, xq, dx, xb, yf)
#define RES_SPLIT_CASE(N)                                                                      \
  case N:                                                                                      \
    if (mode == 0) RES_SPLIT(N, 0);                                                            \
    else if (mode == 1) RES_SPLIT(N, 1);                                                       \
    else if (mode == 2) RES_SPLIT(N, 2);                                                       \
    else if (mode == 3) RES_SPLIT(N, 3);                                                       \
    else RES_SPLIT(N, 4);                                                                      \
    break;
    switch (nv) {
      RES_SPLIT_CASE(1)
      RES_SPLIT_CASE(2)
      RES_SPLIT_CASE(3)
      RES_SPLIT_CASE(4)
      default:
        return hipErrorInvalidValue;
    }
#undef RES_SPLIT_CASE
#undef RES_SPLIT
    return hipGetLastError();
  }
  const int nw = norm_waves(rows);
  const unsigned grid = (unsigned)((rows + nw - 1) / nw);
  const size_t lds = (size_t)nw * (dim + 32) * sizeof(float);
  const int nv = (int)((dim + 255) / 256);
  const int mode = xb != nullptr ? 3 : xq == nullptr ? 0 : (plain_q ? 2 : 1);
#define RES_LAUNCH(N, MODE)                                                                    \
  residual_norm_kernel<N, MODE><<<grid, 64 * nw, lds, s>>>(x, w_post, h, w_next, scalar, eps,  \
                                                          rows, (int)dim, xq, dx, xb)
#define RES_CASE(N)                                                                            \
  case N:                                                                                      \
    if (mode == 0) RES_LAUNCH(N, 0);                                                           \
    else if (mode == 1) RES_LAUNCH(N, 1);                                                      \
    else if (mode == 2) RES_LAUNCH(N, 2);                                                      \
    else RES_LAUNCH(N, 3);                                                                     \
    break;
  switch (nv) {
    RES_CASE(1)
    RES_CASE(2)
    RES_CASE(3)
    RES_CASE(4)
    default:
      return hipErrorInvalidValue;
  }
#undef RES_CASE
#undef RES_LAUNCH
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// GeGLU elementwise (cpu_geglu).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) geglu_kernel(const float* g, const float* u, float* out,
                                                    int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    out[i] = geglu_scalar(g[i], u[i]);
}

hipError_t launch_geglu(const float* g, const float* u, float* out, int64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  int64_t grid = (n + 255) / 256;
  if (grid > 65536) grid = 65536;
  geglu_kernel<<<(unsigned)grid, 256, 0, s>>>(g, u, out, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// candle's Tensor * f64 on f32 (affine(mul, 0)): y = v * f32(mul) + 0.0f, two
// roundings (the + 0 turns a -0 product into +0).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) affine_kernel(float* x, int64_t n, float mul) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    x[i] = x[i] * mul + 0.0f;
}

hipError_t launch_affine(float* x, int64_t n, float mul, hipStream_t s) {
  if (n == 0) return hipSuccess;
  int64_t grid = (n + 255) / 256;
  if (grid > 65536) grid = 65536;
  affine_kernel<<<(unsigned)grid, 256, 0, s>>>(x, n, mul);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// TextPLEBlock's cpu_geglu(gate, per_layer_input) (ple.rs:136-138) followed by
// BlockQ8_0::from_float of each 32-block: the proj GEMM's int8 operand.  gate
// [rows][dim] contiguous; row r of the per-layer input at u + r * u_stride.
// Eight lanes per 32-block, four elements each (the quantizer's layout).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) geglu_quant_kernel(const float* __restrict__ g,
                                                          const float* __restrict__ u,
                                                          int64_t u_stride, int64_t rows, int dim,
                                                          int8_t* __restrict__ hq,
                                                          float* __restrict__ dh) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int nbr = dim / QK;
  const int64_t b = gid >> 3;
  const int j = threadIdx.x & 7;
  const bool ok = b < rows * nbr;
  const int64_t r = ok ? b / nbr : 0;
  const int col = ok ? (int)(b - r * nbr) * QK + 4 * j : 0;
  v4f hv = {0, 0, 0, 0};
  if (ok) {
    const v4f gv = *reinterpret_cast<const v4f*>(g + r * dim + col);
    const v4f uv = *reinterpret_cast<const v4f*>(u + r * u_stride + col);
#pragma unroll
    for (int e = 0; e < 4; e++) hv[e] = geglu_scalar(gv[e], uv[e]);
  }
  float a = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; e++) a = fmaxf(a, fabsf(hv[e]));
  a = max8(a);
  const QScale sc = q8_scale(a);
  uint32_t packed = 0;
#pragma unroll
  for (int e = 0; e < 4; e++) packed |= ((uint32_t)(quant_round(hv[e] * sc.id) & 0xFF)) << (8 * e);
  if (ok) {
    *reinterpret_cast<uint32_t*>(hq + r * dim + col) = packed;
    if (j == 0) dh[r * nbr + col / QK] = sc.dq;
  }
}

hipError_t launch_geglu_quant(const float* g, const float* u, int64_t u_stride, int64_t rows,
                              int64_t dim, int8_t* hq, float* dh, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  if (dim % QK != 0 || u_stride % 4 != 0) return hipErrorInvalidValue;
  const int64_t threads = rows * (dim / QK) * 8;
  geglu_quant_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(g, u, u_stride, rows,
                                                                       (int)dim, hq, dh);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// pool_and_normalize (model.rs:654-705): f32 mean over the valid tokens, L2
// with the 1e-12 clamp, MRL narrow + renormalise.  candle sums the token axis
// sequentially; a sequential sum is one dependent chain of t loads per column
// (latency-bound: milliseconds at t = 8192), so the sum here is chunked:
// pool_partial sums POOL_CHUNK-token chunks per column (sequentially inside a
// chunk), pool_finalize adds the chunk sums in chunk order, divides, and runs
// the norms with block-wide tree reductions.  Deterministic (fixed order) and
// within a few f32 ulps of the sequential sums; tested against float64.
// ---------------------------------------------------------------------------
constexpr int POOL_CHUNK = 64;

// seg (nullable): the segment table of several sequences at 64-aligned row
// offsets ({start, length} per row, see launch_qkv_post); a chunk then ends at
// its sequence's last token, and chunks of padding rows sum to 0.
__global__ void __launch_bounds__(256) pool_partial_kernel(const float* __restrict__ tok,
                                                           const uint8_t* __restrict__ mask,
                                                           int64_t t, int64_t d,
                                                           float* __restrict__ partial,
                                                           const int2* __restrict__ seg) {
  const int64_t col = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t chunk = blockIdx.y;
  if (col >= d) return;
  const int64_t r0 = chunk * POOL_CHUNK;
  int64_t end = t;
  if (seg) {
    const int2 sg = seg[r0];
    end = (int64_t)sg.x + sg.y;
  }
  const int64_t r1 = r0 + POOL_CHUNK < end ? r0 + POOL_CHUNK : end;
  float s = 0.0f;
  if (mask) {
    for (int64_t j = r0; j < r1; j++) s += tok[j * d + col] * (mask[j] ? 1.0f : 0.0f);
  } else {
#pragma unroll 16
    for (int64_t j = r0; j < r1; j++) s += tok[j * d + col];
  }
  partial[chunk * d + col] = s;
}

// Sum of v over the 1024 threads of the block (fixed tree: wave shuffles,
// then the 16 wave sums in order).  Every thread gets the total.
__device__ __forceinline__ float block_sum_1024(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; i++) t += red[i];
  return t;
}

// seqs (nullable): {row offset, length} per sequence; block b then pools
// sequence b from its own chunks into out[b][td] (pooled: d floats per block).
// count_div: divide the sum by the token count, as the reference's masked
// mean does for a batch of mixed lengths (model.rs:671-680, lib.rs:902-941);
// otherwise multiply by 1/t as its mean (a homogeneous batch, one sequence).
__global__ void __launch_bounds__(1024) pool_finalize_kernel(const float* __restrict__ partial,
                                                             const uint8_t* __restrict__ mask,
                                                             int64_t t, int64_t d, int64_t trunc,
                                                             float* __restrict__ out,
                                                             float* __restrict__ pooled,
                                                             const int32_t* __restrict__ seqs,
                                                             bool count_div = false) {
  __shared__ float red[16];
  const int64_t td_out = (trunc > 0 && trunc < d) ? trunc : d;
  if (seqs) {
    const int64_t b = blockIdx.x;
    const int64_t off = seqs[2 * b];
    t = seqs[2 * b + 1];
    partial += (off / POOL_CHUNK) * d;
    out += b * td_out;
    pooled += b * d;
    mask = nullptr;
  }
  const int64_t nchunk = (t + POOL_CHUNK - 1) / POOL_CHUNK;
  float cnt = 0.0f;
  if (mask) {
    float c = 0.0f;
    for (int64_t j = threadIdx.x; j < t; j += blockDim.x) c += mask[j] ? 1.0f : 0.0f;
    cnt = block_sum_1024(c, red);
    if (cnt < 1e-9f) cnt = 1e-9f;
  }
  const float inv_t = (float)(1.0 / (double)t);
  float ss = 0.0f;
  for (int64_t i = threadIdx.x; i < d; i += blockDim.x) {
    float s = 0.0f;
    for (int64_t c = 0; c < nchunk; c++) s += partial[c * d + i];
    const float v = mask ? s / cnt : count_div ? s / (float)t : s * inv_t + 0.0f;
    pooled[i] = v;
    ss += v * v;
  }
  const float n1 = sqrtf(block_sum_1024(ss, red));
  const float nrm = n1 < 1e-12f ? 1e-12f : n1;
  const int64_t td = (trunc > 0 && trunc < d) ? trunc : d;
  if (td == d) {
    for (int64_t i = threadIdx.x; i < d; i += blockDim.x) out[i] = pooled[i] / nrm;
    return;
  }
  // MRL: keep the first td of the normalised vector and normalise again
  float ss2 = 0.0f;
  for (int64_t i = threadIdx.x; i < td; i += blockDim.x) {
    const float v = pooled[i] / nrm;
    pooled[i] = v;
    ss2 += v * v;
  }
  const float n2 = sqrtf(block_sum_1024(ss2, red));
  const float nrm2 = n2 < 1e-12f ? 1e-12f : n2;
  for (int64_t i = threadIdx.x; i < td; i += blockDim.x) out[i] = pooled[i] / nrm2;
}

size_t pool_scratch_floats(int64_t t, int64_t d) {
  return (size_t)(((t + POOL_CHUNK - 1) / POOL_CHUNK) * d + d);
}

hipError_t launch_pool(const float* tok, const uint8_t* mask, int64_t t, int64_t d, int64_t trunc,
                       float* out, float* scratch, hipStream_t s) {
  const int64_t nchunk = (t + POOL_CHUNK - 1) / POOL_CHUNK;
  float* partial = scratch;
  float* pooled = scratch + nchunk * d;
  dim3 g1((unsigned)((d + 255) / 256), (unsigned)nchunk);
  pool_partial_kernel<<<g1, 256, 0, s>>>(tok, mask, t, d, partial, nullptr);
  pool_finalize_kernel<<<1, 1024, 0, s>>>(partial, mask, t, d, trunc, out, pooled, nullptr);
  return hipGetLastError();
}

size_t pool_segments_scratch_floats(int64_t rows, int64_t n_seqs, int64_t d) {
  return (size_t)(((rows + POOL_CHUNK - 1) / POOL_CHUNK) * d + n_seqs * d);
}

hipError_t launch_pool_segments(const float* tok, int64_t rows, const int32_t* seg,
                                const int32_t* seqs, int64_t n_seqs, int64_t d, int64_t trunc,
                                float* out, float* scratch, hipStream_t s, bool mixed) {
  if (rows % POOL_CHUNK != 0) return hipErrorInvalidValue;
  const int64_t nchunk = rows / POOL_CHUNK;
  float* partial = scratch;
  float* pooled = scratch + nchunk * d;
  dim3 g1((unsigned)((d + 255) / 256), (unsigned)nchunk);
  pool_partial_kernel<<<g1, 256, 0, s>>>(tok, nullptr, rows, d, partial,
                                         reinterpret_cast<const int2*>(seg));
  pool_finalize_kernel<<<(unsigned)n_seqs, 1024, 0, s>>>(partial, nullptr, rows, d, trunc, out,
                                                          pooled, seqs, mixed);
  return hipGetLastError();
}

}  // namespace glypr
