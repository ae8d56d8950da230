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

namespace glypr {

// Sum of squares of one row in the reference's order, returned to all 8 lanes
// of the row's group.  j = lane & 7.
__device__ __forceinline__ float row_sumsq(const float* xr, int dim, int j,
                                           bool valid) {
  float acc = 0.0f;
  const int head = dim & ~7;
  if (valid) {
#pragma unroll 8
    for (int c = j; c < head; c += 8) {
      float v = xr[c];
      acc = fmaf(v, v, acc);
    }
  }
  float s = acc + __shfl_down(acc, 4, 8);  // j<4: l_j + l_{j+4}
  float t = s + __shfl_down(s, 2, 8);      // j<2: s_j + s_{j+2}
  float sum = t + __shfl_down(t, 1, 8);    // j=0: t_0 + t_1
  sum = __shfl(sum, 0, 8);
  if (valid)
    for (int c = head; c < dim; c++) sum += xr[c] * xr[c];
  return sum;
}

__device__ __forceinline__ float rms_inv(float sum, int dim, float eps) {
  return 1.0f / sqrtf(sum / (float)dim + eps);
}

// Plain RMSNorm, f32 out.  256 threads = 4 waves = 32 rows per block.
__global__ void __launch_bounds__(256) rmsnorm_kernel(const float* x, const float* w, float eps,
                                                      float* y, int64_t rows, int dim) {
  int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  int j = threadIdx.x & 7;
  bool valid = row < rows;
  const float* xr = x + row * dim;
  float sum = row_sumsq(xr, dim, j, valid);
  if (!valid) return;
  float inv = rms_inv(sum, dim, eps);
  float* yr = y + row * dim;
  // x may alias y: every lane finished reading x in row_sumsq's loop before the
  // shuffles that follow it, and each lane only rewrites its own elements here.
  if (w) {
    for (int c = j; c < dim; c += 8) yr[c] = (xr[c] * inv) * w[c];
  } else {
    for (int c = j; c < dim; c += 8) yr[c] = xr[c] * inv;
  }
}

hipError_t launch_rmsnorm(const float* x, const float* w, float eps, float* y, int64_t rows,
                          int64_t dim, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  rmsnorm_kernel<<<(unsigned)((rows + 31) / 32), 256, 0, s>>>(x, w, eps, y, rows, (int)dim);
  return hipGetLastError();
}

// RMSNorm prologue emitting Q8_0 activations (int8 [rows][dim] + f32 f16-rounded
// scales [rows][dim/32]) exactly as k_quants::matmul would quantize the
// normalised rows.  After the sum, the row's 8 lanes re-read it in the
// quantizer's layout: per 32-block, lane j owns values 4j..4j+3.
__global__ void __launch_bounds__(256) rmsnorm_quant_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            float eps, int64_t rows, int dim,
                                                            int8_t* __restrict__ xq,
                                                            float* __restrict__ dx) {
  int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  int j = threadIdx.x & 7;
  bool valid = row < rows;
  const float* xr = x + row * dim;
  float sum = row_sumsq(xr, dim, j, valid);
  float inv = rms_inv(sum, dim, eps);
  const int nb = dim / QK;
  for (int b = 0; b < nb; b++) {
    v4f v = valid ? *reinterpret_cast<const v4f*>(xr + b * QK + 4 * j) : v4f{0, 0, 0, 0};
    v4f wv = w ? *reinterpret_cast<const v4f*>(w + b * QK + 4 * j) : v4f{1, 1, 1, 1};
    v4f yv;
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      yv[e] = w ? (v[e] * inv) * wv[e] : v[e] * inv;
      a = fmaxf(a, fabsf(yv[e]));
    }
    a = fmaxf(a, __shfl_xor(a, 1, 8));
    a = fmaxf(a, __shfl_xor(a, 2, 8));
    a = fmaxf(a, __shfl_xor(a, 4, 8));
    QScale sc = q8_scale(a);
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; e++)
      packed |= ((uint32_t)(quant_round(yv[e] * sc.id) & 0xFF)) << (8 * e);
    if (valid) {
      *reinterpret_cast<uint32_t*>(xq + row * dim + b * QK + 4 * j) = packed;
      if (j == 0) dx[row * nb + b] = sc.dq;
    }
  }
}

hipError_t launch_rmsnorm_quant(const float* x, const float* w, float eps, int64_t rows,
                                int64_t dim, int8_t* xq, float* dx, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  rmsnorm_quant_kernel<<<(unsigned)((rows + 31) / 32), 256, 0, s>>>(x, w, eps, rows, (int)dim, xq,
                                                                    dx);
  return hipGetLastError();
}

__device__ __forceinline__ uint32_t bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) r = (u >> 16) | 0x40u;
  return r;
}

// RMSNorm prologue for the bf16-dequant GEMM: normalised rows rounded to bf16.
__global__ void __launch_bounds__(256) rmsnorm_bf16_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           float eps, int64_t rows, int dim,
                                                           uint16_t* __restrict__ xb) {
  int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  int j = threadIdx.x & 7;
  bool valid = row < rows;
  const float* xr = x + row * dim;
  float sum = row_sumsq(xr, dim, j, valid);
  if (!valid) return;
  float inv = rms_inv(sum, dim, eps);
  for (int c = 4 * j; c < dim; c += 32) {
    v4f v = *reinterpret_cast<const v4f*>(xr + c);
    v4f wv = w ? *reinterpret_cast<const v4f*>(w + c) : v4f{1, 1, 1, 1};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = bf16_rne(w ? (v[e] * inv) * wv[e] : v[e] * inv);
    uint32_t* dst = reinterpret_cast<uint32_t*>(xb + row * dim + c);
    dst[0] = o[0] | (o[1] << 16);
    dst[1] = o[2] | (o[3] << 16);
  }
}

hipError_t launch_rmsnorm_bf16(const float* x, const float* w, float eps, int64_t rows,
                               int64_t dim, uint16_t* xb, hipStream_t s) {
  if (rows == 0) return hipSuccess;
  rmsnorm_bf16_kernel<<<(unsigned)((rows + 31) / 32), 256, 0, s>>>(x, w, eps, rows, (int)dim, xb);
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
// pool_and_normalize (model.rs:654-705).  candle sums over the token axis in
// token order per column and L2-reduces the last axis sequentially; each
// column's sum is one thread's sequential loop, the norms are one lane's loop,
// so the result is bit-identical to the CPU path.  One 256-thread block.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) pool_kernel(const float* __restrict__ tok,
                                                   const uint8_t* __restrict__ mask, int64_t t,
                                                   int64_t d, int64_t trunc,
                                                   float* __restrict__ out,
                                                   float* __restrict__ pooled) {
  __shared__ float s_norm;
  float cnt = 0.0f;
  if (mask) {
    for (int64_t j = 0; j < t; j++) cnt += mask[j] ? 1.0f : 0.0f;
    if (cnt < 1e-9f) cnt = 1e-9f;
  }
  const float inv_t = (float)(1.0 / (double)t);
  for (int64_t i = threadIdx.x; i < d; i += blockDim.x) {
    float s = 0.0f;
    if (mask) {
      for (int64_t j = 0; j < t; j++) s += tok[j * d + i] * (mask[j] ? 1.0f : 0.0f);
      pooled[i] = s / cnt;
    } else {
      for (int64_t j = 0; j < t; j++) s += tok[j * d + i];
      pooled[i] = s * inv_t + 0.0f;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float ss = 0.0f;
    for (int64_t i = 0; i < d; i++) ss += pooled[i] * pooled[i];
    float n = sqrtf(ss);
    s_norm = n < 1e-12f ? 1e-12f : n;
  }
  __syncthreads();
  const int64_t td = (trunc > 0 && trunc < d) ? trunc : d;
  float nrm = s_norm;
  if (td == d) {
    for (int64_t i = threadIdx.x; i < d; i += blockDim.x) out[i] = pooled[i] / nrm;
    return;
  }
  for (int64_t i = threadIdx.x; i < d; i += blockDim.x) pooled[i] = pooled[i] / nrm;
  __syncthreads();
  if (threadIdx.x == 0) {
    float ss = 0.0f;
    for (int64_t i = 0; i < td; i++) ss += pooled[i] * pooled[i];
    float n = sqrtf(ss);
    s_norm = n < 1e-12f ? 1e-12f : n;
  }
  __syncthreads();
  nrm = s_norm;
  for (int64_t i = threadIdx.x; i < td; i += blockDim.x) out[i] = pooled[i] / nrm;
}

hipError_t launch_pool(const float* tok, const uint8_t* mask, int64_t t, int64_t d, int64_t trunc,
                       float* out, float* scratch, hipStream_t s) {
  pool_kernel<<<1, 256, 0, s>>>(tok, mask, t, d, trunc, out, scratch);
  return hipGetLastError();
}

}  // namespace glypr
