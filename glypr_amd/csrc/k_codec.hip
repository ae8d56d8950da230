// k_codec.hip — Q8_0 codec kernels: load-time repack, dequantize, token-row
// gather, activation quantization.  All are HBM-bound byte/integer work:
// 16-byte vector loads/stores, no LDS.
#include <cstring>

#include "device_common.hpp"
#include "internal.hpp"

namespace glypr {

// ---------------------------------------------------------------------------
// Repack GGUF Q8_0 blocks [rows][nb][34] into qs int8 [rows][k] + dw f32
// [rows][nb].  One thread per block; the 34-byte source blocks are 2-byte
// aligned, so they are read as 17 halfwords.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) repack_kernel(const uint16_t* __restrict__ src,
                                                     int8_t* __restrict__ qs,
                                                     float* __restrict__ dw, int64_t nblocks) {
  int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint16_t* s = src + b * (BLOCK_BYTES / 2);
  uint16_t h[17];
#pragma unroll
  for (int i = 0; i < 17; i++) h[i] = s[i];
  dw[b] = f16_bits_to_f32(h[0]);
  v4i lo, hi;
  lo[0] = (int)h[1] | ((int)h[2] << 16);
  lo[1] = (int)h[3] | ((int)h[4] << 16);
  lo[2] = (int)h[5] | ((int)h[6] << 16);
  lo[3] = (int)h[7] | ((int)h[8] << 16);
  hi[0] = (int)h[9] | ((int)h[10] << 16);
  hi[1] = (int)h[11] | ((int)h[12] << 16);
  hi[2] = (int)h[13] | ((int)h[14] << 16);
  hi[3] = (int)h[15] | ((int)h[16] << 16);
  v4i* d = reinterpret_cast<v4i*>(qs + b * QK);
  d[0] = lo;
  d[1] = hi;
}

hipError_t launch_repack(const uint8_t* gguf, int8_t* qs, float* dw, int64_t rows, int64_t k,
                         hipStream_t s) {
  int64_t nblocks = rows * (k / QK);
  if (nblocks == 0) return hipSuccess;
  int64_t grid = (nblocks + 255) / 256;
  repack_kernel<<<dim3((unsigned)grid), dim3(256), 0, s>>>(
      reinterpret_cast<const uint16_t*>(gguf), qs, dw, nblocks);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dequantize (BlockQ8_0::to_float): out = (float)q * f32(d).  One 16-byte
// chunk (16 values, half a block) per thread, grid-stride.
// Gather: the same per token row, times embed_scale as candle's affine
// (v * mul + 0).
// ---------------------------------------------------------------------------
template <bool GATHER>
__global__ void __launch_bounds__(256) dequant_rows_kernel(const int8_t* __restrict__ qs,
                                                           const float* __restrict__ dw,
                                                           int64_t k,
                                                           const uint32_t* __restrict__ ids,
                                                           int64_t rows, float scale,
                                                           float* __restrict__ out) {
  const int64_t cpr = k / 16;  // 16-byte chunks per row
  const int64_t total = rows * cpr;
  const int64_t nb = k / QK;
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < total;
       c += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = c / cpr;
    int64_t j = c - r * cpr;
    int64_t src = GATHER ? (int64_t)ids[r] : r;
    v4i q = *reinterpret_cast<const v4i*>(qs + src * k + j * 16);
    float d = dw[src * nb + (j >> 1)];
    v4f o[4];
#pragma unroll
    for (int w = 0; w < 4; w++) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int8_t v = (int8_t)((q[w] >> (8 * e)) & 0xFF);
        float y = (float)v * d;
        if (GATHER) y = y * scale + 0.0f;
        o[w][e] = y;
      }
    }
    v4f* dst = reinterpret_cast<v4f*>(out + r * k + j * 16);
#pragma unroll
    for (int w = 0; w < 4; w++) dst[w] = o[w];
  }
}

static unsigned grid_for(int64_t work, int threads, int64_t cap) {
  int64_t g = (work + threads - 1) / threads;
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return (unsigned)g;
}

hipError_t launch_dequant(const int8_t* qs, const float* dw, int64_t rows, int64_t k, float* out,
                          hipStream_t s) {
  int64_t work = rows * (k / 16);
  if (work == 0) return hipSuccess;
  dequant_rows_kernel<false><<<grid_for(work, 256, 65536), 256, 0, s>>>(qs, dw, k, nullptr, rows,
                                                                        1.0f, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Token-row gather (Embedding::forward x embed_scale): out[r] =
// ((float)q * f32(d)) * scale + 0 for table row ids[r], the dequant kernel's
// arithmetic.  The write of the f32 rows is 80 % of the bytes, so every store
// instruction covers 1 KB of contiguous output: lane l of a wave handles 4
// int8 values (one 32-bit load) and writes them as one 16-byte store, and a
// block of k/4 lanes covers a row.  Each block walks GATHER_ROWS rows with all
// their loads issued before the stores, so several rows are in flight per
// wave; the row ids are block-uniform scalar loads.
// ---------------------------------------------------------------------------
constexpr int GATHER_ROWS = 8;

template <class Ids>
__global__ void __launch_bounds__(256) gather_rows_kernel(const int8_t* __restrict__ qs,
                                                          const float* __restrict__ dw, int k,
                                                          Ids ids, int64_t rows, float scale,
                                                          float* __restrict__ out) {
  const int lanes_per_row = k >> 2;
  const int c = threadIdx.x;   // 4-value column group
  if (c >= lanes_per_row) return;
  const int64_t r0 = (int64_t)blockIdx.x * GATHER_ROWS;
  const int nb = k >> 5;
  int q[GATHER_ROWS];
  float d[GATHER_ROWS];
#pragma unroll
  for (int i = 0; i < GATHER_ROWS; i++) {
    const int64_t r = r0 + i;
    if (r < rows) {
      const int64_t src = (int64_t)ids[r];
      q[i] = *reinterpret_cast<const int*>(qs + src * k + 4 * c);
      d[i] = dw[src * nb + (c >> 3)];
    }
  }
#pragma unroll
  for (int i = 0; i < GATHER_ROWS; i++) {
    const int64_t r = r0 + i;
    if (r >= rows) break;
    v4f o;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float y = (float)(int8_t)((q[i] >> (8 * e)) & 0xFF) * d[i];
      o[e] = y * scale + 0.0f;
    }
    *reinterpret_cast<v4f*>(out + r * k + 4 * c) = o;
  }
}

static bool gather_rows_ok(int64_t k) { return k % 32 == 0 && k / 4 <= 256; }

hipError_t launch_gather(const int8_t* qs, const float* dw, int64_t k, const uint32_t* ids,
                         int64_t n_ids, float scale, float* out, hipStream_t s) {
  if (n_ids == 0) return hipSuccess;
  if (gather_rows_ok(k)) {
    const int threads = (int)((k / 4 + 63) / 64 * 64);
    const int64_t blocks = (n_ids + GATHER_ROWS - 1) / GATHER_ROWS;
    gather_rows_kernel<const uint32_t*><<<(unsigned)blocks, threads, 0, s>>>(
        qs, dw, (int)k, ids, n_ids, scale, out);
    return hipGetLastError();
  }
  const int64_t work = n_ids * (k / 16);
  dequant_rows_kernel<true><<<grid_for(work, 256, 65536), 256, 0, s>>>(qs, dw, k, ids, n_ids,
                                                                       scale, out);
  return hipGetLastError();
}

bool gather_host_ids_ok(int64_t k, int64_t n_ids) {
  return gather_rows_ok(k) && n_ids > 0 && n_ids <= GATHER_ARG_IDS;
}

hipError_t launch_gather_host_ids(const int8_t* qs, const float* dw, int64_t k,
                                  const uint32_t* host_ids, int64_t n_ids, float scale, float* out,
                                  hipStream_t s) {
  if (!gather_host_ids_ok(k, n_ids)) return hipErrorInvalidValue;
  GatherIds ids;
  memcpy(ids.v, host_ids, (size_t)n_ids * 4);
  const int threads = (int)((k / 4 + 63) / 64 * 64);
  const int64_t blocks = (n_ids + GATHER_ROWS - 1) / GATHER_ROWS;
  gather_rows_kernel<GatherIds><<<(unsigned)blocks, threads, 0, s>>>(qs, dw, (int)k, ids, n_ids,
                                                                     scale, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Activation quantization (BlockQ8_0::from_float).  Eight lanes per 32-value
// block, four values (one float4) per lane: amax by three xor-shuffles (max is
// order independent, so exact), then each lane rounds its four values and
// stores them as one 32-bit word.  A wave covers 8 consecutive blocks: 1 KB of
// contiguous f32 reads and 256 B of contiguous int8 writes.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) quantize_planar_kernel(const float* __restrict__ x,
                                                              int64_t nblocks,
                                                              int8_t* __restrict__ xq,
                                                              float* __restrict__ dx) {
  int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t b = gid >> 3;
  int j = threadIdx.x & 7;
  bool ok = b < nblocks;
  v4f v = ok ? *reinterpret_cast<const v4f*>(x + b * QK + 4 * j) : v4f{0, 0, 0, 0};
  float a = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; e++) a = fmaxf(a, fabsf(v[e]));
  a = max8(a);
  QScale sc = q8_scale(a);
  uint32_t packed = 0;
#pragma unroll
  for (int e = 0; e < 4; e++) packed |= ((uint32_t)(quant_round(v[e] * sc.id) & 0xFF)) << (8 * e);
  if (ok) {
    *reinterpret_cast<uint32_t*>(xq + b * QK + 4 * j) = packed;
    if (j == 0) dx[b] = sc.dq;
  }
}

hipError_t launch_quantize_planar(const float* x, int64_t m, int64_t k, int8_t* xq, float* dx,
                                  hipStream_t s) {
  int64_t nblocks = m * (k / QK);
  if (nblocks == 0) return hipSuccess;
  int64_t threads = nblocks * 8;
  quantize_planar_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(x, nblocks, xq, dx);
  return hipGetLastError();
}

// Same arithmetic, GGUF block output (34 bytes per block, 2-byte aligned):
// the 8 lanes of a block each write two halfwords of qs; lane 0 writes d.
__global__ void __launch_bounds__(256) quantize_gguf_kernel(const float* __restrict__ x,
                                                            int64_t nblocks,
                                                            uint16_t* __restrict__ out) {
  int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t b = gid >> 3;
  int j = threadIdx.x & 7;
  bool ok = b < nblocks;
  v4f v = ok ? *reinterpret_cast<const v4f*>(x + b * QK + 4 * j) : v4f{0, 0, 0, 0};
  float a = 0.0f;
#pragma unroll
  for (int e = 0; e < 4; e++) a = fmaxf(a, fabsf(v[e]));
  a = max8(a);
  QScale sc = q8_scale(a);
  uint32_t q0 = (uint32_t)(quant_round(v[0] * sc.id) & 0xFF);
  uint32_t q1 = (uint32_t)(quant_round(v[1] * sc.id) & 0xFF);
  uint32_t q2 = (uint32_t)(quant_round(v[2] * sc.id) & 0xFF);
  uint32_t q3 = (uint32_t)(quant_round(v[3] * sc.id) & 0xFF);
  if (ok) {
    uint16_t* blk = out + b * (BLOCK_BYTES / 2);
    blk[1 + 2 * j] = (uint16_t)(q0 | (q1 << 8));
    blk[2 + 2 * j] = (uint16_t)(q2 | (q3 << 8));
    if (j == 0) blk[0] = sc.dbits;
  }
}

hipError_t launch_quantize_gguf(const float* x, int64_t m, int64_t k, uint8_t* out,
                                hipStream_t s) {
  int64_t nblocks = m * (k / QK);
  if (nblocks == 0) return hipSuccess;
  int64_t threads = nblocks * 8;
  quantize_gguf_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(
      x, nblocks, reinterpret_cast<uint16_t*>(out));
  return hipGetLastError();
}

// f32 -> bf16 (round to nearest even) for the bf16-dequant GEMM's activations.
__global__ void __launch_bounds__(256) to_bf16_kernel(const float* __restrict__ x, int64_t n4,
                                                      uint32_t* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * blockDim.x) {
    v4f v = reinterpret_cast<const v4f*>(x)[i];
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      uint32_t u = __float_as_uint(v[e]);
      uint32_t r = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
      if ((u & 0x7FFFFFFFu) > 0x7F800000u) r = (u >> 16) | 0x40u;  // quiet NaN
      w[e] = r;
    }
    out[2 * i] = w[0] | (w[1] << 16);
    out[2 * i + 1] = w[2] | (w[3] << 16);
  }
}

hipError_t launch_to_bf16(const float* x, int64_t n, uint16_t* out, hipStream_t s) {
  int64_t n4 = n / 4;
  if (n4 == 0) return hipSuccess;
  to_bf16_kernel<<<grid_for(n4, 256, 65536), 256, 0, s>>>(x, n4, reinterpret_cast<uint32_t*>(out));
  return hipGetLastError();
}

}  // namespace glypr
