// k_vec.hip — output-vector codecs for the serving path (glypr-core util.rs:
// 52-197): 1-bit and symmetric int8 quantization of embeddings, and all-pairs
// similarity between a query set and a database of encoded vectors.
//
//  - quantize_binary: bit i of word i/64 is (x[i] > 0).  With dim % 256 == 0
//    a lane loads 4 consecutive elements (one 16-byte load, 1 KB per wave),
//    forms their nibble, and 16 lanes' nibbles shift-or into one word;
//    otherwise lane i holds element 64 w + i and the wave's ballot IS word w.
//    Grid-stride loops, 4 (8) loads in flight per wave.
//  - quantize_int8: (x * 127).round().clamp(-127, 127) as i8, NaN -> 0.
//  - hamming / binary cosine: one thread per database row, the row's words in
//    registers, the query words read wave-uniformly (scalar loads); every
//    database byte is read once from HBM.  The binary cosine looks up
//    cos(pi * h / dim) in a host-built table (h takes only dim + 1 values),
//    staged in LDS per workgroup.
//  - int8 dot / int8 cosine: the all-pairs product is an int8 GEMM with exact
//    i32 sums, so it runs on v_mfma_i32_16x16x64_i8: a wave holds 16 database
//    rows against up to 64 queries, streaming K in 64-byte steps (16 bytes per
//    lane); the database is read once per 64-query group, and for the cosine
//    its row norms are summed from the same fragments.  Integer sums are
//    order-free, so the result equals the reference's 4-lane sum bit for bit.
#include "device_common.hpp"
#include "internal.hpp"

namespace glypr {

namespace {


constexpr int BIN_CPW = 4;   // 256-element chunks per wave per iteration (4 words each)

// Lane l loads elements 4 l .. 4 l + 3 of a 256-element chunk as one float4
// (1 KB per wave load) and forms their 4-bit nibble; word j of the chunk is
// the nibbles of lanes 16 j .. 16 j + 15 in lane order, gathered by three
// shift-or steps down each 16-lane group into lane 16 j.
__global__ void __launch_bounds__(256) quantize_binary_kernel(const float* __restrict__ x,
                                                              int64_t words,
                                                              unsigned long long* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t chunks = words >> 2;   // words % 4 == 0 (dim % 256 == 0)
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t c0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * BIN_CPW; c0 < chunks;
       c0 += nwaves * BIN_CPW) {
    v4f v[BIN_CPW];
#pragma unroll
    for (int t = 0; t < BIN_CPW; t++)
      v[t] = c0 + t < chunks ? *reinterpret_cast<const v4f*>(x + (c0 + t) * 256 + 4 * lane)
                             : v4f{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < BIN_CPW; t++) {
      const uint32_t n = (uint32_t)(v[t][0] > 0.0f) | ((uint32_t)(v[t][1] > 0.0f) << 1) |
                         ((uint32_t)(v[t][2] > 0.0f) << 2) | ((uint32_t)(v[t][3] > 0.0f) << 3);
      const uint32_t n2 = n | ((uint32_t)__shfl_down((int)n, 1, 16) << 4);      // 8 bits
      const uint32_t n4 = n2 | ((uint32_t)__shfl_down((int)n2, 2, 16) << 8);    // 16 bits
      const uint32_t n8 = n4 | ((uint32_t)__shfl_down((int)n4, 4, 16) << 16);   // 32 bits
      const uint32_t hi = (uint32_t)__shfl_down((int)n8, 8, 16);               // next 32
      if ((lane & 15) == 0 && c0 + t < chunks)
        out[(c0 + t) * 4 + (lane >> 4)] = (unsigned long long)n8 | ((unsigned long long)hi << 32);
    }
  }
}

// Any dim % 64 == 0: lane i holds element 64 w + i, so the ballot IS word w.
constexpr int BIN_WPW = 8;   // words per wave per iteration
__global__ void __launch_bounds__(256) quantize_binary_word_kernel(
    const float* __restrict__ x, int64_t words, unsigned long long* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t w0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * BIN_WPW; w0 < words;
       w0 += nwaves * BIN_WPW) {
    float v[BIN_WPW];
#pragma unroll
    for (int t = 0; t < BIN_WPW; t++)
      v[t] = w0 + t < words ? x[(w0 + t) * 64 + lane] : 0.0f;
    unsigned long long mine = 0;
#pragma unroll
    for (int t = 0; t < BIN_WPW; t++) {
      const unsigned long long bits = __ballot(v[t] > 0.0f);
      if (lane == t) mine = bits;
    }
    if (lane < BIN_WPW && w0 + lane < words) out[w0 + lane] = mine;
  }
}

__global__ void __launch_bounds__(256) quantize_int8_kernel(const float* __restrict__ x,
                                                            int64_t n, int8_t* __restrict__ out) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  auto q = [](float v) -> int {
    const float r = roundf(v * 127.0f);
    if (r != r) return 0;
    return (int)fminf(fmaxf(r, -127.0f), 127.0f);
  };
  if (i + 4 <= n) {
    const v4f v = *reinterpret_cast<const v4f*>(x + i);
    const uint32_t packed = (uint32_t)(q(v[0]) & 0xFF) | ((uint32_t)(q(v[1]) & 0xFF) << 8) |
                            ((uint32_t)(q(v[2]) & 0xFF) << 16) | ((uint32_t)(q(v[3]) & 0xFF) << 24);
    *reinterpret_cast<uint32_t*>(out + i) = packed;
  } else {
    for (int64_t e = i; e < n; e++) out[e] = (int8_t)q(x[e]);
  }
}

// out[i][j] = popcount(a_i ^ b_j) (u32) or table[that] (f32).  W words per row.
// The cosine table (64 W + 1 floats) is staged in LDS: every output looks it
// up at a lane-dependent index.
template <int W, bool COS>
__global__ void __launch_bounds__(256) hamming_kernel(const unsigned long long* __restrict__ a,
                                                      int64_t na,
                                                      const unsigned long long* __restrict__ b,
                                                      int64_t nb, uint32_t* __restrict__ out_h,
                                                      const float* __restrict__ table,
                                                      float* __restrict__ out_c) {
  __shared__ float tab[COS ? 64 * W + 1 : 1];
  if constexpr (COS) {
    for (int i = threadIdx.x; i <= 64 * W; i += 256) tab[i] = table[i];
    __syncthreads();
  }
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= nb) return;
  unsigned long long row[W];
#pragma unroll
  for (int w = 0; w < W; w++) row[w] = b[j * W + w];
  for (int64_t i = 0; i < na; i++) {
    uint32_t h = 0;
#pragma unroll
    for (int w = 0; w < W; w++) h += (uint32_t)__popcll(a[i * W + w] ^ row[w]);
    if (COS) out_c[i * nb + j] = tab[h];
    else out_h[i * nb + j] = h;
  }
}

// Any word count: the row is re-read per query (from the cache).
template <bool COS>
__global__ void __launch_bounds__(256) hamming_generic_kernel(
    const unsigned long long* __restrict__ a, int64_t na, const unsigned long long* __restrict__ b,
    int64_t nb, int64_t words, uint32_t* __restrict__ out_h, const float* __restrict__ table,
    float* __restrict__ out_c) {
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= nb) return;
  const unsigned long long* row = b + j * words;
  for (int64_t i = 0; i < na; i++) {
    uint32_t h = 0;
    for (int64_t w = 0; w < words; w++) h += (uint32_t)__popcll(a[i * words + w] ^ row[w]);
    if (COS) out_c[i * nb + j] = table[h];
    else out_h[i * nb + j] = h;
  }
}

// Sum of squares of each int8 row (exact i32): one wave per row.
__global__ void __launch_bounds__(256) int8_row_norms_kernel(const int8_t* __restrict__ x,
                                                             int64_t rows, int64_t dim,
                                                             int32_t* __restrict__ out) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const int8_t* p = x + r * dim;
  int32_t s = 0;
  for (int64_t e = lane; e < dim; e += 64) s += (int32_t)p[e] * (int32_t)p[e];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
  if (lane == 0) out[r] = s;
}

// 16 bytes of row `row` at byte k (zero past dim).  FAST: dim % 16 == 0 and
// 16-byte aligned rows, so a k < dim chunk is whole.
template <bool FAST>
__device__ __forceinline__ v4i load16(const int8_t* base, int64_t row, int64_t dim, int64_t k) {
  const int8_t* p = base + row * dim + k;
  if (FAST) return k < dim ? *reinterpret_cast<const v4i*>(p) : v4i{0, 0, 0, 0};
  v4i v = {0, 0, 0, 0};
#pragma unroll
  for (int e = 0; e < 16; e++)
    if (k + e < dim) v[e >> 2] |= (int)(uint8_t)p[e] << (8 * (e & 3));
  return v;
}

__device__ __forceinline__ int32_t sq_sum16(v4i v) {
  int32_t s = 0;
#pragma unroll
  for (int e = 0; e < 16; e++) {
    const int32_t b = (int8_t)(v[e >> 2] >> (8 * (e & 3)));
    s += b * b;
  }
  return s;
}

// All-pairs int8 dot on MFMA.  A wave: database rows j0 .. j0+15 (output
// column = lane & 15) against MT tiles of 16 queries (output rows
// 16 t + 4 (lane >> 4) + r).  Lane (l16, lq) feeds bytes k0 + 16 lq .. +15 of
// its rows to both operands.  COS: the epilogue applies
// int8_cosine_similarity with the queries' norms and the database rows' norms
// summed here from the same fragments.
template <int MT, bool FAST, bool COS>
__global__ void __launch_bounds__(256) int8_pairs_kernel(
    const int8_t* __restrict__ a, int64_t na, const int8_t* __restrict__ b, int64_t nb,
    int64_t dim, int32_t* __restrict__ out_d, const int32_t* __restrict__ norm_a,
    float* __restrict__ out_c) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, lq = lane >> 4;
  const int64_t j0 = ((int64_t)blockIdx.x * 4 + wave) * 16;
  if (j0 >= nb) return;   // whole wave exits together
  const int64_t i0 = (int64_t)blockIdx.y * 16 * MT;
  const int64_t jr = j0 + l16 < nb ? j0 + l16 : nb - 1;
  int64_t ir[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) ir[t] = i0 + 16 * t + l16 < na ? i0 + 16 * t + l16 : na - 1;
  v4i acc[MT];
#pragma unroll
  for (int t = 0; t < MT; t++) acc[t] = v4i{0, 0, 0, 0};
  int32_t nsq = 0;
#pragma unroll 2
  for (int64_t k0 = 0; k0 < dim; k0 += 64) {
    const int64_t k = k0 + 16 * lq;
    const v4i bf = load16<FAST>(b, jr, dim, k);
    if (COS) nsq += sq_sum16(bf);
#pragma unroll
    for (int t = 0; t < MT; t++) {
      const v4i af = load16<FAST>(a, ir[t], dim, k);
      acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf, acc[t], 0, 0, 0);
    }
  }
  if (COS) {   // row l16's norm: its four 16-byte slices sit in lanes l16 + 16 lq
    nsq += __shfl_xor(nsq, 16);
    nsq += __shfl_xor(nsq, 32);
  }
  const int64_t j = j0 + l16;
  if (j >= nb) return;
#pragma unroll
  for (int t = 0; t < MT; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int64_t i = i0 + 16 * t + 4 * lq + r;
      if (i >= na) continue;
      if (!COS) {
        out_d[i * nb + j] = acc[t][r];
      } else {
        const int32_t nai = norm_a[i];
        float c = 0.0f;
        if (nai != 0 && nsq != 0) {
          const float denom = sqrtf((float)nai) * sqrtf((float)nsq);
          c = fminf(fmaxf((float)acc[t][r] / denom, -1.0f), 1.0f);
        }
        out_c[i * nb + j] = c;
      }
    }
}

template <bool COS>
hipError_t run_hamming(const unsigned long long* a, int64_t na, const unsigned long long* b,
                       int64_t nb, int64_t words, uint32_t* out_h, const float* table,
                       float* out_c, hipStream_t s) {
  const unsigned grid = (unsigned)((nb + 255) / 256);
#define GLYPR_HAMMING_W(w)                                                                     \
  case w:                                                                                      \
    hamming_kernel<w, COS><<<grid, 256, 0, s>>>(a, na, b, nb, out_h, table, out_c);           \
    return hipGetLastError();
  switch (words) {
    GLYPR_HAMMING_W(1)
    GLYPR_HAMMING_W(2)
    GLYPR_HAMMING_W(4)
    GLYPR_HAMMING_W(8)
    GLYPR_HAMMING_W(12)
    GLYPR_HAMMING_W(16)
    default:
      hamming_generic_kernel<COS><<<grid, 256, 0, s>>>(a, na, b, nb, words, out_h, table, out_c);
      return hipGetLastError();
  }
#undef GLYPR_HAMMING_W
}

template <int MT, bool COS>
hipError_t run_int8_pairs_mt(const int8_t* a, int64_t na, const int8_t* b, int64_t nb,
                             int64_t dim, int32_t* out_d, const int32_t* norm_a, float* out_c,
                             hipStream_t s) {
  const dim3 grid((unsigned)((nb + 63) / 64), (unsigned)((na + 16 * MT - 1) / (16 * MT)));
  if (dim % 16 == 0)
    int8_pairs_kernel<MT, true, COS><<<grid, 256, 0, s>>>(a, na, b, nb, dim, out_d, norm_a,
                                                          out_c);
  else
    int8_pairs_kernel<MT, false, COS><<<grid, 256, 0, s>>>(a, na, b, nb, dim, out_d, norm_a,
                                                           out_c);
  return hipGetLastError();
}

// Query tiles per wave: just enough 16-row tiles for na (at most 4 per pass).
template <bool COS>
hipError_t run_int8_pairs(const int8_t* a, int64_t na, const int8_t* b, int64_t nb, int64_t dim,
                          int32_t* out_d, const int32_t* norm_a, float* out_c, hipStream_t s) {
  if (na <= 16) return run_int8_pairs_mt<1, COS>(a, na, b, nb, dim, out_d, norm_a, out_c, s);
  if (na <= 32) return run_int8_pairs_mt<2, COS>(a, na, b, nb, dim, out_d, norm_a, out_c, s);
  return run_int8_pairs_mt<4, COS>(a, na, b, nb, dim, out_d, norm_a, out_c, s);
}

}  // namespace

hipError_t launch_quantize_binary(const float* x, int64_t n, int64_t dim, uint64_t* out,
                                  hipStream_t s) {
  const int64_t words = n * (dim / 64);
  if (words == 0) return hipSuccess;
  if (dim % 256 == 0) {
    const int64_t blocks = (words / 4 + 4 * BIN_CPW - 1) / (4 * BIN_CPW);
    quantize_binary_kernel<<<(unsigned)(blocks < 16384 ? blocks : 16384), 256, 0, s>>>(
        x, words, reinterpret_cast<unsigned long long*>(out));
  } else {
    const int64_t blocks = (words + 4 * BIN_WPW - 1) / (4 * BIN_WPW);
    quantize_binary_word_kernel<<<(unsigned)(blocks < 16384 ? blocks : 16384), 256, 0, s>>>(
        x, words, reinterpret_cast<unsigned long long*>(out));
  }
  return hipGetLastError();
}

hipError_t launch_quantize_int8(const float* x, int64_t count, int8_t* out, hipStream_t s) {
  if (count == 0) return hipSuccess;
  quantize_int8_kernel<<<(unsigned)((count + 1023) / 1024), 256, 0, s>>>(x, count, out);
  return hipGetLastError();
}

hipError_t launch_hamming(const uint64_t* a, int64_t na, const uint64_t* b, int64_t nb,
                          int64_t words, uint32_t* out, hipStream_t s) {
  if (na == 0 || nb == 0) return hipSuccess;
  return run_hamming<false>(reinterpret_cast<const unsigned long long*>(a), na,
                            reinterpret_cast<const unsigned long long*>(b), nb, words, out,
                            nullptr, nullptr, s);
}

hipError_t launch_binary_cosine(const uint64_t* a, int64_t na, const uint64_t* b, int64_t nb,
                                int64_t words, const float* table, float* out, hipStream_t s) {
  if (na == 0 || nb == 0) return hipSuccess;
  return run_hamming<true>(reinterpret_cast<const unsigned long long*>(a), na,
                           reinterpret_cast<const unsigned long long*>(b), nb, words, nullptr,
                           table, out, s);
}

hipError_t launch_int8_dot(const int8_t* a, int64_t na, const int8_t* b, int64_t nb, int64_t dim,
                           int32_t* out, hipStream_t s) {
  if (na == 0 || nb == 0) return hipSuccess;
  return run_int8_pairs<false>(a, na, b, nb, dim, out, nullptr, nullptr, s);
}

hipError_t launch_int8_cosine(const int8_t* a, int64_t na, const int8_t* b, int64_t nb,
                              int64_t dim, int32_t* norms, float* out, hipStream_t s) {
  if (na == 0 || nb == 0) return hipSuccess;
  int8_row_norms_kernel<<<(unsigned)((na + 3) / 4), 256, 0, s>>>(a, na, dim, norms);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return run_int8_pairs<true>(a, na, b, nb, dim, nullptr, norms, out, s);
}

}  // namespace glypr
