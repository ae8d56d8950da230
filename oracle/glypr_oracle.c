/*
 * glypr_oracle.c — CPU restatement of glypr's CPU Q8_0 path (oracle + CPU baseline).
 *
 * TEST INFRASTRUCTURE ONLY (see glypr_oracle.h).  Build: oracle/Makefile
 * (gcc -O3 -march=x86-64-v3 -ffp-contract=off -fopenmp).  -ffp-contract=off is
 * load-bearing: Rust never contracts a*b+c into an FMA, so neither may we,
 * except where the reference itself uses mul_add (RMSNorm lanes).
 *
 * Citations are path:line inside the reference tree (phrozen/glypr v0.3.0).
 */
#include "glypr_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int orc_threads(int threads) {
#ifdef _OPENMP
  return threads > 0 ? threads : omp_get_max_threads();
#else
  (void)threads;
  return 1;
#endif
}

/* ======================================================================== */
/* f16 codec.  glypr stores Q8_0 scales as IEEE binary16 (half 2.7.1,        */
/* Cargo.lock:1341-1344): f32 -> f16 rounds to nearest even, overflow -> inf. */
/* ======================================================================== */

uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) {             /* inf / NaN */
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    return (uint16_t)(sign | 0x7C00u);
  }
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
  if (ax < 0x38800000u) {              /* below 2^-14: f16 subnormal or zero */
    if (ax < 0x33000000u) return (uint16_t)sign;            /* < 2^-25 -> 0 */
    uint32_t e = ax >> 23;
    uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e;         /* value / 2^-24 = mant >> shift */
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t r = ax - 0x38000000u;       /* rebias exponent 127 -> 15 */
  r += 0xFFFu + ((r >> 13) & 1u);      /* round 23 -> 10 mantissa bits, ties to even */
  return (uint16_t)(sign | (r >> 13));
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  uint32_t bits;
  if (e == 0x1Fu) {
    bits = sign | 0x7F800000u | (m << 13);
  } else if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {                           /* subnormal: m * 2^-24 */
      float v = (float)m * 5.9604644775390625e-08f;
      memcpy(&bits, &v, 4);
      bits |= sign;
    }
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

void orc_f32_to_f16_array(const float* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = orc_f32_to_f16(x[i]);
}
void orc_f16_to_f32_array(const uint16_t* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = orc_f16_to_f32(x[i]);
}

/* ======================================================================== */
/* Q8_0 codec (candle k_quants::BlockQ8_0, restated from the GGML Q8_0 def.) */
/* ======================================================================== */

static inline uint16_t blk_d(const uint8_t* b) { return (uint16_t)(b[0] | (b[1] << 8)); }
static inline const int8_t* blk_qs(const uint8_t* b) { return (const int8_t*)(b + 2); }

/* Rust `f32::round(v) as i8`: round half away from zero, saturating cast, NaN -> 0. */
static inline int8_t round_to_i8(float v) {
  if (v != v) return 0;
  float r = roundf(v);
  if (r > 127.0f) return 127;
  if (r < -128.0f) return -128;
  return (int8_t)r;
}

/* BlockQ8_0::from_float: per block amax = max|x| (f32::max ignores NaN),
 * d = amax / 127 (f32), id = d != 0 ? 1/d : 0 (from the f32 d, not the f16 one),
 * qs[j] = round(x[j] * id), d stored as f16.  Reached for activations from
 * k_quants::matmul via LinearOp::forward (linear.rs:153-162). */
void orc_q8_0_quantize_row(const float* x, int64_t k, uint8_t* blocks) {
  int64_t nb = k / ORC_QK8_0;
  for (int64_t b = 0; b < nb; b++) {
    const float* xs = x + b * ORC_QK8_0;
    uint8_t* out = blocks + b * ORC_BLOCK_BYTES;
    float amax = 0.0f;
    for (int j = 0; j < ORC_QK8_0; j++) {
      float a = fabsf(xs[j]);
      if (a > amax) amax = a;   /* f32::max: a NaN operand is ignored */
    }
    float d = amax / 127.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    uint16_t dh = orc_f32_to_f16(d);
    out[0] = (uint8_t)(dh & 0xFF);
    out[1] = (uint8_t)(dh >> 8);
    int8_t* qs = (int8_t*)(out + 2);
    for (int j = 0; j < ORC_QK8_0; j++) qs[j] = round_to_i8(xs[j] * id);
  }
}

void orc_q8_0_quantize_rows(const float* x, int64_t m, int64_t k, uint8_t* blocks) {
  int64_t rb = (k / ORC_QK8_0) * ORC_BLOCK_BYTES;
  for (int64_t i = 0; i < m; i++) orc_q8_0_quantize_row(x + i * k, k, blocks + i * rb);
}

/* BlockQ8_0::to_float (QTensor::dequantize, model.rs:252-254): y = (f32)q * f32(d). */
void orc_q8_0_dequantize_row(const uint8_t* blocks, int64_t k, float* y) {
  int64_t nb = k / ORC_QK8_0;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t* blk = blocks + b * ORC_BLOCK_BYTES;
    float d = orc_f16_to_f32(blk_d(blk));
    const int8_t* qs = blk_qs(blk);
    for (int j = 0; j < ORC_QK8_0; j++) y[b * ORC_QK8_0 + j] = (float)qs[j] * d;
  }
}

void orc_q8_0_dequantize_rows(const uint8_t* blocks, int64_t rows, int64_t k, float* y) {
  int64_t rb = (k / ORC_QK8_0) * ORC_BLOCK_BYTES;
  for (int64_t i = 0; i < rows; i++) orc_q8_0_dequantize_row(blocks + i * rb, k, y + i * k);
}

/* BlockQ8_0::vec_dot_unopt, the path a default x86-64 build of glypr takes
 * (no target_feature=avx in the reference's build config): per block an
 * exact i32 sum, then sumf += sum_i as f32 * d_w * d_x, left to right. */
float orc_q8_0_vec_dot(int64_t k, const uint8_t* wblocks, const uint8_t* xblocks) {
  int64_t nb = k / ORC_QK8_0;
  float sumf = 0.0f;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t* wb = wblocks + b * ORC_BLOCK_BYTES;
    const uint8_t* xb = xblocks + b * ORC_BLOCK_BYTES;
    const int8_t* wq = blk_qs(wb);
    const int8_t* xq = blk_qs(xb);
    int32_t isum = 0;
    for (int j = 0; j < ORC_QK8_0; j++) isum += (int32_t)wq[j] * (int32_t)xq[j];
    sumf += (float)isum * orc_f16_to_f32(blk_d(wb)) * orc_f16_to_f32(blk_d(xb));
  }
  return sumf;
}

/* k_quants::matmul::<BlockQ8_0> (call site linear.rs:153-162): rows of x are
 * quantized serially, then every output is one vec_dot(W[n], Xq[m]).  candle
 * runs the columns of each row in parallel (Rayon, 128..512 per task); the
 * arithmetic of each output is independent of the schedule. */
void orc_q8_0_matmul_preq(const uint8_t* xq, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                          float* y, int threads) {
  int64_t rb = (k / ORC_QK8_0) * ORC_BLOCK_BYTES;
  int nt = orc_threads(threads);
  const int64_t chunk = 128;
  int64_t nchunks = (n + chunk - 1) / chunk;
  int64_t total = m * nchunks;
#pragma omp parallel for num_threads(nt) schedule(dynamic, 4)
  for (int64_t t = 0; t < total; t++) {
    int64_t i = t / nchunks;
    int64_t c0 = (t % nchunks) * chunk;
    int64_t c1 = c0 + chunk < n ? c0 + chunk : n;
    const uint8_t* xr = xq + i * rb;
    for (int64_t c = c0; c < c1; c++) y[i * n + c] = orc_q8_0_vec_dot(k, w + c * rb, xr);
  }
}

void orc_q8_0_matmul(const float* x, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                     float* y, int threads) {
  int64_t rb = (k / ORC_QK8_0) * ORC_BLOCK_BYTES;
  uint8_t* xq = (uint8_t*)malloc((size_t)(m * rb > 0 ? m * rb : 1));
  orc_q8_0_quantize_rows(x, m, k, xq);   /* serial, as in candle */
  orc_q8_0_matmul_preq(xq, m, k, w, n, y, threads);
  free(xq);
}

/* The INT8_FMA variant (no counterpart in the reference): vec_dot_unopt's
 * operands and block order, with the last two roundings of each block fused,
 * sumf = fmaf((float)isum * d_w, d_x, sumf).  fmaf is the C99 correctly
 * rounded fused multiply-add. */
float orc_q8_0_vec_dot_fma(int64_t k, const uint8_t* wblocks, const uint8_t* xblocks) {
  int64_t nb = k / ORC_QK8_0;
  float sumf = 0.0f;
  for (int64_t b = 0; b < nb; b++) {
    const uint8_t* wb = wblocks + b * ORC_BLOCK_BYTES;
    const uint8_t* xb = xblocks + b * ORC_BLOCK_BYTES;
    const int8_t* wq = blk_qs(wb);
    const int8_t* xq = blk_qs(xb);
    int32_t isum = 0;
    for (int j = 0; j < ORC_QK8_0; j++) isum += (int32_t)wq[j] * (int32_t)xq[j];
    const float t = (float)isum * orc_f16_to_f32(blk_d(wb));
    sumf = fmaf(t, orc_f16_to_f32(blk_d(xb)), sumf);
  }
  return sumf;
}

void orc_q8_0_matmul_fma(const float* x, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                         float* y, int threads) {
  int64_t rb = (k / ORC_QK8_0) * ORC_BLOCK_BYTES;
  uint8_t* xq = (uint8_t*)malloc((size_t)(m * rb > 0 ? m * rb : 1));
  orc_q8_0_quantize_rows(x, m, k, xq);
  int nt = orc_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int64_t i = 0; i < m; i++)
    for (int64_t c = 0; c < n; c++) y[i * n + c] = orc_q8_0_vec_dot_fma(k, w + c * rb, xq + i * rb);
  free(xq);
}

void orc_q8_0_matmul_f64(const uint8_t* xq, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                         double* y) {
  int64_t nb = k / ORC_QK8_0;
  int64_t rb = nb * ORC_BLOCK_BYTES;
  for (int64_t i = 0; i < m; i++)
    for (int64_t c = 0; c < n; c++) {
      double acc = 0.0;
      for (int64_t b = 0; b < nb; b++) {
        const uint8_t* wb = w + c * rb + b * ORC_BLOCK_BYTES;
        const uint8_t* xb = xq + i * rb + b * ORC_BLOCK_BYTES;
        long isum = 0;
        for (int j = 0; j < ORC_QK8_0; j++) isum += (long)blk_qs(wb)[j] * (long)blk_qs(xb)[j];
        acc += (double)isum * (double)orc_f16_to_f32(blk_d(wb)) * (double)orc_f16_to_f32(blk_d(xb));
      }
      y[i * n + c] = acc;
    }
}

void orc_q8_0_matmul_dequant_f64(const float* x, int64_t m, int64_t k, const uint8_t* w,
                                 int64_t n, double* y, int threads) {
  float* wd = (float*)malloc((size_t)(n * k) * sizeof(float));
  orc_q8_0_dequantize_rows(w, n, k, wd);
  int nt = orc_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int64_t i = 0; i < m; i++)
    for (int64_t c = 0; c < n; c++) {
      double acc = 0.0;
      const float* xr = x + i * k;
      const float* wr = wd + c * k;
      for (int64_t j = 0; j < k; j++) acc += (double)xr[j] * (double)wr[j];
      y[i * n + c] = acc;
    }
  free(wd);
}

/* ======================================================================== */
/* RMSNorm: simd_rmsnorm_row_f32 (cpu_simd/rmsnorm.rs:6-47) as pulp runs it  */
/* on x86-64-v3 (AVX2+FMA, f32x8; pulp 0.22 without the x86-v4 feature):     */
/*   8 lane accumulators, lane j: acc_j = fma(x[8c+j], x[8c+j], acc_j);      */
/*   reduce_sum_f32s: s_j = l_j + l_{j+4}; ((s0+s2) + (s1+s3));             */
/*   tail: sum += x*x; inv = 1 / sqrt(sum/d + eps); y = (x*inv)*w.           */
/* ======================================================================== */

void orc_rmsnorm_row(const float* x, const float* weight, float eps, float* y, int64_t d) {
  float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t head = (d / 8) * 8;
  for (int64_t c = 0; c < head; c += 8)
    for (int j = 0; j < 8; j++) lane[j] = fmaf(x[c + j], x[c + j], lane[j]);
  float s0 = lane[0] + lane[4], s1 = lane[1] + lane[5], s2 = lane[2] + lane[6],
        s3 = lane[3] + lane[7];
  float sum = (s0 + s2) + (s1 + s3);
  for (int64_t c = head; c < d; c++) sum += x[c] * x[c];
  float inv = 1.0f / sqrtf(sum / (float)d + eps);
  if (weight) {
    for (int64_t i = 0; i < d; i++) y[i] = (x[i] * inv) * weight[i];
  } else {
    for (int64_t i = 0; i < d; i++) y[i] = x[i] * inv;
  }
}

/* CpuRMSNormOp::cpu_fwd (cpu_simd/rmsnorm.rs:59-118): rows in parallel. */
void orc_rmsnorm(const float* x, const float* weight, float eps, float* y, int64_t rows,
                 int64_t d, int threads) {
  int nt = orc_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static)
  for (int64_t r = 0; r < rows; r++) orc_rmsnorm_row(x + r * d, weight, eps, y + r * d, d);
}

/* ======================================================================== */
/* tanh.  glypr calls f32::tanh (platform libm: glibc on Linux, Apple libm on */
/* macOS), so its GeGLU bits are platform dependent.  The oracle and the GPU  */
/* share one definition instead, written only with IEEE +,-,*,/ and fma so    */
/* both sides round identically:                                              */
/*   tanh|x| = -t / (t + 2),  t = expm1(-2|x|)                                */
/* expm1 by Cody-Waite reduction y = k ln2 + r (fdlibm's float ln2 hi/lo      */
/* split), |r| <= ln2/2, degree-8 Taylor polynomial (truncation < 2e-10),     */
/* then expm1(y) = 2^k p + (2^k - 1).  Accuracy is measured against double    */
/* tanh in tests (a few ulp).  The HIP kernels carry an independent copy.     */
/* ======================================================================== */

static float orc_expm1_nonpos(float y) {  /* y <= 0 */
  if (y < -30.0f) return -1.0f;
  const float LOG2E = 1.44269504088896341f;
  const float LN2_HI = 6.93145751953125e-01f;   /* 0x3f317200 */
  const float LN2_LO = 1.42860682030941723e-06f; /* 0x35bfbe8e */
  float kf = rintf(y * LOG2E);
  float r = fmaf(-kf, LN2_HI, y);
  r = fmaf(-kf, LN2_LO, r);
  float p = fmaf(r, 2.48015873015873016e-05f, 1.98412698412698413e-04f); /* 1/40320, 1/5040 */
  p = fmaf(r, p, 1.38888888888888889e-03f);                              /* 1/720 */
  p = fmaf(r, p, 8.33333333333333333e-03f);                              /* 1/120 */
  p = fmaf(r, p, 4.16666666666666667e-02f);                              /* 1/24 */
  p = fmaf(r, p, 1.66666666666666667e-01f);                              /* 1/6 */
  p = fmaf(r, p, 0.5f);
  p = fmaf(r * r, p, r);
  int k = (int)kf;
  if (k == 0) return p;
  uint32_t sb = (uint32_t)(k + 127) << 23;
  float s;
  memcpy(&s, &sb, 4);
  return fmaf(s, p, s - 1.0f);
}

float orc_tanhf(float x) {
  float ax = fabsf(x);
  if (x != x) return x;
  if (ax >= 10.0f) return copysignf(1.0f, x);
  if (ax < 2.44140625e-04f) return x;  /* |x| < 2^-12: tanh(x) rounds to x */
  float t = orc_expm1_nonpos(-2.0f * ax);
  float r = -t / (t + 2.0f);
  return copysignf(r, x);
}

/* geglu_scalar_f32 (cpu_simd/geglu.rs:6-18), tanh as above. */
float orc_geglu_scalar(float g, float u) {
  if (g <= -10.0f) return 0.0f;
  if (g >= 10.0f) return g * u;
  float g3 = g * g * g;
  float inner = 0.7978846f * (g + 0.044715f * g3);
  float th = orc_tanhf(inner);
  float act = 0.5f * g * (1.0f + th);
  return act * u;
}

float orc_geglu_scalar_libm(float g, float u) {
  if (g <= -10.0f) return 0.0f;
  if (g >= 10.0f) return g * u;
  float g3 = g * g * g;
  float inner = 0.7978846f * (g + 0.044715f * g3);
  float th = tanhf(inner);
  float act = 0.5f * g * (1.0f + th);
  return act * u;
}

/* orc_geglu with the platform tanhf: glypr's CPU numerics where libm's tanhf
 * is glibc's (the reference's Rust f32::tanh). */
void orc_geglu_libm(const float* gate, const float* up, float* out, int64_t n, int threads) {
  int nt = orc_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static, 1024)
  for (int64_t i = 0; i < n; i++) out[i] = orc_geglu_scalar_libm(gate[i], up[i]);
}

/* CpuGeGLUOp::cpu_fwd (cpu_simd/geglu.rs:27-113): chunks of 1024 in parallel. */
void orc_geglu(const float* gate, const float* up, float* out, int64_t n, int threads) {
  int nt = orc_threads(threads);
#pragma omp parallel for num_threads(nt) schedule(static, 1024)
  for (int64_t i = 0; i < n; i++) out[i] = orc_geglu_scalar(gate[i], up[i]);
}

/* ======================================================================== */
/* Token embedding: table dequantized at load (model.rs:252-254), gathered by */
/* candle_nn::Embedding (model.rs:507), times embed_scale = sqrt(hidden) as a */
/* candle affine (v * mul + add, add = 0) in f32 (model.rs:255, 508).         */
/* ======================================================================== */

int orc_embed_gather(const uint8_t* table, int64_t vocab, int64_t d, const uint32_t* ids,
                     int64_t n_ids, float scale, float* out) {
  int64_t rb = (d / ORC_QK8_0) * ORC_BLOCK_BYTES;
  for (int64_t t = 0; t < n_ids; t++)
    if ((int64_t)ids[t] >= vocab) return -1;
  for (int64_t t = 0; t < n_ids; t++) {
    float* o = out + t * d;
    orc_q8_0_dequantize_row(table + (int64_t)ids[t] * rb, d, o);
    for (int64_t i = 0; i < d; i++) o[i] = o[i] * scale + 0.0f;
  }
  return 0;
}

/* ======================================================================== */
/* pool_and_normalize (model.rs:654-705): f32 mean over tokens (candle sum   */
/* over dim 1 then affine * f32(1/t)), or masked sum / clamp(count, 1e-9),   */
/* L2 with clamp(norm, 1e-12), MRL narrow + renormalise.                      */
/* ======================================================================== */

void orc_pool_normalize(const float* tokens, const uint8_t* mask, int64_t t, int64_t d,
                        int64_t trunc, float* out) {
  float* pooled = (float*)malloc((size_t)d * sizeof(float));
  if (mask) {
    float cnt = 0.0f;
    for (int64_t j = 0; j < t; j++) cnt += mask[j] ? 1.0f : 0.0f;
    if (cnt < 1e-9f) cnt = 1e-9f;
    for (int64_t i = 0; i < d; i++) {
      float s = 0.0f;
      for (int64_t j = 0; j < t; j++) s += tokens[j * d + i] * (mask[j] ? 1.0f : 0.0f);
      pooled[i] = s / cnt;
    }
  } else {
    float inv_t = (float)(1.0 / (double)t);
    for (int64_t i = 0; i < d; i++) {
      float s = 0.0f;
      for (int64_t j = 0; j < t; j++) s += tokens[j * d + i];
      pooled[i] = s * inv_t + 0.0f;
    }
  }
  float ss = 0.0f;
  for (int64_t i = 0; i < d; i++) ss += pooled[i] * pooled[i];
  float nrm = sqrtf(ss);
  if (nrm < 1e-12f) nrm = 1e-12f;
  for (int64_t i = 0; i < d; i++) pooled[i] = pooled[i] / nrm;
  int64_t td = (trunc > 0 && trunc < d) ? trunc : d;
  if (td < d) {
    float s2 = 0.0f;
    for (int64_t i = 0; i < td; i++) s2 += pooled[i] * pooled[i];
    float n2 = sqrtf(s2);
    if (n2 < 1e-12f) n2 = 1e-12f;
    for (int64_t i = 0; i < td; i++) out[i] = pooled[i] / n2;
  } else {
    for (int64_t i = 0; i < d; i++) out[i] = pooled[i];
  }
  free(pooled);
}

/* Rust's `Sum for f32` (core::iter, Rust >= 1.83; the reference is edition
 * 2024, so Rust >= 1.85) is a sequential fold that starts from -0.0: the sum
 * of no terms, or of -0.0 terms only, is -0.0. */
static float rust_sum_start(void) { return -0.0f; }

/* l2_normalize (util.rs:22-29): norm = sqrt(sequential f32 sum of x*x); a
 * zero norm returns the input unchanged (no clamp); else x / norm. */
void orc_l2_normalize(const float* x, int64_t n, float* y) {
  float s = rust_sum_start();
  for (int64_t i = 0; i < n; i++) s = s + x[i] * x[i];
  float nrm = sqrtf(s);
  for (int64_t i = 0; i < n; i++) y[i] = nrm == 0.0f ? x[i] : x[i] / nrm;
}

/* cosine_similarity (util.rs:32-41): three sequential f32 sums (dot, |a|^2,
 * |b|^2), sqrt of each norm, 0.0 when either norm is 0, else
 * (dot / (norm_a * norm_b)) clamped to [-1, 1]. */
float orc_cosine(const float* a, const float* b, int64_t n) {
  float dot = rust_sum_start(), sa = rust_sum_start(), sb = rust_sum_start();
  for (int64_t i = 0; i < n; i++) dot = dot + a[i] * b[i];
  for (int64_t i = 0; i < n; i++) sa = sa + a[i] * a[i];
  for (int64_t i = 0; i < n; i++) sb = sb + b[i] * b[i];
  float na = sqrtf(sa), nb = sqrtf(sb);
  if (na == 0.0f || nb == 0.0f) return 0.0f;
  float c = dot / (na * nb);
  /* f32::clamp(-1, 1): NaN stays NaN */
  if (c < -1.0f) c = -1.0f;
  if (c > 1.0f) c = 1.0f;
  return c;
}

/* ======================================================================== */
/* Output-vector codecs (glypr-core util.rs:52-197).                         */
/* ======================================================================== */

/* quantize_binary (util.rs:52-71): dim % 64 != 0 is an error (-1); bit i of
 * word i / 64 is set when x[i] > 0.0 (false for NaN and -0.0). */
int orc_quantize_binary(const float* x, int64_t dim, uint64_t* words) {
  if (dim % 64 != 0) return -1;
  for (int64_t w = 0; w < dim / 64; w++) words[w] = 0;
  for (int64_t i = 0; i < dim; i++)
    if (x[i] > 0.0f) words[i / 64] |= (uint64_t)1 << (i % 64);
  return 0;
}

/* hamming_distance (util.rs:75-109): total popcount of a XOR b.  The
 * reference's four-lane partial sums are integers, so the order is free. */
uint32_t orc_hamming(const uint64_t* a, const uint64_t* b, int64_t words) {
  uint32_t s = 0;
  for (int64_t w = 0; w < words; w++) s += (uint32_t)__builtin_popcountll(a[w] ^ b[w]);
  return s;
}

/* binary_cosine_similarity (util.rs:112-119): dim = 64 words; dim 0 -> 1.0;
 * (PI * (h as f32 / dim as f32)).cos() in f32 with the platform cosf, as
 * Rust's f32::cos calls it. */
float orc_binary_cosine(const uint64_t* a, const uint64_t* b, int64_t words) {
  const int64_t dim = words * 64;
  if (dim == 0) return 1.0f;
  const float h = (float)orc_hamming(a, b, words);
  return cosf(3.14159265358979323846f * (h / (float)dim));
}

/* quantize_int8 (util.rs:128-133): (v * 127.0).round().clamp(-127.0, 127.0)
 * as i8.  f32 round is half away from zero (roundf); the saturating `as i8`
 * cast maps NaN to 0. */
void orc_quantize_int8(const float* x, int64_t n, int8_t* q) {
  for (int64_t i = 0; i < n; i++) {
    float r = roundf(x[i] * 127.0f);
    if (r != r) {
      q[i] = 0;
      continue;
    }
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    q[i] = (int8_t)r;
  }
}

/* int8_dot_product (util.rs:137-176): i32 sum of products.  Rust release
 * arithmetic wraps, so the sum is taken mod 2^32 (order-free). */
int32_t orc_int8_dot(const int8_t* a, const int8_t* b, int64_t n) {
  uint32_t s = 0;
  for (int64_t i = 0; i < n; i++) s += (uint32_t)((int32_t)a[i] * (int32_t)b[i]);
  return (int32_t)s;
}

/* int8_cosine_similarity (util.rs:181-197): 0 when either squared norm is 0,
 * else (dot as f32 / (sqrt(na as f32) * sqrt(nb as f32))).clamp(-1, 1). */
float orc_int8_cosine(const int8_t* a, const int8_t* b, int64_t n) {
  const int32_t na = orc_int8_dot(a, a, n), nb = orc_int8_dot(b, b, n);
  if (na == 0 || nb == 0) return 0.0f;
  const int32_t dot = orc_int8_dot(a, b, n);
  const float denom = sqrtf((float)na) * sqrtf((float)nb);
  float c = (float)dot / denom;
  if (c < -1.0f) c = -1.0f;
  if (c > 1.0f) c = 1.0f;
  return c;
}

/* ======================================================================== */
/* Seeded synthetic inputs: SplitMix64, Box-Muller in double.                */
/* ======================================================================== */

uint64_t orc_splitmix64(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static double orc_unit(uint64_t* s) { /* (0, 1] */
  return ((double)(orc_splitmix64(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void orc_fill_normal(float* out, int64_t n, uint64_t seed, float mean, float stddev) {
  uint64_t s = seed;
  const double two_pi = 6.283185307179586476925;
  int64_t i = 0;
  while (i < n) {
    double u1 = orc_unit(&s), u2 = orc_unit(&s);
    double r = sqrt(-2.0 * log(u1));
    out[i++] = (float)(mean + stddev * r * cos(two_pi * u2));
    if (i < n) out[i++] = (float)(mean + stddev * r * sin(two_pi * u2));
  }
}

void orc_fill_uniform_ids(uint32_t* ids, int64_t n, uint64_t seed, uint32_t vocab) {
  uint64_t s = seed;
  for (int64_t i = 0; i < n; i++) ids[i] = (uint32_t)(orc_splitmix64(&s) % vocab);
}

void orc_make_q8_0_weight(uint8_t* blocks, int64_t n, int64_t k, uint64_t seed, float sigma) {
  int64_t nb = k / ORC_QK8_0;
  uint64_t s = seed;
  const double two_pi = 6.283185307179586476925;
  for (int64_t i = 0; i < n * nb; i++) {
    uint8_t* b = blocks + i * ORC_BLOCK_BYTES;
    double u1 = orc_unit(&s), u2 = orc_unit(&s);
    double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    float d = (float)(fabs(z) * sigma / 127.0);
    uint16_t dh = orc_f32_to_f16(d);
    b[0] = (uint8_t)(dh & 0xFF);
    b[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < ORC_QK8_0; j++) {
      int v = (int)(orc_splitmix64(&s) % 255u) - 127;
      b[2 + j] = (uint8_t)(int8_t)v;
    }
  }
}

/* ======================================================================== */
/* Backbone (configs 4-5).  EncoderLayer::forward (layer.rs:20-50) without    */
/* the PLE block and layer scalar, SelfAttention::forward (attention/mod.rs:  */
/* 166-277), RoPE (rope.rs:14-106), attention (attention/standard.rs:10-83;  */
/* chunked.rs:64-172 == band |i-j| <= W), scale 1.0, f32 softmax.            */
/* ======================================================================== */

int orc_layer_is_full(int64_t layer_idx) { return ((layer_idx + 1) % 6) == 0; }

/* RotaryEmbedding::new + get_cos_sin: inv_freq in f64 cast to f32, positions
 * as f32, freqs = pos * inv_freq in f32, emb = cat(freqs, freqs), cos/sin f32. */
void orc_rope_tables(int64_t head_dim, double theta, int64_t t, float* cos_t, float* sin_t) {
  int64_t half = head_dim / 2;
  float* inv = (float*)malloc((size_t)half * sizeof(float));
  for (int64_t i = 0; i < half; i++) {
    double e = (double)(2 * i) / (double)head_dim;
    inv[i] = (float)(1.0 / pow(theta, e));
  }
  for (int64_t p = 0; p < t; p++)
    for (int64_t i = 0; i < head_dim; i++) {
      float f = (float)p * inv[i % half];
      cos_t[p * head_dim + i] = cosf(f);
      sin_t[p * head_dim + i] = sinf(f);
    }
  free(inv);
}

/* apply_rotary_pos_emb (rope.rs:99-106): x*cos + rotate_half(x)*sin. */
static void orc_rope_apply(float* x, const float* c, const float* s, int64_t hd) {
  int64_t half = hd / 2;
  float tmp[1024];
  for (int64_t i = 0; i < hd; i++) {
    float rot = i < half ? -x[i + half] : x[i - half];
    tmp[i] = x[i] * c[i] + rot * s[i];
  }
  memcpy(x, tmp, (size_t)hd * sizeof(float));
}

void orc_attention(const float* q, const float* k, const float* v, int64_t n_heads,
                   int64_t n_kv, int64_t t, int64_t hd, int64_t window, float* ctx, int threads) {
  int nt = orc_threads(threads);
  int64_t rep = n_heads / n_kv;
#pragma omp parallel num_threads(nt)
  {
    float* sc = (float*)malloc((size_t)t * sizeof(float));
    double* acc = (double*)malloc((size_t)hd * sizeof(double));
#pragma omp for schedule(dynamic, 8)
    for (int64_t hi = 0; hi < n_heads * t; hi++) {
      int64_t h = hi / t, i = hi % t;
      int64_t kvh = h / rep;   /* repeat_kv (attention/mod.rs:22-31) */
      const float* qi = q + (h * t + i) * hd;
      int64_t j0 = 0, j1 = t;
      if (window > 0 && t > window) {
        j0 = i - window > 0 ? i - window : 0;
        j1 = i + window + 1 < t ? i + window + 1 : t;
      }
      float mx = -FLT_MAX;
      for (int64_t j = j0; j < j1; j++) {
        const float* kj = k + (kvh * t + j) * hd;
        double s = 0.0;
        for (int64_t e = 0; e < hd; e++) s += (double)qi[e] * (double)kj[e];
        sc[j] = (float)s;
        if (sc[j] > mx) mx = sc[j];
      }
      float den = 0.0f;
      for (int64_t j = j0; j < j1; j++) {
        sc[j] = expf(sc[j] - mx);
        den += sc[j];
      }
      for (int64_t e = 0; e < hd; e++) acc[e] = 0.0;
      for (int64_t j = j0; j < j1; j++) {
        float p = sc[j] / den;
        const float* vj = v + (kvh * t + j) * hd;
        for (int64_t e = 0; e < hd; e++) acc[e] += (double)p * (double)vj[e];
      }
      float* o = ctx + i * (n_heads * hd) + h * hd;
      for (int64_t e = 0; e < hd; e++) o[e] = (float)acc[e];
    }
    free(sc);
    free(acc);
  }
}

static void orc_linear(const uint8_t* w, int64_t n, int64_t k, const float* x, int64_t m, float* y,
                       int threads) {
  orc_q8_0_matmul(x, m, k, w, n, y, threads);
}

void orc_encoder_layer(const orc_model_config* cfg, const orc_layer_weights* w, int64_t layer_idx,
                       float* hidden, const float* per_layer_input, int64_t t, int threads) {
  int full = cfg->layer_types ? cfg->layer_types[layer_idx] != 0 : orc_layer_is_full(layer_idx);
  /* per-layer geometry: full-attention layers take their own head_dim and kv
   * head count (TextConfig::get_head_dim / get_num_kv_heads, config.rs:142-169,
   * 208-230; model.rs:286-287), the RoPE table of their head_dim */
  int64_t H = cfg->hidden, F = cfg->ffn, nh = cfg->n_heads,
          nkv = full && cfg->full_n_kv_heads ? cfg->full_n_kv_heads : cfg->n_kv_heads,
          hd = full && cfg->full_head_dim ? cfg->full_head_dim : cfg->head_dim;
  float* normed = (float*)malloc((size_t)(t * H) * sizeof(float));
  float* qb = (float*)malloc((size_t)(t * nh * hd) * sizeof(float));
  float* kb = (float*)malloc((size_t)(t * nkv * hd) * sizeof(float));
  float* vb = (float*)malloc((size_t)(t * nkv * hd) * sizeof(float));
  float* qh = (float*)malloc((size_t)(t * nh * hd) * sizeof(float));
  float* kh = (float*)malloc((size_t)(t * nkv * hd) * sizeof(float));
  float* vh = (float*)malloc((size_t)(t * nkv * hd) * sizeof(float));
  float* ctxb = (float*)malloc((size_t)(t * nh * hd) * sizeof(float));
  float* attn = (float*)malloc((size_t)(t * H) * sizeof(float));
  float* gate = (float*)malloc((size_t)(t * F) * sizeof(float));
  float* up = (float*)malloc((size_t)(t * F) * sizeof(float));
  float* cos_t = (float*)malloc((size_t)(t * hd) * sizeof(float));
  float* sin_t = (float*)malloc((size_t)(t * hd) * sizeof(float));
  orc_rope_tables(hd, full ? cfg->rope_theta_full : cfg->rope_theta_sliding, t, cos_t, sin_t);

  /* 1. attention block */
  orc_rmsnorm(hidden, w->input_norm, cfg->eps, normed, t, H, threads);
  orc_linear(w->q, nh * hd, H, normed, t, qb, threads);
  orc_linear(w->k, nkv * hd, H, normed, t, kb, threads);
  orc_linear(w->v, nkv * hd, H, normed, t, vb, threads);
  /* q/k/v norms on [t, heads, hd], then transpose to [heads, t, hd], RoPE on q, k */
  for (int64_t i = 0; i < t; i++) {
    for (int64_t h = 0; h < nh; h++) {
      float* dst = qh + (h * t + i) * hd;
      orc_rmsnorm_row(qb + (i * nh + h) * hd, w->q_norm, cfg->eps, dst, hd);
      orc_rope_apply(dst, cos_t + i * hd, sin_t + i * hd, hd);
    }
    for (int64_t h = 0; h < nkv; h++) {
      float* dk = kh + (h * t + i) * hd;
      orc_rmsnorm_row(kb + (i * nkv + h) * hd, w->k_norm, cfg->eps, dk, hd);
      orc_rope_apply(dk, cos_t + i * hd, sin_t + i * hd, hd);
      orc_rmsnorm_row(vb + (i * nkv + h) * hd, NULL, cfg->eps, vh + (h * t + i) * hd, hd);
    }
  }
  orc_attention(qh, kh, vh, nh, nkv, t, hd, full ? 0 : cfg->sliding_window, ctxb, threads);
  orc_linear(w->o, H, nh * hd, ctxb, t, attn, threads);
  /* forward_residual_add (norm.rs:65-95): residual + RMSNorm(x) */
  orc_rmsnorm(attn, w->post_attn_norm, cfg->eps, normed, t, H, threads);
  for (int64_t i = 0; i < t * H; i++) hidden[i] = hidden[i] + normed[i];

  /* 2. feed-forward block: MLP::forward CPU arm (mlp.rs:53-65) */
  orc_rmsnorm(hidden, w->pre_ffn_norm, cfg->eps, normed, t, H, threads);
  orc_linear(w->gate, F, H, normed, t, gate, threads);
  orc_linear(w->up, F, H, normed, t, up, threads);
  orc_geglu(gate, up, gate, t * F, threads);
  orc_linear(w->down, H, F, gate, t, attn, threads);
  orc_rmsnorm(attn, w->post_ffn_norm, cfg->eps, normed, t, H, threads);
  for (int64_t i = 0; i < t * H; i++) hidden[i] = hidden[i] + normed[i];

  /* 3. TextPLEBlock::forward_with_scalar (ple.rs:118-145): gate = inp_gate(h),
   * cpu_geglu(gate, per_layer_input), proj, then post_norm.forward_residual_add
   * with the layer scalar (norm.rs:65-95): (h + RMSNorm(p)) * scalar. */
  if (cfg->ple_dim > 0) {
    const int64_t P = cfg->ple_dim;
    float* pg = (float*)malloc((size_t)(t * P) * sizeof(float));
    orc_linear(w->ple_gate, P, H, hidden, t, pg, threads);
    orc_geglu(pg, per_layer_input, pg, t * P, threads);
    orc_linear(w->ple_proj, H, P, pg, t, attn, threads);
    orc_rmsnorm(attn, w->ple_post_norm, cfg->eps, normed, t, H, threads);
    const float sc = w->layer_scalar ? w->layer_scalar[0] : 1.0f;
    for (int64_t i = 0; i < t * H; i++) {
      const float sum = hidden[i] + normed[i];
      hidden[i] = w->layer_scalar ? sum * sc : sum;
    }
    free(pg);
  }

  free(normed); free(qb); free(kb); free(vb); free(qh); free(kh); free(vh);
  free(ctxb); free(attn); free(gate); free(up); free(cos_t); free(sin_t);
}

int orc_model_forward(const orc_model_config* cfg, const uint8_t* embed_table,
                      const orc_layer_weights* layers, const float* final_norm,
                      const uint8_t* ple_model_proj, const float* ple_proj_norm,
                      const uint8_t* out_proj, const uint32_t* ids, int64_t t, int64_t trunc,
                      float* out, float* hidden_out, int threads) {
  int64_t H = cfg->hidden, L = cfg->n_layers, P = cfg->ple_dim;
  float* hidden = (float*)malloc((size_t)(t * H) * sizeof(float));
  float scale = (float)sqrt((double)H);   /* embed_scale f64 -> affine mul as f32 */
  if (orc_embed_gather(embed_table, cfg->vocab, H, ids, t, scale, hidden) != 0) {
    free(hidden);
    return -1;
  }
  /* TextPLE::project_and_norm_per_layer (ple.rs:48-85): projection of the
   * scaled embeddings, * hidden^-0.5 (f64 powf, applied as an f32 affine mul),
   * RMSNorm over ple_dim, then each layer's [t][ple_dim] slice. */
  float* ple = NULL;
  float* slice = NULL;
  if (P > 0) {
    float* raw = (float*)malloc((size_t)(t * L * P) * sizeof(float));
    ple = (float*)malloc((size_t)(t * L * P) * sizeof(float));
    slice = (float*)malloc((size_t)(t * P) * sizeof(float));
    orc_linear(ple_model_proj, L * P, H, hidden, t, raw, threads);
    const float ps = (float)pow((double)H, -0.5);
    for (int64_t i = 0; i < t * L * P; i++) raw[i] = raw[i] * ps + 0.0f;
    orc_rmsnorm(raw, ple_proj_norm, cfg->eps, ple, t * L, P, threads);
    free(raw);
  }
  for (int64_t l = 0; l < L; l++) {
    if (P > 0)
      for (int64_t i = 0; i < t; i++)
        memcpy(slice + i * P, ple + (i * L + l) * P, (size_t)P * sizeof(float));
    orc_encoder_layer(cfg, &layers[l], l, hidden, P > 0 ? slice : NULL, t, threads);
  }
  float* normed = (float*)malloc((size_t)(t * H) * sizeof(float));
  orc_rmsnorm(hidden, final_norm, cfg->eps, normed, t, H, threads);  /* model.rs:576 */
  /* embedding_projection.forward (model.rs:577) */
  int64_t D = H;
  float* tokens = normed;
  float* projected = NULL;
  if (cfg->out_dim > 0) {
    D = cfg->out_dim;
    projected = (float*)malloc((size_t)(t * D) * sizeof(float));
    orc_linear(out_proj, D, H, normed, t, projected, threads);
    tokens = projected;
  }
  if (hidden_out) memcpy(hidden_out, tokens, (size_t)(t * D) * sizeof(float));
  orc_pool_normalize(tokens, NULL, t, D, trunc, out);
  free(hidden);
  free(normed);
  free(projected);
  free(ple);
  free(slice);
  return 0;
}
