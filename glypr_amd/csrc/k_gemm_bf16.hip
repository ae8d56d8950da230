// k_gemm_bf16.hip — Q8_0 GEMM with in-register dequantization to bf16 and
// CDNA4 bf16 MFMA (v_mfma_f32_32x32x16_bf16), f32 accumulation.
//
// The semantics of glypr's Metal Q8_0 kernels (dequantize the weight, multiply
// unquantized activations, f32 accumulate; fused_ops.metal:574-581, 649-758)
// and of candle's CANDLE_DEQUANTIZE_ALL path, at bf16 operand precision.
// Weights stay Q8_0 in HBM (1.125 B/value); each 16-byte int8 chunk is turned
// into 16 bf16 values on the way into LDS: q ^ 0x80 as an unsigned byte
// (v_cvt_f32_ubyteN) then fma(q+128, d, -128 d) = q*d exactly, then
// v_cvt_pk_bf16_f32 (round to nearest even).  Activations arrive as bf16 from
// the RMSNorm prologue (or a conversion pass).
#include "device_common.hpp"
#include "internal.hpp"

namespace glypr {

namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

constexpr int BKE = 64;  // K elements per LDS stage (2 Q8_0 blocks); 128-byte bf16 rows

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  v2bf r;
  r[0] = (__bf16)a;
  r[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, r);
}

// 16 int8 -> 16 bf16 (32 bytes) scaled by d.
__device__ __forceinline__ void dequant16(v4i q, float d, v4i& lo, v4i& hi) {
  const float c = -128.0f * d;
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    uint32_t u = (uint32_t)q[i] ^ 0x80808080u;
    float f0 = fmaf((float)(u & 0xFFu), d, c);
    float f1 = fmaf((float)((u >> 8) & 0xFFu), d, c);
    float f2 = fmaf((float)((u >> 16) & 0xFFu), d, c);
    float f3 = fmaf((float)(u >> 24), d, c);
    w[2 * i] = pack_bf16x2(f0, f1);
    w[2 * i + 1] = pack_bf16x2(f2, f3);
  }
  lo = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  hi = v4i{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
}

template <int BM, int BN, int WM, int WN, bool GEGLU>
__global__ void __launch_bounds__(WM * WN * 64)
gemm_bf16_kernel(const uint16_t* __restrict__ A, const int8_t* __restrict__ B,
                 const float* __restrict__ dB, float* __restrict__ C, uint16_t* __restrict__ Hb,
                 int M, int N, int K, int ldc, int F) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int ROWB = BKE * 2;  // bytes per LDS row (bf16)
  constexpr int A_LD = BM * 8 / NT;  // 16-byte bf16 chunks
  constexpr int B_LD = BN * 4 / NT;  // 16-byte int8 chunks
  static_assert(BM * 8 % NT == 0 && BN * 4 % NT == 0, "tile/thread mismatch");
  static_assert(!GEGLU || WTN % 64 == 0, "GeGLU needs gate/up tile pairs per wave");

  __shared__ __attribute__((aligned(16))) uint8_t As[2][BM * ROWB];
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][BN * ROWB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int nb = K / QK;
  const int nstage = (K + BKE - 1) / BKE;

  auto b_src = [&](int nl, bool& ok) -> int {
    if (!GEGLU) {
      ok = n0 + nl < N;
      return n0 + nl;
    }
    int c = (n0 >> 1) + (nl >> 6) * 32 + (nl & 31);
    ok = c < F;
    return ((nl >> 5) & 1) ? F + c : c;
  };

  v4i ra[A_LD], rb[B_LD];
  float rd[B_LD];

  auto load_stage = [&](int s) {
#pragma unroll
    for (int i = 0; i < A_LD; i++) {
      int idx = tid + i * NT;
      int row = idx >> 3, ch = idx & 7;
      int gk = s * BKE + ch * 8;
      int gm = m0 + row;
      ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const v4i*>(A + (int64_t)gm * K + gk)
                                 : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < B_LD; i++) {
      int idx = tid + i * NT;
      int row = idx >> 2, ch = idx & 3;
      int gk = s * BKE + ch * 16;
      bool ok;
      int gn = b_src(row, ok);
      ok = ok && gk < K;
      rb[i] = ok ? *reinterpret_cast<const v4i*>(B + (int64_t)gn * K + gk) : v4i{0, 0, 0, 0};
      rd[i] = ok ? dB[(int64_t)gn * nb + (gk >> 5)] : 0.0f;
    }
  };

  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LD; i++) {
      int idx = tid + i * NT;
      int row = idx >> 3, ch = idx & 7;
      *reinterpret_cast<v4i*>(&As[buf][row * ROWB + ((ch ^ (row & 7)) * 16)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LD; i++) {
      int idx = tid + i * NT;
      int row = idx >> 2, ch = idx & 3;
      v4i lo, hi;
      dequant16(rb[i], rd[i], lo, hi);
      *reinterpret_cast<v4i*>(&Bs[buf][row * ROWB + (((2 * ch) ^ (row & 7)) * 16)]) = lo;
      *reinterpret_cast<v4i*>(&Bs[buf][row * ROWB + (((2 * ch + 1) ^ (row & 7)) * 16)]) = hi;
    }
  };

  v16f acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int tn = 0; tn < TN; tn++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[tm][tn][r] = 0.0f;

  const int lrow = lane & 31;
  const int lhalf = lane >> 5;

  load_stage(0);
  store_stage(0);
  __syncthreads();

  for (int s = 0; s < nstage; s++) {
    const int buf = s & 1;
    if (s + 1 < nstage) load_stage(s + 1);
#pragma unroll
    for (int ks = 0; ks < BKE / 16; ks++) {
      const int ch = ks * 2 + lhalf;
      v8bf af[TM], bfr[TN];
#pragma unroll
      for (int tm = 0; tm < TM; tm++) {
        int row = wm * WTM + tm * 32 + lrow;
        af[tm] = *reinterpret_cast<const v8bf*>(&As[buf][row * ROWB + ((ch ^ (row & 7)) * 16)]);
      }
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        int row = wn * WTN + tn * 32 + lrow;
        bfr[tn] = *reinterpret_cast<const v8bf*>(&Bs[buf][row * ROWB + ((ch ^ (row & 7)) * 16)]);
      }
#pragma unroll
      for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int tn = 0; tn < TN; tn++)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[tm], bfr[tn], acc[tm][tn], 0, 0, 0);
    }
    if (s + 1 < nstage) store_stage(buf ^ 1);
    __syncthreads();
  }

  if constexpr (!GEGLU) {
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        const int gn = n0 + wn * WTN + tn * 32 + lrow;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int gm = m0 + wm * WTM + tm * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
          if (gm < M && gn < N) C[(int64_t)gm * ldc + gn] = acc[tm][tn][r];
        }
      }
  } else {
#pragma unroll
    for (int p = 0; p < TN / 2; p++) {
      const int hc = (n0 >> 1) + ((wn * WTN) >> 6) * 32 + p * 32 + lrow;
#pragma unroll
      for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int gm = m0 + wm * WTM + tm * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
          float h = geglu_scalar(acc[tm][2 * p][r], acc[tm][2 * p + 1][r]);
          if (gm < M && hc < F) Hb[(int64_t)gm * F + hc] = __builtin_bit_cast(uint16_t, (__bf16)h);
        }
    }
  }
}

template <int BM, int BN, int WM, int WN, bool GEGLU>
hipError_t run(const uint16_t* xb, const int8_t* wq, const float* dw, float* y, uint16_t* hb,
               int64_t M, int64_t Nrows, int64_t K, int64_t ldc, int64_t F, hipStream_t s) {
  dim3 grid((unsigned)((Nrows + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  gemm_bf16_kernel<BM, BN, WM, WN, GEGLU><<<grid, WM * WN * 64, 0, s>>>(
      xb, wq, dw, y, hb, (int)M, (int)Nrows, (int)K, (int)ldc, (int)F);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_bf16(const uint16_t* xb, const int8_t* wq, const float* dw, float* y,
                            int64_t M, int64_t N, int64_t K, int64_t ldc, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  int64_t big_tiles = ((M + 255) / 256) * ((N + 127) / 128);
  if (big_tiles >= 256)
    return run<256, 128, 4, 2, false>(xb, wq, dw, y, nullptr, M, N, K, ldc, 0, s);
  return run<64, 64, 2, 2, false>(xb, wq, dw, y, nullptr, M, N, K, ldc, 0, s);
}

hipError_t launch_gemm_bf16_geglu(const uint16_t* xb, const int8_t* wq, const float* dw,
                                  uint16_t* hb, int64_t M, int64_t F, int64_t K, hipStream_t s) {
  if (M == 0 || F == 0) return hipSuccess;
  int64_t big_tiles = ((M + 255) / 256) * ((2 * F + 127) / 128);
  if (big_tiles >= 256)
    return run<256, 128, 4, 2, true>(xb, wq, dw, nullptr, hb, M, 2 * F, K, 0, F, s);
  return run<64, 128, 2, 2, true>(xb, wq, dw, nullptr, hb, M, 2 * F, K, 0, F, s);
}

}  // namespace glypr
