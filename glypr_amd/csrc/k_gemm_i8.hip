// k_gemm_i8.hip — Q8_0 x Q8_0 GEMM on CDNA4 int8 MFMA, bit-exact with glypr's
// CPU path (candle k_quants::matmul + BlockQ8_0::vec_dot_unopt).
//
//   y[m,n] = sum_b ((float)S_b * d_w[n,b]) * d_x[m,b],   S_b = sum_{j<32} qw*qx
//
// summed in f32 in block order b = 0, 1, ... exactly like the scalar vec_dot.
// One v_mfma_i32_32x32x32_i8 covers one Q8_0 block (K = 32) of a 32x32 output
// tile, so every MFMA result is an exact block sum S_b.  The MFMA accumulates
// onto the constant 0x4B400000 (1.5 * 2^23 as f32): |S_b| <= 32*128*128 < 2^22,
// so the result's bit pattern IS the f32 1.5*2^23 + S_b, and
//   fma(f, d_w, -1.5*2^23*d_w) = round(S_b * d_w)
// exactly (-1.5*2^23*d_w is exact for an f16-derived d_w).  That leaves
// one mul (x d_x) and one add per output per block: three VALU ops, all
// rounding like the reference.  Operand tiles go HBM -> registers -> LDS
// (XOR-swizzled 16-byte chunks, conflict-free ds_read_b128) double-buffered,
// 128 bytes of K (4 blocks) per stage.  Per-block scales ride along in LDS.
//
// GEGLU epilogue (MLP::forward, mlp.rs:53-65): the B operand is the try_concat
// of [gate; up] (2F rows).  Each 64-row group of a tile holds 32 gate rows and
// the 32 matching up rows, so a lane holds gate and up for the same (m, j);
// h = geglu(gate, up) is quantized to Q8_0 in registers (block amax over the
// 32 lanes that hold one row's 32 consecutive j) and written as the down
// projection's int8 operand: the f32 h never reaches HBM.
#include "device_common.hpp"
#include "internal.hpp"

namespace glypr {

namespace {

constexpr int BK = 128;        // K bytes per LDS stage
constexpr int KB = BK / QK;    // Q8_0 blocks per stage
constexpr int MAGIC = 0x4B400000;
constexpr float NEG_MAGIC = -12582912.0f;  // -(1.5 * 2^23)

template <int BM, int BN, int WM, int WN, bool GEGLU>
__global__ void __launch_bounds__(WM * WN * 64)
gemm_i8_kernel(const int8_t* __restrict__ A, const float* __restrict__ dA,
               const int8_t* __restrict__ B, const float* __restrict__ dB,
               float* __restrict__ C, int8_t* __restrict__ Hq, float* __restrict__ dH, int M,
               int N, int K, int ldc, int F) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  constexpr int CPR = BK / 16;  // 16-byte chunks per tile row
  constexpr int A_LD = BM * CPR / NT, B_LD = BN * CPR / NT;
  constexpr int SA_LD = (BM * KB + NT - 1) / NT, SB_LD = (BN * KB + NT - 1) / NT;
  static_assert(BM * CPR % NT == 0 && BN * CPR % NT == 0, "tile/thread mismatch");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be 32-aligned");
  static_assert(!GEGLU || WTN % 64 == 0, "GeGLU needs gate/up tile pairs per wave");

  __shared__ __attribute__((aligned(16))) int8_t As[2][BM * BK];
  __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN * BK];
  __shared__ __attribute__((aligned(16))) float dAs[2][KB][BM];
  __shared__ __attribute__((aligned(16))) float dBs[2][KB][BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int nb = K / QK;
  const int nstage = (nb + KB - 1) / KB;

  // Global row of local B row nl, and whether it exists.
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
  float rsa[SA_LD], rsb[SB_LD];

  auto load_stage = [&](int s) {
#pragma unroll
    for (int i = 0; i < A_LD; i++) {
      int idx = tid + i * NT;
      int row = idx / CPR, ch = idx % CPR;
      int gk = s * BK + ch * 16;
      int gm = m0 + row;
      ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const v4i*>(A + (int64_t)gm * K + gk)
                                 : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < B_LD; i++) {
      int idx = tid + i * NT;
      int row = idx / CPR, ch = idx % CPR;
      int gk = s * BK + ch * 16;
      bool ok;
      int gn = b_src(row, ok);
      rb[i] = (ok && gk < K) ? *reinterpret_cast<const v4i*>(B + (int64_t)gn * K + gk)
                             : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < SA_LD; i++) {
      int idx = tid + i * NT;
      int row = idx / KB, kb = idx % KB;
      int gb = s * KB + kb, gm = m0 + row;
      rsa[i] = (idx < BM * KB && gm < M && gb < nb) ? dA[(int64_t)gm * nb + gb] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < SB_LD; i++) {
      int idx = tid + i * NT;
      int row = idx / KB, kb = idx % KB;
      int gb = s * KB + kb;
      bool ok = false;
      int gn = idx < BN * KB ? b_src(row, ok) : 0;
      rsb[i] = (idx < BN * KB && ok && gb < nb) ? dB[(int64_t)gn * nb + gb] : 0.0f;
    }
  };

  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LD; i++) {
      int idx = tid + i * NT;
      int row = idx / CPR, ch = idx % CPR;
      *reinterpret_cast<v4i*>(&As[buf][row * BK + ((ch ^ (row & 7)) * 16)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LD; i++) {
      int idx = tid + i * NT;
      int row = idx / CPR, ch = idx % CPR;
      *reinterpret_cast<v4i*>(&Bs[buf][row * BK + ((ch ^ (row & 7)) * 16)]) = rb[i];
    }
#pragma unroll
    for (int i = 0; i < SA_LD; i++) {
      int idx = tid + i * NT;
      if (idx < BM * KB) dAs[buf][idx % KB][idx / KB] = rsa[i];
    }
#pragma unroll
    for (int i = 0; i < SB_LD; i++) {
      int idx = tid + i * NT;
      if (idx < BN * KB) dBs[buf][idx % KB][idx / KB] = rsb[i];
    }
  };

  v16i magic;
#pragma unroll
  for (int i = 0; i < 16; i++) magic[i] = MAGIC;

  float acc[TM][TN][16];
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
    const int kbn = (nb - s * KB) < KB ? (nb - s * KB) : KB;
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      if (kb < kbn) {
        v4i af[TM], bfr[TN];
        const int ch = kb * 2 + lhalf;
#pragma unroll
        for (int tm = 0; tm < TM; tm++) {
          int row = wm * WTM + tm * 32 + lrow;
          af[tm] = *reinterpret_cast<const v4i*>(&As[buf][row * BK + ((ch ^ (row & 7)) * 16)]);
        }
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
          int row = wn * WTN + tn * 32 + lrow;
          bfr[tn] = *reinterpret_cast<const v4i*>(&Bs[buf][row * BK + ((ch ^ (row & 7)) * 16)]);
        }
        float wd[TN], wc[TN];
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
          wd[tn] = dBs[buf][kb][wn * WTN + tn * 32 + lrow];
          wc[tn] = wd[tn] * NEG_MAGIC;
        }
#pragma unroll
        for (int tm = 0; tm < TM; tm++) {
          v4f xd[4];
#pragma unroll
          for (int g = 0; g < 4; g++)
            xd[g] = *reinterpret_cast<const v4f*>(
                &dAs[buf][kb][wm * WTM + tm * 32 + 8 * g + 4 * lhalf]);
#pragma unroll
          for (int tn = 0; tn < TN; tn++) {
            v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[tm], bfr[tn], magic, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) {
              float t = fmaf(__int_as_float(d[r]), wd[tn], wc[tn]);  // round(S * d_w)
              float u = t * xd[r >> 2][r & 3];                        // round(. * d_x)
              acc[tm][tn][r] = acc[tm][tn][r] + u;                    // round(acc + .)
            }
          }
        }
      }
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
    const int nbh = F / QK;
#pragma unroll
    for (int p = 0; p < TN / 2; p++) {
      const int hc = (n0 >> 1) + ((wn * WTN) >> 6) * 32 + p * 32 + lrow;
#pragma unroll
      for (int tm = 0; tm < TM; tm++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int gm = m0 + wm * WTM + tm * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
          float h = geglu_scalar(acc[tm][2 * p][r], acc[tm][2 * p + 1][r]);
          float a = fmaxf(0.0f, fabsf(h));
          a = fmaxf(a, __shfl_xor(a, 1));
          a = fmaxf(a, __shfl_xor(a, 2));
          a = fmaxf(a, __shfl_xor(a, 4));
          a = fmaxf(a, __shfl_xor(a, 8));
          a = fmaxf(a, __shfl_xor(a, 16));
          QScale sc = q8_scale(a);
          int q = quant_round(h * sc.id);
          if (gm < M && hc < F) {
            Hq[(int64_t)gm * F + hc] = (int8_t)q;
            if (lrow == 0) dH[(int64_t)gm * nbh + (hc >> 5)] = sc.dq;
          }
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, bool GEGLU>
hipError_t run(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw, float* y,
               int8_t* hq, float* dh, int64_t M, int64_t Nrows, int64_t K, int64_t ldc,
               int64_t F, hipStream_t s) {
  dim3 grid((unsigned)((Nrows + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  gemm_i8_kernel<BM, BN, WM, WN, GEGLU><<<grid, WM * WN * 64, 0, s>>>(
      xq, dx, wq, dw, y, hq, dh, (int)M, (int)Nrows, (int)K, (int)ldc, (int)F);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_i8(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                          float* y, int64_t M, int64_t N, int64_t K, int64_t ldc,
                          hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  int64_t big_tiles = ((M + 127) / 128) * ((N + 127) / 128);
  if (big_tiles >= 512)
    return run<128, 128, 2, 2, false>(xq, dx, wq, dw, y, nullptr, nullptr, M, N, K, ldc, 0, s);
  return run<64, 64, 2, 2, false>(xq, dx, wq, dw, y, nullptr, nullptr, M, N, K, ldc, 0, s);
}

hipError_t launch_gemm_i8_geglu(const int8_t* xq, const float* dx, const int8_t* wq,
                                const float* dw, int8_t* hq, float* dh, int64_t M, int64_t F,
                                int64_t K, hipStream_t s) {
  if (M == 0 || F == 0) return hipSuccess;
  int64_t big_tiles = ((M + 127) / 128) * ((2 * F + 127) / 128);
  if (big_tiles >= 512)
    return run<128, 128, 2, 2, true>(xq, dx, wq, dw, nullptr, hq, dh, M, 2 * F, K, 0, F, s);
  return run<64, 128, 2, 2, true>(xq, dx, wq, dw, nullptr, hq, dh, M, 2 * F, K, 0, F, s);
}

}  // namespace glypr
