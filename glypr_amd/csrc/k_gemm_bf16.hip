// k_gemm_bf16.hip — Q8_0 GEMM with in-register dequantization to bf16 and
// CDNA4 bf16 MFMA (v_mfma_f32_32x32x16_bf16), f32 accumulation.
//
// The semantics of glypr's Metal Q8_0 kernels (dequantize the weight, multiply
// unquantized activations, f32 accumulate; fused_ops.metal:574-581, 649-758)
// and of candle's CANDLE_DEQUANTIZE_ALL path, at bf16 operand precision.
// Weights stay Q8_0 in HBM (1.125 B/value); each 16-byte int8 chunk is turned
// into 16 bf16 values in registers: the signed byte to f32 (an SDWA byte
// select of v_cvt_f32_i32), q*d (exact), then v_cvt_pk_bf16_f32 (round to
// nearest even).  Activations arrive as bf16 from
// the RMSNorm prologue (or a conversion pass).
#include "device_common.hpp"
#include "internal.hpp"
#include "qkv_epilogue.hpp"

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

// GeGLU of the BF16_DEQUANT path, whose h is rounded to bf16 (relative
// error up to 2^-9): 0.5 g (1 + tanh(z)) = g sigmoid(2 z), evaluated as
// g u / (1 + exp2(-2 log2(e) z)) on the hardware exp2 and reciprocal (~1e-6
// relative, and no cancellation for negative z, where 1 + tanh(z) would
// lose its low bits); the tanh-GELU constants and the +-10 clamps of
// geglu_scalar_f32 (cpu_simd/geglu.rs:6-18).  Straight-line: the formula is
// evaluated for every g (it cannot trap) and the clamps select, so a wave's
// lanes need no divergent branches.
__device__ __forceinline__ float geglu_bf16(float g, float u) {
  // -2 log2(e) * 0.7978846
  const float z2 = -2.3022083f * (g + 0.044715f * (g * g * g));
  const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z2));
  const float mid = materialize((g * u) * s);
  return g <= -10.0f ? 0.0f : (g >= 10.0f ? g * u : mid);
}

// 16 int8 -> 16 bf16 (32 bytes) scaled by d: the sign-extending byte select of
// v_cvt_f32_i32 (SDWA), the exact product q*d (8 x 11 significant bits), then
// v_cvt_pk_bf16_f32 (round to nearest even).
__device__ __forceinline__ void dequant16(v4i q, float d, v4i& lo, v4i& hi) {
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t u = (uint32_t)q[i];
    const float f0 = (float)(int)(signed char)(u & 0xFFu) * d;
    const float f1 = (float)(int)(signed char)((u >> 8) & 0xFFu) * d;
    const float f2 = (float)(int)(signed char)((u >> 16) & 0xFFu) * d;
    const float f3 = (float)(int)(signed char)(u >> 24) * d;
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
          float h = geglu_bf16(acc[tm][2 * p][r], acc[tm][2 * p + 1][r]);
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

// ---------------------------------------------------------------------------
// Large-M variant (M > 2048, K % 64 == 0).  128 x 128 tiles on 4 waves side
// by side along N, 128 x 32 outputs each (4 v_mfma_f32_32x32x16_bf16 tiles
// stacked along M), so every B column is dequantized by exactly one wave;
// every 64-K stage arrives by LDS DMA into a two-slot ring:
//   A  [128 rows][128 B] bf16, 16-byte chunk c of row r at c ^ ((r >> 1) & 7);
//   B  [128 rows][64 B]  int8, chunk c of row r at c ^ ((r >> 2) & 3);
//   dB [2 blocks][128 rows] f32.
// Per 32-K block a lane reads 16 consecutive K of its A row (two b128) and
// of its B column (one b128 of int8), dequantizes the latter in registers
// (dequant16: the exact q*d, then bf16 round-to-nearest-even, as the staged
// path) and runs two MFMA k-steps on K {0..7, 16..23} and {8..15, 24..31} of
// the block; A and B use the same order, so every product is formed once.
// XCD-aware tile order as in the int8 large-M kernel; 50 KB of LDS and ~120
// VGPRs, so three workgroups share a CU.  The 128-column tile (rather than
// 256) keeps the grids of the C3 projections near whole rounds of 768
// workgroup slots.
// GEGLU: the 32 B rows of wave w are gate columns hc0 + 16 w .. + 15, then
// the up columns of the same h columns, so lanes l and l + 16 hold gate and
// up of one h element; one v_permlane16_swap per register pair brings them
// together, and each lane evaluates half of its 16 rows per MFMA tile.
// ---------------------------------------------------------------------------
constexpr int BFB_BN = 128, BFB_BK = 64;

// TM 32-row MFMA tiles per wave (BM = 32 TM rows per workgroup).
template <bool GEGLU, int TM>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
gemm_bf16_big_kernel(const uint16_t* __restrict__ A, const int8_t* __restrict__ B,
                     const float* __restrict__ dB, float* __restrict__ C,
                     uint16_t* __restrict__ Hb, int M, int N, int K, int ldc, int F,
                     int tiles_n) {
  constexpr int NW = 4, BFB_BM = 32 * TM;
  constexpr int UA = BFB_BM / 8;         // 1 KB units: 8 A rows of 128 B
  constexpr int UB = BFB_BN / 16;        // 1 KB units: 16 B rows of 64 B
  constexpr int USB = 2 * BFB_BN / 64;   // 256 B units: 64 scales of one block
  constexpr int NU = UA + UB + USB, UPW = NU / NW;
  constexpr int OFF_B = UA * 1024, OFF_SB = OFF_B + UB * 1024;
  constexpr int SLOT = OFF_SB + 2 * BFB_BN * 4;
  static_assert(UA % NW == 0 && UB % NW == 0 && USB % NW == 0,
                "every unit index j must be of one kind across the waves");
  __shared__ __attribute__((aligned(16))) uint8_t ring[2 * SLOT];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave;
  // XCD-aware tile id: workgroup i runs on XCD i % 8 (the grid is exactly
  // the tile count, taken from the arguments rather than gridDim)
  const int nblk = ((M + BFB_BM - 1) / BFB_BM) * tiles_n, id = blockIdx.x;
  const int xq8 = nblk >> 3, xr8 = nblk & 7, xcd = id & 7;
  const int W = xcd * xq8 + (xcd < xr8 ? xcd : xr8) + (id >> 3);
  const int tmi = W / tiles_n;
  const int m0 = tmi * BFB_BM, n0 = (W - tmi * tiles_n) * BFB_BN;
  const int hc0 = n0 >> 1;
  const int nb = K / QK, nst = K / BFB_BK;

  // GEGLU: 32-row group t holds gate then up of h columns hc0 + 16 t .. + 15.
  auto b_row = [&](int nl) -> int {
    if (!GEGLU) return n0 + nl < N ? n0 + nl : N - 1;
    int c = hc0 + 16 * (nl >> 5) + (nl & 15);
    if (c >= F) c = F - 1;
    return (nl & 16) ? F + c : c;
  };
  auto a_row = [&](int ml) -> int { return m0 + ml < M ? m0 + ml : M - 1; };

  // this wave's DMA units, unit u = 4 j + wave: [0, UA) A, [UA, UA + UB) B,
  // then the B scales of block u / 2 of the stage, 64 rows each.
  const int8_t* ubase[UPW];
  int uvoff[UPW];
#pragma unroll
  for (int j = 0; j < UPW; j++) {
    const int u = j * NW + wave;
    if (j * NW < UA) {
      const int row = u * 8 + (lane >> 3), c = lane & 7;
      ubase[j] = reinterpret_cast<const int8_t*>(A);
      uvoff[j] = a_row(row) * (2 * K) + ((c ^ ((row >> 1) & 7)) << 4);
    } else if (j * NW < UA + UB) {
      const int row = (u - UA) * 16 + (lane >> 2), c = lane & 3;
      ubase[j] = B;
      uvoff[j] = b_row(row) * K + ((c ^ ((row >> 2) & 3)) << 4);
    } else {
      const int v = u - UA - UB, kb = v / (BFB_BN / 64);
      ubase[j] = reinterpret_cast<const int8_t*>(dB);
      uvoff[j] = (b_row((v % (BFB_BN / 64)) * 64 + lane) * nb + kb) * 4;
    }
  }
  auto issue = [&](int st, int slot) {
    uint8_t* base = ring + slot * SLOT;
#pragma unroll
    for (int j = 0; j < UPW; j++) {
      const int u = j * NW + wave;
      if (j * NW < UA)
        dma16(ubase[j] + st * (2 * BFB_BK), uvoff[j], lds_u32(base + u * 1024));
      else if (j * NW < UA + UB)
        dma16(ubase[j] + st * BFB_BK, uvoff[j], lds_u32(base + OFF_B + (u - UA) * 1024));
      else
        dma4(ubase[j] + st * 8, uvoff[j], lds_u32(base + OFF_SB + (u - UA - UB) * 256));
    }
  };
  issue(0, 0);

  // fragment offsets; the swizzles depend on lrow only (tile rows are
  // multiples of 32)
  const int lrow = lane & 31, lhalf = lane >> 5;
  int offA[TM][2][2], offB[2], offS[2];
#pragma unroll
  for (int p = 0; p < 2; p++) {
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int row = 32 * tm + lrow, q = 4 * p + 2 * lhalf + h;
        offA[tm][p][h] = row * 128 + ((q ^ ((row >> 1) & 7)) << 4);
      }
    const int row = 32 * wn + lrow, c = 2 * p + lhalf;
    offB[p] = OFF_B + row * 64 + ((c ^ ((row >> 2) & 3)) << 4);
    offS[p] = OFF_SB + (p * BFB_BN + row) * 4;
  }
  v16f acc[TM];
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[tm][r] = 0.0f;

#pragma unroll 1
  for (int st = 0; st < nst; st++) {
    const int r = st & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (st + 1 < nst) issue(st + 1, r ^ 1);
    const uint8_t* slot = ring + r * SLOT;
#pragma unroll
    for (int p = 0; p < 2; p++) {
      v8bf a[TM][2];
#pragma unroll
      for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int h = 0; h < 2; h++)
          a[tm][h] = *reinterpret_cast<const v8bf*>(slot + offA[tm][p][h]);
      const v4i q = *reinterpret_cast<const v4i*>(slot + offB[p]);
      const float d = *reinterpret_cast<const float*>(slot + offS[p]);
      v4i lo, hi;
      dequant16(q, d, lo, hi);
      const v8bf b0 = __builtin_bit_cast(v8bf, lo), b1 = __builtin_bit_cast(v8bf, hi);
#pragma unroll
      for (int tm = 0; tm < TM; tm++) {
        acc[tm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[tm][0], b0, acc[tm], 0, 0, 0);
        acc[tm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[tm][1], b1, acc[tm], 0, 0, 0);
      }
    }
  }

  // output rows of register r: 8 (r >> 2) + 4 lhalf + (r & 3) of the 32-row tile
  if constexpr (!GEGLU) {
    const int gn = n0 + 32 * wn + lrow;
    float* crow = C + (int64_t)(m0 + 4 * lhalf) * ldc + gn;
    if (m0 + BFB_BM <= M && n0 + BFB_BN <= N) {  // whole tile in range (uniform)
#pragma unroll
      for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          st_nt(&crow[(int64_t)(32 * tm + 8 * (r >> 2) + (r & 3)) * ldc], (float)acc[tm][r]);
    } else {
#pragma unroll
      for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int gm = m0 + 32 * tm + 8 * (r >> 2) + 4 * lhalf + (r & 3);
          if (gm < M && gn < N)
            st_nt(&crow[(int64_t)(32 * tm + 8 * (r >> 2) + (r & 3)) * ldc], (float)acc[tm][r]);
        }
    }
  } else {
    // Lane l < 16 (of each 16-lane row pair) holds gate, lane l + 16 up, of
    // h column hc.  v_permlane16_swap on registers (i, 8 + i) swaps the odd
    // 16-lane rows of the first with the even rows of the second, leaving
    // gate in the first and up in the second, for tile row 8 (i >> 2) +
    // 4 lhalf + (i & 3) in lanes l < 16 and that row + 16 in lanes l + 16.
    const int hc = hc0 + 16 * wn + (lrow & 15);
    uint16_t hv[TM][8];
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
      for (int i = 0; i < 8; i++) {
        // (copied to scalars first: __builtin_bit_cast of an ext_vector
        // element reads element 0 with this compiler)
        const float x = acc[tm][i], y = acc[tm][8 + i];
        const auto gu = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x),
                                                         __builtin_bit_cast(uint32_t, y), false, false);
        const float h = geglu_bf16(__builtin_bit_cast(float, (uint32_t)gu[0]),
                                   __builtin_bit_cast(float, (uint32_t)gu[1]));
        hv[tm][i] = __builtin_bit_cast(uint16_t, (__bf16)h);
      }
    uint16_t* hrow = Hb + (int64_t)(m0 + (lrow & 16) + 4 * lhalf) * F + hc;
    if (m0 + BFB_BM <= M && hc0 + BFB_BN / 2 <= F) {  // whole tile in range (uniform)
#pragma unroll
      for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int i = 0; i < 8; i++)
          hrow[(int64_t)(32 * tm + 8 * (i >> 2) + (i & 3)) * F] = hv[tm][i];
    } else {
#pragma unroll
      for (int tm = 0; tm < TM; tm++)
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const int gm = m0 + 32 * tm + 8 * (i >> 2) + (lrow & 16) + 4 * lhalf + (i & 3);
          if (gm < M && hc < F) hrow[(int64_t)(32 * tm + 8 * (i >> 2) + (i & 3)) * F] = hv[tm][i];
        }
    }
  }
}

template <bool GEGLU, int TM>
hipError_t run_big(const uint16_t* xb, const int8_t* wq, const float* dw, float* y, uint16_t* hb,
                   int64_t M, int64_t Nrows, int64_t K, int64_t ldc, int64_t F, hipStream_t s) {
  constexpr int BM = 32 * TM;
  const int64_t tiles_n = (Nrows + BFB_BN - 1) / BFB_BN;
  const int64_t tiles = ((M + BM - 1) / BM) * tiles_n;
  gemm_bf16_big_kernel<GEGLU, TM><<<dim3((unsigned)tiles), 256, 0, s>>>(
      xb, wq, dw, y, hb, (int)M, (int)Nrows, (int)K, (int)ldc, (int)F, (int)tiles_n);
  return hipGetLastError();
}

// The large-M kernel addresses operands with 32-bit offsets.
inline bool big_ok(int64_t M, int64_t Nrows, int64_t K) {
  return M > 2048 && K % BFB_BK == 0 && 2 * M * K < (int64_t(1) << 31) &&
         Nrows * K < (int64_t(1) << 31);
}

// ---------------------------------------------------------------------------
// Dense bf16 weights (LinearOp over an F16/BF16 GGUF tensor, linear.rs:48-54,
// at bf16): C = A . B^T with A bf16 [M][K] and B bf16 [N][K], f32 accumulate.
// 128 x 128 tiles on a 2 x 2 grid of waves (64 x 64 outputs each, 2 x 2
// v_mfma_f32_32x32x16_bf16 tiles).  K streams through an LDS ring of RING
// slots, BKE K per stage (one or two 32-K blocks), A and B each [128 rows]
// [2 BKE bytes] by LDS DMA, 16-byte chunk c of row r at c ^ swz(r); the waits
// count exactly the units issued after each stage, so RING - 1 stages are in
// flight.  Per 32-K block a lane takes 16 consecutive K of its A row and B
// column (two b128 each) as two MFMA k-steps, the same order on both sides.
// GEGLU: 32-row tiles alternate gate and up of the same 32 h columns; h =
// geglu(gate, up) leaves as bf16.
// ---------------------------------------------------------------------------
constexpr int BFW_BM = 128, BFW_BN = 128;

template <bool GEGLU, int BKE, int RING, bool VEC>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
gemm_bf16w_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                  float* __restrict__ C, uint16_t* __restrict__ Hb, int M, int N, int K,
                  int ldc, int F, int tiles_n) {
  constexpr int NW = 4, TM = 2, TN = 2;
  constexpr int ROWB = 2 * BKE;                 // bytes per LDS row per stage
  constexpr int CPR = ROWB / 16;                // 16-byte chunks per row (4 or 8)
  constexpr int RPU = 1024 / ROWB;              // rows per 1 KB DMA unit
  constexpr int UA = BFW_BM / RPU, UB = BFW_BN / RPU;
  constexpr int UPW = (UA + UB) / NW;
  constexpr int SLOT = (UA + UB) * 1024;
  constexpr int NBLK = BKE / 32;                // 32-K blocks per stage
  static_assert(BKE == 32 || BKE == 64, "stage of one or two 32-K blocks");
  static_assert(UA % NW == 0 && UB % NW == 0 && RING >= 2, "unit kinds per j; ring");
  // 8 chunks per row: swizzle by (r >> 1) & 7; 4 chunks: by (r >> 2) & 3.
  // Either keeps any 16 consecutive rows' b128 reads on distinct banks.
  auto swz = [](int r) -> int { return CPR == 8 ? (r >> 1) & 7 : (r >> 2) & 3; };
  __shared__ __attribute__((aligned(16))) uint8_t ring[RING * SLOT];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  // the grid is exactly the tile count (from the arguments, not gridDim)
  const int nblk = ((M + BFW_BM - 1) / BFW_BM) * tiles_n, id = blockIdx.x;
  const int xq8 = nblk >> 3, xr8 = nblk & 7, xcd = id & 7;
  const int W = xcd * xq8 + (xcd < xr8 ? xcd : xr8) + (id >> 3);
  const int tmi = W / tiles_n;
  const int m0 = tmi * BFW_BM, n0 = (W - tmi * tiles_n) * BFW_BN;
  const int hc0 = n0 >> 1;
  const int nst = K / BKE;

  auto b_row = [&](int nl) -> int {
    if (!GEGLU) return n0 + nl < N ? n0 + nl : N - 1;
    const int t = nl >> 5;
    int c = hc0 + (t >> 1) * 32 + (nl & 31);
    if (c >= F) c = F - 1;
    return (t & 1) ? F + c : c;
  };
  auto a_row = [&](int ml) -> int { return m0 + ml < M ? m0 + ml : M - 1; };

  const int8_t* ubase[UPW];
  int uvoff[UPW];
#pragma unroll
  for (int j = 0; j < UPW; j++) {
    const int u = j * NW + wave;
    const int row = (u < UA ? u : u - UA) * RPU + lane / CPR, c = lane % CPR;
    const int grow = u < UA ? a_row(row) : b_row(row);
    ubase[j] = reinterpret_cast<const int8_t*>(u < UA ? A : B);
    uvoff[j] = grow * (2 * K) + ((c ^ swz(row)) << 4);
  }
  auto issue = [&](int st, int slot) {
#pragma unroll
    for (int j = 0; j < UPW; j++)
      dma16(ubase[j] + st * ROWB, uvoff[j], lds_u32(ring + slot * SLOT + (j * NW + wave) * 1024));
  };
#pragma unroll
  for (int st = 0; st < RING - 1; st++)
    if (st < nst) issue(st, st);

  const int lrow = lane & 31, lhalf = lane >> 5;
  int offA[TM][NBLK][2], offB[TN][NBLK][2];
#pragma unroll
  for (int p = 0; p < NBLK; p++)
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int q = 4 * p + 2 * lhalf + h;
#pragma unroll
      for (int tm = 0; tm < TM; tm++) {
        const int row = 64 * wm + 32 * tm + lrow;
        offA[tm][p][h] = row * ROWB + ((q ^ swz(row)) << 4);
      }
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        const int row = 64 * wn + 32 * tn + lrow;
        offB[tn][p][h] = UA * 1024 + row * ROWB + ((q ^ swz(row)) << 4);
      }
    }
  v16f acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int tn = 0; tn < TN; tn++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[tm][tn][r] = 0.0f;

#pragma unroll 1
  for (int g = 0; g < nst; g += RING) {
#pragma unroll
    for (int r = 0; r < RING; r++) {
      const int st = g + r;
      if (st < nst) {
        const int later = (st + RING - 2 < nst - 1 ? st + RING - 2 : nst - 1) - st;
        vm_wait_units<UPW, RING - 2>(later);
        __syncthreads();
        if (st + RING - 1 < nst) issue(st + RING - 1, (r + RING - 1) % RING);
        const uint8_t* slot = ring + r * SLOT;
#pragma unroll
        for (int p = 0; p < NBLK; p++) {
          v8bf a[TM][2], b[TN][2];
#pragma unroll
          for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
              a[tm][h] = *reinterpret_cast<const v8bf*>(slot + offA[tm][p][h]);
#pragma unroll
            for (int tn = 0; tn < TN; tn++)
              b[tn][h] = *reinterpret_cast<const v8bf*>(slot + offB[tn][p][h]);
          }
#pragma unroll
          for (int h = 0; h < 2; h++)
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
              for (int tn = 0; tn < TN; tn++)
                acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[tm][h], b[tn][h],
                                                                      acc[tm][tn], 0, 0, 0);
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Output rows of register r: 8 (r >> 2) + 4 lhalf + (r & 3) of the 32-row
  // tile, column lrow.  VEC (the host checked that N, ldc or F are multiples
  // of 4 and the output 16- or 8-byte aligned): a quad transpose of registers
  // 4g .. 4g + 3 gives lane 4k + i row 8g + 4 lhalf + i, columns 4k .. 4k + 3,
  // one 16-byte (8-byte for bf16 h) store instead of four scalar ones.
  const int qi = lane & 3, qc = lrow & ~3;
  if constexpr (!GEGLU) {
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        const int gn = n0 + 64 * wn + 32 * tn + (VEC ? qc : lrow);
#pragma unroll
        for (int g = 0; g < 4; g++) {
          float v[4] = {acc[tm][tn][4 * g], acc[tm][tn][4 * g + 1], acc[tm][tn][4 * g + 2],
                        acc[tm][tn][4 * g + 3]};
          const int gr = m0 + 64 * wm + 32 * tm + 8 * g + 4 * lhalf;
          if constexpr (VEC) {
            quad_transpose4(v);
            if (gr + qi < M && gn < N)
              *reinterpret_cast<float4*>(C + (int64_t)(gr + qi) * ldc + gn) =
                  make_float4(v[0], v[1], v[2], v[3]);
          } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
              if (gr + j < M && gn < N) C[(int64_t)(gr + j) * ldc + gn] = v[j];
          }
        }
      }
  } else {
    // tiles 0 and 1 of the wave are gate and up of h columns hc0 + 32 wn ..
    const int hc = hc0 + 32 * wn + (VEC ? qc : lrow);
#pragma unroll
    for (int tm = 0; tm < TM; tm++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = geglu_bf16(acc[tm][0][4 * g + j], acc[tm][1][4 * g + j]);
        const int gr = m0 + 64 * wm + 32 * tm + 8 * g + 4 * lhalf;
        if constexpr (VEC) {
          quad_transpose4(v);
          const uint32_t lo = __builtin_bit_cast(uint16_t, (__bf16)v[0]) |
                              (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v[1]) << 16;
          const uint32_t hi = __builtin_bit_cast(uint16_t, (__bf16)v[2]) |
                              (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v[3]) << 16;
          if (gr + qi < M && hc < F)
            *reinterpret_cast<uint2*>(Hb + (int64_t)(gr + qi) * F + hc) = make_uint2(lo, hi);
        } else {
#pragma unroll
          for (int j = 0; j < 4; j++)
            if (gr + j < M && hc < F)
              Hb[(int64_t)(gr + j) * F + hc] = __builtin_bit_cast(uint16_t, (__bf16)v[j]);
        }
      }
  }
}

// ---------------------------------------------------------------------------
// The dense-bf16 q|k|v projection with the attention prologue as epilogue
// (the bf16-weight model's SelfAttention::forward up to the attention,
// attention/mod.rs:192-214): the dense kernel's main loop on (64 WMW tokens,
// head slot of 256 columns) tiles, 4 WMW waves of 64 x 64 (WMW along M, 4
// along N) over the same two-slot ring of 64-K stages, then the f32 tile
// through LDS in two halves of 32 WMW rows and qkv_epilogue_rows.
// The f32 products are those of gemm_bf16w_kernel (same MFMA order), so the
// operands equal gemm_bf16w + qkv_post bit for bit.  WMW 2 (128 rows, 96 KB)
// or 3 (192 rows, 112 KB): one workgroup per CU.
// ---------------------------------------------------------------------------
template <int WMW>
__global__ void __launch_bounds__(WMW * 4 * 64) __attribute__((amdgpu_waves_per_eu(WMW)))
gemm_bf16w_qkv_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, int K,
                      int T, int Tp, int nq, int nkv, const float* __restrict__ qnw,
                      const float* __restrict__ knw, float eps, const float* __restrict__ cos_t,
                      const float* __restrict__ sin_t, _Float16* __restrict__ q16,
                      _Float16* __restrict__ k16, _Float16* __restrict__ vt16,
                      const int2* __restrict__ seg) {
  constexpr int NW = 4 * WMW, TM = 2, TN = 2, BKE = 64;
  constexpr int BM = 64 * WMW, BN = QKV_HD;
  constexpr int ROWB = 2 * BKE, CPR = ROWB / 16, RPU = 1024 / ROWB;   // 128 B, 8, 8
  constexpr int UA = BM / RPU, UB = BN / RPU;                         // 1 KB units
  constexpr int NU = UA + UB, UPW = (NU + NW - 1) / NW;
  constexpr int SLOT = NU * 1024;
  constexpr int NBLK = BKE / 32;
  constexpr int HALF = BM / 2;
  static_assert(WMW == 2 || WMW == 3, "128 or 192 rows");
  static_assert(HALF == 8 * NW && HALF * QKV_SP * 4 <= 2 * SLOT, "epilogue halves");
  auto swz = [](int r) -> int { return (r >> 1) & 7; };   // 8 chunks per row
  __shared__ __attribute__((aligned(16))) uint8_t ring[2 * SLOT];
  __shared__ float sinv[HALF];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  int mi, slot;
  xcd_tile((Tp + BM - 1) / BM, nq + 2 * nkv, false, mi, slot);
  const int m0 = mi * BM, n0 = slot * BN;
  const int nst = K / BKE;
  auto a_row = [&](int ml) -> int { return m0 + ml < T ? m0 + ml : T - 1; };

  // this wave's DMA units u = NW j + wave (uniform per wave): [0, UA) A rows,
  // [UA, NU) B rows, RPU rows of 128 B each, + 128 B per stage
  const int8_t* ubase[UPW];
  int uvoff[UPW];
#pragma unroll
  for (int j = 0; j < UPW; j++) {
    const int u = j * NW + wave;
    const int row = (u < UA ? u : u - UA) * RPU + lane / CPR, c = lane % CPR;
    ubase[j] = reinterpret_cast<const int8_t*>(u < UA ? A : B);
    uvoff[j] = (u < UA ? a_row(row) : n0 + row) * (2 * K) + ((c ^ swz(row)) << 4);
  }
  auto issue = [&](int st, int sl) {
#pragma unroll
    for (int j = 0; j < UPW; j++) {
      const int u = j * NW + wave;
      if (u < NU)
        dma16(ubase[j] + st * ROWB, uvoff[j], lds_u32(ring + sl * SLOT + u * 1024));
    }
  };
  issue(0, 0);

  const int lrow = lane & 31, lhalf = lane >> 5;
  int offA[TM][NBLK][2], offB[TN][NBLK][2];
#pragma unroll
  for (int p = 0; p < NBLK; p++)
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int q = 4 * p + 2 * lhalf + h;
#pragma unroll
      for (int tm = 0; tm < TM; tm++) {
        const int row = 64 * wm + 32 * tm + lrow;
        offA[tm][p][h] = row * ROWB + ((q ^ swz(row)) << 4);
      }
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        const int row = 64 * wn + 32 * tn + lrow;
        offB[tn][p][h] = UA * 1024 + row * ROWB + ((q ^ swz(row)) << 4);
      }
    }
  v16f acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; tm++)
#pragma unroll
    for (int tn = 0; tn < TN; tn++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[tm][tn][r] = 0.0f;

#pragma unroll 1
  for (int st = 0; st < nst; st++) {
    const int r = st & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // stage st has landed
    __syncthreads();   // ... for every wave; the other slot is free
    if (st + 1 < nst) issue(st + 1, r ^ 1);
    const uint8_t* sl = ring + r * SLOT;
#pragma unroll
    for (int p = 0; p < NBLK; p++) {
      v8bf a[TM][2], b[TN][2];
#pragma unroll
      for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
          a[tm][h] = *reinterpret_cast<const v8bf*>(sl + offA[tm][p][h]);
#pragma unroll
        for (int tn = 0; tn < TN; tn++)
          b[tn][h] = *reinterpret_cast<const v8bf*>(sl + offB[tn][p][h]);
      }
#pragma unroll
      for (int h = 0; h < 2; h++)
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
          for (int tn = 0; tn < TN; tn++)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[tm][h], b[tn][h],
                                                                  acc[tm][tn], 0, 0, 0);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();   // every wave is past its last ring read

  float* stg = reinterpret_cast<float*>(ring);
#pragma unroll 1
  for (int hf = 0; hf < 2; hf++) {
    // register r of MFMA tile (tm, tn) is row 64 wm + 32 tm + 8 (r >> 2) +
    // 4 lhalf + (r & 3), column 64 wn + 32 tn + lrow; each 32-row tile lies
    // in one half
    const int r0 = m0 + HALF * hf;
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
      const int lr = 64 * wm + 32 * tm - HALF * hf;   // first row of the MFMA tile in the half
      if (lr >= 0 && lr < HALF) {
#pragma unroll
        for (int tn = 0; tn < TN; tn++)
#pragma unroll
          for (int r = 0; r < 16; r++)
            stg[(lr + 8 * (r >> 2) + 4 * lhalf + (r & 3)) * QKV_SP + 64 * wn + 32 * tn + lrow] =
                acc[tm][tn][r];
      }
    }
    __syncthreads();
    qkv_epilogue_rows<NW>(stg, sinv, r0, T, Tp, slot, nq, nkv, qnw, knw, eps, cos_t, sin_t, q16,
                          k16, vt16, seg);
    __syncthreads();   // the half is consumed before the next one is staged
  }
}

template <bool GEGLU>
hipError_t run_dense(const uint16_t* xb, const uint16_t* wb, float* y, uint16_t* hb, int64_t M,
                     int64_t Nrows, int64_t K, int64_t ldc, int64_t F, hipStream_t s) {
  const int64_t tiles_n = (Nrows + BFW_BN - 1) / BFW_BN;
  const int64_t tiles = ((M + BFW_BM - 1) / BFW_BM) * tiles_n;
  const bool vec = GEGLU ? F % 4 == 0 && (reinterpret_cast<uintptr_t>(hb) & 7) == 0
                         : Nrows % 4 == 0 && ldc % 4 == 0 &&
                               (reinterpret_cast<uintptr_t>(y) & 15) == 0;
  if (vec)
    gemm_bf16w_kernel<GEGLU, 64, 2, true><<<dim3((unsigned)tiles), 256, 0, s>>>(
        xb, wb, y, hb, (int)M, (int)Nrows, (int)K, (int)ldc, (int)F, (int)tiles_n);
  else
    gemm_bf16w_kernel<GEGLU, 64, 2, false><<<dim3((unsigned)tiles), 256, 0, s>>>(
        xb, wb, y, hb, (int)M, (int)Nrows, (int)K, (int)ldc, (int)F, (int)tiles_n);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_bf16(const uint16_t* xb, const int8_t* wq, const float* dw, float* y,
                            int64_t M, int64_t N, int64_t K, int64_t ldc, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  if (big_ok(M, N, K)) return run_big<false, 4>(xb, wq, dw, y, nullptr, M, N, K, ldc, 0, s);
  int64_t big_tiles = ((M + 255) / 256) * ((N + 127) / 128);
  if (big_tiles >= 256)
    return run<256, 128, 4, 2, false>(xb, wq, dw, y, nullptr, M, N, K, ldc, 0, s);
  return run<64, 64, 2, 2, false>(xb, wq, dw, y, nullptr, M, N, K, ldc, 0, s);
}

hipError_t launch_gemm_bf16_geglu(const uint16_t* xb, const int8_t* wq, const float* dw,
                                  uint16_t* hb, int64_t M, int64_t F, int64_t K, hipStream_t s) {
  if (M == 0 || F == 0) return hipSuccess;
  if (big_ok(M, 2 * F, K)) return run_big<true, 4>(xb, wq, dw, nullptr, hb, M, 2 * F, K, 0, F, s);
  int64_t big_tiles = ((M + 255) / 256) * ((2 * F + 127) / 128);
  if (big_tiles >= 256)
    return run<256, 128, 4, 2, true>(xb, wq, dw, nullptr, hb, M, 2 * F, K, 0, F, s);
  return run<64, 128, 2, 2, true>(xb, wq, dw, nullptr, hb, M, 2 * F, K, 0, F, s);
}

}  // namespace glypr

namespace glypr {

bool gemm_bf16w_ok(int64_t M, int64_t Nrows, int64_t K) {
  return K % 64 == 0 && 2 * M * K < (int64_t(1) << 31) && 2 * Nrows * K < (int64_t(1) << 31);
}

hipError_t launch_gemm_bf16w(const uint16_t* xb, const uint16_t* wb, float* y, int64_t M,
                             int64_t N, int64_t K, int64_t ldc, hipStream_t s) {
  if (M == 0 || N == 0) return hipSuccess;
  if (!gemm_bf16w_ok(M, N, K)) return hipErrorInvalidValue;
  return run_dense<false>(xb, wb, y, nullptr, M, N, K, ldc, 0, s);
}

hipError_t launch_gemm_bf16w_geglu(const uint16_t* xb, const uint16_t* wb, uint16_t* hb,
                                   int64_t M, int64_t F, int64_t K, hipStream_t s) {
  if (M == 0 || F == 0) return hipSuccess;
  if (!gemm_bf16w_ok(M, 2 * F, K) || F % 32 != 0) return hipErrorInvalidValue;
  return run_dense<true>(xb, wb, nullptr, hb, M, 2 * F, K, 0, F, s);
}

// From 2048 rows the fused launch beats gemm_bf16w + qkv_post (2048: 18.9
// against 22.9 us; 8192: 32.8 against 46.8 us); below, its 128-row blocks
// leave most CUs idle (512: 18.0 against 15.3 us).
bool gemm_bf16w_qkv_ok(int64_t T, int64_t Tp, int64_t K, int64_t hd) {
  return hd == QKV_HD && Tp % 64 == 0 && Tp >= T && T > 0 && Tp >= 2048 && K > 0 &&
         K % 64 == 0 && 2 * T * K < (int64_t(1) << 31);
}

hipError_t launch_gemm_bf16w_qkv(const uint16_t* xb, const uint16_t* wb, int64_t T, int64_t Tp,
                                 int64_t K, int64_t nq, int64_t nkv, int64_t hd, const float* qnw,
                                 const float* knw, float eps, const float* cos_t,
                                 const float* sin_t, uint16_t* q16, uint16_t* k16, uint16_t* vt16,
                                 const int32_t* seg, hipStream_t s) {
  const int64_t slots = nq + 2 * nkv;
  if (!gemm_bf16w_qkv_ok(T, Tp, K, hd) || 2 * slots * hd * K >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  _Float16* q = reinterpret_cast<_Float16*>(q16);
  _Float16* k = reinterpret_cast<_Float16*>(k16);
  _Float16* v = reinterpret_cast<_Float16*>(vt16);
  const int2* sg = reinterpret_cast<const int2*>(seg);
  // one workgroup per CU: the row block (128 or 192) with the fewest rows per
  // CU over its rounds of 256 workgroups
  auto cost = [&](int64_t bm) { return ((Tp + bm - 1) / bm * slots + 255) / 256 * bm; };
  if (cost(192) < cost(128))
    gemm_bf16w_qkv_kernel<3><<<(unsigned)(slots * ((Tp + 191) / 192)), 768, 0, s>>>(
        xb, wb, (int)K, (int)T, (int)Tp, (int)nq, (int)nkv, qnw, knw, eps, cos_t, sin_t, q, k, v,
        sg);
  else
    gemm_bf16w_qkv_kernel<2><<<(unsigned)(slots * ((Tp + 127) / 128)), 512, 0, s>>>(
        xb, wb, (int)K, (int)T, (int)Tp, (int)nq, (int)nkv, qnw, knw, eps, cos_t, sin_t, q, k, v,
        sg);
  return hipGetLastError();
}

}  // namespace glypr
