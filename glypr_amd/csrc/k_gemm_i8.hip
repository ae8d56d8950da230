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
#include "qkv_epilogue.hpp"

namespace glypr {

namespace {

constexpr int BK = 128;        // K bytes per LDS stage
constexpr int KB = BK / QK;    // Q8_0 blocks per stage
constexpr int MAGIC = 0x4B400000;
constexpr float NEG_MAGIC = -12582912.0f;  // -(1.5 * 2^23)

// One Q8_0 block's term added to an output.  `sb` is the MFMA accumulator
// word MAGIC + S (S the block's integer dot product), wc = wd * NEG_MAGIC, so
// the first FMA is round(S * d_w) exactly.  EXACT (F2 = false) then rounds
// the product by d_x and the sum separately, the reference's vec_dot order;
// F2 fuses the last two into one FMA (GLYPR_Q8_INT8_FMA: 2 VALU ops per
// output and block instead of 3, one rounding fewer).
template <bool F2>
__device__ __forceinline__ float q8_term(float acc, int sb, float wd, float wc, float xd) {
  const float t = fmaf(__int_as_float(sb), wd, wc);  // round(S * d_w)
  if constexpr (F2) return fmaf(t, xd, acc);         // round(acc + . * d_x)
  const float u = t * xd;                            // round(. * d_x)
  return acc + u;                                    // round(acc + .)
}

template <int BM, int BN, int WM, int WN, bool GEGLU, bool F2>
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
        v16i d[TM][TN];
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
          for (int tn = 0; tn < TN; tn++)
            d[tm][tn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[tm], bfr[tn], magic, 0, 0, 0);
#pragma unroll
        for (int tm = 0; tm < TM; tm++) {
          v4f xd[4];
#pragma unroll
          for (int g = 0; g < 4; g++)
            xd[g] = *reinterpret_cast<const v4f*>(
                &dAs[buf][kb][wm * WTM + tm * 32 + 8 * g + 4 * lhalf]);
#pragma unroll
          for (int tn = 0; tn < TN; tn++) {
#pragma unroll
            for (int r = 0; r < 16; r++)
              acc[tm][tn][r] =
                  q8_term<F2>(acc[tm][tn][r], d[tm][tn][r], wd[tn], wc[tn], xd[r >> 2][r & 3]);
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
    // h = geglu(gate, up); a row's 32-wide Q8_0 block of h is one 32-lane
    // half-wave.  The 32 lanes reduce the block amax together, then one lane
    // per row derives the scale (through a per-wave LDS table in the
    // now-free A tile) instead of all 32 repeating the two divisions.
    const int nbh = F / QK;
    float* t_amax = reinterpret_cast<float*>(&As[0][0]) + wave * (3 * WTM);
    float* t_id = t_amax + WTM;
    float* t_dq = t_amax + 2 * WTM;
#pragma unroll
    for (int p = 0; p < TN / 2; p++) {
      const int hc = (n0 >> 1) + ((wn * WTN) >> 6) * 32 + p * 32 + lrow;
      float h[TM][16];
#pragma unroll
      for (int tm = 0; tm < TM; tm++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          h[tm][r] = geglu_scalar(acc[tm][2 * p][r], acc[tm][2 * p + 1][r]);
          const float a = max32_hi(fmaxf(0.0f, fabsf(h[tm][r])));
          if (lrow == 31) t_amax[tm * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3)] = a;
        }
      }
      // LDS serves a wave's accesses in order; the fences keep the compiler
      // from moving the table reads above the writes.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      for (int row = lane; row < WTM; row += 64) {
        const QScale q = q8_scale(t_amax[row]);
        t_id[row] = q.id;
        t_dq[row] = q.dq;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int tm = 0; tm < TM; tm++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int lr = tm * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
          const int gm = m0 + wm * WTM + lr;
          const int q = quant_round(h[tm][r] * t_id[lr]);
          if (gm < M && hc < F) {
            Hq[(int64_t)gm * F + hc] = (int8_t)q;
            if (lrow == 0) dH[(int64_t)gm * nbh + (hc >> 5)] = t_dq[lr];
          }
        }
      }
      __builtin_amdgcn_wave_barrier();   // the table is reused by the next pair
    }
  }
}


// ---------------------------------------------------------------------------
// Small-M variant (T <= ~2K tokens: one sequence through a layer).  There the
// big-tile grid has fewer waves than the chip has SIMDs, and the exact
// epilogue (3 VALU ops per output and block) is the bound.  This kernel:
//  - uses v_mfma_i32_16x16x32_i8 (still one Q8_0 block per MFMA) so each wave
//    owns a 16 x 16*TNW tile: many small waves spread over all SIMDs;
//  - streams K in 128-byte stages through a RING-slot LDS ring filled by
//    global_load_lds_dwordx4 (LDS DMA, no register staging).  The DMAs are
//    issued from inline asm: the compiler then does not see them and adds no
//    vmcnt(0) before the ds_reads of earlier stages.  Every loop iteration
//    issues exactly UPW DMAs per wave (past the last stage it reloads the last
//    stage into the slot just freed), so "stage s has landed" is the single
//    constant wait vmcnt((RING-2)*UPW) followed by a barrier;
//  - stages the per-block scales once, coalesced, in their natural [row][b]
//    layout (dA rows of the tile, then dB rows).
// LDS layout of a ring slot: A rows then B rows, each [row][128 B] with the
// 16-byte chunk c of row r stored at chunk c ^ sm_swz(r).  One DMA writes 1 KB
// linearly (lane i -> row i/8, physical chunk i%8), so lane i reads global
// chunk (i%8) ^ sm_swz(row).  Rows past M/N are clamped to a valid row (their
// outputs are never stored).
// ---------------------------------------------------------------------------
constexpr int SMALL_NB_MAX = 64;   // K <= 2048
// Row swizzle of the small-M kernels' 128-byte LDS rows.  The fragment reads
// (ds_read_b64: rows l16 of a 16-row tile, chunk 2 kb + (lq >> 1), half lq & 1)
// measured 2 SQ_LDS_BANK_CONFLICT cycles per read with r & 7 and none with
// (r >> 1) & 7.
__device__ __forceinline__ int sm_swz(int r) { return (r >> 1) & 7; }

// WM x WN waves; wave (wm, wn) owns rows 16 wm.. and TNW 16-row B tiles.
// GEGLU: TNW == 2 (gate tile, up tile of the same 16 h columns) and WN == 2:
// the 32-wide Q8_0 block of h spans waves wn = 0, 1, which exchange their
// amax through LDS.  NB = K / 32 blocks, NB % 4 == 0.
//
// Scales stay in their natural [row][b] layout in LDS, so the four blocks of
// a stage are 16 contiguous bytes of a row: per stage a lane reads its four
// row scales and its TNW column scales with 4 + TNW ds_read_b128.  The stage
// loop is unrolled by RING so ring slots are compile-time LDS offsets.
// Argument order: everything the first DMAs need (operands, scales, M, N)
// comes first, so that it lies within the 14 argument dwords the hardware
// preloads into SGPRs; the outputs, used at the end, follow.
template <int WM, int WN, int TNW, bool GEGLU, bool F2, int RING, int NB>
__global__ void __launch_bounds__(WM * WN * 64)
gemm_i8_small_kernel(const int8_t* __restrict__ A, const float* __restrict__ dA,
                     const int8_t* __restrict__ B, const float* __restrict__ dB, int M, int N,
                     int ldc, int F, float* __restrict__ C, int8_t* __restrict__ Hq,
                     float* __restrict__ dH) {
  constexpr int K = NB * QK, NST = NB / KB;
  constexpr int NW = WM * WN;
  constexpr int BM = WM * 16;
  constexpr int BN = WN * 16 * TNW;         // B rows per tile
  constexpr int UA = BM / 8, UB = BN / 8;   // 1 KB DMA units per stage
  constexpr int UPW = (UA + UB) / NW;
  constexpr int SA = NB * BM, SB = NB * BN;
  static_assert(NB % KB == 0 && NB <= SMALL_NB_MAX, "K must be a multiple of 128, <= 2048");
  static_assert((UA + UB) % NW == 0, "stage units must split evenly over the waves");
  static_assert(RING >= 2, "ring needs >= 2 slots");
  static_assert(!GEGLU || (TNW == 2 && WN == 2), "GeGLU tile: 2 waves x (gate, up)");
  constexpr int SLOT = (BM + BN) * BK;
  __shared__ __attribute__((aligned(16))) uint8_t ring[RING * SLOT];
  __shared__ __attribute__((aligned(16))) float sc[SA + SB + 256];
  __shared__ float amax_x[GEGLU ? WN * BM : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  // consecutive workgroups are the N tiles of one M block, so they start on
  // different XCDs together (measured faster here than the prologue kernel's
  // XCD order, which re-reads less)
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;   // GEGLU: virtual column index (2 per h column)
  const int hc0 = n0 >> 1;

  // B row of tile-local row nl.  GEGLU: [gate hc0..+15, up hc0..+15,
  // gate hc0+16..+31, up hc0+16..+31].
  auto b_row = [&](int nl) -> int {
    if (!GEGLU) return n0 + nl < N ? n0 + nl : N - 1;
    int t = nl >> 4;
    int c = hc0 + (t >> 1) * 16 + (nl & 15);
    if (c >= F) c = F - 1;
    return (t & 1) ? F + c : c;
  };

  // ---- scales: dA rows [BM][NB] then dB rows [BN][NB], 16 B (four blocks)
  // per lane; the last unit's spare lanes repeat the last chunk into the slack
  constexpr int NQ = NB / 4;                    // 16-byte chunks per row
  constexpr int SCH = (SA + SB) / 4;            // chunks in all
  for (int c0 = wave * 64; c0 < SCH; c0 += NW * 64) {
    const int c = c0 + lane < SCH ? c0 + lane : SCH - 1;
    const float* src;
    if (c < SA / 4) {
      const int r = c / NQ, q = c - r * NQ;
      const int gm = m0 + r < M ? m0 + r : M - 1;
      src = dA + (int64_t)gm * NB + 4 * q;
    } else {
      const int f = c - SA / 4, r = f / NQ, q = f - r * NQ;
      src = dB + (int64_t)b_row(r) * NB + 4 * q;
    }
    dma16_flat(src, lds_u32(sc + 4 * c0));
  }
  // ---- this wave's DMA units: uniform base (A or B) + per-lane row offset
  const int rsub = lane >> 3, pch = lane & 7;
  const int8_t* ubase[UPW];
  int uvoff[UPW];
#pragma unroll
  for (int j = 0; j < UPW; j++) {
    const int u = j * NW + wave;
    const int row = (u < UA ? u : u - UA) * 8 + rsub;
    const int grow = u < UA ? (m0 + row < M ? m0 + row : M - 1) : b_row(row);
    ubase[j] = u < UA ? A : B;
    uvoff[j] = grow * K + ((pch ^ sm_swz(row)) << 4);
  }
  // stage st into ring slot `slot`
  auto issue = [&](int st, int slot) {
#pragma unroll
    for (int j = 0; j < UPW; j++)
      dma16(ubase[j] + st * BK, uvoff[j], lds_u32(ring + slot * SLOT + (j * NW + wave) * 1024));
  };
#pragma unroll
  for (int st = 0; st < RING - 1; st++)
    if (st < NST) issue(st, st);

  const int l16 = lane & 15, lq = lane >> 4;   // lq: 8-byte K slice (operands) / row quad (out)
  const int arow = wm * 16 + l16;
  int offA[KB], offB[TNW][KB];
#pragma unroll
  for (int kb = 0; kb < KB; kb++) {
    const int ch = 2 * kb + (lq >> 1);
    offA[kb] = arow * BK + ((ch ^ sm_swz(arow)) << 4) + ((lq & 1) << 3);
#pragma unroll
    for (int t = 0; t < TNW; t++) {
      const int brow = wn * 16 * TNW + t * 16 + l16;
      offB[t][kb] = (BM + brow) * BK + ((ch ^ sm_swz(brow)) << 4) + ((lq & 1) << 3);
    }
  }
  const float* xrow = sc + (wm * 16 + 4 * lq) * NB;   // row 4 lq + r at xrow + r * NB
  const float* wrow = sc + SA + (wn * 16 * TNW + l16) * NB;  // tile t at wrow + 16 t NB
  const v4i magic = {MAGIC, MAGIC, MAGIC, MAGIC};
  float acc[TNW][4];
#pragma unroll
  for (int t = 0; t < TNW; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) acc[t][r] = 0.0f;

  // Every wait counts exactly the DMA units issued after stage st (a uniform
  // branch picks the immediate in the last RING - 2 stages): no stage is
  // fetched twice.
#pragma unroll 1
  for (int g = 0; g < NST; g += RING) {
#pragma unroll
    for (int r = 0; r < RING; r++) {
      const int st = g + r;
      if (st < NST) {
        const int later = (st + RING - 2 < NST - 1 ? st + RING - 2 : NST - 1) - st;
        vm_wait_units<UPW, RING - 2>(later);
        __syncthreads();
        if (st + RING - 1 < NST) issue(st + RING - 1, (r + RING - 1) % RING);
        const uint8_t* slot = ring + r * SLOT;
        v4i d[KB][TNW];
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
          const v1l af = *reinterpret_cast<const v1l*>(slot + offA[kb]);
#pragma unroll
          for (int t = 0; t < TNW; t++) {
            const v1l bf = *reinterpret_cast<const v1l*>(slot + offB[t][kb]);
            d[kb][t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, bf, magic, 0, 0, 0);
          }
        }
        v4f xq[4], wq[TNW];
#pragma unroll
        for (int rr = 0; rr < 4; rr++)
          xq[rr] = *reinterpret_cast<const v4f*>(xrow + rr * NB + st * KB);
#pragma unroll
        for (int t = 0; t < TNW; t++)
          wq[t] = *reinterpret_cast<const v4f*>(wrow + t * 16 * NB + st * KB);
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
          for (int t = 0; t < TNW; t++) {
            const float wd = wq[t][kb];
            const float wc = wd * NEG_MAGIC;
#pragma unroll
            for (int rr = 0; rr < 4; rr++)
              acc[t][rr] = q8_term<F2>(acc[t][rr], d[kb][t][rr], wd, wc, xq[rr][kb]);
          }
      }
    }
  }
  // the reloads issued past the last stage must land before the LDS is released
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const int grow0 = m0 + wm * 16 + 4 * lq;
  if constexpr (!GEGLU) {
#pragma unroll
    for (int t = 0; t < TNW; t++) {
      const int gn = n0 + wn * 16 * TNW + t * 16 + l16;
#pragma unroll
      for (int r = 0; r < 4; r++)
        if (grow0 + r < M && gn < N) C[(int64_t)(grow0 + r) * ldc + gn] = acc[t][r];
    }
  } else {
    // h = geglu(gate, up); a row's 32-wide block spans waves wn = 0, 1: each
    // wave reduces its 16 columns and publishes the row maxima; after the one
    // barrier, lane l16 = r of each 16-lane group derives the scale of row
    // 4 lq + r and the group broadcasts it.
    const int nbh = F / QK;
    const int hc = hc0 + wn * 16 + l16;
    float h[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      h[r] = geglu_scalar(acc[0][r], acc[1][r]);
      const float v = max16_nonneg(fmaxf(0.0f, fabsf(h[r])));
      if (l16 == 0) amax_x[wn * BM + wm * 16 + 4 * lq + r] = v;
    }
    __syncthreads();
    const int lrs = wm * 16 + 4 * lq + (l16 & 3);
    const QScale q = q8_scale(fmaxf(amax_x[lrs], amax_x[BM + lrs]));
    const float ids[4] = {bcast16<0>(q.id), bcast16<1>(q.id), bcast16<2>(q.id),
                          bcast16<3>(q.id)};
    if (hc < F) {
#pragma unroll
      for (int r = 0; r < 4; r++)
        if (grow0 + r < M) Hq[(int64_t)(grow0 + r) * F + hc] = (int8_t)quant_round(h[r] * ids[r]);
      if (wn == 0 && l16 < 4 && grow0 + l16 < M)
        dH[(int64_t)(grow0 + l16) * nbh + (hc >> 5)] = q.dq;
    }
  }
}

template <int WM, int WN, int TNW, bool GEGLU, bool F2, int RING, int NB>
hipError_t run_small_nb(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                        float* y, int8_t* hq, float* dh, int64_t M, int64_t Nrows, int64_t ldc,
                        int64_t F, hipStream_t s) {
  constexpr int BM = WM * 16, BN = WN * 16 * TNW;
  dim3 grid((unsigned)((Nrows + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  gemm_i8_small_kernel<WM, WN, TNW, GEGLU, F2, RING, NB><<<grid, WM * WN * 64, 0, s>>>(
      xq, dx, wq, dw, (int)M, (int)Nrows, (int)ldc, (int)F, y, hq, dh);
  return hipGetLastError();
}

// K is a multiple of 128 and <= 2048 (small_ok): the BASELINE widths (768,
// 1152) and the released EmbeddingGemma-2's (512; 2048 for its down and
// full-layer o projections).
template <int WM, int WN, int TNW, bool GEGLU, bool F2, int RING>
hipError_t run_small(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                     float* y, int8_t* hq, float* dh, int64_t M, int64_t Nrows, int64_t K,
                     int64_t ldc, int64_t F, hipStream_t s) {
#define GLYPR_SMALL_NB(nb)                                                                 \
  case nb:                                                                                 \
    return run_small_nb<WM, WN, TNW, GEGLU, F2, RING, nb>(xq, dx, wq, dw, y, hq, dh, M,     \
                                                          Nrows, ldc, F, s);
  switch (K / QK) {
    GLYPR_SMALL_NB(4)
    GLYPR_SMALL_NB(8)
    GLYPR_SMALL_NB(12)
    GLYPR_SMALL_NB(16)
    GLYPR_SMALL_NB(20)
    GLYPR_SMALL_NB(24)
    GLYPR_SMALL_NB(28)
    GLYPR_SMALL_NB(32)
    GLYPR_SMALL_NB(36)
    GLYPR_SMALL_NB(48)
    GLYPR_SMALL_NB(64)
    default:
      return hipErrorInvalidValue;
  }
#undef GLYPR_SMALL_NB
}

// Small-M kernels stream K through an LDS ring; the scales of the whole K
// range stay in LDS ((BM + BN) * K/32 floats).  Their DMA offsets into the
// weight (row * K) are 32-bit: larger weights take the int64-offset kernel.
constexpr int64_t SMALL_M_MAX = 2048;
constexpr int64_t SMALL_K_MAX = 32 * SMALL_NB_MAX;
inline bool small_ok(int64_t M, int64_t Nrows, int64_t K) {
  const int64_t nb = K / QK;
  return M <= SMALL_M_MAX && K <= SMALL_K_MAX && K % BK == 0 &&
         (nb <= 36 || nb == 48 || nb == 64) && Nrows * K < (int64_t(1) << 31);
}

// ---------------------------------------------------------------------------
// GeGLU gate/up for few rows, one 16-column MFMA tile per wave whose columns
// are 8 gate rows of W and the 8 matching up rows: a wave owns 16 rows x 8 h
// columns and a workgroup of four waves one whole Q8_0 block of h (16 rows x
// 32 h columns).  The exact epilogue's VALU work binds these launches, so
// what matters is the work of the busiest SIMD: at M = 512, F = 1152 this is
// 4608 waves on 1024 SIMDs (at most 5 where the mean is 4.5), where 16 h
// columns per wave (gemm_i8_small_kernel's GeGLU tile) give 2304 waves (at
// most 3 where the mean is 2.25).
//   Gate and up of one h column meet in lanes j and j + 8 of a 16-lane row;
// one DPP row rotation by 8 trades them so that lane j < 8 holds rows
// 4 lq, 4 lq + 1 and lane j + 8 rows 4 lq + 2, 4 lq + 3 of that column, and
// every lane evaluates two h values.  A row's 32-wide amax is 8 lanes of
// each of the four waves, merged through LDS after one barrier.
//   Ring and scales as gemm_i8_small_kernel: A rows (16) then B rows (64) per
// 128-byte K stage, ten 1 KB DMA units per stage, three for waves 0 and 1
// and two for waves 2 and 3.  Same arithmetic per output, so Q8_0(h) is
// bit-identical to gemm_i8_small_kernel's GeGLU route.
// ---------------------------------------------------------------------------
template <bool F2, int RING, int NB>
__global__ void __launch_bounds__(256)
gemm_i8_geglu8_kernel(const int8_t* __restrict__ A, const float* __restrict__ dA,
                      const int8_t* __restrict__ B, const float* __restrict__ dB,
                      int8_t* __restrict__ Hq, float* __restrict__ dH, int M, int F) {
  constexpr int K = NB * QK, NST = NB / KB;
  constexpr int NW = 4, BM = 16, BN = 64;
  constexpr int UA = BM / 8, UB = BN / 8, UN = UA + UB;   // 2 + 8 DMA units per stage
  constexpr int SA = NB * BM, SB = NB * BN;
  static_assert(NB % KB == 0 && NB <= SMALL_NB_MAX, "K must be a multiple of 128, <= 2048");
  static_assert(RING >= 2, "ring needs >= 2 slots");
  constexpr int SLOT = (BM + BN) * BK;
  __shared__ __attribute__((aligned(16))) uint8_t ring[RING * SLOT];
  __shared__ __attribute__((aligned(16))) float sc[SA + SB + 256];
  __shared__ float amax_w[NW][BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hb = blockIdx.x;            // Q8_0 block of h: columns 32 hb ..
  const int m0 = blockIdx.y * BM;
  const int hc0 = hb * QK;
  // B row of tile-local row nl: wave nl / 16, gate (nl % 16 < 8) or up
  auto b_row = [&](int nl) -> int {
    const int c = hc0 + 8 * (nl >> 4) + (nl & 7);
    return (nl & 8) ? F + c : c;
  };

  constexpr int NQ = NB / 4;
  constexpr int SCH = (SA + SB) / 4;
  for (int c0 = wave * 64; c0 < SCH; c0 += NW * 64) {
    const int c = c0 + lane < SCH ? c0 + lane : SCH - 1;
    const float* src;
    if (c < SA / 4) {
      const int r = c / NQ, q = c - r * NQ;
      const int gm = m0 + r < M ? m0 + r : M - 1;
      src = dA + (int64_t)gm * NB + 4 * q;
    } else {
      const int f = c - SA / 4, r = f / NQ, q = f - r * NQ;
      src = dB + (int64_t)b_row(r) * NB + 4 * q;
    }
    dma16_flat(src, lds_u32(sc + 4 * c0));
  }
  // DMA units u = wave, wave + 4, wave + 8 (< UN): three for waves 0, 1
  const int rsub = lane >> 3, pch = lane & 7;
  const bool three = wave + 8 < UN;
  const int8_t* ubase[3];
  int uvoff[3];
#pragma unroll
  for (int j = 0; j < 3; j++) {
    const int u = j * NW + wave < UN ? j * NW + wave : UN - 1;
    const int row = (u < UA ? u : u - UA) * 8 + rsub;
    const int grow = u < UA ? (m0 + row < M ? m0 + row : M - 1) : b_row(row);
    ubase[j] = u < UA ? A : B;
    uvoff[j] = grow * K + ((pch ^ sm_swz(row)) << 4);
  }
  auto issue = [&](int st, int slot) {
#pragma unroll
    for (int j = 0; j < 3; j++)
      if (j < 2 || three)
        dma16(ubase[j] + st * BK, uvoff[j],
              lds_u32(ring + slot * SLOT + (j * NW + wave) * 1024));
  };
#pragma unroll
  for (int st = 0; st < RING - 1; st++)
    if (st < NST) issue(st, st);

  const int l16 = lane & 15, lq = lane >> 4;
  int offA[KB], offB[KB];
#pragma unroll
  for (int kb = 0; kb < KB; kb++) {
    const int ch = 2 * kb + (lq >> 1);
    offA[kb] = l16 * BK + ((ch ^ sm_swz(l16)) << 4) + ((lq & 1) << 3);
    const int brow = wave * 16 + l16;
    offB[kb] = (BM + brow) * BK + ((ch ^ sm_swz(brow)) << 4) + ((lq & 1) << 3);
  }
  const float* xrow = sc + (4 * lq) * NB;
  const float* wrow = sc + SA + (wave * 16 + l16) * NB;
  const v4i magic = {MAGIC, MAGIC, MAGIC, MAGIC};
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll 1
  for (int g = 0; g < NST; g += RING) {
#pragma unroll
    for (int r = 0; r < RING; r++) {
      const int st = g + r;
      if (st < NST) {
        const int later = (st + RING - 2 < NST - 1 ? st + RING - 2 : NST - 1) - st;
        if (three)
          vm_wait_units<3, RING - 2>(later);
        else
          vm_wait_units<2, RING - 2>(later);
        __syncthreads();
        if (st + RING - 1 < NST) issue(st + RING - 1, (r + RING - 1) % RING);
        const uint8_t* slot = ring + r * SLOT;
        v4i d[KB];
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
          const v1l af = *reinterpret_cast<const v1l*>(slot + offA[kb]);
          const v1l bf = *reinterpret_cast<const v1l*>(slot + offB[kb]);
          d[kb] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, bf, magic, 0, 0, 0);
        }
        v4f xq[4];
#pragma unroll
        for (int rr = 0; rr < 4; rr++)
          xq[rr] = *reinterpret_cast<const v4f*>(xrow + rr * NB + st * KB);
        const v4f wq = *reinterpret_cast<const v4f*>(wrow + st * KB);
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
          const float wd = wq[kb];
          const float wc = wd * NEG_MAGIC;
#pragma unroll
          for (int rr = 0; rr < 4; rr++)
            acc[rr] = q8_term<F2>(acc[rr], d[kb][rr], wd, wc, xq[rr][kb]);
        }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // lane j < 8: gate rows 4 lq .. 4 lq + 3 of column j; lane j + 8: up rows
  const bool hi = (l16 & 8) != 0;
  const float s0 = hi ? acc[0] : acc[2];
  const float s1 = hi ? acc[1] : acc[3];
  const float r0 = dpp_mov<0x128>(s0, s0);   // row_ror:8 (lane j <-> j ^ 8)
  const float r1 = dpp_mov<0x128>(s1, s1);
  const float g0 = hi ? r0 : acc[0], g1 = hi ? r1 : acc[1];
  const float u0 = hi ? acc[2] : r0, u1 = hi ? acc[3] : r1;
  float h[2];
  h[0] = geglu_scalar(g0, u0);
  h[1] = geglu_scalar(g1, u1);
  // rows of h[e]: 4 lq + 2 hi + e; their 8 columns of this wave are one
  // aligned group of 8 lanes
  const int rbase = 4 * lq + (hi ? 2 : 0);
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const float v = max8_nonneg(fmaxf(0.0f, fabsf(h[e])));
    if ((l16 & 7) == 0) amax_w[wave][rbase + e] = v;
  }
  __syncthreads();
  // lane 8 k + e' of a group derives the scale of row rbase + (e' & 1)
  const int rs = rbase + (l16 & 1);
  const QScale q =
      q8_scale(fmaxf(fmaxf(amax_w[0][rs], amax_w[1][rs]), fmaxf(amax_w[2][rs], amax_w[3][rs])));
  const float id0 = bcast8<0>(q.id), id1 = bcast8<1>(q.id);
  const int hc = hc0 + 8 * wave + (l16 & 7);
  const int nbh = F / QK;
  if (m0 + rbase < M) Hq[(int64_t)(m0 + rbase) * F + hc] = (int8_t)quant_round(h[0] * id0);
  if (m0 + rbase + 1 < M) Hq[(int64_t)(m0 + rbase + 1) * F + hc] = (int8_t)quant_round(h[1] * id1);
  if (wave == 0 && (l16 & 7) < 2 && m0 + rs < M) dH[(int64_t)(m0 + rs) * nbh + hb] = q.dq;
}

template <bool F2, int RING, int NB>
hipError_t run_geglu8_nb(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                         int8_t* hq, float* dh, int64_t M, int64_t F, hipStream_t s) {
  dim3 grid((unsigned)(F / QK), (unsigned)((M + 15) / 16));
  gemm_i8_geglu8_kernel<F2, RING, NB><<<grid, 256, 0, s>>>(xq, dx, wq, dw, hq, dh, (int)M,
                                                            (int)F);
  return hipGetLastError();
}

template <bool F2, int RING>
hipError_t run_geglu8(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                      int8_t* hq, float* dh, int64_t M, int64_t F, int64_t K, hipStream_t s) {
#define GLYPR_GEGLU8_NB(nb) \
  case nb:                  \
    return run_geglu8_nb<F2, RING, nb>(xq, dx, wq, dw, hq, dh, M, F, s);
  switch (K / QK) {
    GLYPR_GEGLU8_NB(4)
    GLYPR_GEGLU8_NB(8)
    GLYPR_GEGLU8_NB(12)
    GLYPR_GEGLU8_NB(16)
    GLYPR_GEGLU8_NB(20)
    GLYPR_GEGLU8_NB(24)
    GLYPR_GEGLU8_NB(28)
    GLYPR_GEGLU8_NB(32)
    GLYPR_GEGLU8_NB(36)
    GLYPR_GEGLU8_NB(48)
    GLYPR_GEGLU8_NB(64)
    default:
      return hipErrorInvalidValue;
  }
#undef GLYPR_GEGLU8_NB
}

// ---------------------------------------------------------------------------
// Small-M GEMM with the activation prologue fused (one launch per op): the
// workgroup reads its 16 rows of f32 x and builds their Q8_0 operand in LDS
// itself, while the weight stages stream in by LDS DMA.
//   PRO_QUANT: BlockQ8_0::from_float of x (QMatMul::forward's quantization);
//   PRO_NORM:  the same of RMSNorm(x; w) (RmsNorm::forward, then QMatMul).
// The prologue's arithmetic is the standalone kernels' (rmsnorm_row_kernel,
// quantize_planar_kernel) op for op, so the int8 operand and its scales are
// bit-identical to the two-launch path:
//  - chain lanes: lane j of a row runs the reference's FMA chain j over
//    x[8c + j] (c in order) straight from global memory, then the AVX2
//    horizontal sum ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)) and
//    inv = 1/sqrt(sum/K + eps);
//  - quantization: eight lanes per 32-block, four values each.
// Every workgroup along N repeats its rows' prologue, so the tile is wide
// (BN = 128 B rows on 4 waves) to keep that repetition at N/128.
// The int8 tile stays resident for the whole K range in the ring-slot layout
// (stage-major [stage][16 rows][128 B], XOR-swizzled chunks), so the MFMA
// operand reads are those of gemm_i8_small_kernel.
// Tiles are dealt to the XCDs in contiguous runs (xcd_tile): at the C2 shape
// each XCD takes whole M blocks, so the f32 rows that every N tile of a block
// re-reads come from one XCD's L2 instead of several (o projection at
// M = 512: 2.25x its algorithmic bytes from memory, against 3.63x with the N
// tiles of a block on different XCDs, at the same time per launch; cutting
// the grid into 4 x 2 XCD regions read 1.98x but took ~0.5 us longer).
// ---------------------------------------------------------------------------
enum { PRO_QUANT = 1, PRO_NORM = 2 };

template <int PRO, bool F2, int WN, int TNW, int RING, int NB>
__global__ void __launch_bounds__(WN * 64)
gemm_i8_pro_kernel(const float* __restrict__ X, const float* __restrict__ nw, float eps,
                   const int8_t* __restrict__ B, const float* __restrict__ dB,
                   float* __restrict__ C, int M, int N, int ldc, int nmajor) {
  constexpr int K = NB * QK, NST = NB / KB;
  constexpr int NW = WN, BM = 16;
  constexpr int BN = WN * 16 * TNW;
  constexpr int UB = BN / 8;               // 1 KB DMA units per stage
  constexpr int UPW = UB / NW;
  constexpr int SA = NB * BM, SB = NB * BN;
  constexpr int SLOT = BN * BK;
  constexpr int LPR = NW * 64 / BM;        // lanes per row in the prologue
  constexpr int PARTS = LPR / 8;           // 8-lane groups per row
  constexpr int BPP = NB / PARTS;          // blocks per group
  static_assert(NB % KB == 0 && NB <= SMALL_NB_MAX, "K must be a multiple of 128, <= 2048");
  static_assert(UB % NW == 0 && RING >= 2, "stage units must split evenly over the waves");
  static_assert(LPR >= 8 && LPR <= 64 && NB % PARTS == 0, "prologue lane layout");
  __shared__ __attribute__((aligned(16))) uint8_t ring[RING * SLOT];
  __shared__ __attribute__((aligned(16))) uint8_t ares[BM * K];
  __shared__ __attribute__((aligned(16))) float sc[SA + SB + 256];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave;
  int mi, ni;
  xcd_tile((M + BM - 1) / BM, (N + BN - 1) / BN, nmajor != 0, mi, ni);
  const int m0 = mi * BM;
  const int n0 = ni * BN;
  // B row of tile-local row nl (rows past N repeat the last one; never stored)
  auto b_row = [&](int nl) -> int { return n0 + nl < N ? n0 + nl : N - 1; };

  // ---- B scales [BN][NB] by DMA, 16 B (four blocks) per lane
  constexpr int NQ = NB / 4;
  constexpr int SCB = SB / 4;
  for (int c0 = wave * 64; c0 < SCB; c0 += NW * 64) {
    const int c = c0 + lane < SCB ? c0 + lane : SCB - 1;
    const int r = c / NQ, q = c - r * NQ;
    dma16_flat(dB + (int64_t)b_row(r) * NB + 4 * q, lds_u32(sc + SA + 4 * c0));
  }
  // ---- B stages: this wave's DMA units (8 rows x 128 B each)
  const int rsub = lane >> 3, pch = lane & 7;
  int uvoff[UPW];
#pragma unroll
  for (int j = 0; j < UPW; j++) {
    const int row = (j * NW + wave) * 8 + rsub;
    uvoff[j] = b_row(row) * K + ((pch ^ sm_swz(row)) << 4);
  }
  auto issue = [&](int st, int slot) {
#pragma unroll
    for (int j = 0; j < UPW; j++)
      dma16(B + st * BK, uvoff[j], lds_u32(ring + slot * SLOT + (j * NW + wave) * 1024));
  };
#pragma unroll
  for (int st = 0; st < RING - 1; st++)
    if (st < NST) issue(st, st);

  // ---- prologue: row pr of the tile on lanes [pr * LPR, pr * LPR + LPR);
  // 8-lane group `part` quantizes blocks [part * BPP, part * BPP + BPP).
  {
    const int pr = tid / LPR, pl = tid % LPR;
    const int pj = pl & 7, part = pl >> 3;
    const int gm = m0 + pr < M ? m0 + pr : M - 1;
    const float* xr = X + (int64_t)gm * K;
    // every operand of the lane is loaded before any is used: one memory
    // latency, not one per block (ones for a missing norm weight: x * 1 is x)
    constexpr bool NORM = PRO == PRO_NORM;
    v4f xv[BPP], wv[NORM ? BPP : 1];
#pragma unroll
    for (int i = 0; i < BPP; i++) {
      const int col = QK * (part * BPP + i) + 4 * pj;
      xv[i] = *reinterpret_cast<const v4f*>(xr + col);
      if constexpr (NORM)
        wv[i] = nw ? *reinterpret_cast<const v4f*>(nw + col) : v4f{1.0f, 1.0f, 1.0f, 1.0f};
    }
    float inv = 1.0f;
    if constexpr (NORM) {
      float acc = 0.0f;
      if (part == 0) {
#pragma unroll
        for (int c = 0; c < K / 8; c++) {
          const float e = xr[8 * c + pj];
          acc = fmaf(e, e, acc);
        }
      }
      const float s = acc + __shfl_down(acc, 4, 8);
      const float t = s + __shfl_down(s, 2, 8);
      const float sum = __shfl(t + __shfl_down(t, 1, 8), lane - pl);
      inv = 1.0f / sqrtf(sum / (float)K + eps);
    }
    // Blocks go in groups of up to 8.  The 8 lanes of a block hold the same
    // amax, so lane j derives the scale of block g0 + j once (two IEEE
    // divisions) and the group broadcasts the inverses, instead of every lane
    // dividing for every block.
#pragma unroll
    for (int g0 = 0; g0 < BPP; g0 += 8) {
      const int G = BPP - g0 < 8 ? BPP - g0 : 8;
      v4f yv[8];
      float am[8];
#pragma unroll
      for (int i = 0; i < G; i++) {
        yv[i] = xv[g0 + i];
        if constexpr (NORM) {
#pragma unroll
          for (int e = 0; e < 4; e++) yv[i][e] = (xv[g0 + i][e] * inv) * wv[g0 + i][e];
        }
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) a = fmaxf(a, fabsf(yv[i][e]));
        am[i] = max8_nonneg(a);
      }
      float asel = am[0];
#pragma unroll
      for (int i = 1; i < G; i++) asel = pj == i ? am[i] : asel;
      const QScale q = q8_scale(asel);
      if (pj < G) sc[pr * NB + part * BPP + g0 + pj] = q.dq;
#pragma unroll
      for (int i = 0; i < G; i++) {
        const float id = bcast8(q.id, i);
        uint32_t packed = 0;
#pragma unroll
        for (int e = 0; e < 4; e++)
          packed |= ((uint32_t)(quant_round(yv[i][e] * id) & 0xFF)) << (8 * e);
        const int col = QK * (part * BPP + g0 + i) + 4 * pj;
        const int st = col >> 7, qb = col & (BK - 1);
        *reinterpret_cast<uint32_t*>(ares + st * (BM * BK) + pr * BK +
                                     (((qb >> 4) ^ sm_swz(pr)) << 4) + (qb & 15)) = packed;
      }
    }
  }

  const int l16 = lane & 15, lq = lane >> 4;
  int offA[KB], offB[TNW][KB];
#pragma unroll
  for (int kb = 0; kb < KB; kb++) {
    const int ch = 2 * kb + (lq >> 1);
    offA[kb] = l16 * BK + ((ch ^ sm_swz(l16)) << 4) + ((lq & 1) << 3);
#pragma unroll
    for (int t = 0; t < TNW; t++) {
      const int brow = wn * 16 * TNW + t * 16 + l16;
      offB[t][kb] = brow * BK + ((ch ^ sm_swz(brow)) << 4) + ((lq & 1) << 3);
    }
  }
  const float* xrow = sc + (4 * lq) * NB;                    // row 4 lq + r at xrow + r NB
  const float* wrow = sc + SA + (wn * 16 * TNW + l16) * NB;  // tile t at wrow + 16 t NB
  const v4i magic = {MAGIC, MAGIC, MAGIC, MAGIC};
  float acc[TNW][4];
#pragma unroll
  for (int t = 0; t < TNW; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) acc[t][r] = 0.0f;

  // The prologue's own loads have all been consumed, so the DMA waits below
  // count only ring units.  The first barrier also publishes the prologue's
  // LDS writes.
#pragma unroll 1
  for (int g = 0; g < NST; g += RING) {
#pragma unroll
    for (int r = 0; r < RING; r++) {
      const int st = g + r;
      if (st < NST) {
        const int later = (st + RING - 2 < NST - 1 ? st + RING - 2 : NST - 1) - st;
        vm_wait_units<UPW, RING - 2>(later);
        __syncthreads();
        if (st + RING - 1 < NST) issue(st + RING - 1, (r + RING - 1) % RING);
        const uint8_t* slot = ring + r * SLOT;
        const uint8_t* aslot = ares + st * (BM * BK);
        v4i d[KB][TNW];
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
          const v1l af = *reinterpret_cast<const v1l*>(aslot + offA[kb]);
#pragma unroll
          for (int t = 0; t < TNW; t++) {
            const v1l bf = *reinterpret_cast<const v1l*>(slot + offB[t][kb]);
            d[kb][t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, bf, magic, 0, 0, 0);
          }
        }
        v4f xq[4], wq[TNW];
#pragma unroll
        for (int rr = 0; rr < 4; rr++)
          xq[rr] = *reinterpret_cast<const v4f*>(xrow + rr * NB + st * KB);
#pragma unroll
        for (int t = 0; t < TNW; t++)
          wq[t] = *reinterpret_cast<const v4f*>(wrow + t * 16 * NB + st * KB);
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
          for (int t = 0; t < TNW; t++) {
            const float wd = wq[t][kb];
            const float wc = wd * NEG_MAGIC;
#pragma unroll
            for (int rr = 0; rr < 4; rr++)
              acc[t][rr] = q8_term<F2>(acc[t][rr], d[kb][t][rr], wd, wc, xq[rr][kb]);
          }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const int grow0 = m0 + 4 * lq;
#pragma unroll
  for (int t = 0; t < TNW; t++) {
    const int gn = n0 + wn * 16 * TNW + t * 16 + l16;
#pragma unroll
    for (int r = 0; r < 4; r++)
      if (grow0 + r < M && gn < N) C[(int64_t)(grow0 + r) * ldc + gn] = acc[t][r];
  }
}

template <int PRO, bool F2, int WN, int TNW, int RING>
hipError_t run_pro(const float* x, const float* nw, float eps, const int8_t* wq, const float* dw,
                   float* y, int64_t M, int64_t N, int64_t K, int64_t ldc, hipStream_t s) {
  constexpr int BN = WN * 16 * TNW;
  const dim3 grid((unsigned)(((N + BN - 1) / BN) * ((M + 15) / 16)));
  // XCD order (xcd_tile): re-read the smaller of x as f32 (4 B per value) and
  // the weight as Q8_0 (1.125 B)
  const int nmajor = 4 * M * 8 < 9 * N ? 1 : 0;
#define GLYPR_PRO_NB(nb)                                                                  \
  case nb:                                                                                \
    gemm_i8_pro_kernel<PRO, F2, WN, TNW, RING, nb><<<grid, WN * 64, 0, s>>>(              \
        x, nw, eps, wq, dw, y, (int)M, (int)N, (int)ldc, nmajor);                         \
    break;
  switch (K / QK) {
    GLYPR_PRO_NB(4)
    GLYPR_PRO_NB(8)
    GLYPR_PRO_NB(12)
    GLYPR_PRO_NB(16)
    GLYPR_PRO_NB(20)
    GLYPR_PRO_NB(24)
    GLYPR_PRO_NB(28)
    GLYPR_PRO_NB(32)
    GLYPR_PRO_NB(36)
    default:
      return hipErrorInvalidValue;
  }
#undef GLYPR_PRO_NB
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Large-M variant (M > 2048: batched sequences, long contexts).  The exact
// epilogue (3 VALU ops per output and block) binds.  On gfx950 the MFMA pipe
// and the VALU do not overlap for this MFMA -> dependent-epilogue pattern, so
// the cost per output and block is (VALU ops + MFMA cycles): the kernel uses
// the full-rate v_mfma_i32_32x32x32_i8 (2 cycles per output and block, half
// of the 16x16x32 form).  Structure:
//  - 4 waves stacked along M; wave w owns rows 32w..32w+31 of a 128 x 128
//    tile and all 128 columns (4 MFMA tiles of 32 x 32, 64 accumulators);
//  - every stage (128 bytes of K = 4 blocks) arrives by LDS DMA into a
//    two-slot ring: A tile [128][128 B] and B tile [128][128 B] (16-byte
//    chunk c of row r at c ^ ((r >> 1) & 7): conflict-free ds_read_b128),
//    then the A and B scales of the stage as [block][row] f32 (dword DMA), so
//    the 16 row scales of a lane's 32 x 32 outputs are 4 ds_read_b128;
//    48 units, 12 per wave: "stage s has landed" is vmcnt(0) + barrier and
//    the next stage streams in under the current stage's compute;
//  - 2 workgroups per CU (72 KB LDS, <= 256 VGPRs each);
//  - the tile order is XCD-aware: the 8 XCDs get contiguous ranges of the
//    row-major tile list, so the tiles sharing an A row block share an L2.
// Rows past M/N are clamped to a valid row (their outputs are never stored).
//
// GEGLU: B rows of a tile are [gate c..c+31, up c..c+31, gate c+32..c+63,
// up c+32..c+63], so a Q8_0 block of h is one MFMA tile pair: the block amax
// is a 32-lane reduction, and each wave derives its 64 (row, block) scales one
// per lane through a per-wave LDS table instead of repeating the divisions.
// ---------------------------------------------------------------------------
constexpr int BIG_BM = 128, BIG_BN = 128;

__device__ __forceinline__ int big_swz(int row) { return (row >> 1) & 7; }

template <bool GEGLU, bool F2>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
gemm_i8_big_kernel(const int8_t* __restrict__ A, const float* __restrict__ dA,
                   const int8_t* __restrict__ B, const float* __restrict__ dB,
                   float* __restrict__ C, int8_t* __restrict__ Hq, float* __restrict__ dH,
                   int M, int N, int K, int ldc, int F, int tiles_n) {
  constexpr int NW = 4, TN = 4;
  constexpr int UA = BIG_BM / 8, UB = BIG_BN / 8;        // 1 KB operand units
  constexpr int USA = KB * BIG_BM / 64, USB = KB * BIG_BN / 64;   // 256 B scale units
  constexpr int NU = UA + UB + USA + USB;
  constexpr int UPW = NU / NW;
  constexpr int OFF_SA = (UA + UB) * 1024, OFF_SB = OFF_SA + KB * BIG_BM * 4;
  constexpr int SLOT = OFF_SB + KB * BIG_BN * 4;
  static_assert(NU % NW == 0 && (UA + UB) % NW == 0 && USA % NW == 0,
                "every unit index j must be of one kind across the waves");
  __shared__ __attribute__((aligned(16))) uint8_t ring[2 * SLOT];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware tile id: workgroup i runs on XCD i % 8 (the grid is exactly
  // the tile count, taken from the arguments rather than gridDim)
  const int nblk = ((M + BIG_BM - 1) / BIG_BM) * tiles_n, id = blockIdx.x;
  const int xq8 = nblk >> 3, xr8 = nblk & 7, xcd = id & 7;
  const int W = xcd * xq8 + (xcd < xr8 ? xcd : xr8) + (id >> 3);
  const int tmi = W / tiles_n;
  const int m0 = tmi * BIG_BM, n0 = (W - tmi * tiles_n) * BIG_BN;
  const int hc0 = n0 >> 1;
  const int nb = K / QK, nst = K / BK;

  auto b_row = [&](int nl) -> int {
    if (!GEGLU) return n0 + nl < N ? n0 + nl : N - 1;
    const int t = nl >> 5;
    int c = hc0 + (t >> 1) * 32 + (nl & 31);
    if (c >= F) c = F - 1;
    return (t & 1) ? F + c : c;
  };
  auto a_row = [&](int ml) -> int { return m0 + ml < M ? m0 + ml : M - 1; };

  // this wave's DMA units: uniform base + per-lane offset.  Unit u = 4 j + wave:
  // [0, UA) A rows, [UA, UA+UB) B rows (8 rows x 128 B, +128 B per stage),
  // then A scales and B scales (64 rows of one block, +16 B per stage).
  const int rsub = lane >> 3, pch = lane & 7;
  const int8_t* ubase[UPW];
  int uvoff[UPW];
#pragma unroll
  for (int j = 0; j < UPW; j++) {
    const int u = j * NW + wave;
    if (u < UA) {
      const int row = u * 8 + rsub;
      ubase[j] = A;
      uvoff[j] = a_row(row) * K + ((pch ^ big_swz(row)) << 4);
    } else if (u < UA + UB) {
      const int row = (u - UA) * 8 + rsub;
      ubase[j] = B;
      uvoff[j] = b_row(row) * K + ((pch ^ big_swz(row)) << 4);
    } else if (u < UA + UB + USA) {
      const int v = u - UA - UB, kb = v / (BIG_BM / 64);
      ubase[j] = reinterpret_cast<const int8_t*>(dA);
      uvoff[j] = (a_row((v % (BIG_BM / 64)) * 64 + lane) * nb + kb) * 4;
    } else {
      const int v = u - UA - UB - USA, kb = v / (BIG_BN / 64);
      ubase[j] = reinterpret_cast<const int8_t*>(dB);
      uvoff[j] = (b_row((v % (BIG_BN / 64)) * 64 + lane) * nb + kb) * 4;
    }
  }
  auto lds_unit = [&](int slot, int u) -> uint32_t {
    int off;
    if (u < UA + UB) off = u * 1024;
    else off = OFF_SA + (u - UA - UB) * 256;   // A then B scales, [block][row]
    return lds_u32(ring + slot * SLOT + off);
  };
  auto issue = [&](int st, int slot) {
#pragma unroll
    for (int j = 0; j < UPW; j++) {
      const int u = j * NW + wave;
      if (j * NW < UA + UB) dma16(ubase[j] + st * BK, uvoff[j], lds_unit(slot, u));
      else dma4(ubase[j] + st * KB * 4, uvoff[j], lds_unit(slot, u));
    }
  };
  issue(0, 0);

  const int lrow = lane & 31, lhalf = lane >> 5;
  const int arow = wave * 32 + lrow;
  // operand chunk of block kb: bytes 32 kb + 16 lhalf of the row
  int offA[KB], offB[KB];
#pragma unroll
  for (int kb = 0; kb < KB; kb++) {
    const int ch = 2 * kb + lhalf;
    offA[kb] = arow * BK + ((ch ^ big_swz(arow)) << 4);
    offB[kb] = (BIG_BM + lrow) * BK + ((ch ^ big_swz(lrow)) << 4);   // tile tn: + 32 tn rows
  }
  // A scales of rows 32 w + 8 g + 4 lhalf + (0..3): b128 g at + 32 g
  const int offX = OFF_SA + (wave * 32 + 4 * lhalf) * 4;
  const int offW = OFF_SB + lrow * 4;   // B scale of tile tn, block kb: + (kb * 128 + 32 tn) * 4
  v16i magic;
#pragma unroll
  for (int i = 0; i < 16; i++) magic[i] = MAGIC;
  float acc[TN][16];
#pragma unroll
  for (int tn = 0; tn < TN; tn++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[tn][r] = 0.0f;

  auto stage = [&](const uint8_t* slot) {
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      const v4i af = *reinterpret_cast<const v4i*>(slot + offA[kb]);
      v4f xv[4];
#pragma unroll
      for (int g = 0; g < 4; g++)
        xv[g] = *reinterpret_cast<const v4f*>(slot + offX + kb * BIG_BM * 4 + 32 * g);
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        const v4i bf = *reinterpret_cast<const v4i*>(slot + offB[kb] + 32 * BK * tn);
        const float wd = *reinterpret_cast<const float*>(slot + offW + (kb * BIG_BN + 32 * tn) * 4);
        const float wc = wd * NEG_MAGIC;
        const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, magic, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; r++)
          acc[tn][r] = q8_term<F2>(acc[tn][r], d[r], wd, wc, xv[r >> 2][r & 3]);
      }
    }
  };

#pragma unroll 1
  for (int st = 0; st < nst; st++) {
    const int r = st & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (st + 1 < nst) issue(st + 1, r ^ 1);
    stage(ring + r * SLOT);
  }

  // output rows of register r: 32 w + 8 (r >> 2) + 4 lhalf + (r & 3)
  const int row0 = m0 + wave * 32 + 4 * lhalf;
  if constexpr (!GEGLU) {
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
      const int gn = n0 + 32 * tn + lrow;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int gm = row0 + 8 * (r >> 2) + (r & 3);
        if (gm < M && gn < N) st_nt(&C[(int64_t)gm * ldc + gn], (float)acc[tn][r]);
      }
    }
  } else {
    // h block p (columns c + 32 p .. +31) of row (r, lhalf) is lane lrow's
    // value of geglu(acc[2p][r], acc[2p+1][r]).  Scale table per wave in the
    // ring slot of stage nst - 2, which every wave finished before the last
    // barrier: amax[lhalf][p][r], then (id, dq) per entry.
    const int nbh = F / QK;
    float* tab = reinterpret_cast<float*>(ring + (((nst - 1) & 1) ^ 1) * SLOT) + wave * 192;
    float h[2][16];
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        h[p][r] = geglu_scalar(acc[2 * p][r], acc[2 * p + 1][r]);
        const float v = max32_hi(fmaxf(0.0f, fabsf(h[p][r])));
        if (lrow == 31) tab[lhalf * 32 + p * 16 + r] = v;
      }
    // LDS serves a wave's accesses in order; the fences keep the compiler
    // from moving the table accesses across each other.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    {
      const QScale q = q8_scale(tab[lane]);
      tab[64 + lane] = q.id;
      tab[128 + lane] = q.dq;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int c = hc0;
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int hb = c + 32 * p;   // first column of the h block
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int gm = row0 + 8 * (r >> 2) + (r & 3);
        const int e = lhalf * 32 + p * 16 + r;
        if (gm < M && hb < F) {
          Hq[(int64_t)gm * F + hb + lrow] = (int8_t)quant_round(h[p][r] * tab[64 + e]);
          if (lrow == 0) dH[(int64_t)gm * nbh + (hb >> 5)] = tab[128 + e];
        }
      }
    }
  }
}

template <bool GEGLU, bool F2>
hipError_t run_big(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                   float* y, int8_t* hq, float* dh, int64_t M, int64_t Nrows, int64_t K,
                   int64_t ldc, int64_t F, hipStream_t s) {
  const int64_t tiles_n = (Nrows + BIG_BN - 1) / BIG_BN;
  const int64_t tiles = ((M + BIG_BM - 1) / BIG_BM) * tiles_n;
  gemm_i8_big_kernel<GEGLU, F2><<<dim3((unsigned)tiles), 256, 0, s>>>(
      xq, dx, wq, dw, y, hq, dh, (int)M, (int)Nrows, (int)K, (int)ldc, (int)F, (int)tiles_n);
  return hipGetLastError();
}

// The large-M kernel addresses operands with 32-bit offsets.
inline bool big_ok(int64_t M, int64_t Nrows, int64_t K) {
  return K % BK == 0 && M * K < (int64_t(1) << 31) && Nrows * K < (int64_t(1) << 31);
}

template <int BM, int BN, int WM, int WN, bool GEGLU, bool F2>
hipError_t run(const int8_t* xq,const float* dx, const int8_t* wq, const float* dw, float* y,
               int8_t* hq, float* dh, int64_t M, int64_t Nrows, int64_t K, int64_t ldc,
               int64_t F, hipStream_t s) {
  dim3 grid((unsigned)((Nrows + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  gemm_i8_kernel<BM, BN, WM, WN, GEGLU, F2><<<grid, WM * WN * 64, 0, s>>>(
      xq, dx, wq, dw, y, hq, dh, (int)M, (int)Nrows, (int)K, (int)ldc, (int)F);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The fused q|k|v projection with the attention prologue as its epilogue
// (SelfAttention::forward up to the attention itself, attention/mod.rs:
// 192-214 with the per-head RMSNorm and rope.rs:99-106): the small-M GEMM
// above, one workgroup per (16 tokens, head slot of 256 columns), 8 waves of
// 16 x 32 outputs, then the head's f32 tile is staged in LDS and turned into
// the attention operands exactly as qkv_post_kernel (k_attn.hip) does it:
//   q / k slots: RMSNorm over the head (eight FMA chains in the reference's
//     order), times q_norm / k_norm, RoPE x*cos + rot*sin with both products
//     rounded, f16 -> q [nq][Tp][256] / k [nkv][Tp][256];
//   v slots: weightless RMSNorm, f16 -> vt [nkv][256][Tp] (transposed);
//   rows that hold no token (past T, or past their sequence in a segment
//   table) are written as zeros.
// The f32 q|k|v rows never reach HBM and qkv_post's launch goes away.  Grid:
// (head slot, 16-row block of the Tp padded rows), the slots being the q
// heads, then the k heads, then the v heads.  Stage DMA: 2 A units and 32 B
// units per 128-byte K stage; wave w issues B units 4 w .. 4 w + 3 and waves
// 0 and 1 one A unit each.
// ---------------------------------------------------------------------------
constexpr int QKV_NW = 8;
constexpr int QKV_RING = 3;

template <bool F2, int NB>
__global__ void __launch_bounds__(QKV_NW * 64)
gemm_i8_qkv_kernel(const int8_t* __restrict__ A, const float* __restrict__ dA,
                   const int8_t* __restrict__ B, const float* __restrict__ dB, int T, int Tp,
                   int nq, int nkv, const float* __restrict__ qnw, const float* __restrict__ knw,
                   float eps, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                   _Float16* __restrict__ q16, _Float16* __restrict__ k16,
                   _Float16* __restrict__ vt16, const int2* __restrict__ seg) {
  constexpr int K = NB * QK, NST = NB / KB;
  constexpr int BM = 16, BN = QKV_HD, TNW = 2;
  constexpr int UA = BM / 8, UB = BN / 8;   // 2 and 32 units of 1 KB per stage
  constexpr int UBW = UB / QKV_NW;          // B units per wave
  constexpr int SA = NB * BM, SB = NB * BN;
  constexpr int SLOT = (BM + BN) * BK;
  static_assert(NB % KB == 0 && NB <= SMALL_NB_MAX, "K must be a multiple of 128, <= 2048");
  static_assert(UB % QKV_NW == 0 && UA <= QKV_NW && BM * QKV_SP * 4 <= SLOT, "layout");
  __shared__ __attribute__((aligned(16))) uint8_t ring[QKV_RING * SLOT];
  __shared__ __attribute__((aligned(16))) float sc[SA + SB + 256];
  __shared__ float sinv[BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave;
  // Workgroup i runs on XCD i % 8: each XCD takes a contiguous run of the
  // slot-major order, so it streams the weight rows of one or two head
  // slots rather than all of them.
  int rb, slot;
  xcd_tile(Tp / BM, nq + 2 * nkv, true, rb, slot);
  const int m0 = rb * BM;                 // first row (token) of the block
  const int n0 = slot * BN;
  const int M = T;                        // rows with activations

  // ---- scales: dA rows [BM][NB], then dB rows [BN][NB]
  constexpr int NQ = NB / 4;
  constexpr int SCH = (SA + SB) / 4;
  for (int c0 = wave * 64; c0 < SCH; c0 += QKV_NW * 64) {
    const int c = c0 + lane < SCH ? c0 + lane : SCH - 1;
    const float* src;
    if (c < SA / 4) {
      const int r = c / NQ, q = c - r * NQ;
      const int gm = m0 + r < M ? m0 + r : M - 1;
      src = dA + (int64_t)gm * NB + 4 * q;
    } else {
      const int f = c - SA / 4, r = f / NQ, q = f - r * NQ;
      src = dB + (int64_t)(n0 + r) * NB + 4 * q;
    }
    dma16_flat(src, lds_u32(sc + 4 * c0));
  }
  // ---- this wave's stage units: B units UA + UBW w .. (+ A unit w for w < UA)
  const int rsub = lane >> 3, pch = lane & 7;
  int boff[UBW];
#pragma unroll
  for (int j = 0; j < UBW; j++) {
    const int row = (UBW * wave + j) * 8 + rsub;
    boff[j] = (n0 + row) * K + ((pch ^ sm_swz(row)) << 4);
  }
  const bool has_a = wave < UA;
  int aoff;
  {
    const int row = (has_a ? wave : 0) * 8 + rsub;
    const int gm = m0 + row < M ? m0 + row : M - 1;
    aoff = gm * K + ((pch ^ sm_swz(row)) << 4);
  }
  auto issue = [&](int st, int sl) {
    uint8_t* base = ring + sl * SLOT;
    if (has_a) dma16(A + st * BK, aoff, lds_u32(base + wave * 1024));
#pragma unroll
    for (int j = 0; j < UBW; j++)
      dma16(B + st * BK, boff[j], lds_u32(base + (UA + UBW * wave + j) * 1024));
  };
#pragma unroll
  for (int st = 0; st < QKV_RING - 1; st++)
    if (st < NST) issue(st, st);

  const int l16 = lane & 15, lq = lane >> 4;
  int offA[KB], offB[TNW][KB];
#pragma unroll
  for (int kb = 0; kb < KB; kb++) {
    const int ch = 2 * kb + (lq >> 1);
    offA[kb] = l16 * BK + ((ch ^ sm_swz(l16)) << 4) + ((lq & 1) << 3);
#pragma unroll
    for (int t = 0; t < TNW; t++) {
      const int brow = wn * 16 * TNW + t * 16 + l16;
      offB[t][kb] = (BM + brow) * BK + ((ch ^ sm_swz(brow)) << 4) + ((lq & 1) << 3);
    }
  }
  const float* xrow = sc + (4 * lq) * NB;
  const float* wrow = sc + SA + (wn * 16 * TNW + l16) * NB;
  const v4i magic = {MAGIC, MAGIC, MAGIC, MAGIC};
  float acc[TNW][4];
#pragma unroll
  for (int t = 0; t < TNW; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) acc[t][r] = 0.0f;

  // q / k epilogue operands of this wave's rows 2 w, 2 w + 1 (dims 4 l ..):
  // the norm weight and the RoPE rows, loaded now so that their latency
  // passes under the K loop
  const bool qk_slot = slot < nq + nkv;
  v4f ep_w = {1.0f, 1.0f, 1.0f, 1.0f}, ep_cos[2], ep_sin[2];
  bool ep_valid[2];
  if (qk_slot) {
    const float* w = slot < nq ? qnw : knw;
    if (w) ep_w = *reinterpret_cast<const v4f*>(w + 4 * lane);
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int pos = seg_row_pos(seg, m0 + 2 * wave + k, T, &ep_valid[k]);
      ep_cos[k] = ep_valid[k] ? *reinterpret_cast<const v4f*>(cos_t + (int64_t)pos * QKV_HD + 4 * lane)
                              : v4f{0.0f, 0.0f, 0.0f, 0.0f};
      ep_sin[k] = ep_valid[k] ? *reinterpret_cast<const v4f*>(sin_t + (int64_t)pos * QKV_HD + 4 * lane)
                              : v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }

#pragma unroll 1
  for (int g = 0; g < NST; g += QKV_RING) {
#pragma unroll
    for (int r = 0; r < QKV_RING; r++) {
      const int st = g + r;
      if (st < NST) {
        const int later = (st + QKV_RING - 2 < NST - 1 ? st + QKV_RING - 2 : NST - 1) - st;
        if (has_a)
          vm_wait_units<UBW + 1, QKV_RING - 2>(later);
        else
          vm_wait_units<UBW, QKV_RING - 2>(later);
        __syncthreads();
        if (st + QKV_RING - 1 < NST) issue(st + QKV_RING - 1, (r + QKV_RING - 1) % QKV_RING);
        const uint8_t* sl = ring + r * SLOT;
        v4i d[KB][TNW];
#pragma unroll
        for (int kb = 0; kb < KB; kb++) {
          const v1l af = *reinterpret_cast<const v1l*>(sl + offA[kb]);
#pragma unroll
          for (int t = 0; t < TNW; t++) {
            const v1l bf = *reinterpret_cast<const v1l*>(sl + offB[t][kb]);
            d[kb][t] = __builtin_amdgcn_mfma_i32_16x16x32_i8(af, bf, magic, 0, 0, 0);
          }
        }
        v4f xq[4], wq[TNW];
#pragma unroll
        for (int rr = 0; rr < 4; rr++)
          xq[rr] = *reinterpret_cast<const v4f*>(xrow + rr * NB + st * KB);
#pragma unroll
        for (int t = 0; t < TNW; t++)
          wq[t] = *reinterpret_cast<const v4f*>(wrow + t * 16 * NB + st * KB);
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
          for (int t = 0; t < TNW; t++) {
            const float wd = wq[t][kb];
            const float wc = wd * NEG_MAGIC;
#pragma unroll
            for (int rr = 0; rr < 4; rr++)
              acc[t][rr] = q8_term<F2>(acc[t][rr], d[kb][t][rr], wd, wc, xq[rr][kb]);
          }
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();   // every wave is past its last ring read

  // ---- the head's f32 tile [16 rows][256] into LDS (ring slot 0)
  float* stg = reinterpret_cast<float*>(ring);
#pragma unroll
  for (int t = 0; t < TNW; t++)
#pragma unroll
    for (int r = 0; r < 4; r++)
      stg[(4 * lq + r) * QKV_SP + wn * 16 * TNW + t * 16 + l16] = acc[t][r];
  __syncthreads();

  // Reference-order 1/rms of staged row i, on lanes 8 c + j (chain j of the
  // row held by lane group c): every read ahead of the chain, DPP sum.
  auto row_inv = [&](int i) -> float {
    float e[QKV_HD / 8];
#pragma unroll
    for (int c = 0; c < QKV_HD / 8; c++) e[c] = stg[i * QKV_SP + 8 * c + (lane & 7)];
    __builtin_amdgcn_sched_barrier(0);
    float a = 0.0f;
#pragma unroll
    for (int c = 0; c < QKV_HD / 8; c++) a = fmaf(e[c], e[c], a);
    const float sum = hsum8_avx2(a);
    return 1.0f / sqrtf(sum / (float)QKV_HD + eps);   // valid on lanes 8 c
  };

  if (qk_slot) {
    // q / k: wave w handles rows 2 w and 2 w + 1; lane l holds dims 4 l .. 4 l + 3
    const bool is_q = slot < nq;
    const int head = is_q ? slot : slot - nq;
    const float* w = is_q ? qnw : knw;
    _Float16* outp = is_q ? q16 : k16;
    // lanes 0..7 run row 2 w's chains, lanes 8..15 row 2 w + 1's
    const float invp = row_inv(2 * wave + ((lane >> 3) & 1));
    const float inv0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(invp), 0));
    const float inv1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(invp), 8));
    const v4f wv = ep_w;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int i = 2 * wave + k;
      const int t = m0 + i;
      const bool valid = ep_valid[k];
      const float inv = k == 0 ? inv0 : inv1;
      const v4f x = *reinterpret_cast<const v4f*>(stg + i * QKV_SP + 4 * lane);
      float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (valid) {
#pragma unroll
        for (int e = 0; e < 4; e++) y[e] = w ? (x[e] * inv) * wv[e] : x[e] * inv;
        const v4f cv = ep_cos[k];
        const v4f sv = ep_sin[k];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          // lanes l and l ^ 32 hold dims d and d +- 128 (rotate_half's pairs)
          const float ye = y[e];
          const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(ye), __float_as_uint(ye),
                                                          false, false);
          const float rt = lane < 32 ? -__uint_as_float(p[1]) : __uint_as_float(p[0]);
          const float a = ye * cv[e];
          const float b = rt * sv[e];
          y[e] = a + b;
        }
      }
      typedef _Float16 h4 __attribute__((ext_vector_type(4)));
      const h4 yh = {(_Float16)y[0], (_Float16)y[1], (_Float16)y[2], (_Float16)y[3]};
      *reinterpret_cast<h4*>(outp + ((int64_t)head * Tp + t) * QKV_HD + 4 * lane) = yh;
    }
  } else {
    // v: the 16 rows' 1/rms first, then thread (dim d, token half) writes 8
    // consecutive tokens of vt row d as one 16-byte store
    const int head = slot - nq - nkv;
    const float invp = row_inv(2 * wave + ((lane >> 3) & 1));
    if (lane == 0) sinv[2 * wave] = invp;
    if (lane == 8) sinv[2 * wave + 1] = invp;
    __syncthreads();
    const int d = tid >> 1, th = tid & 1;
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 yh;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int i = 8 * th + j;
      bool valid;
      (void)seg_row_pos(seg, m0 + i, T, &valid);
      // the f32 product is rounded first, then converted (qkv_post's two
      // roundings): left free, the compiler folds multiply and conversion
      // into one v_fma_mixlo_f16, which rounds once
      float p = stg[i * QKV_SP + d] * sinv[i];
      asm volatile("" : "+v"(p));
      yh[j] = valid ? (_Float16)p : (_Float16)0.0f;
    }
    *reinterpret_cast<h8*>(vt16 + ((int64_t)head * QKV_HD + d) * Tp + m0 + 8 * th) = yh;
  }
}

template <bool F2, int NB>
hipError_t run_qkv_nb(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                      int64_t T, int64_t Tp, int64_t nq, int64_t nkv, const float* qnw,
                      const float* knw, float eps, const float* cos_t, const float* sin_t,
                      _Float16* q16, _Float16* k16, _Float16* vt16, const int2* seg,
                      hipStream_t s) {
  const unsigned grid = (unsigned)((nq + 2 * nkv) * (Tp / 16));
  gemm_i8_qkv_kernel<F2, NB><<<grid, QKV_NW * 64, 0, s>>>(
      xq, dx, wq, dw, (int)T, (int)Tp, (int)nq, (int)nkv, qnw, knw, eps, cos_t, sin_t, q16, k16,
      vt16, seg);
  return hipGetLastError();
}


// ---------------------------------------------------------------------------
// The fused q|k|v projection for many rows (Tp > 2048: long sequences and
// batches of sequences): the large-M kernel's main loop with the attention
// prologue as epilogue, as gemm_i8_qkv_kernel does it for few rows.  One
// workgroup per (128 tokens, head slot of 256 columns), 8 waves: wave w owns
// rows 32 (w & 3) .. +31 and columns 128 (w >> 2) .. +127 as 4 MFMA tiles of
// 32 x 32 (the large-M kernel's wave tile and exact epilogue); every 128-byte
// K stage arrives by LDS DMA into a two-slot ring (A [128][128 B], B
// [256][128 B], then the A and B scales as [block][row] f32).  After the loop
// the f32 tile goes through LDS in two halves of 64 rows, each turned into
// the attention operands exactly as qkv_post_kernel (k_attn.hip) does:
// RMSNorm over the head in the reference's chain order, q_norm / k_norm,
// RoPE with both products rounded, f16 (q, k) or transposed f16 (v); rows
// that hold no token are written as zeros, rows past Tp not at all.
// ---------------------------------------------------------------------------
// WMW waves along M (4 or 6: 128 or 192 rows), 2 along N; one workgroup per CU
// either way (110 or 126 KB of LDS), 2 or 3 waves per SIMD.
template <int WMW, bool F2>
__global__ void __launch_bounds__(WMW * 2 * 64) __attribute__((amdgpu_waves_per_eu(WMW / 2)))
gemm_i8_qkv_big_kernel(const int8_t* __restrict__ A, const float* __restrict__ dA,
                       const int8_t* __restrict__ B, const float* __restrict__ dB, int K, int T,
                       int Tp, int nq, int nkv, const float* __restrict__ qnw,
                       const float* __restrict__ knw, float eps, const float* __restrict__ cos_t,
                       const float* __restrict__ sin_t, _Float16* __restrict__ q16,
                       _Float16* __restrict__ k16, _Float16* __restrict__ vt16,
                       const int2* __restrict__ seg) {
  constexpr int NW = 2 * WMW, BM = 32 * WMW, BN = QKV_HD, TN = 4;
  constexpr int UA = BM / 8, UB = BN / 8;                  // 1 KB operand units
  constexpr int USA = KB * BM / 64, USB = KB * BN / 64;    // 256 B scale units
  constexpr int NU = UA + UB + USA + USB, UPW = NU / NW;
  static_assert(NU % NW == 0 && BM % 64 == 0, "stage units split evenly over the waves");
  constexpr int OFF_SA = (UA + UB) * 1024, OFF_SB = OFF_SA + KB * BM * 4;
  constexpr int SLOT = OFF_SB + KB * BN * 4;
  constexpr int HALF = BM / 2;                             // rows per epilogue pass
  static_assert(WMW == 4 || WMW == 6, "128 or 192 rows");
  static_assert(HALF * QKV_SP * 4 <= 2 * SLOT, "an epilogue half fits the ring");
  __shared__ __attribute__((aligned(16))) uint8_t ring[2 * SLOT];
  __shared__ float sinv[HALF];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WMW, wn = wave / WMW;
  const int slots = nq + 2 * nkv;
  // Workgroup i runs on XCD i % 8: each XCD takes a contiguous run of the
  // (row block, head slot) list, so the slots of a row block share its A rows
  // in one L2.
  int mi, slot;
  xcd_tile((Tp + BM - 1) / BM, slots, false, mi, slot);
  const int m0 = mi * BM, n0 = slot * BN;
  const int nb = K / QK, nst = K / BK;
  auto a_row = [&](int ml) -> int { return m0 + ml < T ? m0 + ml : T - 1; };

  // this wave's DMA units: unit u = NW j + wave (uniform per wave): [0, UA)
  // A rows, [UA, UA+UB) B rows (8 rows x 128 B, +128 B per stage), then the
  // A and B scales (64 rows of one block, +16 B per stage)
  const int rsub = lane >> 3, pch = lane & 7;
  const int8_t* ubase[UPW];
  int uvoff[UPW];
#pragma unroll
  for (int j = 0; j < UPW; j++) {
    const int u = j * NW + wave;
    if (u < UA) {
      const int row = u * 8 + rsub;
      ubase[j] = A;
      uvoff[j] = a_row(row) * K + ((pch ^ big_swz(row)) << 4);
    } else if (u < UA + UB) {
      const int row = (u - UA) * 8 + rsub;
      ubase[j] = B;
      uvoff[j] = (n0 + row) * K + ((pch ^ big_swz(row)) << 4);
    } else if (u < UA + UB + USA) {
      const int v = u - UA - UB, kb = v / (BM / 64);
      ubase[j] = reinterpret_cast<const int8_t*>(dA);
      uvoff[j] = (a_row((v % (BM / 64)) * 64 + lane) * nb + kb) * 4;
    } else {
      const int v = u - UA - UB - USA, kb = v / (BN / 64);
      ubase[j] = reinterpret_cast<const int8_t*>(dB);
      uvoff[j] = ((n0 + (v % (BN / 64)) * 64 + lane) * nb + kb) * 4;
    }
  }
  auto issue = [&](int st, int sl) {
#pragma unroll
    for (int j = 0; j < UPW; j++) {
      const int u = j * NW + wave;
      if (u < UA + UB)
        dma16(ubase[j] + st * BK, uvoff[j], lds_u32(ring + sl * SLOT + u * 1024));
      else
        dma4(ubase[j] + st * KB * 4, uvoff[j],
             lds_u32(ring + sl * SLOT + OFF_SA + (u - UA - UB) * 256));
    }
  };
  issue(0, 0);

  const int lrow = lane & 31, lhalf = lane >> 5;
  const int arow = wm * 32 + lrow;
  int offA[KB], offB[KB];
#pragma unroll
  for (int kb = 0; kb < KB; kb++) {
    const int ch = 2 * kb + lhalf;
    offA[kb] = arow * BK + ((ch ^ big_swz(arow)) << 4);
    // B row wn 128 + 32 tn + lrow: its swizzle depends on lrow only
    offB[kb] = (BM + wn * 128 + lrow) * BK + ((ch ^ big_swz(lrow)) << 4);
  }
  const int offX = OFF_SA + (wm * 32 + 4 * lhalf) * 4;
  const int offW = OFF_SB + (wn * 128 + lrow) * 4;   // tile tn, block kb: + (kb BN + 32 tn) 4
  v16i magic;
#pragma unroll
  for (int i = 0; i < 16; i++) magic[i] = MAGIC;
  float acc[TN][16];
#pragma unroll
  for (int tn = 0; tn < TN; tn++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[tn][r] = 0.0f;

#pragma unroll 1
  for (int st = 0; st < nst; st++) {
    const int r = st & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (st + 1 < nst) issue(st + 1, r ^ 1);
    const uint8_t* sl = ring + r * SLOT;
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      const v4i af = *reinterpret_cast<const v4i*>(sl + offA[kb]);
      v4f xv[4];
#pragma unroll
      for (int g = 0; g < 4; g++)
        xv[g] = *reinterpret_cast<const v4f*>(sl + offX + kb * BM * 4 + 32 * g);
#pragma unroll
      for (int tn = 0; tn < TN; tn++) {
        const v4i bf = *reinterpret_cast<const v4i*>(sl + offB[kb] + 32 * BK * tn);
        const float wd = *reinterpret_cast<const float*>(sl + offW + (kb * BN + 32 * tn) * 4);
        const float wc = wd * NEG_MAGIC;
        const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, magic, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 16; q++)
          acc[tn][q] = q8_term<F2>(acc[tn][q], d[q], wd, wc, xv[q >> 2][q & 3]);
      }
    }
  }
  __syncthreads();   // every wave is past its last ring read

  float* stg = reinterpret_cast<float*>(ring);
  static_assert(HALF == 8 * NW, "the epilogue takes 8 rows per wave");
#pragma unroll 1
  for (int hf = 0; hf < 2; hf++) {
    const int r0 = m0 + HALF * hf;   // first token of this half
    // the half's rows: waves wm / (WMW / 2) == hf stage theirs; register q of
    // tile tn is row 32 wm + 8 (q >> 2) + 4 lhalf + (q & 3), column
    // 128 wn + 32 tn + lrow
    if (wm / (WMW / 2) == hf) {
#pragma unroll
      for (int tn = 0; tn < TN; tn++)
#pragma unroll
        for (int q = 0; q < 16; q++)
          stg[(32 * (wm % (WMW / 2)) + 8 * (q >> 2) + 4 * lhalf + (q & 3)) * QKV_SP + wn * 128 +
              32 * tn + lrow] = acc[tn][q];
    }
    __syncthreads();
    qkv_epilogue_rows<NW>(stg, sinv, r0, T, Tp, slot, nq, nkv, qnw, knw, eps, cos_t, sin_t, q16,
                          k16, vt16, seg);
    __syncthreads();   // the half is consumed before the next one is staged
  }
}

template <bool F2>
hipError_t run_qkv_big(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                       int64_t K, int64_t T, int64_t Tp, int64_t nq, int64_t nkv,
                       const float* qnw, const float* knw, float eps, const float* cos_t,
                       const float* sin_t, _Float16* q16, _Float16* k16, _Float16* vt16,
                       const int2* seg, hipStream_t s) {
  // one workgroup per CU: pick the row block (128 or 192) whose rounds of 256
  // workgroups take the fewest rows per CU (8192 rows: 320 blocks of 128 are
  // two rounds, 215 of 192 one)
  const int64_t slots = nq + 2 * nkv;
  auto cost = [&](int64_t bm) { return ((Tp + bm - 1) / bm * slots + 255) / 256 * bm; };
  if (cost(192) < cost(128)) {
    const unsigned grid = (unsigned)(slots * ((Tp + 191) / 192));
    gemm_i8_qkv_big_kernel<6, F2><<<grid, 768, 0, s>>>(xq, dx, wq, dw, (int)K, (int)T, (int)Tp,
                                                   (int)nq, (int)nkv, qnw, knw, eps, cos_t, sin_t,
                                                   q16, k16, vt16, seg);
  } else {
    const unsigned grid = (unsigned)(slots * ((Tp + 127) / 128));
    gemm_i8_qkv_big_kernel<4, F2><<<grid, 512, 0, s>>>(xq, dx, wq, dw, (int)K, (int)T, (int)Tp,
                                                   (int)nq, (int)nkv, qnw, knw, eps, cos_t, sin_t,
                                                   q16, k16, vt16, seg);
  }
  return hipGetLastError();
}

}  // namespace

int gemm_i8_route(int64_t M, int64_t Nrows, int64_t K) {
  if (small_ok(M, Nrows, K)) return GEMM_ROUTE_SMALL;
  if (big_ok(M, Nrows, K)) return GEMM_ROUTE_BIG;
  return ((M + 127) / 128) * ((Nrows + 127) / 128) >= 512 ? GEMM_ROUTE_REG128 : GEMM_ROUTE_REG64;
}

namespace {

template <bool F2>
hipError_t gemm_i8_routed(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                          float* y, int64_t M, int64_t N, int64_t K, int64_t ldc,
                          hipStream_t s) {
  switch (gemm_i8_route(M, N, K)) {
    case GEMM_ROUTE_SMALL:
      return run_small<1, 2, 1, false, F2, 3>(xq, dx, wq, dw, y, nullptr, nullptr, M, N, K, ldc,
                                              0, s);
    case GEMM_ROUTE_BIG:
      return run_big<false, F2>(xq, dx, wq, dw, y, nullptr, nullptr, M, N, K, ldc, 0, s);
    case GEMM_ROUTE_REG128:
      return run<128, 128, 2, 2, false, F2>(xq, dx, wq, dw, y, nullptr, nullptr, M, N, K, ldc, 0,
                                            s);
    default:
      return run<64, 64, 2, 2, false, F2>(xq, dx, wq, dw, y, nullptr, nullptr, M, N, K, ldc, 0, s);
  }
}

template <bool F2>
hipError_t geglu_i8_routed(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                           int8_t* hq, float* dh, int64_t M, int64_t F, int64_t K,
                           hipStream_t s) {
  switch (gemm_i8_route(M, 2 * F, K)) {
    case GEMM_ROUTE_SMALL:
      if (F % QK == 0) return run_geglu8<F2, 2>(xq, dx, wq, dw, hq, dh, M, F, K, s);
      return run_small<2, 2, 2, true, F2, 3>(xq, dx, wq, dw, nullptr, hq, dh, M, 2 * F, K, 0, F,
                                             s);
    case GEMM_ROUTE_BIG:
      return run_big<true, F2>(xq, dx, wq, dw, nullptr, hq, dh, M, 2 * F, K, 0, F, s);
    case GEMM_ROUTE_REG128:
      return run<128, 128, 2, 2, true, F2>(xq, dx, wq, dw, nullptr, hq, dh, M, 2 * F, K, 0, F, s);
    default:
      return run<64, 128, 2, 2, true, F2>(xq, dx, wq, dw, nullptr, hq, dh, M, 2 * F, K, 0, F, s);
  }
}

}  // namespace

hipError_t launch_gemm_i8(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                          float* y, int64_t M, int64_t N, int64_t K, int64_t ldc, hipStream_t s,
                          bool fma2) {
  if (M == 0 || N == 0) return hipSuccess;
  return fma2 ? gemm_i8_routed<true>(xq, dx, wq, dw, y, M, N, K, ldc, s)
              : gemm_i8_routed<false>(xq, dx, wq, dw, y, M, N, K, ldc, s);
}

// Few rows: the small-M form (16-row blocks); many rows, or a K the small
// form is not built for: the large-M form (128-row blocks, runtime K).
static bool qkv_small_ok(int64_t Tp, int64_t K) {
  const int64_t nb = K / QK;
  return Tp <= SMALL_M_MAX && (nb == 16 || nb == 24 || nb == 32 || nb == 36);
}

bool gemm_i8_qkv_ok(int64_t T, int64_t Tp, int64_t K, int64_t hd) {
  return hd == QKV_HD && Tp % 64 == 0 && Tp >= T && T > 0 && K > 0 && K % BK == 0 &&
         (qkv_small_ok(Tp, K) || T * K < (int64_t(1) << 31));
}

namespace {

template <bool F2>
hipError_t qkv_routed(const int8_t* xq, const float* dx, const int8_t* wq, const float* dw,
                      int64_t T, int64_t Tp, int64_t K, int64_t nq, int64_t nkv, const float* qnw,
                      const float* knw, float eps, const float* cos_t, const float* sin_t,
                      _Float16* q, _Float16* k, _Float16* v, const int2* sg, hipStream_t s) {
  if (!qkv_small_ok(Tp, K))
    return run_qkv_big<F2>(xq, dx, wq, dw, K, T, Tp, nq, nkv, qnw, knw, eps, cos_t, sin_t, q, k,
                           v, sg, s);
  switch (K / QK) {
    case 16:
      return run_qkv_nb<F2, 16>(xq, dx, wq, dw, T, Tp, nq, nkv, qnw, knw, eps, cos_t, sin_t, q, k,
                                v, sg, s);
    case 24:
      return run_qkv_nb<F2, 24>(xq, dx, wq, dw, T, Tp, nq, nkv, qnw, knw, eps, cos_t, sin_t, q, k,
                                v, sg, s);
    case 32:
      return run_qkv_nb<F2, 32>(xq, dx, wq, dw, T, Tp, nq, nkv, qnw, knw, eps, cos_t, sin_t, q, k,
                                v, sg, s);
    case 36:
      return run_qkv_nb<F2, 36>(xq, dx, wq, dw, T, Tp, nq, nkv, qnw, knw, eps, cos_t, sin_t, q, k,
                                v, sg, s);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_gemm_i8_qkv(const int8_t* xq, const float* dx, const int8_t* wq,
                              const float* dw, int64_t T, int64_t Tp, int64_t K, int64_t nq,
                              int64_t nkv, int64_t hd, const float* qnw, const float* knw,
                              float eps, const float* cos_t, const float* sin_t, uint16_t* q16,
                              uint16_t* k16, uint16_t* vt16, const int32_t* seg, hipStream_t s,
                              bool fma2) {
  if (!gemm_i8_qkv_ok(T, Tp, K, hd) || (nq + 2 * nkv) * hd * K >= (int64_t(1) << 31))
    return hipErrorInvalidValue;
  _Float16* q = reinterpret_cast<_Float16*>(q16);
  _Float16* k = reinterpret_cast<_Float16*>(k16);
  _Float16* v = reinterpret_cast<_Float16*>(vt16);
  const int2* sg = reinterpret_cast<const int2*>(seg);
  return fma2 ? qkv_routed<true>(xq, dx, wq, dw, T, Tp, K, nq, nkv, qnw, knw, eps, cos_t, sin_t,
                                 q, k, v, sg, s)
              : qkv_routed<false>(xq, dx, wq, dw, T, Tp, K, nq, nkv, qnw, knw, eps, cos_t, sin_t,
                                  q, k, v, sg, s);
}

// The prologue is repeated by every workgroup along N, so fusing pays only
// while the saved launch outweighs that repetition (measured on MI355X at
// EmbeddingGemma widths: quantize up to M = 1024, RMSNorm up to M = 256).
bool gemm_i8_pro_ok(int64_t M, int64_t N, int64_t K, bool norm) {
  return small_ok(M, N, K) && K <= 1152 && M <= (norm ? 256 : 1024);
}

hipError_t launch_gemm_i8_pro(const float* x, const float* nw, float eps, bool norm,
                              const int8_t* wq, const float* dw, float* y, int64_t M, int64_t N,
                              int64_t K, int64_t ldc, hipStream_t s, bool fma2) {
  if (M == 0 || N == 0) return hipSuccess;
  if (!gemm_i8_pro_ok(M, N, K, norm)) return hipErrorInvalidValue;
  if (fma2) {
    if (norm) return run_pro<PRO_NORM, true, 4, 2, 3>(x, nw, eps, wq, dw, y, M, N, K, ldc, s);
    return run_pro<PRO_QUANT, true, 4, 2, 3>(x, nullptr, 0.0f, wq, dw, y, M, N, K, ldc, s);
  }
  if (norm) return run_pro<PRO_NORM, false, 4, 2, 3>(x, nw, eps, wq, dw, y, M, N, K, ldc, s);
  return run_pro<PRO_QUANT, false, 4, 2, 3>(x, nullptr, 0.0f, wq, dw, y, M, N, K, ldc, s);
}

hipError_t launch_gemm_i8_geglu(const int8_t* xq, const float* dx, const int8_t* wq,
                                const float* dw, int8_t* hq, float* dh, int64_t M, int64_t F,
                                int64_t K, hipStream_t s, bool fma2) {
  if (M == 0 || F == 0) return hipSuccess;
  return fma2 ? geglu_i8_routed<true>(xq, dx, wq, dw, hq, dh, M, F, K, s)
              : geglu_i8_routed<false>(xq, dx, wq, dw, hq, dh, M, F, K, s);
}

}  // namespace glypr
