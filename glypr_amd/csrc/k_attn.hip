// k_attn.hip — the attention side of one encoder layer (backbone configs):
//   qkv_post: q/k/v RMSNorm per head (q_norm, k_norm, weightless v_norm), RoPE,
//             and the f16 Q / K / V^T operands the MFMA attention consumes;
//   attention: bidirectional GQA flash attention, scale 1.0, f32 softmax,
//             optional band mask |i - j| <= W (sliding layers).
// Head dims 256 and 512 (the released model's full-attention layers), one
// sequence or several at 64-aligned row offsets (a segment table).
//
// Reference semantics: SelfAttention::forward (attention/mod.rs:166-277):
// q/k/v projections -> per-head RMSNorm on [T, heads, hd] -> transpose ->
// apply_rotary_pos_emb (rope.rs:99-106: x*cos + rotate_half(x)*sin) ->
// repeat_kv -> StandardAttention / ChunkedSlidingAttention (softmax in f32 of
// q k^T + mask, no 1/sqrt(d) scale) -> context @ o_proj.
//
// Precision: Q, K, V and the probabilities P enter f16 MFMAs (2^-11 relative
// rounding each) with f32 accumulation; max, exp, sums and the final
// normalisation are f32.  The K and V roundings dominate: carrying Q and P in
// two f16 parts as well would cut the context error by only ~20 % at twice the
// MFMA work.
#include "device_common.hpp"
#include "internal.hpp"

namespace glypr {

namespace {
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 f16;

}  // namespace

// ---------------------------------------------------------------------------
// qkv_post, for head dims HD = 256 and 512 (DPL = HD / 64 dims per lane).
// q and k: one wave per (token, head slot); slots 0..nq-1 are q heads,
// nq..nq+nkv-1 k heads.  Lane l holds dims DPL l .. DPL l + DPL-1 and writes
// them as one 8- (HD 256) or 16-byte (HD 512) store.  v (the blocks after the
// q/k blocks): one wave per 4 consecutive tokens of a head, so each lane
// writes its DPL dims of the transposed vt as DPL 8-byte runs of 4 tokens; the
// same eight chains and horizontal sum per token, run by lanes 8 i + j (token
// i, chain j).  RMSNorm follows simd_rmsnorm_row_f32's order (eight FMA
// chains, chain j = dims j, j+8, ...; see k_norm.hip) so it is bit-exact with
// the CPU path; RoPE is x*cos + rot*sin with both products rounded (no FMA),
// rot = -x[i+HD/2] for i < HD/2 and x[i-HD/2] otherwise: lane l's partner is
// l ^ 32 for either HD.
// Outputs (token rows padded to Tp, padding zero-filled):
//   q [nq][Tp][HD], k [nkv][Tp][HD], vt [nkv][HD][Tp] (f16).
// ---------------------------------------------------------------------------
constexpr int QKV_V_TOK = 4;   // tokens per v wave (8 lanes each)
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

template <int HD>
struct QkvGeom {
  static constexpr int DPL = HD / 64;                        // dims per lane
  static constexpr int S = HD / 8 + 4;                       // chain stride (k_norm.hip)
  static constexpr int V_LDS = QKV_V_TOK * 8 * S;            // floats per v wave
  static constexpr int LDS = V_LDS > HD ? V_LDS : HD;        // per-wave staging
};

template <int HD>
__global__ void __launch_bounds__(256) qkv_post_kernel(
    const float* __restrict__ qkv, int T, int Tp, int nq, int nkv, const float* __restrict__ qnw,
    const float* __restrict__ knw, float eps, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, f16* __restrict__ q16,
    f16* __restrict__ k16, f16* __restrict__ vt16, int qk_blocks, const int2* __restrict__ seg) {
  using Gm = QkvGeom<HD>;
  constexpr int DPL = Gm::DPL;
  constexpr int NV4 = DPL / 4;   // float4s per lane
  __shared__ __attribute__((aligned(16))) float lds_rows[4][Gm::LDS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slots = nq + 2 * nkv;
  if ((int)blockIdx.x >= qk_blocks) {
    // v: wave = QKV_V_TOK consecutive tokens of one head; lane 8 i + j runs
    // chain j of token i from the chain-major LDS copy, then lane l stores dims
    // DPL l .. DPL l + DPL-1 of the tokens as DPL runs of vt rows.
    const int64_t vtask = (int64_t)((int)blockIdx.x - qk_blocks) * 4 + wave;
    const int per_head = Tp / QKV_V_TOK;
    if (vtask >= (int64_t)nkv * per_head) return;
    const int head = (int)(vtask / per_head), t0 = (int)(vtask % per_head) * QKV_V_TOK;
    constexpr int S = Gm::S;
    float* lv = lds_rows[wave];
    v4f x[QKV_V_TOK][NV4];
#pragma unroll
    for (int i = 0; i < QKV_V_TOK; i++) {
      const int t = t0 + i;
      bool valid;
      (void)seg_row_pos(seg, t, T, &valid);
#pragma unroll
      for (int c = 0; c < NV4; c++) {
        x[i][c] = valid ? *reinterpret_cast<const v4f*>(
                              qkv + (int64_t)t * slots * HD + (int64_t)(nq + nkv + head) * HD +
                              DPL * lane + 4 * c)
                        : v4f{0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int d = DPL * lane + 4 * c + k;   // chain d & 7, position d >> 3
          lv[i * 8 * S + (d & 7) * S + (d >> 3)] = x[i][c][k];
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    // lanes past 8 QKV_V_TOK repeat a staged token (their sums are unused)
    const int ti = (lane >> 3) % QKV_V_TOK;
    const v4f* src = reinterpret_cast<const v4f*>(lv + ti * 8 * S + (lane & 7) * S);
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < HD / 32; c++) {
      const v4f e = src[c];
      acc = fmaf(e[0], e[0], acc);
      acc = fmaf(e[1], e[1], acc);
      acc = fmaf(e[2], e[2], acc);
      acc = fmaf(e[3], e[3], acc);
    }
    const float sum = hsum8_avx2(acc);
    const float inv = 1.0f / sqrtf(sum / (float)HD + eps);   // valid on lanes 8 i
    v4h yh[DPL];
#pragma unroll
    for (int i = 0; i < QKV_V_TOK; i++) {
      const float inv_i = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), 8 * i));
#pragma unroll
      for (int e = 0; e < DPL; e++) yh[e][i] = (f16)(x[i][e / 4][e % 4] * inv_i);
    }
#pragma unroll
    for (int e = 0; e < DPL; e++)
      *reinterpret_cast<v4h*>(vt16 + ((int64_t)head * HD + DPL * lane + e) * Tp + t0) = yh[e];
    return;
  }
  const int qk_slots = nq + nkv;
  const int64_t task = (int64_t)blockIdx.x * 4 + wave;
  if (task >= (int64_t)Tp * qk_slots) return;
  const int t = (int)(task / qk_slots), slot = (int)(task % qk_slots);
  const int kind = slot < nq ? 0 : 1;
  const int head = kind == 0 ? slot : slot - nq;

  float y[DPL];
#pragma unroll
  for (int e = 0; e < DPL; e++) y[e] = 0.0f;
  bool valid;
  const int pos = seg_row_pos(seg, t, T, &valid);
  if (valid) {
    const float* src = qkv + (int64_t)t * (nq + 2 * nkv) * HD + (int64_t)slot * HD;
    v4f x[NV4];
    float* lrow = lds_rows[wave];
#pragma unroll
    for (int c = 0; c < NV4; c++) {
      x[c] = *reinterpret_cast<const v4f*>(src + DPL * lane + 4 * c);
      *reinterpret_cast<v4f*>(lrow + DPL * lane + 4 * c) = x[c];
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    // lanes 0..7 run the eight chains, every read issued before the chain
    float sum = 0.0f;
    if (lane < 8) {
      float e[HD / 8];
#pragma unroll
      for (int c = 0; c < HD / 8; c++) e[c] = lrow[8 * c + lane];
      __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the chain
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < HD / 8; c++) acc = fmaf(e[c], e[c], acc);
      sum = hsum8_avx2(acc);
    }
    sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sum), 0));
    const float inv = 1.0f / sqrtf(sum / (float)HD + eps);
    const float* w = kind == 0 ? qnw : knw;
#pragma unroll
    for (int c = 0; c < NV4; c++) {
      const v4f wv = w ? *reinterpret_cast<const v4f*>(w + DPL * lane + 4 * c) : v4f{1, 1, 1, 1};
#pragma unroll
      for (int e = 0; e < 4; e++) y[4 * c + e] = w ? (x[c][e] * inv) * wv[e] : x[c][e] * inv;
    }
#pragma unroll
    for (int c = 0; c < NV4; c++) {
      const v4f cv = *reinterpret_cast<const v4f*>(cos_t + (int64_t)pos * HD + DPL * lane + 4 * c);
      const v4f sv = *reinterpret_cast<const v4f*>(sin_t + (int64_t)pos * HD + DPL * lane + 4 * c);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        // v_permlane32_swap of y with itself: lanes < 32 get (own, lane + 32),
        // lanes >= 32 get (lane - 32, own)
        const float ye = y[4 * c + e];
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(ye), __float_as_uint(ye),
                                                        false, false);
        const float r = lane < 32 ? -__uint_as_float(p[1]) : __uint_as_float(p[0]);
        const float a = ye * cv[e];
        const float b = r * sv[e];
        y[4 * c + e] = a + b;
      }
    }
  }
  f16* out = (kind == 0 ? q16 : k16) + ((int64_t)head * Tp + t) * HD + DPL * lane;
#pragma unroll
  for (int c = 0; c < NV4; c++) {
    const v4h yh = {(f16)y[4 * c], (f16)y[4 * c + 1], (f16)y[4 * c + 2], (f16)y[4 * c + 3]};
    *reinterpret_cast<v4h*>(out + 4 * c) = yh;
  }
}

hipError_t launch_qkv_post(const float* qkv, int64_t T, int64_t Tp, int64_t nq, int64_t nkv,
                           int64_t hd, const float* qnw, const float* knw, float eps,
                           const float* cos_t, const float* sin_t, uint16_t* q16, uint16_t* k16,
                           uint16_t* vt16, hipStream_t s, const int32_t* seg) {
  if (Tp % 64 != 0) return hipErrorInvalidValue;
  const int64_t qk_blocks = (Tp * (nq + nkv) + 3) / 4;
  const int64_t v_blocks = (nkv * (Tp / QKV_V_TOK) + 3) / 4;
  const unsigned grid = (unsigned)(qk_blocks + v_blocks);
  if (hd == 256)
    qkv_post_kernel<256><<<grid, 256, 0, s>>>(
        qkv, (int)T, (int)Tp, (int)nq, (int)nkv, qnw, knw, eps, cos_t, sin_t,
        reinterpret_cast<f16*>(q16), reinterpret_cast<f16*>(k16), reinterpret_cast<f16*>(vt16),
        (int)qk_blocks, reinterpret_cast<const int2*>(seg));
  else if (hd == 512)
    qkv_post_kernel<512><<<grid, 256, 0, s>>>(
        qkv, (int)T, (int)Tp, (int)nq, (int)nkv, qnw, knw, eps, cos_t, sin_t,
        reinterpret_cast<f16*>(q16), reinterpret_cast<f16*>(k16), reinterpret_cast<f16*>(vt16),
        (int)qk_blocks, reinterpret_cast<const int2*>(seg));
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Flash attention, split over keys.
// attn_partial: block = (16 AQS-query block, key partition, kv group) with
//   AQS x G waves: wave (qs, hh) owns queries q0 + 16 qs .. +15 of q head
//   g G + hh, so every K/V tile staged in LDS serves 16 AQS queries of all G
//   heads of the group (GQA).  K/V tiles (32 keys) stream through a three-slot LDS
//   ring filled by LDS DMA (global_load_lds_dwordx4 from inline asm, so the
//   compiler adds no vmcnt waits of its own).
//   Transposed formulation: S^T = K Q^T and O^T = V^T P^T with
//   v_mfma_f32_16x16x32_f16, so a lane owns ONE query (q0 + 16 qs + l16) in S,
//   P and O: its running max and sum are scalars, the key reductions need two
//   shuffles (lanes l16 + 16 lq'), and P^T goes from the S^T accumulator
//   straight into the B operand of the PV product.  Row m of S^T tile kt is
//   key 8 (m / 4) + 4 kt + m % 4, so the lane's 8 probabilities (tile kt, r)
//   are keys 8 lq + 4 kt + r: one contiguous 16-byte chunk of a V^T row is the
//   matching A operand.  The S^T of tile kb+1 is issued before the softmax of
//   tile kb so the MFMA pipe and the VALU overlap.  Each partition writes its
//   running max m, sum l and unnormalised O for its queries; with a single
//   partition the kernel writes the context itself and no combine runs.
// LDS layouts (16-byte chunks, conflict-free fragment reads):
//   K slot  [32 keys][256 dims]: chunk c of key row r at c ^ kswz(r);
//   V^T slot [256 dims][32 keys]: chunk c of dim row r at c ^ vswz(r).
// attn_combine: one wave per token merges the partitions per head,
//   ctx = sum_p e^{m_p - M} O_p / sum_p e^{m_p - M} l_p, and writes ctx as f32
//   and/or directly as the o projection's Q8_0 operand (BlockQ8_0::from_float).
// MFMA 16x16x32 layouts: A (16 x 32): lane l holds row l%16, k = 8(l/16)..+7;
// B (32 x 16): column l%16, same k; D (16 x 16): column l%16, rows 4(l/16)+r.
// ---------------------------------------------------------------------------
constexpr int AK = ATTN_AK;       // keys per tile
constexpr float ATTN_TAU = 8.0f;  // lazy-rescale threshold (natural log): p <= e^8 ~ 2981
constexpr float ATTN_LOG2E = 1.44269504f;
static_assert(ATTN_TP_ALIGN % 64 == 0, "query blocks (16 or 64) must tile the padded length");

typedef float v4f_ __attribute__((ext_vector_type(4)));

// Lane pairs (l, l ^ 16) and (l, l ^ 32) through gfx950's permlane swaps:
// v_permlane16_swap / v_permlane32_swap of a value with itself return, in
// every lane, the lane's own value and its partner's (in either order), all
// in VALU — no LDS round trip as with ds_bpermute.  max and + over the pair
// are order-independent, so each equals op(v, v[l ^ 16]) (resp. l ^ 32).
__device__ __forceinline__ float pair_max16(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float pair_max32(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float pair_sum16(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float pair_sum32(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// LDS swizzles (16-byte chunk c of row r is stored at chunk c ^ swz(r)),
// chosen by measurement: with them the fragment reads show no
// SQ_LDS_BANK_CONFLICT cycles.
// K rows are 512 B; the S^T tiles read rows 8 (l16 / 4) + 4 kt + l16 % 4.
__device__ __forceinline__ int kswz(int r) { return (r & 3) | ((r >> 1) & 12); }
// V^T rows are 64 B (4 chunks); the O^T tiles read rows 16 t + l16.  Of the
// row functions measured for these ds_read_b128 fragments (SQ_LDS_BANK_CONFLICT
// per read, rows 16 t + l16 for every t), (r >> 1) & 3 is the one with no
// conflict cycles; (r >> 1 ^ r >> 3) & 3, r & 3, (r >> 2) & 3 and no swizzle
// all cost ~4 cycles per read.
__device__ __forceinline__ int vswz(int r) { return (r >> 1) & 3; }

// HD = 512: the K and V^T tiles are 32 KB each, so the ring has two slots
// (128 KB) and each block is one 16-query row of waves (AQS = 1): the next
// tile's DMA overlaps the current tile's S^T, softmax and PV.
template <int HD, int G, int AQS>
__global__ void __launch_bounds__(G * AQS * 64) attn_partial_kernel(
    const f16* __restrict__ q16, const f16* __restrict__ kk, const f16* __restrict__ vt,
    float* __restrict__ part_o, float* __restrict__ part_ml, int T, int Tp, int nq, int nkv,
    int window, int kb_per_part, int kparts, const int2* __restrict__ seg,
    float* __restrict__ ctx, int8_t* __restrict__ cq, float* __restrict__ dc,
    uint16_t* __restrict__ cb) {
  static_assert(HD == 256 || HD == 512, "head dims 256 and 512");
  constexpr int NWV = G * AQS;
  constexpr int AQB = 16 * AQS;
  constexpr int RING = HD == 256 ? 3 : 2;
  constexpr int TILE_H = AK * HD;        // halves per K (or V^T) tile: 16 or 32 KB
  constexpr int KU = HD / 16;            // 1 KB DMA units per K tile (= per V^T tile)
  constexpr int UNITS = 2 * KU;
  constexpr int KLPR = HD / 8;           // lanes (16-byte chunks) per K row
  constexpr int KRPU = 64 / KLPR;        // K rows per unit
  __shared__ __attribute__((aligned(16))) f16 Ks[RING][TILE_H];
  __shared__ __attribute__((aligned(16))) f16 Vs[RING][TILE_H];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  const int hh = w % G, qs = w / G;
  // Blocks are dealt round-robin to the 8 XCDs (block id % 8).  Give each XCD
  // a contiguous run of work items W = (group, partition, query block), so the
  // K/V range one XCD streams (one partition, or the band of neighbouring
  // query blocks) stays in its L2.
  const int nqb = Tp / AQB;
  // the grid is the work items rounded up to a multiple of 8 (run_attention)
  const int n8 = (nkv * kparts * nqb + 7) / 8;
  const int W = (int)(blockIdx.x % 8) * n8 + (int)(blockIdx.x / 8);
  if (W >= nkv * kparts * nqb) return;   // grid padding (whole block)
  const int g = W / (kparts * nqb);
  const int kp = (W / nqb) % kparts;
  const int q0 = (W % nqb) * AQB;
  const int h = g * G + hh;
  const int qw = q0 + 16 * qs;   // this wave's first query
  const int qi = qw + l16;       // this lane's query
  // keys of this query block's sequence: [kstart, kend) (a segment table
  // places each sequence at a 64-aligned row offset; query blocks never
  // straddle two sequences)
  int kstart = 0, kend = T;
  if (seg) {
    const int2 sg = seg[q0];
    kstart = sg.x;
    kend = sg.x + sg.y;
  }
  const bool banded = window > 0 && kend - kstart > window;

  int kb_lo = kstart / AK, kb_hi = (kend + AK - 1) / AK;
  if (banded) {
    const int lo_key = q0 - window, hi_key = q0 + AQB - 1 + window;
    kb_lo = (lo_key > kstart ? lo_key : kstart) / AK;
    kb_hi = (hi_key < kend - 1 ? hi_key : kend - 1) / AK + 1;
  }
  const int kb0 = kb_lo + kp * kb_per_part;
  const int kb1 = kb0 + kb_per_part < kb_hi ? kb0 + kb_per_part : kb_hi;

  // Q fragments (B operand of S^T = K Q^T): query qi, dims 32 s + 8 lq .. +7
  v8h qf[HD / 32];
  {
    const int64_t off = ((int64_t)h * Tp + qi) * HD + 8 * lq;
#pragma unroll
    for (int s = 0; s < HD / 32; s++) qf[s] = *reinterpret_cast<const v8h*>(q16 + off + 32 * s);
  }

  const f16* kbase = kk + (int64_t)g * Tp * HD;
  const f16* vbase = vt + (int64_t)g * HD * Tp;
  // A tile is KU K units (KRPU key rows each) + KU V^T units (16 dim rows
  // each), 1 KB per unit; wave w issues units w, w + NWV, ...  Per-lane byte
  // offsets are fixed; the tile moves the (uniform) base.
  constexpr int UPWA = (UNITS + NWV - 1) / NWV;
  int uoff[UPWA];
#pragma unroll
  for (int j = 0; j < UPWA; j++) {
    const int u = w + NWV * j;
    if (u < KU) {
      const int row = KRPU * u + lane / KLPR, pc = lane % KLPR;
      uoff[j] = (row * HD + ((pc ^ kswz(row)) << 3)) * 2;
    } else {
      const int row = 16 * (u - KU) + (lane >> 2), pc = lane & 3;
      uoff[j] = (row * Tp + ((pc ^ vswz(row)) << 3)) * 2;
    }
  }
  auto issue = [&](int kb, int sl) {
    const int k0 = kb * AK;
    const f16* kb_base = kbase + (int64_t)k0 * HD;
    const f16* vb_base = vbase + k0;
#pragma unroll
    for (int j = 0; j < UPWA; j++) {
      const int u = w + NWV * j;
      if (u < UNITS) {
        const f16* dst = u < KU ? &Ks[sl][u * 512] : &Vs[sl][(u - KU) * 512];
        dma16(reinterpret_cast<const int8_t*>(u < KU ? kb_base : vb_base), uoff[j],
              lds_u32(dst));
      }
    }
  };

  float m_run = -INFINITY, l_run = 0.0f;
  v4f_ o[HD / 16];   // O^T: dims 16 t + 4 lq + r of query qi
#pragma unroll
  for (int t = 0; t < HD / 16; t++) o[t] = v4f_{0, 0, 0, 0};

  // S^T of the tile in slot sl: sacc[kt][r] = S[qi][k0 + 8 lq + 4 kt + r]
  auto scores = [&](int sl, v4f_ (&sacc)[2]) {
    const f16* Kt = Ks[sl];
    sacc[0] = v4f_{0, 0, 0, 0};
    sacc[1] = v4f_{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < HD / 32; s++) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        const int row = 8 * (l16 >> 2) + 4 * kt + (l16 & 3);
        const v8h kf = *reinterpret_cast<const v8h*>(Kt + row * HD +
                                                     (((4 * s + lq) ^ kswz(row)) << 3));
        sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[s], sacc[kt], 0, 0, 0);
      }
    }
  };

  // Softmax of one S^T tile (mask, lazy-rescaled online statistics) and
  // O^T += V^T P^T with the tile's V^T in slot sl.
  auto softmax_pv = [&](int kb, int sl, v4f_ (&sacc)[2]) {
    const f16* Vt = Vs[sl];
    const int k0 = kb * AK;
    // ---- mask (only where a key of the tile can be out of range or band)
    const bool edge = k0 + AK > kend ||
                      (banded && (k0 < q0 + AQB - 1 - window || k0 + AK - 1 > q0 + window));
    if (edge) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int key = k0 + 8 * lq + 4 * kt + r;
          bool ok = key < kend;
          if (banded) {
            const int d = qi - key;
            ok = ok && d <= window && -d <= window;
          }
          if (!ok) sacc[kt][r] = -INFINITY;
        }
    }
    // ---- online softmax for query qi
    float mx = fmaxf(fmaxf(fmaxf(sacc[0][0], sacc[0][1]), fmaxf(sacc[0][2], sacc[0][3])),
                     fmaxf(fmaxf(sacc[1][0], sacc[1][1]), fmaxf(sacc[1][2], sacc[1][3])));
    mx = pair_max32(pair_max16(mx));
    // Lazy rescaling: the reference max m_run moves only when a tile's max
    // exceeds it by more than ATTN_TAU (the first finite tile always moves
    // it), so p = e^{s - m_run} <= e^TAU fits f16 with its usual 2^-11
    // relative rounding, and the O rescale below runs on few tiles.  The
    // partition's (m, l, O) all refer to m_run; the combine is unchanged.
    const float m_new = mx > m_run + ATTN_TAU ? mx : m_run;
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __expf(m_run - m_use);   // exactly 1 while m_run holds
    v8h pf;   // P^T B operand: k-slot 4 kt + r = key 8 lq + 4 kt + r
    float ps = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float pv = __expf(sacc[kt][r] - m_use);
        ps += pv;
        pf[4 * kt + r] = (f16)pv;
      }
    ps = pair_sum32(pair_sum16(ps));
    l_run = l_run * alpha + ps;
    m_run = m_new;
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int t = 0; t < HD / 16; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) o[t][r] *= alpha;
    }
    // ---- O^T += V^T P^T: A = V^T[16 t + l16][keys 8 lq .. +7]
#pragma unroll
    for (int t = 0; t < HD / 16; t++) {
      const int row = 16 * t + l16;
      const v8h vf = *reinterpret_cast<const v8h*>(Vt + row * AK + ((lq ^ vswz(row)) << 3));
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf, o[t], 0, 0, 0);
    }
  };

  v4f_ sacc[2];
  if constexpr (RING == 3) {
    // Software pipeline over key tiles, slot = (kb - kb0) % 3: iteration kb
    // issues S^T of tile kb+1, runs the softmax of tile kb, then O^T += V^T P^T
    // for tile kb; tile kb+2 is in flight meanwhile.
    if (kb0 < kb1) issue(kb0, 0);
    if (kb0 + 1 < kb1) issue(kb0 + 1, 1);
    const int my_units = (UNITS - w + NWV - 1) / NWV;   // this wave's DMAs per tile
    if (kb0 < kb1) {
      if (kb0 + 1 >= kb1)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      else if (my_units == (UNITS + NWV - 1) / NWV)
        asm volatile("s_waitcnt vmcnt(%0)" :: "n"((UNITS + NWV - 1) / NWV) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(%0)" :: "n"(UNITS / NWV) : "memory");
      __syncthreads();
      scores(0, sacc);
    }
    for (int kb = kb0, sl = 0; kb < kb1; kb++, sl = sl == RING - 1 ? 0 : sl + 1) {
      const int sl1 = sl == RING - 1 ? 0 : sl + 1;
      v4f_ snext[2];
      if (kb + 1 < kb1) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // tile kb+1 has landed
        __syncthreads();   // ... for every wave; tile kb-1's slot is free
        if (kb + 2 < kb1) issue(kb + 2, sl == 0 ? RING - 1 : sl - 1);
        scores(sl1, snext);
      }
      softmax_pv(kb, sl, sacc);
      sacc[0] = snext[0];
      sacc[1] = snext[1];
    }
  } else {
    // Two slots: iteration kb waits for tile kb, then issues tile kb+1 into the
    // other slot (free: every wave has passed tile kb-1's PV, the barrier
    // says) and runs S^T, softmax and PV of tile kb under that DMA.
    if (kb0 < kb1) issue(kb0, 0);
    for (int kb = kb0, sl = 0; kb < kb1; kb++, sl ^= 1) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // tile kb has landed
      __syncthreads();
      if (kb + 1 < kb1) issue(kb + 1, sl ^ 1);
      scores(sl, sacc);
      softmax_pv(kb, sl, sacc);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if (kparts == 1) {
    // One partition: the combine's merge is the identity (weight e^0 = 1,
    // L = l, acc = O), so the context O / l is written here, in the
    // combine's arithmetic (one division, then per-value products), as f32
    // and / or the o projection's Q8_0 or bf16 operand; rows past T are not
    // outputs.  A Q8_0 block (32 dims: t = 2 b, 2 b + 1) spans the lanes
    // l16 + 16 lq of the query, two permlane swaps give its amax.
    const float inv = 1.0f / l_run;
    const bool live = qi < T;
    const int width = nq * HD;
    const int64_t rowoff = (int64_t)qi * width + (int64_t)h * HD;
#pragma unroll
    for (int t = 0; t < HD / 16; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) o[t][r] = o[t][r] * inv;
    if (ctx && live)
#pragma unroll
      for (int t = 0; t < HD / 16; t++)
        *reinterpret_cast<v4f_*>(ctx + rowoff + 16 * t + 4 * lq) = o[t];
    if (cb && live)
#pragma unroll
      for (int t = 0; t < HD / 16; t++) {
        uint32_t* dst = reinterpret_cast<uint32_t*>(cb + rowoff + 16 * t + 4 * lq);
#pragma unroll
        for (int e = 0; e < 2; e++)
          dst[e] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)o[t][2 * e]) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)o[t][2 * e + 1]) << 16);
      }
    if (cq) {
#pragma unroll
      for (int b = 0; b < HD / 32; b++) {
        float a = 0.0f;
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
          for (int r = 0; r < 4; r++) a = fmaxf(a, fabsf(o[2 * b + tt][r]));
        a = pair_max32(pair_max16(a));
        const QScale sc = q8_scale(a);
        if (live) {
#pragma unroll
          for (int tt = 0; tt < 2; tt++) {
            uint32_t packed = 0;
#pragma unroll
            for (int r = 0; r < 4; r++)
              packed |= ((uint32_t)(quant_round(o[2 * b + tt][r] * sc.id) & 0xFF)) << (8 * r);
            *reinterpret_cast<uint32_t*>(cq + rowoff + 16 * (2 * b + tt) + 4 * lq) = packed;
          }
          if (lq == 0) dc[(int64_t)qi * (width / QK) + (h * HD) / QK + b] = sc.dq;
        }
      }
    }
    return;
  }

  // ---- partial results: query qi, dims 16 t + 4 lq .. +3
  const int64_t prow = (int64_t)kp * Tp + qi;
#pragma unroll
  for (int t = 0; t < HD / 16; t++)
    *reinterpret_cast<v4f_*>(part_o + prow * nq * HD + (int64_t)h * HD + 16 * t + 4 * lq) =
        o[t];
  if (lq == 0) {
    part_ml[(prow * nq + h) * 2] = m_run;
    part_ml[(prow * nq + h) * 2 + 1] = l_run;
  }
}

// One wave per (token, head): merge the partitions in order p = 0, 1, ...;
// emit f32 ctx and/or the head's HD columns of the Q8_0 operand.  Lane p
// holds partition p's (m, l); readlane broadcasts them.  Lane l owns dims
// DPL l .. DPL l + DPL-1 (DPL = HD / 64), so a Q8_0 block is 32 / DPL lanes.
template <int HD>
__global__ void __launch_bounds__(256) attn_combine_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml, int T, int Tp, int nq,
    int kparts, float* __restrict__ ctx, int8_t* __restrict__ cq, float* __restrict__ dc,
    uint16_t* __restrict__ cb) {
  constexpr int DPL = HD / 64;
  const int lane = threadIdx.x & 63;
  const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (task >= (int64_t)T * nq) return;
  const int64_t q = task / nq;
  const int h = (int)(task % nq);
  const int width = nq * HD;
  float mp = -INFINITY, lp = 0.0f;
  if (lane < kparts) {
    const int64_t r = ((int64_t)lane * Tp + q) * nq + h;
    mp = part_ml[r * 2];
    lp = part_ml[r * 2 + 1];
  }
  float M = -INFINITY;
  for (int p = 0; p < kparts; p++)
    M = fmaxf(M, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mp), p)));
  const float wl = mp == -INFINITY ? 0.0f : __expf(mp - M);
  float L = 0.0f;
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; e++) acc[e] = 0.0f;
  const float* src = part_o + q * width + h * HD + DPL * lane;
  // partitions in batches of 8: the batch's loads are all in flight before
  // the first is used (one memory latency per batch, not per partition);
  // the sums still run in partition order
  constexpr int PB = 8;
  for (int p0 = 0; p0 < kparts; p0 += PB) {
    v4f v[PB][DPL / 4];
#pragma unroll
    for (int j = 0; j < PB; j++)
      if (p0 + j < kparts)
#pragma unroll
        for (int c = 0; c < DPL / 4; c++)
          v[j][c] = *reinterpret_cast<const v4f*>(src + (int64_t)(p0 + j) * Tp * width + 4 * c);
#pragma unroll
    for (int j = 0; j < PB; j++) {
      if (p0 + j >= kparts) break;
      const float wgt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), p0 + j));
      L += wgt * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lp), p0 + j));
#pragma unroll
      for (int c = 0; c < DPL / 4; c++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[4 * c + e] += wgt * v[j][c][e];
    }
  }
  const float inv = 1.0f / L;
  float y[DPL];
#pragma unroll
  for (int e = 0; e < DPL; e++) y[e] = acc[e] * inv;
  const int64_t col = (int64_t)h * HD + DPL * lane;
  if (ctx) {
#pragma unroll
    for (int c = 0; c < DPL / 4; c++)
      *reinterpret_cast<v4f*>(ctx + q * width + col + 4 * c) =
          v4f{y[4 * c], y[4 * c + 1], y[4 * c + 2], y[4 * c + 3]};
  }
  if (cb) {
    // bf16, round to nearest even (the dense-bf16 o projection's operand)
    uint32_t* dst = reinterpret_cast<uint32_t*>(cb + q * width + col);
#pragma unroll
    for (int e = 0; e < DPL / 2; e++)
      dst[e] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)y[2 * e]) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)y[2 * e + 1]) << 16);
  }
  if (cq) {
    float a = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; e++) a = fmaxf(a, fabsf(y[e]));
    a = DPL == 4 ? max8(a) : max4(a);
    QScale sc = q8_scale(a);
    uint32_t packed[DPL / 4];
#pragma unroll
    for (int c = 0; c < DPL / 4; c++) {
      packed[c] = 0;
#pragma unroll
      for (int e = 0; e < 4; e++)
        packed[c] |= ((uint32_t)(quant_round(y[4 * c + e] * sc.id) & 0xFF)) << (8 * e);
    }
#pragma unroll
    for (int c = 0; c < DPL / 4; c++)
      *reinterpret_cast<uint32_t*>(cq + q * width + col + 4 * c) = packed[c];
    if ((lane & (32 / DPL - 1)) == 0) dc[q * (width / QK) + (col >> 5)] = sc.dq;
  }
}

// ---------------------------------------------------------------------------
// Short single sequences: one launch, no key partitions, no combine.
// attn_short: block = (kv group g, 16-query block, DS-dim slice sl of the head
//   dims), eight waves, two per SIMD.  Each wave owns a contiguous eighth of
//   the block's keys and walks it in steps of 16 keys: S^T = K Q^T for all G
//   heads of the group (16 keys x 16 queries per head), the lazy online
//   softmax of attn_partial, and O^T += V^T P^T for the slice's DS dims with
//   v_mfma_f32_16x16x16_f16, whose B operand (keys 4 lq .. +3 of query l16)
//   is exactly the lane's S^T accumulator, so P needs no permutation.  The
//   eight waves' (m, l, O) merge through LDS in wave order (the combine's
//   arithmetic), and waves 0..G-1 write head hh's slice of the context:
//   DS / 32 whole Q8_0 blocks of the o projection's operand.
//   Every block reads the group's whole K (T x 512 B) but only DS / 256 of
//   V^T, and repeats the S^T products and the softmax once per slice: the
//   price of writing no f32 partials and running no second launch.  At
//   T = 512 with one kv head and 32-dim slices the grid is 32 query blocks x
//   8 slices = 256 blocks.
//   Operands reach registers through LDS: read straight from global memory
//   in the MFMA fragment layouts (neighbouring lanes on different 512-byte
//   rows) every lane is a cache access of its own, while LDS DMA moves 1 KB
//   of contiguous rows per instruction.  Each wave owns a two-slot ring
//   (16 keys of K, 8 KB, and of the slice's V^T) that only it fills and
//   reads, so the ring needs vmcnt waits but no barriers; the next step's
//   DMA is issued before the current step's fragments are read, and the
//   other wave of the SIMD runs while one waits.  The group's Q
//   (G x 16 rows x 512 B) is staged once in the first waves' second slots.
//   LDS rows of K and Q (512 B) hold 16-byte chunk c at c ^ (row % 16), so
//   the 16 rows a fragment read touches fall on distinct bank groups.
// ---------------------------------------------------------------------------
constexpr int ASH_WAVES = 8;
constexpr int ASH_KS = 16;                  // keys per step
constexpr int ASH_DS = 32;                  // head dims per slice (one Q8_0 block)
constexpr int64_t ATTN_SHORT_TP = 1024;     // padded lengths it runs up to
constexpr int ASH_KU = 8;                   // 1 KB K units per step (2 key rows each)
constexpr int ASH_SLOT_K = ASH_KS * 256 * 2;

typedef _Float16 v4h_ __attribute__((ext_vector_type(4)));

template <int G, int DS>
__global__ void __launch_bounds__(ASH_WAVES * 64) attn_short_kernel(
    const f16* __restrict__ q16, const f16* __restrict__ kk, const f16* __restrict__ vt, int T,
    int Tp, int nq, int nkv, int window, float* __restrict__ ctx, int8_t* __restrict__ cq,
    float* __restrict__ dc, uint16_t* __restrict__ cb) {
  constexpr int HD = 256;
  constexpr int NW = ASH_WAVES;
  constexpr int NSL = HD / DS;          // slices per head
  constexpr int NT = DS / 16;           // O^T tiles (16 dims) per slice
  constexpr int VU = DS / 32;           // 1 KB V^T units per step (32 dim rows of 32 B)
  constexpr int SLOT_V = DS * ASH_KS * 2;
  static_assert(G <= NW / 2, "the first G waves stage one head's Q each (in their second slot)");
  static_assert(DS % 32 == 0 && HD % DS == 0, "slices are whole Q8_0 blocks");
  // K ring [NW][2][8 KB], V^T ring [NW][2][DS x 32 B]; after the key loop
  // the K ring holds the merge buffers.
  __shared__ __attribute__((aligned(16))) char lds[NW * 2 * (ASH_SLOT_K + SLOT_V)];
  static_assert(NW * G * NT * 64 * 16 + 2 * NW * G * 16 * 4 <= NW * 2 * ASH_SLOT_K,
                "merge buffers fit the K ring");
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lq = lane >> 4;
  // one contiguous run of work items per XCD (block id % 8): neighbouring
  // query blocks and their slices, whose K/V ranges overlap, share an L2
  const int nqb = Tp / 16;
  // the grid is the work items rounded up to a multiple of 8 (run_attention)
  const int n8 = (nkv * nqb * NSL + 7) / 8;
  const int W = (int)(blockIdx.x % 8) * n8 + (int)(blockIdx.x / 8);
  if (W >= nkv * nqb * NSL) return;   // grid padding (whole block)
  const int g = W / (nqb * NSL);
  const int q0 = ((W / NSL) % nqb) * 16;
  const int sl = W % NSL;
  const int qi = q0 + l16;   // this lane's query
  const bool banded = window > 0 && T > window;
  int kb_lo = 0, kb_hi = (T + ASH_KS - 1) / ASH_KS;
  if (banded) {
    const int lo_key = q0 - window, hi_key = q0 + 15 + window;
    kb_lo = (lo_key > 0 ? lo_key : 0) / ASH_KS;
    kb_hi = (hi_key < T - 1 ? hi_key : T - 1) / ASH_KS + 1;
  }
  const int per = (kb_hi - kb_lo + NW - 1) / NW;
  const int kw0 = kb_lo + w * per;
  const int kw1 = kw0 + per < kb_hi ? kw0 + per : kb_hi;

  char* kring = lds + w * 2 * ASH_SLOT_K;
  char* vring = lds + NW * 2 * ASH_SLOT_K + w * 2 * SLOT_V;
  // DMA lane offsets.  K (and Q) unit u = rows 2u, 2u + 1 (lane: row
  // 2u + krow, 16-byte chunk kpc of the LDS row, fetched from global chunk
  // kpc ^ (row % 16) = (kpc ^ krow) ^ 2u): byte offset 1024 u (the unit's
  // base) + (kl ^ (2u << 4)).  V^T unit u = dim rows 32u .. 32u + 31 of the
  // slice, 16 keys (32 B) each (lane: row 32u + lane / 2, chunk lane % 2).
  const int krow = lane >> 5, kpc = lane & 31;
  const int kl = 512 * krow + ((kpc ^ krow) << 4);
  // V^T row r of a unit keeps its two 16-byte chunks swapped when bit 3 of r
  // is set (row 32 u + lane / 2: bit 3 is bit 4 of the lane), which keeps the
  // PV fragment reads below free of LDS bank-conflict cycles (measured; the
  // unswizzled rows cost ~2 cycles per ds_read_b64)
  const int vl = (lane >> 1) * Tp * 2 + (((lane & 1) ^ ((lane >> 4) & 1)) << 4);
  const f16* kbase = kk + (int64_t)g * Tp * HD;
  const f16* vbase = vt + ((int64_t)g * HD + DS * sl) * Tp;
  auto issue = [&](int kb, int slot) {
    const int8_t* kb_base = reinterpret_cast<const int8_t*>(kbase + (int64_t)kb * ASH_KS * HD);
    const int8_t* vb_base = reinterpret_cast<const int8_t*>(vbase + (int64_t)kb * ASH_KS);
#pragma unroll
    for (int u = 0; u < ASH_KU; u++)
      dma16(kb_base + 1024 * u, kl ^ (u << 5), lds_u32(kring + slot * ASH_SLOT_K + u * 1024));
#pragma unroll
    for (int u = 0; u < VU; u++)
      dma16(vb_base + (int64_t)64 * u * Tp, vl, lds_u32(vring + slot * SLOT_V + u * 1024));
  };

  // ---- Q of head w (w < G): 16 rows x 512 B into this wave's second K slot
  if (w < G) {
    const int8_t* qb_base =
        reinterpret_cast<const int8_t*>(q16 + ((int64_t)(g * G + w) * Tp + q0) * HD);
#pragma unroll
    for (int u = 0; u < ASH_KU; u++)
      dma16(qb_base + 1024 * u, kl ^ (u << 5), lds_u32(kring + ASH_SLOT_K + u * 1024));
  }
  if (kw0 < kw1) {
    issue(kw0, 0);
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(ASH_KU + VU) : "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  __syncthreads();   // every head's Q has landed
  // Q fragments (B operand of S^T = K Q^T): query qi of head g G + hh,
  // dims 32 s + 8 lq .. +7
  v8h qf[G][HD / 32];
#pragma unroll
  for (int hh = 0; hh < G; hh++) {
    const char* qs = lds + hh * 2 * ASH_SLOT_K + ASH_SLOT_K + l16 * 512;
#pragma unroll
    for (int s = 0; s < HD / 32; s++)
      qf[hh][s] = *reinterpret_cast<const v8h*>(qs + (((4 * s + lq) ^ l16) << 4));
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): Q is in registers
  __syncthreads();                      // ... in every wave: the second slots are free

  float m_run[G], l_run[G], thr[G], mlog[G];
  v4f_ o[G][NT];   // O^T: dims DS sl + 16 t + 4 lq + r of query qi
#pragma unroll
  for (int hh = 0; hh < G; hh++) {
    m_run[hh] = -INFINITY;
    thr[hh] = -INFINITY;
    mlog[hh] = 0.0f;
    l_run[hh] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; t++) o[hh][t] = v4f_{0, 0, 0, 0};
  }
  for (int kb = kw0, slot = 0; kb < kw1; kb++, slot ^= 1) {
    if (kb + 1 < kw1) {
      // the other slot's fragments were read (and used) in the previous step
      issue(kb + 1, slot ^ 1);
      asm volatile("s_waitcnt vmcnt(%0)" :: "n"(ASH_KU + VU) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    const char* ks = kring + slot * ASH_SLOT_K + l16 * 512;
    const char* vs = vring + slot * SLOT_V;
    // K fragments (A operand): key k0 + l16, dims 32 s + 8 lq .. +7
    v8h kf[HD / 32];
#pragma unroll
    for (int s = 0; s < HD / 32; s++)
      kf[s] = *reinterpret_cast<const v8h*>(ks + (((4 * s + lq) ^ l16) << 4));
    // V^T fragments (A operand of the 16x16x16 PV): dim rows 16 t + l16 of
    // the slice, keys 4 lq .. +3 of the step
    v4h_ vf[NT];
#pragma unroll
    for (int t = 0; t < NT; t++)
      vf[t] = *reinterpret_cast<const v4h_*>(vs + (16 * t + l16) * 32 +
                                             ((((lq >> 1) ^ (l16 >> 3)) << 4) | ((lq & 1) << 3)));
    // S^T: sacc[hh][r] = S[qi][k0 + 4 lq + r]
    v4f_ sacc[G];
#pragma unroll
    for (int hh = 0; hh < G; hh++) sacc[hh] = v4f_{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < HD / 32; s++)
#pragma unroll
      for (int hh = 0; hh < G; hh++)
        sacc[hh] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[s], qf[hh][s], sacc[hh], 0, 0, 0);
    const int k0 = kb * ASH_KS;
    const bool edge = k0 + ASH_KS > T ||
                      (banded && (k0 < q0 + 15 - window || k0 + ASH_KS - 1 > q0 + window));
    if (edge) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int key = k0 + 4 * lq + r;
        bool ok = key < T;
        if (banded) {
          const int d = qi - key;
          ok = ok && d <= window && -d <= window;
        }
#pragma unroll
        for (int hh = 0; hh < G; hh++)
          if (!ok) sacc[hh][r] = -INFINITY;
      }
    }
    // Online softmax for query qi of every head with attn_partial's lazy
    // rescale, made lane-local in the common case: m_run (the same in the
    // four lanes of a query) moves only when some S exceeds it by more than
    // ATTN_TAU, which a wave vote on each lane's own four values detects;
    // only then are the lanes' maxima reduced and O and l rescaled.  l is
    // kept per lane (the lane's own keys) and summed over the query's four
    // lanes after the loop.  P = 2^(S log2 e - m log2 e).
#pragma unroll
    for (int hh = 0; hh < G; hh++) {
      const float mloc = fmaxf(fmaxf(sacc[hh][0], sacc[hh][1]), fmaxf(sacc[hh][2], sacc[hh][3]));
      if (__any(mloc > thr[hh])) {
        const float mx = pair_max32(pair_max16(mloc));
        const float m_new = mx > thr[hh] ? mx : m_run[hh];
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __expf(m_run[hh] - m_use);
        l_run[hh] *= alpha;
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
          for (int r = 0; r < 4; r++) o[hh][t][r] *= alpha;
        m_run[hh] = m_new;
        thr[hh] = m_new + ATTN_TAU;
        mlog[hh] = m_use * ATTN_LOG2E;
      }
      v4h_ pf;   // P^T B operand: k-slot r = key 4 lq + r
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[hh][r], ATTN_LOG2E, -mlog[hh]));
        l_run[hh] += pv;
        pf[r] = (f16)pv;
      }
#pragma unroll
      for (int t = 0; t < NT; t++)
        o[hh][t] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf[t], pf, o[hh][t], 0, 0, 0);
    }
  }
#pragma unroll
  for (int hh = 0; hh < G; hh++) l_run[hh] = pair_sum32(pair_sum16(l_run[hh]));

  // ---- merge the eight waves' partial results (wave order), write the slice
  v4f_(*lo)[G][NT][64] = reinterpret_cast<v4f_(*)[G][NT][64]>(lds);
  float(*lm)[G][16] = reinterpret_cast<float(*)[G][16]>(lds + NW * G * NT * 64 * 16);
  float(*ll)[G][16] = lm + NW;
  __syncthreads();   // every wave is done with its ring
#pragma unroll
  for (int hh = 0; hh < G; hh++) {
#pragma unroll
    for (int t = 0; t < NT; t++) lo[w][hh][t][lane] = o[hh][t];
    if (lq == 0) {
      lm[w][hh][l16] = m_run[hh];
      ll[w][hh][l16] = l_run[hh];
    }
  }
  __syncthreads();
  if (w >= G) return;
  const int hh = w;
  float mw[NW];
  float M = -INFINITY;
#pragma unroll
  for (int v = 0; v < NW; v++) {
    mw[v] = lm[v][hh][l16];
    M = fmaxf(M, mw[v]);
  }
  float L = 0.0f;
  v4f_ acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) acc[t] = v4f_{0, 0, 0, 0};
#pragma unroll
  for (int v = 0; v < NW; v++) {
    const float wgt = mw[v] == -INFINITY ? 0.0f : __expf(mw[v] - M);
    L += wgt * ll[v][hh][l16];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const v4f_ ov = lo[v][hh][t][lane];
#pragma unroll
      for (int r = 0; r < 4; r++) acc[t][r] += wgt * ov[r];
    }
  }
  const float inv = 1.0f / L;
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int r = 0; r < 4; r++) acc[t][r] = acc[t][r] * inv;
  const bool live = qi < T;
  const int h = g * G + hh;
  const int width = nq * HD;
  const int64_t off = (int64_t)qi * width + (int64_t)h * HD + DS * sl + 4 * lq;
  if (ctx && live)
#pragma unroll
    for (int t = 0; t < NT; t++) *reinterpret_cast<v4f_*>(ctx + off + 16 * t) = acc[t];
  if (cb && live)
#pragma unroll
    for (int t = 0; t < NT; t++) {
      uint32_t* dst = reinterpret_cast<uint32_t*>(cb + off + 16 * t);
#pragma unroll
      for (int e = 0; e < 2; e++)
        dst[e] = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)acc[t][2 * e]) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)acc[t][2 * e + 1]) << 16);
    }
  if (cq) {
    // Q8_0 block b of the slice = tiles t = 2b, 2b + 1: lanes l16 + 16 lq
#pragma unroll
    for (int b = 0; b < NT / 2; b++) {
      float a = 0.0f;
#pragma unroll
      for (int tt = 0; tt < 2; tt++)
#pragma unroll
        for (int r = 0; r < 4; r++) a = fmaxf(a, fabsf(acc[2 * b + tt][r]));
      a = pair_max32(pair_max16(a));
      const QScale sc = q8_scale(a);
      if (live) {
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
          uint32_t packed = 0;
#pragma unroll
          for (int r = 0; r < 4; r++)
            packed |= ((uint32_t)(quant_round(acc[2 * b + tt][r] * sc.id) & 0xFF)) << (8 * r);
          *reinterpret_cast<uint32_t*>(cq + off + 16 * (2 * b + tt)) = packed;
        }
        if (lq == 0) dc[(int64_t)qi * (width / QK) + (h * HD + DS * sl) / QK + b] = sc.dq;
      }
    }
  }
}

template <int HD>
static hipError_t run_attention(const f16* q, const f16* k, const f16* v, float* scratch,
                                float* ctx, int8_t* cq, float* dc, int64_t T, int64_t Tp,
                                int64_t nq, int64_t nkv, int64_t window, hipStream_t s,
                                uint16_t* cb, const int2* seg, int64_t seg_max) {
  const int64_t G = nq / nkv;
  if (HD == 256 && !seg && Tp <= ATTN_SHORT_TP && G <= 3) {
    // one short sequence: the single-launch slice kernel
    const int64_t items = nkv * (Tp / 16) * (HD / ASH_DS);
    const unsigned grid = (unsigned)((items + 7) / 8 * 8);
#define GLYPR_ASH_CASE(GG)                                                                      \
  if (G == GG)                                                                                  \
    attn_short_kernel<GG, ASH_DS><<<grid, ASH_WAVES * 64, 0, s>>>(                              \
        q, k, v, (int)T, (int)Tp, (int)nq, (int)nkv, (int)window, ctx, cq, dc, cb);
    GLYPR_ASH_CASE(1) else GLYPR_ASH_CASE(2) else GLYPR_ASH_CASE(3)
#undef GLYPR_ASH_CASE
    return hipGetLastError();
  }
  const int64_t Tk = seg ? seg_max : T;   // the longest key range
  const int aqs = attn_qs(Tk, Tp, HD);
  int kparts;
  const int per = attn_kb_per_part(Tk, Tp, HD, nq, nkv, window, &kparts);
  if (kparts > 64) return hipErrorInvalidValue;   // the combine holds one partition per lane
  float* part_o = scratch;
  float* part_ml = scratch + (int64_t)kparts * Tp * nq * HD;
  const int64_t items = nkv * kparts * (Tp / (16 * aqs));
  const unsigned grid = (unsigned)((items + 7) / 8 * 8);
#define GLYPR_ATTN_CASE(GG, QS)                                                                  \
  if (G == GG && aqs == QS)                                                                      \
    attn_partial_kernel<HD, GG, QS><<<grid, GG * QS * 64, 0, s>>>(                               \
        q, k, v, part_o, part_ml, (int)T, (int)Tp, (int)nq, (int)nkv, (int)window, per, kparts, \
        seg, ctx, cq, dc, cb);
  if constexpr (HD == 256) {
    GLYPR_ATTN_CASE(1, 1) else GLYPR_ATTN_CASE(1, 4)
    else GLYPR_ATTN_CASE(2, 1) else GLYPR_ATTN_CASE(2, 4)
    else GLYPR_ATTN_CASE(3, 1) else GLYPR_ATTN_CASE(3, 4)
    else GLYPR_ATTN_CASE(4, 1) else GLYPR_ATTN_CASE(4, 4)
    else return hipErrorInvalidValue;
  } else {
    GLYPR_ATTN_CASE(1, 1) else GLYPR_ATTN_CASE(2, 1)
    else GLYPR_ATTN_CASE(3, 1) else GLYPR_ATTN_CASE(4, 1)
    else return hipErrorInvalidValue;
  }
#undef GLYPR_ATTN_CASE
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || kparts == 1) return e;   // one partition: the partial wrote ctx
  attn_combine_kernel<HD><<<(unsigned)((T * nq + 3) / 4), 256, 0, s>>>(
      part_o, part_ml, (int)T, (int)Tp, (int)nq, kparts, ctx, cq, dc, cb);
  return hipGetLastError();
}

hipError_t launch_attention(const uint16_t* q16, const uint16_t* k16, const uint16_t* vt16,
                            float* scratch, float* ctx, int8_t* cq, float* dc, int64_t T,
                            int64_t Tp, int64_t nq, int64_t nkv, int64_t hd, int64_t window,
                            hipStream_t s, uint16_t* cb, const int32_t* seg, int64_t seg_max) {
  if (Tp % ATTN_TP_ALIGN != 0 || Tp < T || nq % nkv != 0) return hipErrorInvalidValue;
  // the kernels' per-lane DMA offsets into V^T (row Tp + column, in bytes,
  // rows < hd) are 32-bit
  if (!attention_rows_ok(Tp, hd)) return hipErrorInvalidValue;
  if (seg && (seg_max <= 0 || seg_max > Tp)) return hipErrorInvalidValue;
  const f16* q = reinterpret_cast<const f16*>(q16);
  const f16* k = reinterpret_cast<const f16*>(k16);
  const f16* v = reinterpret_cast<const f16*>(vt16);
  const int2* sg = reinterpret_cast<const int2*>(seg);
  if (hd == 256)
    return run_attention<256>(q, k, v, scratch, ctx, cq, dc, T, Tp, nq, nkv, window, s, cb, sg,
                              seg_max);
  if (hd == 512)
    return run_attention<512>(q, k, v, scratch, ctx, cq, dc, T, Tp, nq, nkv, window, s, cb, sg,
                              seg_max);
  return hipErrorInvalidValue;
}

}  // namespace glypr
