// k_attn.hip — the attention side of one encoder layer (backbone configs):
//   qkv_post: q/k/v RMSNorm per head (q_norm, k_norm, weightless v_norm), RoPE,
//             and the f16 hi/lo split the MFMA attention consumes;
//   attention: bidirectional GQA flash attention, scale 1.0, f32 softmax,
//             optional band mask |i - j| <= W (sliding layers).
//
// Reference semantics: SelfAttention::forward (attention/mod.rs:166-277):
// q/k/v projections -> per-head RMSNorm on [T, heads, hd] -> transpose ->
// apply_rotary_pos_emb (rope.rs:99-106: x*cos + rotate_half(x)*sin) ->
// repeat_kv -> StandardAttention / ChunkedSlidingAttention (softmax in f32 of
// q k^T + mask, no 1/sqrt(d) scale) -> context @ o_proj.
//
// Precision: f16 MFMA with f32 accumulation.  Q and the probabilities P are
// split as x = hi + lo (hi = f16(x), lo = f16(x - hi)) and multiplied as
// hi*y + lo*y, so only K and V carry an f16 rounding (2^-11 relative); the
// context matches an f32 computation to ~1e-5 relative.
#include "device_common.hpp"
#include "internal.hpp"

namespace glypr {

namespace {
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 f16;

__device__ __forceinline__ void split_f16(float x, f16& hi, f16& lo) {
  hi = (f16)x;
  lo = (f16)(x - (float)hi);
}
}  // namespace

// ---------------------------------------------------------------------------
// qkv_post.  One wave per (token, head slot); slots 0..nq-1 are q heads,
// nq..nq+nkv-1 k heads, then nkv v heads.  hd == 256: lane l holds dims
// 4l..4l+3.  RMSNorm follows simd_rmsnorm_row_f32's order (eight FMA chains,
// lane j = dims j, j+8, ...; see k_norm.hip) so it is bit-exact with the CPU
// path; RoPE is x*cos + rot*sin with both products rounded (no FMA), rot =
// -x[i+128] for i < 128 and x[i-128] otherwise: lane l's partner is l ^ 32.
// Outputs (token rows padded to Tp, padding zero-filled):
//   q_hi/q_lo [nq][Tp][hd] (split), k [nkv][Tp][hd], vt [nkv][hd][Tp] (f16).
// ---------------------------------------------------------------------------
constexpr int QKV_HD = 256;

__global__ void __launch_bounds__(256) qkv_post_kernel(
    const float* __restrict__ qkv, int T, int Tp, int nq, int nkv, const float* __restrict__ qnw,
    const float* __restrict__ knw, float eps, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, f16* __restrict__ q_hi, f16* __restrict__ q_lo,
    f16* __restrict__ k16, f16* __restrict__ vt16) {
  __shared__ float lrows[4][QKV_HD];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slots = nq + 2 * nkv;
  const int64_t task = (int64_t)blockIdx.x * 4 + wave;
  if (task >= (int64_t)Tp * slots) return;
  const int t = (int)(task / slots), slot = (int)(task % slots);
  const int kind = slot < nq ? 0 : (slot < nq + nkv ? 1 : 2);
  const int head = kind == 0 ? slot : (kind == 1 ? slot - nq : slot - nq - nkv);

  v4f y = {0, 0, 0, 0};
  if (t < T) {
    const float* src = qkv + (int64_t)t * (nq + 2 * nkv) * QKV_HD + (int64_t)slot * QKV_HD;
    v4f x = *reinterpret_cast<const v4f*>(src + 4 * lane);
    float* lrow = lrows[wave];
    *reinterpret_cast<v4f*>(lrow + 4 * lane) = x;
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    float sum = 0.0f;
    if (lane < 8) {
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < QKV_HD / 8; c++) {
        float e = lrow[8 * c + lane];
        acc = fmaf(e, e, acc);
      }
      float s = acc + __shfl_down(acc, 4, 8);
      float u = s + __shfl_down(s, 2, 8);
      sum = u + __shfl_down(u, 1, 8);
    }
    sum = __shfl(sum, 0);
    const float inv = 1.0f / sqrtf(sum / (float)QKV_HD + eps);
    const float* w = kind == 0 ? qnw : (kind == 1 ? knw : nullptr);
    v4f wv = w ? *reinterpret_cast<const v4f*>(w + 4 * lane) : v4f{1, 1, 1, 1};
#pragma unroll
    for (int e = 0; e < 4; e++) y[e] = w ? (x[e] * inv) * wv[e] : x[e] * inv;
    if (kind < 2) {
      v4f c = *reinterpret_cast<const v4f*>(cos_t + (int64_t)t * QKV_HD + 4 * lane);
      v4f s = *reinterpret_cast<const v4f*>(sin_t + (int64_t)t * QKV_HD + 4 * lane);
      v4f r;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float partner = __shfl_xor(y[e], 32);
        r[e] = lane < 32 ? -partner : partner;
      }
#pragma unroll
      for (int e = 0; e < 4; e++) {
        float a = y[e] * c[e];
        float b = r[e] * s[e];
        y[e] = a + b;
      }
    }
  }
  if (kind == 0) {
    const int64_t off = ((int64_t)head * Tp + t) * QKV_HD + 4 * lane;
#pragma unroll
    for (int e = 0; e < 4; e++) split_f16(y[e], q_hi[off + e], q_lo[off + e]);
  } else if (kind == 1) {
    const int64_t off = ((int64_t)head * Tp + t) * QKV_HD + 4 * lane;
#pragma unroll
    for (int e = 0; e < 4; e++) k16[off + e] = (f16)y[e];
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++) vt16[((int64_t)head * QKV_HD + 4 * lane + e) * Tp + t] = (f16)y[e];
  }
}

hipError_t launch_qkv_post(const float* qkv, int64_t T, int64_t Tp, int64_t nq, int64_t nkv,
                           int64_t hd, const float* qnw, const float* knw, float eps,
                           const float* cos_t, const float* sin_t, uint16_t* q_hi, uint16_t* q_lo,
                           uint16_t* k16, uint16_t* vt16, hipStream_t s) {
  if (hd != QKV_HD) return hipErrorInvalidValue;
  const int64_t tasks = Tp * (nq + 2 * nkv);
  qkv_post_kernel<<<(unsigned)((tasks + 3) / 4), 256, 0, s>>>(
      qkv, (int)T, (int)Tp, (int)nq, (int)nkv, qnw, knw, eps, cos_t, sin_t,
      reinterpret_cast<f16*>(q_hi), reinterpret_cast<f16*>(q_lo), reinterpret_cast<f16*>(k16),
      reinterpret_cast<f16*>(vt16));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Flash attention, split over keys.
// attn_partial: block = (16-query block, key partition, kv group); one wave per
//   q head of the group, so the K/V tiles staged in LDS serve all of them
//   (GQA).  Per 32-key tile: S = Q K^T with v_mfma_f32_16x16x32_f16 (8 k-steps
//   x 2 key tiles x {q_hi, q_lo}), band/length mask, online softmax in f32,
//   P (split hi/lo) through LDS into the A-operand layout, O += P V (16 dim
//   tiles x {p_hi, p_lo}).  The next K/V tile is loaded into registers while the
//   current one is consumed (double buffering through registers, single LDS
//   buffer).  Each partition writes its running max m, sum l and unnormalised
//   O for its 16 queries.
// attn_combine: one wave per token merges the partitions per head,
//   ctx = sum_p e^{m_p - M} O_p / sum_p e^{m_p - M} l_p, and writes ctx as f32
//   and/or directly as the o projection's Q8_0 operand (BlockQ8_0::from_float).
// MFMA 16x16x32 layouts: A (16 x 32): lane l holds row l%16, k = 8(l/16)..+7;
// B (32 x 16): column l%16, same k; D (16 x 16): column l%16, rows 4(l/16)+r.
// ---------------------------------------------------------------------------
constexpr int AQ = 16;            // queries per block
constexpr int AK = 32;            // keys per tile
constexpr int KROW = QKV_HD + 8;  // padded K row in LDS (halves): 132 words, conflict-free
constexpr int VROW = AK + 8;      // padded V^T row in LDS (halves): 20 words
constexpr int PROW = AK + 8;

typedef float v4f_ __attribute__((ext_vector_type(4)));

template <int G>
__global__ void __launch_bounds__(G * 64) attn_partial_kernel(
    const f16* __restrict__ q_hi, const f16* __restrict__ q_lo, const f16* __restrict__ kk,
    const f16* __restrict__ vt, float* __restrict__ part_o, float* __restrict__ part_ml, int T,
    int Tp, int nq, int window, int kb_per_part) {
  __shared__ __attribute__((aligned(16))) f16 Ks[AK][KROW];
  __shared__ __attribute__((aligned(16))) f16 Vs[QKV_HD][VROW];
  __shared__ __attribute__((aligned(16))) f16 Ph[G][AQ][PROW];
  __shared__ __attribute__((aligned(16))) f16 Pl[G][AQ][PROW];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l16 = lane & 15, lq = lane >> 4;
  const int q0 = blockIdx.x * AQ;
  const int kp = blockIdx.y;
  const int g = blockIdx.z;
  const int h = g * G + w;
  const bool banded = window > 0 && T > window;

  int kb_lo = 0, kb_hi = (T + AK - 1) / AK;
  if (banded) {
    int lo_key = q0 - window, hi_key = q0 + AQ - 1 + window;
    kb_lo = lo_key > 0 ? lo_key / AK : 0;
    kb_hi = (hi_key < T - 1 ? hi_key : T - 1) / AK + 1;
  }
  const int kb0 = kb_lo + kp * kb_per_part;
  const int kb1 = kb0 + kb_per_part < kb_hi ? kb0 + kb_per_part : kb_hi;

  // Q fragments (A operand): row q0 + l16, dims 32s + 8 lq .. +7
  v8h qh[QKV_HD / 32], ql[QKV_HD / 32];
  {
    const int64_t off = ((int64_t)h * Tp + q0 + l16) * QKV_HD + 8 * lq;
#pragma unroll
    for (int s = 0; s < QKV_HD / 32; s++) {
      qh[s] = *reinterpret_cast<const v8h*>(q_hi + off + 32 * s);
      ql[s] = *reinterpret_cast<const v8h*>(q_lo + off + 32 * s);
    }
  }
  float m_run[4], l_run[4];
  v4f_ o[QKV_HD / 16];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < QKV_HD / 16; t++) o[t] = v4f_{0, 0, 0, 0};

  // K tile: 32 rows x 512 B = 1024 chunks; V^T tile: 256 rows x 64 B = 1024 chunks.
  constexpr int NCH = 2048;
  constexpr int PER = (NCH + G * 64 - 1) / (G * 64);
  const f16* kbase = kk + (int64_t)g * Tp * QKV_HD;
  const f16* vbase = vt + (int64_t)g * QKV_HD * Tp;
  v4i stage[PER];
  auto load_tile = [&](int kb) {
    const int k0 = kb * AK;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int c = tid + i * G * 64;
      if (c < 1024) {
        stage[i] = *reinterpret_cast<const v4i*>(kbase + (int64_t)(k0 + (c >> 5)) * QKV_HD +
                                                 ((c & 31) << 3));
      } else if (c < NCH) {
        const int cc = c - 1024;
        stage[i] = *reinterpret_cast<const v4i*>(vbase + (int64_t)(cc >> 2) * Tp + k0 +
                                                 ((cc & 3) << 3));
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int c = tid + i * G * 64;
      if (c < 1024) {
        *reinterpret_cast<v4i*>(&Ks[c >> 5][(c & 31) << 3]) = stage[i];
      } else if (c < NCH) {
        const int cc = c - 1024;
        *reinterpret_cast<v4i*>(&Vs[cc >> 2][(cc & 3) << 3]) = stage[i];
      }
    }
  };

  if (kb0 < kb1) load_tile(kb0);
  for (int kb = kb0; kb < kb1; kb++) {
    __syncthreads();  // previous tile fully consumed
    store_tile();
    __syncthreads();
    if (kb + 1 < kb1) load_tile(kb + 1);
    const int k0 = kb * AK;
    // ---- S = Q K^T: two 16-key tiles
    v4f_ sacc[2] = {v4f_{0, 0, 0, 0}, v4f_{0, 0, 0, 0}};
#pragma unroll
    for (int s = 0; s < QKV_HD / 32; s++) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        v8h kf = *reinterpret_cast<const v8h*>(&Ks[16 * kt + l16][32 * s + 8 * lq]);
        sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[s], kf, sacc[kt], 0, 0, 0);
        sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[s], kf, sacc[kt], 0, 0, 0);
      }
    }
    // ---- mask + online softmax; rows 4 lq + r, key = k0 + 16 kt + l16
    float alpha[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int qi = q0 + 4 * lq + r;
      float sv[2];
#pragma unroll
      for (int kt = 0; kt < 2; kt++) {
        const int key = k0 + 16 * kt + l16;
        bool ok = key < T;
        if (banded) {
          int d = qi - key;
          ok = ok && d <= window && -d <= window;
        }
        sv[kt] = ok ? sacc[kt][r] : -INFINITY;
      }
      float mx = fmaxf(sv[0], sv[1]);
      mx = fmaxf(mx, __shfl_xor(mx, 1));
      mx = fmaxf(mx, __shfl_xor(mx, 2));
      mx = fmaxf(mx, __shfl_xor(mx, 4));
      mx = fmaxf(mx, __shfl_xor(mx, 8));
      const float m_new = fmaxf(m_run[r], mx);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      alpha[r] = __expf(m_run[r] - m_use);
      const float p0 = __expf(sv[0] - m_use), p1 = __expf(sv[1] - m_use);
      float ps = p0 + p1;
      ps += __shfl_xor(ps, 1);
      ps += __shfl_xor(ps, 2);
      ps += __shfl_xor(ps, 4);
      ps += __shfl_xor(ps, 8);
      l_run[r] = l_run[r] * alpha[r] + ps;
      m_run[r] = m_new;
      split_f16(p0, Ph[w][4 * lq + r][l16], Pl[w][4 * lq + r][l16]);
      split_f16(p1, Ph[w][4 * lq + r][16 + l16], Pl[w][4 * lq + r][16 + l16]);
    }
#pragma unroll
    for (int t = 0; t < QKV_HD / 16; t++)
#pragma unroll
      for (int r = 0; r < 4; r++) o[t][r] *= alpha[r];
    // P was written by other lanes of this wave: LDS executes a wave's
    // accesses in order, so a compiler fence suffices (no s_waitcnt, which
    // would also wait for the next tile's prefetch).
    __builtin_amdgcn_wave_barrier();
    // ---- O += P V
    const v8h ah = *reinterpret_cast<const v8h*>(&Ph[w][l16][8 * lq]);
    const v8h al = *reinterpret_cast<const v8h*>(&Pl[w][l16][8 * lq]);
#pragma unroll
    for (int t = 0; t < QKV_HD / 16; t++) {
      v8h vf = *reinterpret_cast<const v8h*>(&Vs[16 * t + l16][8 * lq]);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, vf, o[t], 0, 0, 0);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, vf, o[t], 0, 0, 0);
    }
  }

  // ---- partial results
  const int64_t row0 = (int64_t)kp * Tp + q0 + 4 * lq;
#pragma unroll
  for (int t = 0; t < QKV_HD / 16; t++)
#pragma unroll
    for (int r = 0; r < 4; r++)
      part_o[(row0 + r) * nq * QKV_HD + (int64_t)h * QKV_HD + 16 * t + l16] = o[t][r];
  if (l16 == 0)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      part_ml[((row0 + r) * nq + h) * 2] = m_run[r];
      part_ml[((row0 + r) * nq + h) * 2 + 1] = l_run[r];
    }
}

// One wave per token: merge partitions per head; emit f32 ctx and/or Q8_0.
__global__ void __launch_bounds__(256) attn_combine_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml, int T, int Tp, int nq,
    int kparts, float* __restrict__ ctx, int8_t* __restrict__ cq, float* __restrict__ dc) {
  const int lane = threadIdx.x & 63;
  const int64_t q = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (q >= T) return;
  const int width = nq * QKV_HD;
  for (int h = 0; h < nq; h++) {
    float M = -INFINITY;
    for (int p = 0; p < kparts; p++) M = fmaxf(M, part_ml[(((int64_t)p * Tp + q) * nq + h) * 2]);
    float L = 0.0f;
    v4f acc = {0, 0, 0, 0};
    for (int p = 0; p < kparts; p++) {
      const int64_t r = (int64_t)p * Tp + q;
      const float mp = part_ml[(r * nq + h) * 2];
      const float wgt = mp == -INFINITY ? 0.0f : __expf(mp - M);
      L += wgt * part_ml[(r * nq + h) * 2 + 1];
      v4f v = *reinterpret_cast<const v4f*>(part_o + r * width + h * QKV_HD + 4 * lane);
#pragma unroll
      for (int e = 0; e < 4; e++) acc[e] += wgt * v[e];
    }
    const float inv = 1.0f / L;
    v4f y;
#pragma unroll
    for (int e = 0; e < 4; e++) y[e] = acc[e] * inv;
    const int64_t col = (int64_t)h * QKV_HD + 4 * lane;
    if (ctx) *reinterpret_cast<v4f*>(ctx + q * width + col) = y;
    if (cq) {
      float a = 0.0f;
#pragma unroll
      for (int e = 0; e < 4; e++) a = fmaxf(a, fabsf(y[e]));
      a = fmaxf(a, __shfl_xor(a, 1, 8));
      a = fmaxf(a, __shfl_xor(a, 2, 8));
      a = fmaxf(a, __shfl_xor(a, 4, 8));
      QScale sc = q8_scale(a);
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 4; e++)
        packed |= ((uint32_t)(quant_round(y[e] * sc.id) & 0xFF)) << (8 * e);
      *reinterpret_cast<uint32_t*>(cq + q * width + col) = packed;
      if ((lane & 7) == 0) dc[q * (width / QK) + (col >> 5)] = sc.dq;
    }
  }
}

static int attn_kb_per_part(int64_t T, int64_t nq, int64_t nkv, int64_t window, int* kparts) {
  const int64_t tp = (T + AK - 1) / AK * AK;
  const int64_t nqb = tp / AQ;
  int64_t nkb = (T + AK - 1) / AK;
  if (window > 0 && T > window) {
    int64_t band = (2 * window + AQ + AK - 1) / AK + 1;
    if (band < nkb) nkb = band;
  }
  int64_t want = (640 + nqb * nkv - 1) / (nqb * nkv);  // ~2.5 blocks per CU
  if (want > (nkb + 1) / 2) want = (nkb + 1) / 2;      // >= 2 key tiles per partition
  if (want < 1) want = 1;
  const int64_t per = (nkb + want - 1) / want;
  *kparts = (int)((nkb + per - 1) / per);
  return (int)per;
}

size_t attention_scratch_floats(int64_t T, int64_t nq, int64_t nkv, int64_t window) {
  int kp;
  attn_kb_per_part(T, nq, nkv, window, &kp);
  const int64_t tp = (T + AK - 1) / AK * AK;
  return (size_t)(kp * tp * nq * (QKV_HD + 2));
}

hipError_t launch_attention(const uint16_t* q_hi, const uint16_t* q_lo, const uint16_t* k16,
                            const uint16_t* vt16, float* scratch, float* ctx, int8_t* cq,
                            float* dc, int64_t T, int64_t Tp, int64_t nq, int64_t nkv, int64_t hd,
                            int64_t window, hipStream_t s) {
  if (hd != QKV_HD || Tp % AK != 0 || nq % nkv != 0) return hipErrorInvalidValue;
  const int64_t G = nq / nkv;
  int kparts;
  const int per = attn_kb_per_part(T, nq, nkv, window, &kparts);
  float* part_o = scratch;
  float* part_ml = scratch + (int64_t)kparts * Tp * nq * QKV_HD;
  dim3 grid((unsigned)(Tp / AQ), (unsigned)kparts, (unsigned)nkv);
  const f16* a = reinterpret_cast<const f16*>(q_hi);
  const f16* b = reinterpret_cast<const f16*>(q_lo);
  const f16* c = reinterpret_cast<const f16*>(k16);
  const f16* d = reinterpret_cast<const f16*>(vt16);
  switch (G) {
    case 1:
      attn_partial_kernel<1><<<grid, 64, 0, s>>>(a, b, c, d, part_o, part_ml, (int)T, (int)Tp,
                                                 (int)nq, (int)window, per);
      break;
    case 2:
      attn_partial_kernel<2><<<grid, 128, 0, s>>>(a, b, c, d, part_o, part_ml, (int)T, (int)Tp,
                                                  (int)nq, (int)window, per);
      break;
    case 3:
      attn_partial_kernel<3><<<grid, 192, 0, s>>>(a, b, c, d, part_o, part_ml, (int)T, (int)Tp,
                                                  (int)nq, (int)window, per);
      break;
    case 4:
      attn_partial_kernel<4><<<grid, 256, 0, s>>>(a, b, c, d, part_o, part_ml, (int)T, (int)Tp,
                                                  (int)nq, (int)window, per);
      break;
    default:
      return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  attn_combine_kernel<<<(unsigned)((T + 3) / 4), 256, 0, s>>>(part_o, part_ml, (int)T, (int)Tp,
                                                              (int)nq, kparts, ctx, cq, dc);
  return hipGetLastError();
}

}  // namespace glypr
