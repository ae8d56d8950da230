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
// Precision: products run on f16 MFMA with every f32 operand split as
// x = hi + lo (hi = f16(x), lo = f16(x - hi)); hi*hi + hi*lo + lo*hi carries
// ~22 bits, so scores and context match an f32 computation to ~1e-6 relative.
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
//   q_hi/q_lo [nq][Tp][hd], k_hi/k_lo [nkv][Tp][hd], vt_hi/vt_lo [nkv][hd][Tp].
// ---------------------------------------------------------------------------
constexpr int QKV_HD = 256;

__global__ void __launch_bounds__(256) qkv_post_kernel(
    const float* __restrict__ qkv, int T, int Tp, int nq, int nkv, const float* __restrict__ qnw,
    const float* __restrict__ knw, float eps, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, f16* __restrict__ q_hi, f16* __restrict__ q_lo,
    f16* __restrict__ k_hi, f16* __restrict__ k_lo, f16* __restrict__ vt_hi,
    f16* __restrict__ vt_lo) {
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
  f16 hi[4], lo[4];
#pragma unroll
  for (int e = 0; e < 4; e++) split_f16(y[e], hi[e], lo[e]);
  if (kind < 2) {
    f16* dh = kind == 0 ? q_hi : k_hi;
    f16* dl = kind == 0 ? q_lo : k_lo;
    const int64_t off = ((int64_t)head * Tp + t) * QKV_HD + 4 * lane;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      dh[off + e] = hi[e];
      dl[off + e] = lo[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int64_t off = ((int64_t)head * QKV_HD + 4 * lane + e) * Tp + t;
      vt_hi[off] = hi[e];
      vt_lo[off] = lo[e];
    }
  }
}

hipError_t launch_qkv_post(const float* qkv, int64_t T, int64_t Tp, int64_t nq, int64_t nkv,
                           int64_t hd, const float* qnw, const float* knw, float eps,
                           const float* cos_t, const float* sin_t, uint16_t* q_hi, uint16_t* q_lo,
                           uint16_t* k_hi, uint16_t* k_lo, uint16_t* vt_hi, uint16_t* vt_lo,
                           hipStream_t s) {
  if (hd != QKV_HD) return hipErrorInvalidValue;
  const int64_t tasks = Tp * (nq + 2 * nkv);
  qkv_post_kernel<<<(unsigned)((tasks + 3) / 4), 256, 0, s>>>(
      qkv, (int)T, (int)Tp, (int)nq, (int)nkv, qnw, knw, eps, cos_t, sin_t,
      reinterpret_cast<f16*>(q_hi), reinterpret_cast<f16*>(q_lo), reinterpret_cast<f16*>(k_hi),
      reinterpret_cast<f16*>(k_lo), reinterpret_cast<f16*>(vt_hi), reinterpret_cast<f16*>(vt_lo));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Flash attention.  Block = (q head, 32-query block), 4 waves; wave w takes the
// key blocks kb = w, w+4, ... inside the band, keeping its own running max m,
// sum l and context O (32 x 256 f32 in MFMA output layout: lane l holds
// column l%32 of each 32-wide tile for rows 8(r/4) + 4(l/32) + r%4).  The four
// partial results are merged through LDS at the end.
//   S = Q K^T : v_mfma_f32_32x32x16_f16, 16 k-steps x (hi*hi + hi*lo + lo*hi)
//   O += P V  : P goes through LDS to the A-operand layout; V is read from the
//               transposed vt layout so each lane loads 8 consecutive keys.
// ---------------------------------------------------------------------------
constexpr int ATT_QB = 32;
constexpr int ATT_KB = 32;
constexpr int ATT_WAVES = 4;

__global__ void __launch_bounds__(ATT_WAVES * 64) attention_kernel(
    const f16* __restrict__ q_hi, const f16* __restrict__ q_lo, const f16* __restrict__ k_hi,
    const f16* __restrict__ k_lo, const f16* __restrict__ vt_hi, const f16* __restrict__ vt_lo,
    float* __restrict__ ctx, int T, int Tp, int nq, int nkv, int window) {
  __shared__ __attribute__((aligned(16))) f16 p_hi[ATT_WAVES][ATT_QB][ATT_KB + 8];
  __shared__ __attribute__((aligned(16))) f16 p_lo[ATT_WAVES][ATT_QB][ATT_KB + 8];
  __shared__ float red_m[ATT_WAVES][ATT_QB];
  __shared__ float red_l[ATT_WAVES][ATT_QB];
  __shared__ __attribute__((aligned(16))) float o_acc[ATT_QB][QKV_HD + 4];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, lh = lane >> 5;
  const int h = blockIdx.y;
  const int kvh = h / (nq / nkv);
  const int q0 = blockIdx.x * ATT_QB;

  // Q fragments for all 16 k-steps (A operand: row q0 + l32, dims 16s + 8lh .. +7)
  v8h qa_hi[QKV_HD / 16], qa_lo[QKV_HD / 16];
  {
    const int64_t qoff = ((int64_t)h * Tp + q0 + l32) * QKV_HD + 8 * lh;
#pragma unroll
    for (int s = 0; s < QKV_HD / 16; s++) {
      qa_hi[s] = *reinterpret_cast<const v8h*>(q_hi + qoff + 16 * s);
      qa_lo[s] = *reinterpret_cast<const v8h*>(q_lo + qoff + 16 * s);
    }
  }

  float m_run[16], l_run[16];
  v16f o[QKV_HD / 32];
#pragma unroll
  for (int r = 0; r < 16; r++) {
    m_run[r] = -INFINITY;
    l_run[r] = 0.0f;
  }
#pragma unroll
  for (int t = 0; t < QKV_HD / 32; t++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[t][r] = 0.0f;

  // key-block range intersecting the band of this query block
  int kb_lo = 0, kb_hi = (T + ATT_KB - 1) / ATT_KB;
  if (window > 0 && T > window) {
    int lo_key = q0 - window;
    int hi_key = q0 + ATT_QB - 1 + window;
    kb_lo = lo_key > 0 ? lo_key / ATT_KB : 0;
    int hk = hi_key < T - 1 ? hi_key : T - 1;
    kb_hi = hk / ATT_KB + 1;
  }

  const f16* kh_base = k_hi + (int64_t)kvh * Tp * QKV_HD;
  const f16* kl_base = k_lo + (int64_t)kvh * Tp * QKV_HD;
  const f16* vh_base = vt_hi + (int64_t)kvh * QKV_HD * Tp;
  const f16* vl_base = vt_lo + (int64_t)kvh * QKV_HD * Tp;

  for (int kb = kb_lo + wave; kb < kb_hi; kb += ATT_WAVES) {
    const int k0 = kb * ATT_KB;
    // ---- S = Q K^T (32 queries x 32 keys)
    v16f sacc = {};
    const int64_t koff = (int64_t)(k0 + l32) * QKV_HD + 8 * lh;
#pragma unroll
    for (int s = 0; s < QKV_HD / 16; s++) {
      v8h bh = *reinterpret_cast<const v8h*>(kh_base + koff + 16 * s);
      v8h bl = *reinterpret_cast<const v8h*>(kl_base + koff + 16 * s);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qa_hi[s], bh, sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qa_hi[s], bl, sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qa_lo[s], bh, sacc, 0, 0, 0);
    }
    // ---- mask: keys past T, and the band for sliding layers
    const int key = k0 + l32;
    float sv[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int qi = q0 + 8 * (r >> 2) + 4 * lh + (r & 3);
      bool ok = key < T;
      if (window > 0 && T > window) {
        int d = qi - key;
        ok = ok && (d <= window && -d <= window);
      }
      sv[r] = ok ? sacc[r] : -INFINITY;
    }
    // ---- online softmax (row = 32 lanes of one half)
    float alpha[16];
#pragma unroll
    for (int r = 0; r < 16; r++) {
      float mx = sv[r];
      mx = fmaxf(mx, __shfl_xor(mx, 1));
      mx = fmaxf(mx, __shfl_xor(mx, 2));
      mx = fmaxf(mx, __shfl_xor(mx, 4));
      mx = fmaxf(mx, __shfl_xor(mx, 8));
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      const float m_new = fmaxf(m_run[r], mx);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      alpha[r] = expf(m_run[r] - m_use);
      const float p = expf(sv[r] - m_use);
      float ps = p;
      ps += __shfl_xor(ps, 1);
      ps += __shfl_xor(ps, 2);
      ps += __shfl_xor(ps, 4);
      ps += __shfl_xor(ps, 8);
      ps += __shfl_xor(ps, 16);
      l_run[r] = l_run[r] * alpha[r] + ps;
      m_run[r] = m_new;
      f16 ph, pl;
      split_f16(p, ph, pl);
      const int row = 8 * (r >> 2) + 4 * lh + (r & 3);
      p_hi[wave][row][l32] = ph;
      p_lo[wave][row][l32] = pl;
    }
#pragma unroll
    for (int t = 0; t < QKV_HD / 32; t++)
#pragma unroll
      for (int r = 0; r < 16; r++) o[t][r] *= alpha[r];
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    // ---- O += P V : 2 key steps of 16
#pragma unroll
    for (int s = 0; s < ATT_KB / 16; s++) {
      v8h ah = *reinterpret_cast<const v8h*>(&p_hi[wave][l32][16 * s + 8 * lh]);
      v8h al = *reinterpret_cast<const v8h*>(&p_lo[wave][l32][16 * s + 8 * lh]);
#pragma unroll
      for (int t = 0; t < QKV_HD / 32; t++) {
        const int64_t voff = (int64_t)(32 * t + l32) * Tp + k0 + 16 * s + 8 * lh;
        v8h bh = *reinterpret_cast<const v8h*>(vh_base + voff);
        v8h bl = *reinterpret_cast<const v8h*>(vl_base + voff);
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, o[t], 0, 0, 0);
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, o[t], 0, 0, 0);
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, o[t], 0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- merge the four waves: common max per row, rescale, sum through LDS
  if (l32 == 0)
#pragma unroll
    for (int r = 0; r < 16; r++) red_m[wave][8 * (r >> 2) + 4 * lh + (r & 3)] = m_run[r];
  __syncthreads();
  float scale[16];
#pragma unroll
  for (int r = 0; r < 16; r++) {
    const int row = 8 * (r >> 2) + 4 * lh + (r & 3);
    float M = red_m[0][row];
#pragma unroll
    for (int w = 1; w < ATT_WAVES; w++) M = fmaxf(M, red_m[w][row]);
    const float m_use = M == -INFINITY ? 0.0f : M;
    scale[r] = m_run[r] == -INFINITY ? 0.0f : expf(m_run[r] - m_use);
  }
  if (l32 == 0)
#pragma unroll
    for (int r = 0; r < 16; r++) red_l[wave][8 * (r >> 2) + 4 * lh + (r & 3)] = l_run[r] * scale[r];
  for (int w = 0; w < ATT_WAVES; w++) {
    if (wave == w) {
#pragma unroll
      for (int t = 0; t < QKV_HD / 32; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = 8 * (r >> 2) + 4 * lh + (r & 3);
          const float v = o[t][r] * scale[r];
          float* dst = &o_acc[row][32 * t + l32];
          *dst = (w == 0) ? v : *dst + v;
        }
    }
    __syncthreads();
  }
  // ---- normalise and store ctx [T][nq*256]
  for (int i = threadIdx.x; i < ATT_QB * (QKV_HD / 4); i += ATT_WAVES * 64) {
    const int row = i / (QKV_HD / 4), c4 = i % (QKV_HD / 4);
    const int qi = q0 + row;
    if (qi >= T) continue;
    float L = red_l[0][row];
#pragma unroll
    for (int w = 1; w < ATT_WAVES; w++) L += red_l[w][row];
    const float invl = 1.0f / L;
    v4f v = *reinterpret_cast<const v4f*>(&o_acc[row][4 * c4]);
    v4f out;
#pragma unroll
    for (int e = 0; e < 4; e++) out[e] = v[e] * invl;
    *reinterpret_cast<v4f*>(ctx + (int64_t)qi * nq * QKV_HD + (int64_t)h * QKV_HD + 4 * c4) = out;
  }
}

hipError_t launch_attention(const uint16_t* q_hi, const uint16_t* q_lo, const uint16_t* k_hi,
                            const uint16_t* k_lo, const uint16_t* vt_hi, const uint16_t* vt_lo,
                            float* ctx, int64_t T, int64_t Tp, int64_t nq, int64_t nkv, int64_t hd,
                            int64_t window, hipStream_t s) {
  if (hd != QKV_HD || Tp % ATT_KB != 0 || nq % nkv != 0) return hipErrorInvalidValue;
  dim3 grid((unsigned)(Tp / ATT_QB), (unsigned)nq);
  attention_kernel<<<grid, ATT_WAVES * 64, 0, s>>>(
      reinterpret_cast<const f16*>(q_hi), reinterpret_cast<const f16*>(q_lo),
      reinterpret_cast<const f16*>(k_hi), reinterpret_cast<const f16*>(k_lo),
      reinterpret_cast<const f16*>(vt_hi), reinterpret_cast<const f16*>(vt_lo), ctx, (int)T,
      (int)Tp, (int)nq, (int)nkv, (int)window);
  return hipGetLastError();
}

}  // namespace glypr
