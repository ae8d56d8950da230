// qkv_epilogue.hpp — the attention prologue of SelfAttention::forward
// (attention/mod.rs:192-214, rope.rs:99-106) as the epilogue of a q|k|v GEMM
// over a staged f32 tile, shared by the large-M fused q|k|v kernels (Q8_0 and
// dense bf16 weights).  Each turns the tile into the attention operands
// exactly as qkv_post_kernel (k_attn.hip) does: RMSNorm over the head in the
// reference's chain order, q_norm / k_norm, RoPE with both products rounded,
// f16 q / k, or the weightless norm and transposed f16 v; rows that hold no
// token are written as zeros, rows past Tp not at all.
#pragma once
#include "device_common.hpp"

namespace glypr {

constexpr int QKV_HD = 256;
// staged row stride (floats): 8 banks of shift per row, so the chain reads of
// two neighbouring rows (lanes 0-7 and 8-15) and the accumulator writes of
// rows 4 apart fall on distinct LDS banks
constexpr int QKV_SP = QKV_HD + 8;

// Rows 0 .. 8 NW - 1 of stg (tokens r0 ..) of head slot `slot`, NW waves of
// the calling workgroup, all of which call this (it holds a barrier); sinv
// holds 8 NW floats of LDS.
template <int NW>
__device__ __forceinline__ void qkv_epilogue_rows(
    const float* stg, float* sinv, int r0, int T, int Tp, int slot, int nq, int nkv,
    const float* __restrict__ qnw, const float* __restrict__ knw, float eps,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, _Float16* __restrict__ q16,
    _Float16* __restrict__ k16, _Float16* __restrict__ vt16, const int2* __restrict__ seg) {
  constexpr int HALF = 8 * NW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool is_v = slot >= nq + nkv;
  const bool is_q = slot < nq;
  const int head = is_q ? slot : (is_v ? slot - nq - nkv : slot - nq);
  const float* w = is_q ? qnw : knw;
  _Float16* outp = is_q ? q16 : k16;
  const v4f wv = (!is_v && w) ? *reinterpret_cast<const v4f*>(w + 4 * lane) : v4f{1, 1, 1, 1};
  // Reference-order 1/rms of staged row 8 wave + l / 8 on lanes 8 c:
  // lane l runs chain l % 8 of that row, the reads of each half of the
  // chain ahead of its FMAs (the caller may hold accumulators live)
  float inv;
  {
    const int i = 8 * wave + (lane >> 3);
    constexpr int CH = QKV_HD / 8, CB = CH / 2;
    float a = 0.0f;
#pragma unroll
    for (int c0 = 0; c0 < CH; c0 += CB) {
      float e[CB];
#pragma unroll
      for (int c = 0; c < CB; c++) e[c] = stg[i * QKV_SP + 8 * (c0 + c) + (lane & 7)];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < CB; c++) a = fmaf(e[c], e[c], a);
    }
    const float sum = hsum8_avx2(a);
    inv = 1.0f / sqrtf(sum / (float)QKV_HD + eps);
  }
  if (!is_v) {
    // wave w writes rows 8 w .. 8 w + 7; lane l holds dims 4 l .. 4 l + 3
#pragma unroll 1
    for (int k = 0; k < 8; k++) {
      const int i = 8 * wave + k;
      const int t = r0 + i;
      if (t >= Tp) break;   // uniform: rows past the padded length are not stored
      bool valid;
      const int pos = seg_row_pos(seg, t, T, &valid);
      const float iv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), 8 * k));
      const v4f x = *reinterpret_cast<const v4f*>(stg + i * QKV_SP + 4 * lane);
      float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (valid) {
#pragma unroll
        for (int e = 0; e < 4; e++) y[e] = w ? (x[e] * iv) * wv[e] : x[e] * iv;
        const v4f cv = *reinterpret_cast<const v4f*>(cos_t + (int64_t)pos * QKV_HD + 4 * lane);
        const v4f sv = *reinterpret_cast<const v4f*>(sin_t + (int64_t)pos * QKV_HD + 4 * lane);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          // lanes l and l ^ 32 hold dims d and d +- 128 (rotate_half's pairs)
          const float ye = y[e];
          const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(ye),
                                                          __float_as_uint(ye), false, false);
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
    // v: the half's HALF 1/rms values through LDS, then thread (dim d,
    // group g of 8 tokens) writes 8 consecutive tokens of vt row d as one
    // 16-byte store
    if ((lane & 7) == 0) sinv[8 * wave + (lane >> 3)] = inv;
    __syncthreads();
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    constexpr int NG = HALF / 8;   // groups of 8 tokens in the half
#pragma unroll 1
    for (int task = tid; task < QKV_HD * NG; task += NW * 64) {
      const int d = task / NG, g = task % NG;
      const int t0 = r0 + 8 * g;
      if (t0 >= Tp) continue;   // Tp is a multiple of 64: whole groups past it
      h8 yh;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        bool valid;
        (void)seg_row_pos(seg, t0 + j, T, &valid);
        // the f32 product is rounded first, then converted (qkv_post's two
        // roundings; left free the compiler would fold both into one
        // v_fma_mixlo_f16)
        float p = stg[(8 * g + j) * QKV_SP + d] * sinv[8 * g + j];
        asm volatile("" : "+v"(p));
        yh[j] = valid ? (_Float16)p : (_Float16)0.0f;
      }
      *reinterpret_cast<h8*>(vt16 + ((int64_t)head * QKV_HD + d) * Tp + t0) = yh;
    }
  }
}

}  // namespace glypr
