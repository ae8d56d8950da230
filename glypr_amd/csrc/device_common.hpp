// device_common.hpp — device helpers shared by the gfx950 kernels.
//
// Everything here must round exactly like glypr's CPU path on x86-64, so the
// library is compiled with -ffp-contract=off (no implicit FMA, as in Rust) and
// uses fmaf only where the reference itself fuses (pulp mul_add in RMSNorm).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace glypr {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int QK = 32;                // Q8_0 block length along K
constexpr int BLOCK_BYTES = 34;       // GGUF Q8_0 block: f16 d + 32 x int8

// f32 -> f16 with round-to-nearest-even (v_cvt_f16_f32 in the default mode),
// overflow to inf, subnormals kept: half 2.7.1's f16::from_f32.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __half_as_ushort(__float2half_rn(f));
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}

// ---------------------------------------------------------------------------
// Cross-lane max through DPP (a VALU operand modifier: no LDS round trip, as
// __shfl_xor's ds_bpermute would be).  Max is order-free, so these give the
// same bits as any other reduction order.  DPP controls: quad_perm 0x00-0xFF,
// row_mirror 0x140, row_half_mirror 0x141, row_bcast:15 0x142 (a row is 16
// lanes).
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_mov(float old, float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL,
                                                    ROW_MASK, 0xF, false));
}
// max over each aligned group of 4 lanes; every lane of the group gets it
__device__ __forceinline__ float max4(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v, v));    // quad_perm [1,0,3,2]
  return fmaxf(v, dpp_mov<0x4E>(v, v));  // quad_perm [2,3,0,1]
}
// max over each aligned group of 8 lanes; every lane of the group gets it
__device__ __forceinline__ float max8(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v, v));    // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4E>(v, v));    // quad_perm [2,3,0,1]
  return fmaxf(v, dpp_mov<0x141>(v, v));  // row_half_mirror: quad 0 <-> quad 1
}
// max8 for values that are >= +0 and never NaN (block amax of |x|, which
// starts from 0 and ignores NaN like Rust's f32::max): their bit patterns
// order like the floats, so the reduction is an integer max.
__device__ __forceinline__ float max8_nonneg(float v) {
  uint32_t u = __float_as_uint(v);
  u = max(u, (uint32_t)__builtin_amdgcn_update_dpp((int)u, (int)u, 0xB1, 0xF, 0xF, false));
  u = max(u, (uint32_t)__builtin_amdgcn_update_dpp((int)u, (int)u, 0x4E, 0xF, 0xF, false));
  u = max(u, (uint32_t)__builtin_amdgcn_update_dpp((int)u, (int)u, 0x141, 0xF, 0xF, false));
  return __uint_as_float(u);
}
// v of lane I of each aligned group of 8 lanes, to every lane of the group
// (ds_swizzle bit mode: lane' = (lane & 0x18) | I within each 32 lanes).
template <int I>
__device__ __forceinline__ float bcast8(float v) {
  static_assert(I >= 0 && I < 8, "lane index");
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x18 | (I << 5)));
}
__device__ __forceinline__ float bcast8(float v, int i) {
  switch (i) {
    case 0: return bcast8<0>(v);
    case 1: return bcast8<1>(v);
    case 2: return bcast8<2>(v);
    case 3: return bcast8<3>(v);
    case 4: return bcast8<4>(v);
    case 5: return bcast8<5>(v);
    case 6: return bcast8<6>(v);
    default: return bcast8<7>(v);
  }
}
// max16 for values that are >= +0 and never NaN (see max8_nonneg)
__device__ __forceinline__ float max16_nonneg(float v) {
  uint32_t u = __float_as_uint(max8_nonneg(v));
  u = max(u, (uint32_t)__builtin_amdgcn_update_dpp((int)u, (int)u, 0x140, 0xF, 0xF, false));
  return __uint_as_float(u);
}
// v of lane I of each aligned group of 16 lanes, to every lane of the group
template <int I>
__device__ __forceinline__ float bcast16(float v) {
  static_assert(I >= 0 && I < 16, "lane index");
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x10 | (I << 5)));
}
// 4 x 4 transpose inside each quad of lanes: lane 4k + i holds v[j] =
// M[i][j] on entry and M[j][i] on exit (two butterfly stages over lane bits
// 0 and 1; each moves the off-diagonal pairs with one quad_perm DPP).  Used to
// turn an MFMA tile's column-per-lane layout into row-contiguous vectors.
__device__ __forceinline__ void quad_transpose4(float (&v)[4]) {
  const int i = __lane_id();
  // stage over lane bit 0: pairs (0,1) and (2,3)
  const bool h1 = (i & 1) != 0;
  const float s0 = h1 ? v[0] : v[1], s2 = h1 ? v[2] : v[3];
  const float r0 = dpp_mov<0xB1>(s0, s0), r2 = dpp_mov<0xB1>(s2, s2);  // quad_perm [1,0,3,2]
  const float a0 = h1 ? r0 : v[0], a1 = h1 ? v[1] : r0;
  const float a2 = h1 ? r2 : v[2], a3 = h1 ? v[3] : r2;
  // stage over lane bit 1: pairs (0,2) and (1,3)
  const bool h2 = (i & 2) != 0;
  const float t0 = h2 ? a0 : a2, t1 = h2 ? a1 : a3;
  const float q0 = dpp_mov<0x4E>(t0, t0), q1 = dpp_mov<0x4E>(t1, t1);  // quad_perm [2,3,0,1]
  v[0] = h2 ? q0 : a0;
  v[1] = h2 ? q1 : a1;
  v[2] = h2 ? a2 : q0;
  v[3] = h2 ? a3 : q1;
}
// v of lane i + N within each row of 16 lanes (DPP row_shl:N); lanes whose
// source lies past the end of the row keep their own v.
template <int N>
__device__ __forceinline__ float dpp_row_shl(float v) {
  static_assert(N >= 1 && N <= 15, "row shift");
  return dpp_mov<0x100 + N>(v, v);
}
// The AVX2 horizontal sum of simd_rmsnorm_row_f32 over eight chain
// accumulators held by lanes 8g + j (j = 0..7):
//   ((l0 + l4) + (l2 + l6)) + ((l1 + l5) + (l3 + l7)),
// valid in lane 8g.  Lane j < 4 first adds l(j+4), lanes 0 and 1 then add
// lanes 2 and 3, lane 0 adds lane 1: the same three levels of f32 adds, in
// VALU with DPP row shifts (no LDS round trips).
__device__ __forceinline__ float hsum8_avx2(float acc) {
  const float s = acc + dpp_row_shl<4>(acc);
  const float t = s + dpp_row_shl<2>(s);
  return t + dpp_row_shl<1>(t);
}
// max over each row of 16 lanes; every lane of the row gets it
__device__ __forceinline__ float max16(float v) {
  v = max8(v);
  return fmaxf(v, dpp_mov<0x140>(v, v));  // row_mirror: 8-lane halves swap
}
// max over lanes 0-31 and over lanes 32-63; valid in lanes 16-31 and 48-63
__device__ __forceinline__ float max32_hi(float v) {
  v = max16(v);
  return fmaxf(v, dpp_mov<0x142, 0xA>(v, v));  // rows 1, 3 take lane 15 of rows 0, 2
}

// Rust `f32::round(v) as i8`: half away from zero, saturating, NaN -> 0.
// s = RN(v + copysign(pred(0.5), v)) truncates to round-half-away(v) for every
// finite v (pred(0.5) = 0.5 - 2^-25 keeps v = pred(0.5) from reaching 1, and
// exact ties still round up because the sum's rounding goes to the even
// neighbour, the integer); v_cvt_i32_f32 truncates, saturates out-of-range
// values and maps NaN to 0; med3 clamps to [-128, 127].  Identical to
// clamp(roundf(v)) with NaN -> 0 for all 2^32 inputs (tests/test_round.py).
__device__ __forceinline__ int quant_round(float v) {
  const float s = v + __builtin_copysignf(0.49999997f, v);
  int i;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(i) : "v"(s));
  return min(max(i, -128), 127);
}

// BlockQ8_0::from_float scale: d = amax / 127; id = d != 0 ? 1/d : 0.
// IEEE division (hipcc's default correctly rounded f32 divide).
struct QScale {
  float d;    // f32 scale (id is derived from it)
  float id;   // inverse used for rounding
  float dq;   // f32(f16(d)): the scale every later dot product sees
  uint16_t dbits;
};
__device__ __forceinline__ QScale q8_scale(float amax) {
  QScale s;
  s.d = amax / 127.0f;
  s.id = (s.d != 0.0f) ? 1.0f / s.d : 0.0f;
  s.dbits = f32_to_f16_bits(s.d);
  s.dq = f16_bits_to_f32(s.dbits);
  return s;
}

// ---------------------------------------------------------------------------
// LDS DMA (global_load_lds): global memory straight into LDS, no register
// round trip.  The helpers set m0 themselves; the compiler keeps m0 reserved
// and the kernels that use them contain no other m0 user (no LDS-DMA
// builtins, GWS or indexed register moves), which the build's assembly shows.
// ---------------------------------------------------------------------------
typedef long v1l;

// 16 bytes per lane, global -> LDS (lane i -> lds_base + 16 i); the address
// is the uniform base plus the lane's 32-bit offset.
__device__ __forceinline__ void dma16(const int8_t* base, int voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(base), "s"(lds_base) : "memory", "m0");
}
// 16 bytes per lane from a per-lane 64-bit address (lane i -> lds_base + 16 i).
__device__ __forceinline__ void dma16_flat(const void* g, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(g), "s"(lds_base) : "memory", "m0");
}
// Non-temporal store (global_store with the nt bit): for the large-M GEMMs'
// outputs (tens of MB that no later access in the launch reads), so that they
// do not sit in L2 as dirty lines until the end-of-kernel write-back.  At
// M = 16384 it took the C3 step's GEMMs ~4 % lower (the N = 768 launches run
// as one round of workgroups that all write their tiles at the end).
template <class T>
__device__ __forceinline__ void st_nt(T* p, T v) {
  __builtin_nontemporal_store(v, p);
}
// 4 bytes per lane (lane i -> lds_base + 4 i).
__device__ __forceinline__ void dma4(const int8_t* base, int voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(base), "s"(lds_base) : "memory", "m0");
}
// Tile (mi, ni) of this workgroup in a 1D grid of tm x tn tiles.  Workgroup
// i runs on XCD i % 8 (eight XCDs, each with its own L2), so the tiles are
// dealt out as one contiguous run per XCD: nmajor runs cover whole columns of
// N tiles (an XCD reads its slice of B once and all of A: 8*A + B bytes from
// memory), otherwise whole rows of M tiles (A + 8*B).  The caller picks the
// order that re-reads the smaller operand.
// The grid is exactly tm x tn blocks (every caller launches that): the block
// count comes from the arguments, not from gridDim, which is a hidden kernel
// argument in memory while the explicit leading ones arrive preloaded in SGPRs.
__device__ __forceinline__ void xcd_tile(int tm, int tn, bool nmajor, int& mi, int& ni) {
  const int nblk = tm * tn, id = blockIdx.x;
  const int xq8 = nblk >> 3, xr8 = nblk & 7, xcd = id & 7;
  const int W = xcd * xq8 + (xcd < xr8 ? xcd : xr8) + (id >> 3);
  if (nmajor) {
    ni = W / tm;
    mi = W - ni * tm;
  } else {
    mi = W / tn;
    ni = W - mi * tn;
  }
}

__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

// s_waitcnt vmcnt(min(later, L) * U): wait until at most `later` stages of U
// DMA units each are still in flight (`later` is wave-uniform; the immediate
// must be <= 63).
template <int U, int L>
__device__ __forceinline__ void vm_wait_units(int later) {
  static_assert(L * U <= 63, "vmcnt immediate out of range");
  if constexpr (L <= 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else {
    if (later >= L) asm volatile("s_waitcnt vmcnt(%0)" :: "n"(L * U) : "memory");
    else vm_wait_units<U, L - 1>(later);
  }
}

// Row t's RoPE position and whether it holds a token: with a segment table
// (several sequences at 64-aligned row offsets, seg[t] = {start, length} of
// row t's sequence) the position restarts at each sequence and the rows past
// a sequence's length are padding; without one, row t is position t of one
// sequence of T tokens.
__device__ __forceinline__ int seg_row_pos(const int2* __restrict__ seg, int t, int T,
                                           bool* valid) {
  if (!seg) {
    *valid = t < T;
    return t;
  }
  const int2 sg = seg[t];
  const int p = t - sg.x;
  *valid = p < sg.y;
  return p;
}

// ---------------------------------------------------------------------------
// tanh for GeGLU.  glypr's geglu_scalar_f32 calls the platform libm tanh, so
// its bits differ between glibc and Apple libm.  The backend defines tanh as
//   tanh|x| = -t / (t + 2),  t = expm1(-2|x|),
// expm1 by Cody-Waite reduction y = k*ln2 + r (float ln2 hi/lo split as in
// fdlibm), |r| <= ln2/2, degree-8 Taylor polynomial in Horner form with fma,
// expm1(y) = 2^k * p + (2^k - 1).  Only IEEE +,-,*,/ and fma appear, so the
// CPU oracle computes the same bits.  Max error ~2.5 ulp vs exact tanh.
// ---------------------------------------------------------------------------
// Straight-line code: every case is computed and the result picked by
// selects (v_cndmask), so the four h elements a lane holds run interleaved
// instead of one after another behind per-element branches.  Each select
// returns exactly what the branch of the CPU statement (orc_tanhf) returns.
// materialize(v) pins v to a register at that point (an empty asm that reads
// and writes it), so the compiler cannot sink v's computation into a branch
// around the select.
__device__ __forceinline__ float materialize(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// expm1(y) for y in [-20, -2^-11] (tanh_glypr's range): the oracle's
// orc_expm1_nonpos without its two early returns, which cannot change a bit
// here: y >= -20 never takes the y < -30 one, and for k == 0 the general
// result fma(1, p, 1 - 1) = p + 0 equals p (p < 0 for these y).
__device__ __forceinline__ float expm1_nonpos(float y) {
  const float LOG2E = 1.44269504088896341f;
  const float LN2_HI = 6.93145751953125e-01f;
  const float LN2_LO = 1.42860682030941723e-06f;
  float kf = rintf(y * LOG2E);
  float r = fmaf(-kf, LN2_HI, y);
  r = fmaf(-kf, LN2_LO, r);
  float p = fmaf(r, 2.48015873015873016e-05f, 1.98412698412698413e-04f);
  p = fmaf(r, p, 1.38888888888888889e-03f);
  p = fmaf(r, p, 8.33333333333333333e-03f);
  p = fmaf(r, p, 4.16666666666666667e-02f);
  p = fmaf(r, p, 1.66666666666666667e-01f);
  p = fmaf(r, p, 0.5f);
  p = fmaf(r * r, p, r);
  const int k = (int)kf;
  const float sc = __int_as_float((k + 127) << 23);
  return fmaf(sc, p, sc - 1.0f);
}

// orc_tanhf's value for every input.  The general path runs on |x| clamped to
// [2^-12, 10]: at 10 it gives expm1(-20) = -1.0f exactly and so +-1, which is
// orc_tanhf's |x| >= 10 result; the NaN and |x| < 2^-12 cases (-> x) are
// selects.
__device__ __forceinline__ float tanh_glypr(float x) {
  const float ax = fabsf(x);
  const float axc = fminf(fmaxf(ax, 2.44140625e-04f), 10.0f);
  const float t = expm1_nonpos(-2.0f * axc);
  const float r = materialize(copysignf(-t / (t + 2.0f), x));
  return (x != x || ax < 2.44140625e-04f) ? x : r;
}

// geglu_scalar_f32 (cpu_simd/geglu.rs:6-18).  For g >= 10 the general path
// already gives g * u (tanh = 1, so act = (0.5 g) * 2 = g); g <= -10 gives
// +-0 there, where the reference returns +0, hence the select.
__device__ __forceinline__ float geglu_scalar(float g, float u) {
  float g3 = g * g * g;
  float inner = 0.7978846f * (g + 0.044715f * g3);
  float th = tanh_glypr(inner);
  float act = 0.5f * g * (1.0f + th);
  const float mid = materialize(act * u);
  return g <= -10.0f ? 0.0f : mid;
}

}  // namespace glypr
