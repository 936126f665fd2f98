// Shared device helpers for the gfx950 int4 decode path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mtl_gptq.h"

namespace mtl {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two float32 -> packed bf16 bits (lo | hi << 16), round to nearest even: one
// v_cvt_pk_bf16_f32.  NaN bits are whatever the instruction makes of them, so this is for
// values that stay in registers (MFMA operands, intermediate roundings).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// float32 -> bf16 bits, round to nearest even; every NaN -> 0x7FC0 (c10 rule).
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  const uint32_t b = cvt_pk_bf16(f, 0.f) & 0xffffu;
  return f != f ? 0x7fc0u : b;
}

// Round a float32 to the nearest bf16 value, kept in float32 (a NaN stays a NaN).
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_to_f32(cvt_pk_bf16(f, 0.f) & 0xffffu);
}

// Round two float32 values to bf16, kept in float32, with one conversion.
__device__ __forceinline__ void round_bf16x2(float lo, float hi, float& rlo, float& rhi) {
  const uint32_t p = cvt_pk_bf16(lo, hi);
  rlo = __uint_as_float(p << 16);
  rhi = __uint_as_float(p & 0xffff0000u);
}

// bf16(silu(bf16 g) * bf16 u): F.silu on a bf16 tensor then a bf16 product (fast.py:170-171).
// silu(g) = g / (1 + e^-g) in fp32 from the hardware exp2 and reciprocal (v_exp_f32 of
// -g * log2(e), v_rcp_f32, each about 1 ulp): within a few fp32 ulps of the correctly
// rounded quotient, so the bf16 result differs from it only where the quotient lies within
// those ulps of a bf16 rounding boundary (a few in 10^5).  Every kernel uses this one form.
// It sits on the tail of the SiLU*up GEMV launches, where the libm exp and the IEEE
// division cost 0.3 us.  g -> -inf gives -0 (e = inf, rcp = 0), g -> +inf gives g.
__device__ __forceinline__ uint32_t silu_mul_bf16(float g, float u) {
  g = round_bf16(g);
  const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
  const float sg = round_bf16(g * __builtin_amdgcn_rcpf(1.0f + e));
  return f32_to_bf16(sg * round_bf16(u));
}

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)bits16);
}

// c + a.lo*b.lo + a.hi*b.hi with both operands bf16 pairs (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// Butterfly sum over the 64 lanes of a wave (fixed order: bitwise repeatable).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Sums of squares of the residual stream h travel between kernels as one slot per
// 16-column block: slots[b] = sum over h[16b .. 16b+15] of h^2, formed as four fma chains
// over 4 consecutive columns (lanes 4i .. 4i+3) joined by slot_combine.  Every producer
// uses that order, so every launch plan sees the same slot values.  The RMSNorm that
// consumes them sums the ceil(n/16) slots with one wave (slot_issue, slot_finish, wave_sum).
constexpr int kSlotCols = 16;
constexpr int kMaxSlots = 1024;   // hidden <= 16384

__device__ __forceinline__ float slot_combine(float ss) {
  ss += __shfl_xor(ss, 1);
  return ss + __shfl_xor(ss, 2);
}

// A wave reads the slots as float4 chunks: lane l sums slots 4l .. 4l+3, then +256, ...
// (fixed order).  slot_issue only loads (uniform branches, clamped in-bounds addresses), so
// a kernel can put the loads in flight and sum them once other loads are issued too.
// A slot buffer holds ceil(ns / 4) * 4 floats, ns = ceil(n / 16).
struct SlotLoad {
  float4 v[kMaxSlots / 256];
};

__device__ __forceinline__ void slot_issue(const float* slots, int n, int lane, SlotLoad& sl) {
  const int ns = (n + kSlotCols - 1) / kSlotCols;
  const int nch = (ns + 255) / 256;
#pragma unroll
  for (int it = 0; it < kMaxSlots / 256; ++it) {
    if (it < nch) {
      const int b = 4 * lane + 256 * it;
      sl.v[it] = *reinterpret_cast<const float4*>(slots + (b < ns ? b : 0));
    }
  }
}

__device__ __forceinline__ float slot_finish(const SlotLoad& sl, int n, int lane) {
  const int ns = (n + kSlotCols - 1) / kSlotCols;
  const int nch = (ns + 255) / 256;
  float s = 0.f;
#pragma unroll
  for (int it = 0; it < kMaxSlots / 256; ++it) {
    if (it < nch) {
      const int b = 4 * lane + 256 * it;
      const float4 v = sl.v[it];
      s += ((b < ns ? v.x : 0.f) + (b + 1 < ns ? v.y : 0.f)) +
           ((b + 2 < ns ? v.z : 0.f) + (b + 3 < ns ? v.w : 0.f));
    }
  }
  return s;
}

__device__ __forceinline__ float slot_total(const float* slots, int n, int lane) {
  SlotLoad sl;
  slot_issue(slots, n, lane, sl);
  return wave_sum(slot_finish(sl, n, lane));
}

__device__ __forceinline__ float lo_bf(uint32_t w) { return bf16_to_f32(w & 0xffffu); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return bf16_to_f32(w >> 16); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// The same cross-lane steps on the VALU, for code where all 64 lanes are active: a
// __shfl_xor is a ds_bpermute, an LDS round trip of about 85 cycles that the next step
// waits for; these are a few cycles each.  xor 32 and xor 16 come from v_permlane32_swap /
// v_permlane16_swap (after the swap of two copies of x, the two registers hold x[i] and
// x[i ^ 16] in some order, and addition and max are commutative); xor 8 and xor 4 are DPP
// row rotations, which equal them once the values depend only on the lane modulo 16 and 8
// (true after the larger steps of a butterfly that goes 32, 16, 8, 4, 2, 1); xor 2 and 1
// are DPP quad permutations.  So wave_sum_valu / wave_max_valu give the bits of wave_sum /
// wave_max.  The swaps are inline asm with both registers in and out (the compiler's
// builtin loses the second result when both inputs are the same value), with the wait
// states around them explicit.
__device__ __forceinline__ void permlane_swap16(uint32_t& a, uint32_t& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

__device__ __forceinline__ void permlane_swap32(uint32_t& a, uint32_t& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

__device__ __forceinline__ float xor16_add(float v) {
  uint32_t a = __float_as_uint(v), b = a;
  permlane_swap16(a, b);
  return __uint_as_float(a) + __uint_as_float(b);
}

__device__ __forceinline__ float xor32_add(float v) {
  uint32_t a = __float_as_uint(v), b = a;
  permlane_swap32(a, b);
  return __uint_as_float(a) + __uint_as_float(b);
}

__device__ __forceinline__ float xor16_max(float v) {
  uint32_t a = __float_as_uint(v), b = a;
  permlane_swap16(a, b);
  return fmaxf(__uint_as_float(a), __uint_as_float(b));
}

__device__ __forceinline__ float xor32_max(float v) {
  uint32_t a = __float_as_uint(v), b = a;
  permlane_swap32(a, b);
  return fmaxf(__uint_as_float(a), __uint_as_float(b));
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}

constexpr int kDppRor8 = 0x128, kDppRor4 = 0x124;          // row_ror:8, row_ror:4
constexpr int kDppXor2 = 0x4E, kDppXor1 = 0xB1;            // quad_perm [2,3,0,1], [1,0,3,2]

__device__ __forceinline__ float wave_sum_valu(float v) {
  v = xor32_add(v);
  v = xor16_add(v);
  v += dpp_f32<kDppRor8>(v);
  v += dpp_f32<kDppRor4>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<kDppXor1>(v);
  return v;
}

// Sum over aligned groups of G lanes (G = 2, 4, ..., 64), every lane ending with its group's
// sum: the butterfly xor 1, 2, 4, ... in that order on the VALU (quad permutations; the
// mirrors within 8 and within 16 lanes, which equal xor 4 and xor 8 once each quad and each 8
// lanes hold one value; then the permlane swaps), so the bits of
// `for (o = 1; o < G; o <<= 1) v += __shfl_xor(v, o)`.  All 64 lanes active.
constexpr int kDppHalfMirror = 0x141, kDppMirror = 0x140;  // row_half_mirror, row_mirror

template <int G>
__device__ __forceinline__ float group_sum_valu(float v) {
  static_assert(G == 2 || G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "power of two");
  v += dpp_f32<kDppXor1>(v);
  if (G >= 4) v += dpp_f32<kDppXor2>(v);
  if (G >= 8) v += dpp_f32<kDppHalfMirror>(v);
  if (G >= 16) v += dpp_f32<kDppMirror>(v);
  if (G >= 32) v = xor16_add(v);
  if (G >= 64) v = xor32_add(v);
  return v;
}

// slot_combine on the VALU (the same bits; all lanes active).
__device__ __forceinline__ float slot_combine_valu(float ss) { return group_sum_valu<4>(ss); }

// slot_total on the VALU (the same bits; all lanes active).
__device__ __forceinline__ float slot_total_valu(const float* slots, int n, int lane) {
  SlotLoad sl;
  slot_issue(slots, n, lane, sl);
  return wave_sum_valu(slot_finish(sl, n, lane));
}

__device__ __forceinline__ float wave_max_valu(float v) {
  v = xor32_max(v);
  v = xor16_max(v);
  v = fmaxf(v, dpp_f32<kDppRor8>(v));
  v = fmaxf(v, dpp_f32<kDppRor4>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  return v;
}

// RMSNorm over the 128 dims of one head (lane t holds dims t and t+64), then RoPE:
// q*cos + rotate_half(q)*sin, each product and the sum rounded to bf16 as separate bf16
// tensor ops (model.py:34-44, fast.py:141-144).
// The same with the lane's operands already loaded: norm weights w0 = w[t], w1 = w[t+64],
// cos c0 = cr[t], c1 = cr[t+64], sin s0 = sr[t], s1 = sr[t+64] (bf16 values in fp32).
// VALU: the sum of squares with wave_sum_valu (all 64 lanes active; the same bits).
template <bool VALU = false>
__device__ __forceinline__ void norm_rope_vals(float x0, float x1, float w0, float w1, float c0,
                                               float c1, float s0, float s1, float eps,
                                               float& o0, float& o1) {
  float ss = fmaf(x0, x0, x1 * x1);
  ss = VALU ? wave_sum_valu(ss) : wave_sum(ss);
  const float r = rsqrtf(ss / 128.f + eps);
  const float n0 = round_bf16(w0 * round_bf16(x0 * r));
  const float n1 = round_bf16(w1 * round_bf16(x1 * r));
  o0 = round_bf16(round_bf16(n0 * c0) + round_bf16(-n1 * s0));
  o1 = round_bf16(round_bf16(n1 * c1) + round_bf16(n0 * s1));
}

__device__ __forceinline__ void norm_rope_pair(float x0, float x1, const uint16_t* w,
                                               const uint16_t* cr, const uint16_t* sr, int t,
                                               float eps, float& o0, float& o1) {
  norm_rope_vals(x0, x1, bf16_to_f32(w[t]), bf16_to_f32(w[t + 64]), bf16_to_f32(cr[t]),
                 bf16_to_f32(cr[t + 64]), bf16_to_f32(sr[t]), bf16_to_f32(sr[t + 64]), eps, o0,
                 o1);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int launch_status() {
  return hipGetLastError() == hipSuccess ? MTL_OK : MTL_ERR_LAUNCH;
}

}  // namespace mtl
