// Inner pieces shared by the int4 GEMV kernels for gfx950 (mtl_w4gemm.hip: split-K tiles,
// mtl_w4strip.hip: full-K column strips): code unpacking into MFMA operands, x staging
// transforms, and the activation sources.
#pragma once

#include "mtl_common.h"

namespace mtl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld_f4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}

// Where a GEMV kernel reads its activation row from.
enum : int {
  XSRC_BF16 = 0,      // x bf16 [M, K]
  XSRC_PERM = 1,      // x bf16 [M, K] read through the act-order index: x[:, perm[k]]
  XSRC_SILU_PART = 2, // x = SiLU(gate) * up from the fp32 split-K partials of an
                      // interleaved gate|up GEMV (the down projection's input)
  XSRC_RMSNORM = 3    // x = bf16(w * bf16(h * r)): RMSNorm applied while staging, from the
                      // residual stream h and norm weight w (both already in the weight's
                      // act-order input order) and r = rsqrt(sum(slots)/K + eps)
};

// The 8 codes of one qweight word as the bf16 MFMA operand (128+q_j, 128+q_{j+4}),
// j = 0..3: one v_and_or_b32 per pair (plus a shift for j > 0).
// Plain integer code (not the inline-asm and_or): the compiler must see these VALU
// writes to insert the wait states an MFMA operand read needs after them.  `lo` and
// `magic` are held in VGPRs (vgpr_const), so each pair selects to one v_and_or_b32.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t v) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "s"(v));
  return r;
}

__device__ __forceinline__ bf16x8_t unpack_codes8(uint32_t w, uint32_t lo, uint32_t magic) {
  const u32x4 p{(w & lo) | magic, ((w >> 4) & lo) | magic, ((w >> 8) & lo) | magic,
                ((w >> 12) & lo) | magic};
  return __builtin_bit_cast(bf16x8_t, p);
}

// x item (8 channels) in pair order (x0,x4),(x1,x5),(x2,x6),(x3,x7), and its sum.
__device__ __forceinline__ u32x4 pair_order(u32x4 v, float& sum) {
  const uint32_t e0 = v.x & 0xffffu, e1 = v.x >> 16, e2 = v.y & 0xffffu, e3 = v.y >> 16;
  const uint32_t e4 = v.z & 0xffffu, e5 = v.z >> 16, e6 = v.w & 0xffffu, e7 = v.w >> 16;
  sum = ((bf16_to_f32(e0) + bf16_to_f32(e1)) + (bf16_to_f32(e2) + bf16_to_f32(e3))) +
        ((bf16_to_f32(e4) + bf16_to_f32(e5)) + (bf16_to_f32(e6) + bf16_to_f32(e7)));
  return u32x4{e0 | (e4 << 16), e1 | (e5 << 16), e2 | (e6 << 16), e3 | (e7 << 16)};
}

// The same pair order with v_perm_b32 (one per output word) and the item's sum as a chain
// of four v_dot2_f32_bf16 against (1, 1): cheaper, and the sum's rounding differs from
// pair_order's fixed tree (a kernel uses one of the two throughout).
__device__ __forceinline__ u32x4 pair_order_dot(u32x4 v, float& sum) {
  const uint32_t ones = 0x3f803f80u;    // bf16 (1, 1)
  sum = dot2_bf16(v.x, ones, 0.f);
  sum = dot2_bf16(v.y, ones, sum);
  sum = dot2_bf16(v.z, ones, sum);
  sum = dot2_bf16(v.w, ones, sum);
  return u32x4{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
               __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
}

// x = bf16(w * bf16(h * r)) on 8 packed bf16 values (RMSNorm, model.py:34-40), two values
// per v_cvt_pk_bf16_f32.  The result is an MFMA operand, so NaN bits are not normalised.
__device__ __forceinline__ u32x4 rmsnorm8(u32x4 h, u32x4 w, float r) {
  const uint32_t hh[4] = {h.x, h.y, h.z, h.w};
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
  uint32_t o[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float nlo, nhi;
    round_bf16x2(__uint_as_float(hh[c] << 16) * r, __uint_as_float(hh[c] & 0xffff0000u) * r,
                 nlo, nhi);
    o[c] = cvt_pk_bf16(__uint_as_float(ww[c] << 16) * nlo,
                       __uint_as_float(ww[c] & 0xffff0000u) * nhi);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// Strip-ordered group metadata (mtl_w4_strip_meta): record rec (a strip's 128-channel
// block, or block pair at g = 256) holds the MB = max(1, 128/g) fp16 scales of each of the
// strip's 16 columns contiguously and their zero nibbles (MB = 4: 16 bits per column,
// MB = 2: 8 bits, MB = 1: a nibble, two columns a byte).  Lane column lj loads its
// column's metadata of a record with one scale load and one zero load.
template <int MB>
struct StripMeta {
  uint32_t s[MB == 4 ? 2 : 1];   // MB packed fp16 scales
  uint32_t z;                    // MB zero nibbles (MB = 1: the record byte)
};

template <int MB>
__device__ __forceinline__ void strip_meta_load(__amdgpu_buffer_rsrc_t srsrc,
                                                __amdgpu_buffer_rsrc_t zrsrc, int lj, int rec,
                                                StripMeta<MB>& m) {
  if (MB == 4) {
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                  srsrc, lj * 8, rec * 128, 0));
    m.s[0] = v.x;
    m.s[MB == 4 ? 1 : 0] = v.y;
    m.z = __builtin_amdgcn_raw_buffer_load_b16(zrsrc, lj * 2, rec * 32, 0);
  } else if (MB == 2) {
    m.s[0] = __builtin_amdgcn_raw_buffer_load_b32(srsrc, lj * 4, rec * 64, 0);
    m.z = __builtin_amdgcn_raw_buffer_load_b8(zrsrc, lj, rec * 16, 0);
  } else {
    m.s[0] = __builtin_amdgcn_raw_buffer_load_b16(srsrc, lj * 2, rec * 32, 0);
    m.z = __builtin_amdgcn_raw_buffer_load_b8(zrsrc, lj >> 1, rec * 8, 0);
  }
}

// Scale and 128 + zero + zero_offset of the record's MB groups for column lj.
template <int MB>
__device__ __forceinline__ void strip_meta_decode(const StripMeta<MB>& m, int lj,
                                                  int zero_offset, float (&gs)[MB],
                                                  float (&gz)[MB]) {
  const uint32_t zsh = MB == 1 ? (lj & 1) * 4 : 0;
#pragma unroll
  for (int g = 0; g < MB; ++g) {
    gs[g] = f16_to_f32((m.s[g >> 1] >> (16 * (g & 1))) & 0xffffu);
    gz[g] = (float)(128 + (int)((m.z >> (zsh + 4 * g)) & 0xfu) + zero_offset);
  }
}

// Group metadata of the strip-layout kernels.
enum : int {
  STRIP_META_GPTQ = 0,  // fp16 scales and zero nibbles in the strip order of mtl_w4_strip_meta:
                        // w = (q - z - zero_offset) * s
  STRIP_META_QSZ = 1    // the reference's qsz bf16 [K/g, N, 2] (scale, zero) pairs, in place:
                        // w = (q - 8) * scale + zero (moss_tts_lite/gptq.py:87-97)
};

// One (scale, zero) pair of the reference's qsz for group gidx of column col: 4 bytes at
// (gidx * N + col) * 4 (a per-lane column offset and a uniform group offset).
__device__ __forceinline__ uint32_t qsz_load(__amdgpu_buffer_rsrc_t qrsrc, int col, int gidx,
                                             int N) {
  return __builtin_amdgcn_raw_buffer_load_b32(qrsrc, col * 4, gidx * N * 4, 0);
}

// The group correction of both contracts.  The MFMA accumulates A = sum (128 + q) * x over
// the group exactly in fp32 products; with X the group's sum of x, the group adds
// s * (A - c * X) + d * X: (s, 128 + z + zero_offset, 0) for GPTQ metadata, and
// (scale, 136, zero) for the reference's qsz (136 = 128 + 8).
__device__ __forceinline__ void qsz_decode(uint32_t sz, float& s, float& c, float& d) {
  s = __uint_as_float(sz << 16);
  c = 136.0f;
  d = __uint_as_float(sz & 0xffff0000u);
}

// Arguments of the full-K strip GEMV (mtl_w4strip.hip), M = 1.  The source of x is xpart
// (SiLU*up), else hn (RMSNorm), else x (gathered through perm when set, GPTQ metadata and
// the store epilogue only); the epilogue is SiLU*up into act when act is set
// (RMSNorm source only), the residual add when h is set, else a store to y (fp32) or y16
// (bf16).  fmt is the group metadata (STRIP_META_*): with STRIP_META_QSZ, scales points at
// the reference's qsz and qzeros is unused.
struct StripArgs {
  const u32x4* w;             // strip layout of mtl_w4_strip
  const uint16_t* scales;     // strip-ordered fp16 scales, or the qsz pairs
  const uint32_t* qzeros;     // strip-ordered zero nibbles (GPTQ metadata)
  const uint16_t* x;          // bf16 [K] in the weight's input order, or (perm set) in
  const uint16_t* perm;       //   the checkpoint's order: row k of the weight is x[perm[k]]
  const float* xpart;         // gate|up partials [xsplits, xpart_ld]
  const uint16_t* hn;         // residual stream h [K] (input order), norm weight [K],
  const uint16_t* wn;         //   sums of squares of h per 16 columns
  const float* slots;
  float* y;                   // fp32 [N]
  uint16_t* y16;              // bf16 [N] (store epilogue, when set instead of y)
  uint16_t* h;                // bf16 [N], updated in place
  const int32_t* scatter;     // h_ord[scatter[n]] = h[n] (NULL: identity)
  uint16_t* h_ord;            // may be NULL
  float* slots_out;           // one sum of squares per 16 columns
  uint16_t* act;              // bf16 [N/2]: silu(gate) * up, 32-column gate|up interleave
  int xsplits, xpart_ld;
  float eps;
  int K, N, group;
  int16_t zero_offset, kblocks, xcd_order, fmt;
  int16_t xhalves;            // xpart splits hold [gate K | up K] (else the 32-column interleave)
  mtl_strip_geometry geom;    // requested launch shape (all 0: automatic)
};
// The launch passes StripArgs by value: its 184 bytes put the kernel's arguments at 440
// bytes with the hidden ones; at 448 (8 bytes more) every strip launch measured about
// 0.25 us slower.
static_assert(sizeof(StripArgs) == 184, "StripArgs size");

enum : int { STRIP_EPI_STORE = 0, STRIP_EPI_RESID = 1, STRIP_EPI_SILU = 2 };

// Blocks (128 input channels) per wave of the strip GEMV for this K with ct strips per
// workgroup at this group size; 0: unsupported.
int strip_blocks_per_wave(int64_t K, int ct, int group);
// Launch the strip GEMV; shapes, pointers and alignment are checked by the caller.
int strip_launch(const StripArgs& a, hipStream_t stream);
struct Bf16RowsArgs;
// The RMSNorm-staged strip GEMV and a bf16 kept projection (gb workgroups of its rows) in
// one launch; MTL_ERR_UNSUPPORTED where that launch shape does not apply.
int strip_launch_bf16(const StripArgs& a, const Bf16RowsArgs& b, int gb, hipStream_t stream);

// The skinny-batch strip GEMM (mtl_w4rows.hip) for 1 <= M <= 16 rows: fmt is STRIP_META_*,
// perm (GPTQ metadata only) gathers x's channels; checks shapes and alignment itself.
int strip_rows(const void* x, int64_t M, int64_t ldx, int64_t K, const int32_t* perm,
               const int32_t* strip_weight, const void* meta, const int32_t* qzeros, int64_t N,
               int32_t group_size, int32_t zero_offset, int fmt, void* y, int64_t ldy,
               int32_t out_dtype, void* stream);

// Whether the skinny-batch strip GEMM pays at M rows over N columns (without an act-order
// gather): measured on MI355X it is ahead of the prompt-length GEMM at every M <= 16 on the
// four decode shapes, g32 and g128 (q|k|v 6.5-9.1 against 14.2-17.7 us, down 9.8-21.9
// against 19.9-25.6 us, weights rotated past the Infinity Cache).
inline bool strip_rows_pays(int64_t M, int64_t /*N*/) { return M <= 16; }

// The residual add of the decode step (fast.py:168-171) on 4 consecutive columns:
// h = bf16(bf16(acc) + h); returns their sum of squares (fixed fma order).
__device__ __forceinline__ float residual4(const float acc[4], float hv[4]) {
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    hv[c] = round_bf16(round_bf16(acc[c]) + hv[c]);
    ss = fmaf(hv[c], hv[c], ss);
  }
  return ss;
}

}  // namespace mtl
