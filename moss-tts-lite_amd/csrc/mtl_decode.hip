// Decode-step kernels around the int4 GEMV (gfx950): RMSNorm, embedding sum, q/k norm +
// RoPE + KV-cache write, GQA decode attention, bf16 head GEMV with greedy argmax.
//
// Rounding follows the reference's bf16 tensor ops step by step (every bf16 tensor op
// computes in fp32 and rounds to bf16); reductions run in a fixed order, so every
// launch is bitwise repeatable.
#include "mtl_common.h"
#include "mtl_bf16rows.h"
#include "mtl_decode.h"

namespace mtl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ----------------------------------------------------------------------------------
// RMSNorm (model.py:34-40): fp32 sum of squares, x * rsqrt(mean + eps) rounded to
// bf16, then the bf16 weight product rounded to bf16.
// ----------------------------------------------------------------------------------
__global__ void __launch_bounds__(256) rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w,
                                                      uint16_t* out, int n, float eps) {
  __shared__ float red[4];
  const uint16_t* xr = x + (size_t)blockIdx.x * n;
  uint16_t* orow = out + (size_t)blockIdx.x * n;
  float ss = 0.f;
  for (int i = threadIdx.x * 8; i < n; i += 256 * 8) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + i);
    const uint32_t a[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float f0 = lo_bf(a[j]), f1 = hi_bf(a[j]);
      ss = fmaf(f0, f0, ss);
      ss = fmaf(f1, f1, ss);
    }
  }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float r = rsqrtf(total / (float)n + eps);
  for (int i = threadIdx.x * 8; i < n; i += 256 * 8) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + i);
    const u32x4 g = *reinterpret_cast<const u32x4*>(w + i);
    const uint32_t a[4] = {v.x, v.y, v.z, v.w};
    const uint32_t b[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float y0 = round_bf16(lo_bf(b[j]) * round_bf16(lo_bf(a[j]) * r));
      const float y1 = round_bf16(hi_bf(b[j]) * round_bf16(hi_bf(a[j]) * r));
      o[j] = f32_to_bf16(y0) | (f32_to_bf16(y1) << 16);
    }
    *reinterpret_cast<u32x4*>(orow + i) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// ----------------------------------------------------------------------------------
// Residual add + RMSNorm for the fused step (fast.py:168-169 then model.py:34-40): the
// residual stream h gets bf16(bf16(sum of the split-K partials of the projection) + h),
// then x = RMSNorm(h) is written in the order the next int4 GEMV reads its input
// (x_out[j] = x[gather[j]] for an act-order layer).  One 1024-thread workgroup.
// ----------------------------------------------------------------------------------
constexpr int kNormThreads = 1024;
constexpr int kNormMaxQuads = 4;   // n <= 16384

__global__ void __launch_bounds__(kNormThreads) residual_rmsnorm_kernel(
    const float* __restrict__ part, int splits, const uint16_t* resid, uint16_t* h_out,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ x_out,
    const int32_t* __restrict__ gather, int n, float eps) {
  extern __shared__ uint16_t xs[];   // n bf16 normalised values
  __shared__ float red[kNormThreads / 64];
  const int t = threadIdx.x;
  const int quads = n / 4;
  float hv[kNormMaxQuads][4];
  float ss = 0.f;
#pragma unroll
  for (int qi = 0; qi < kNormMaxQuads; ++qi) {
    const int q = t + qi * kNormThreads;
    if (q < quads) {
      const uint2 rr = *reinterpret_cast<const uint2*>(resid + 4 * q);
      const float r4[4] = {lo_bf(rr.x), hi_bf(rr.x), lo_bf(rr.y), hi_bf(rr.y)};
      if (part) {
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < splits; s0 += 8) {   // 8 independent loads, summed in order
          float4 pv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j)
            pv[j] = *reinterpret_cast<const float4*>(
                part + (size_t)(s0 + j < splits ? s0 + j : splits - 1) * n + 4 * q);
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (s0 + j < splits) {
              acc[0] += pv[j].x; acc[1] += pv[j].y; acc[2] += pv[j].z; acc[3] += pv[j].w;
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) hv[qi][c] = round_bf16(round_bf16(acc[c]) + r4[c]);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) hv[qi][c] = r4[c];
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) ss = fmaf(hv[qi][c], hv[qi][c], ss);
    }
  }
  ss = wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) total += red[i];
  const float r = rsqrtf(total / (float)n + eps);
#pragma unroll
  for (int qi = 0; qi < kNormMaxQuads; ++qi) {
    const int q = t + qi * kNormThreads;
    if (q < quads) {
      const uint2 ww = *reinterpret_cast<const uint2*>(w + 4 * q);
      const float w4[4] = {lo_bf(ww.x), hi_bf(ww.x), lo_bf(ww.y), hi_bf(ww.y)};
      uint32_t hb[4], xb[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        hb[c] = f32_to_bf16(hv[qi][c]);
        xb[c] = f32_to_bf16(round_bf16(w4[c] * round_bf16(hv[qi][c] * r)));
      }
      if (part) *reinterpret_cast<uint2*>(h_out + 4 * q) = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
      if (gather) {
#pragma unroll
        for (int c = 0; c < 4; ++c) xs[4 * q + c] = (uint16_t)xb[c];
      } else {
        *reinterpret_cast<uint2*>(x_out + 4 * q) = make_uint2(xb[0] | (xb[1] << 16), xb[2] | (xb[3] << 16));
      }
    }
  }
  if (gather) {
    __syncthreads();
    for (int j = t; j < n; j += kNormThreads) x_out[j] = xs[gather[j]];
  }
}

// ----------------------------------------------------------------------------------
// Residual add without the norm (the next int4 GEMV applies RMSNorm while staging):
// h = bf16(bf16(sum of split-K partials) + h), one 64-thread workgroup per 256-column
// block; it publishes the sums of squares per 16 columns (slots) and scatters h into the
// next GEMV's act-order input order (h_ord[scatter[i]] = h[i]).
// ----------------------------------------------------------------------------------
constexpr int kResidCols = 256;

__global__ void __launch_bounds__(64) residual_add_kernel(
    const float* __restrict__ part, int splits, uint16_t* h, const int32_t* __restrict__ scatter,
    uint16_t* __restrict__ h_ord, float* __restrict__ slots, int n) {
  const int b = blockIdx.x, t = threadIdx.x;
  const int i = b * kResidCols + 4 * t;   // this thread's 4 columns
  float ss = 0.f;
  if (i < n) {
    const uint2 rr = *reinterpret_cast<const uint2*>(h + i);
    float hv[4] = {lo_bf(rr.x), hi_bf(rr.x), lo_bf(rr.y), hi_bf(rr.y)};
    if (part) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < splits; s0 += 8) {   // 8 independent loads, summed in order
        float4 pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          pv[j] = *reinterpret_cast<const float4*>(
              part + (size_t)(s0 + j < splits ? s0 + j : splits - 1) * n + i);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (s0 + j < splits) {
            acc[0] += pv[j].x; acc[1] += pv[j].y; acc[2] += pv[j].z; acc[3] += pv[j].w;
          }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) hv[c] = round_bf16(round_bf16(acc[c]) + hv[c]);
      *reinterpret_cast<uint2*>(h + i) =
          make_uint2(f32_to_bf16(hv[0]) | (f32_to_bf16(hv[1]) << 16),
                     f32_to_bf16(hv[2]) | (f32_to_bf16(hv[3]) << 16));
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      ss = fmaf(hv[c], hv[c], ss);
      if (h_ord) h_ord[scatter ? scatter[i + c] : i + c] = (uint16_t)f32_to_bf16(hv[c]);
    }
  }
  ss = slot_combine(ss);
  if ((t & 3) == 0 && i < n) slots[i / kSlotCols] = ss;
}

// ----------------------------------------------------------------------------------
// Embedding sum (model.py:156-161): sequential bf16 adds of one row per table.
// ----------------------------------------------------------------------------------
constexpr int kEmbedMaxTables = 64;
constexpr int kEmbedBatch = 17;      // table rows whose loads are in flight together (MOSS: 33 in two)

// STATS: also the first RMSNorm's statistics of the sum and its copy in the first GEMV's
// input order, as residual_add_kernel forms them after a residual add: slots[b] = the sum
// of squares of columns 16b .. 16b+15 (each 4 consecutive columns by a chain of FMAs, the
// four chains joined as slot_combine joins them, so the bits are the same) and
// h_ord[scatter[d]] = out[d] (scatter NULL: h_ord[d]; h_ord NULL: no copy).  Every lane of
// a wave holds a column (hidden % 64 == 0).
template <bool STATS>
__global__ void embed_sum_kernel(const int64_t* __restrict__ ids, int n_tables,
                                 const uint16_t* const* __restrict__ tables,
                                 const int64_t* __restrict__ vocabs, int64_t hidden,
                                 uint16_t* __restrict__ out, const int32_t* __restrict__ scatter,
                                 uint16_t* __restrict__ h_ord, float* __restrict__ slots) {
  // each table's row once per workgroup: its address and its length in bytes, 0 for an id
  // outside the table.  The element reads are buffer loads over that range, so an empty
  // range reads 0 with no branch, and the loads of kEmbedBatch tables go out together.
  __shared__ const uint16_t* rows[kEmbedMaxTables];
  __shared__ int row_bytes[kEmbedMaxTables];
  for (int i = threadIdx.x; i < n_tables; i += blockDim.x) {
    const int64_t id = ids[i];
    const bool ok = id >= 0 && id < vocabs[i];
    rows[i] = ok ? tables[i] + id * hidden : tables[i];
    row_bytes[i] = ok ? (int)(hidden * 2) : 0;
  }
  __syncthreads();
  for (int64_t d = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; d < hidden;
       d += (int64_t)gridDim.x * blockDim.x) {
    float h = 0.f;
    for (int i0 = 0; i0 < n_tables; i0 += kEmbedBatch) {
      float v[kEmbedBatch];
#pragma unroll
      for (int j = 0; j < kEmbedBatch; ++j) {
        const int i = i0 + j < n_tables ? i0 + j : 0;
        // the same LDS word in every lane: wave-uniform, so the descriptor lives in SGPRs
        const uint64_t ra = reinterpret_cast<uint64_t>(rows[i]);
        const uint64_t ru = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(ra >> 32)) << 32) |
                            (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)ra);
        const int nb = __builtin_amdgcn_readfirstlane(i0 + j < n_tables ? row_bytes[i] : 0);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            reinterpret_cast<void*>(ru), (short)0, nb, 0x00020000);
        v[j] = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(rs, (int)(d * 2), 0, 0));
      }
#pragma unroll
      for (int j = 0; j < kEmbedBatch; ++j)   // summed in table order, rounded as before
        if (i0 + j < n_tables) h = (i0 + j == 0) ? v[j] : round_bf16(h + v[j]);
    }
    const uint32_t hb = f32_to_bf16(h);
    out[d] = (uint16_t)hb;
    if constexpr (STATS) {
      const float hv = bf16_to_f32(hb);
      if (h_ord) h_ord[scatter ? scatter[d] : d] = (uint16_t)hb;
      const int lane = threadIdx.x & 63;
      const float h1 = __shfl(hv, lane + 1), h2 = __shfl(hv, lane + 2), h3 = __shfl(hv, lane + 3);
      float ss = fmaf(hv, hv, 0.f);              // lane 4q: columns 4q .. 4q+3 in order
      ss = fmaf(h1, h1, ss);
      ss = fmaf(h2, h2, ss);
      ss = fmaf(h3, h3, ss);
      ss += __shfl_xor(ss, 4);                   // slot_combine over the 4 column quads
      ss += __shfl_xor(ss, 8);
      if ((lane & 15) == 0) slots[d / kSlotCols] = ss;
    }
  }
}

// ----------------------------------------------------------------------------------
// q/k RMSNorm + RoPE + KV write (fast.py:134-147).  One 64-lane workgroup per head;
// lane t owns dims t and t + 64, which are exactly RoPE's rotate-half pair.
// ----------------------------------------------------------------------------------
template <bool PART>
__global__ void __launch_bounds__(64) qk_norm_rope_kv_kernel(
    const uint16_t* __restrict__ qkv, const float* __restrict__ part, int splits, int ncols,
    const uint16_t* __restrict__ qn,
    const uint16_t* __restrict__ kn, const uint16_t* __restrict__ cos_tab,
    const uint16_t* __restrict__ sin_tab, const int64_t* __restrict__ pos_ptr,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    int H, int Hkv, int64_t max_seq, float eps) {
  constexpr int D = 128;
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const int64_t pos = *pos_ptr;
  if (pos < 0 || pos >= max_seq) return;
  float x0, x1;   // the projection outputs (bf16 values) of dims t and t + 64
  if (PART) {       // sum the split-K partials of the q|k|v GEMV in split order, round to bf16
    const float* p0 = part + (size_t)b * D + t;
    float a0 = 0.f, a1 = 0.f;
    for (int s0 = 0; s0 < splits; s0 += 8) {
      float v0[8], v1[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const size_t off = (size_t)(s0 + j < splits ? s0 + j : splits - 1) * ncols;
        v0[j] = p0[off];
        v1[j] = p0[off + 64];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < splits) { a0 += v0[j]; a1 += v1[j]; }
    }
    x0 = round_bf16(a0);
    x1 = round_bf16(a1);
  } else {
    const uint16_t* src = qkv + (size_t)b * D;
    x0 = bf16_to_f32(src[t]);
    x1 = bf16_to_f32(src[t + 64]);
  }
  if (b >= H + Hkv) {   // v head: copied unchanged
    uint16_t* dst = vc + ((size_t)(b - H - Hkv) * max_seq + pos) * D;
    dst[t] = (uint16_t)f32_to_bf16(x0);
    dst[t + 64] = (uint16_t)f32_to_bf16(x1);
    return;
  }
  const uint16_t* w = b < H ? qn : kn;
  float ss = fmaf(x0, x0, x1 * x1);
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / (float)D + eps);
  const float n0 = round_bf16(bf16_to_f32(w[t]) * round_bf16(x0 * r));
  const float n1 = round_bf16(bf16_to_f32(w[t + 64]) * round_bf16(x1 * r));
  const uint16_t* cr = cos_tab + pos * D;
  const uint16_t* sr = sin_tab + pos * D;
  // q*cos + rotate_half(q)*sin, rotate_half(q) = cat(-q[64:], q[:64]); each product and
  // the sum rounded to bf16 as separate bf16 tensor ops.
  const float o0 = round_bf16(round_bf16(n0 * bf16_to_f32(cr[t])) +
                              round_bf16(-n1 * bf16_to_f32(sr[t])));
  const float o1 = round_bf16(round_bf16(n1 * bf16_to_f32(cr[t + 64])) +
                              round_bf16(n0 * bf16_to_f32(sr[t + 64])));
  uint16_t* dst = b < H ? q_out + (size_t)b * D : kc + ((size_t)(b - H) * max_seq + pos) * D;
  dst[t] = (uint16_t)f32_to_bf16(o0);
  dst[t + 64] = (uint16_t)f32_to_bf16(o1);
}

// ----------------------------------------------------------------------------------
// GQA decode attention over positions [0, pos] (fast.py:149-162), split over the
// sequence.  Grid (kv head, chunk): nch = min(ceil(L / 64), 64) chunks of at most
// ceil(L / nch) positions, so for L <= 4096 a workgroup scores at most 64 positions in
// one pass with every K and V load in flight at once.  Wave w of a workgroup serves q
// head kvh * n_rep + w (+4, ...).  Scores are lane-per-position dot products against the
// wave-uniform q; the value sum gives each lane 8 dims of 16 positions (u32x4 loads),
// reduced across the 4 position groups at the end.  Each chunk publishes
// (max, sum, o[128]); the last workgroup of a kv head to finish (agent-scope counter)
// merges that head group's chunks in chunk order, so there is no second launch.
// With FROM_PART, q/k RMSNorm, RoPE and the KV write of position pos run in the
// prologue from the q|k|v split-K partials (fast.py:134-147); the workgroup holding pos
// uses its LDS copy of k/v for that position.
// ----------------------------------------------------------------------------------
constexpr int kAttnBlock = 64;        // positions per pass
constexpr int kAttnMaxChunks = 64;
constexpr int kAttnMaxRep = 8;        // q heads per kv head
constexpr int kAttnPart = 132;        // m, l, 2 pad, o[128]
constexpr int kAttnCounterBytes = 1024;
// The tile kernel's XCD-local hand-off keeps a 64-bit counter per kv head and, in the
// last 8 bytes of the counter area, the number of launches whose chunk workgroups of one
// kv head were found on more than one XCD.
constexpr int kAttnPlacementWord = kAttnCounterBytes - 8;
constexpr int kAttnMaxKvLocal = kAttnPlacementWord / 8;

// XCD (XCC) id of the executing workgroup, hardware register XCC_ID bits [2:0].
__device__ __forceinline__ uint32_t xcc_id() {
  return (uint32_t)__builtin_amdgcn_s_getreg((2 << 11) | (0 << 6) | 20) & 7u;
}

// The first 8 split-K partials of one head's dims (t, t+64), loaded ahead of use; the
// sum (with any further splits) comes later from head_sum.
struct HeadPart {
  float v0[8], v1[8];
};

__device__ __forceinline__ void head_issue(const float* __restrict__ part, int splits, int ncols,
                                           int head, int t, HeadPart& hp) {
  const float* p0 = part + (size_t)head * 128 + t;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const size_t off = (size_t)(j < splits ? j : splits - 1) * ncols;
    hp.v0[j] = p0[off];
    hp.v1[j] = p0[off + 64];
  }
}

__device__ __forceinline__ void head_sum(const float* __restrict__ part, int splits, int ncols,
                                         int head, int t, HeadPart& hp, float& x0, float& x1) {
  float a0 = 0.f, a1 = 0.f;
  for (int s0 = 0; s0 < splits; s0 += 8) {   // splits summed in order
    if (s0 > 0) {
      const float* p0 = part + (size_t)head * 128 + t;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const size_t off = (size_t)(s0 + j < splits ? s0 + j : splits - 1) * ncols;
        hp.v0[j] = p0[off];
        hp.v1[j] = p0[off + 64];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (s0 + j < splits) { a0 += hp.v0[j]; a1 += hp.v1[j]; }
  }
  x0 = round_bf16(a0);
  x1 = round_bf16(a1);
}

struct AttnArgs {
  const uint16_t* q;          // bf16 [H*128] (plain variant)
  const float* qkv_part;      // fp32 [splits, (H+2Hkv)*128] (FROM_PART variant)
  int splits;
  const uint16_t* qn;
  const uint16_t* kn;
  const uint16_t* cos_tab;
  const uint16_t* sin_tab;
  uint16_t* kc;
  uint16_t* vc;
  const int64_t* pos;
  uint16_t* out;
  const int32_t* out_index;
  float* part;                // [H, kAttnMaxChunks, kAttnPart]
  uint32_t* counters;         // [Hkv], zero between launches
  int H, Hkv;
  int64_t max_seq;
  float scale, eps;
  int fixed_chunks;           // chunks are the fixed blocks [64c, 64c + 64)
};


// The merge of one kv head's chunk partials (m, l, o[128]) per q head, in chunk order,
// by the last workgroup of that kv head to finish; out[h*128 + d] (through out_index).
// VALU: the wave reductions on the VALU (wave_max_valu, wave_sum_valu; the same bits).
template <bool VALU, bool LOCAL = false>
__device__ __forceinline__ void attn_merge(const AttnArgs& a, int kvh, int nch, int n_rep,
                                           int wave, int lane, float (*w_lds)[kAttnMaxChunks]) {
  // LOCAL: the partials were written by workgroups of this XCD and sit in its L2; the
  // loads bypass the CU's L1 (sc0) and read them there.  Otherwise the acquire fence of
  // the completing workgroup made them visible and plain loads do.
  constexpr int kPol = LOCAL ? 1 : 0;
  constexpr int D = 128;
  for (int hr = wave; hr < n_rep; hr += 4) {
    const int h = kvh * n_rep + hr;
    const float* ph = a.part + (size_t)h * kAttnMaxChunks * kAttnPart;
    // Every load of the merge is a bounds-checked buffer load issued before any use (the
    // acquire fence of the completing workgroup already made the partials visible): the
    // output columns of dims 2*lane, +1 (a missing out_index reads as 0, replaced below),
    // (m, l) of chunk `lane` and the chunk outputs of dims 2*lane, +1, chunks at or past nch
    // reading as 0.  No load sits under a branch, so none of them waits for another.
    typedef unsigned long long u64;
    const int i0 = h * D + 2 * lane;
    const __amdgpu_buffer_rsrc_t irs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(a.out_index), (short)0, a.out_index ? a.H * D * 4 : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(ph), (short)0, nch * kAttnPart * 4, 0x00020000);
    const u64 oiv = __builtin_bit_cast(u64, __builtin_amdgcn_raw_buffer_load_b64(irs, i0 * 4, 0, 0));
    const u64 ml = __builtin_bit_cast(u64, __builtin_amdgcn_raw_buffer_load_b64(prs, lane * kAttnPart * 4, 0, kPol));
    float mc = __uint_as_float((uint32_t)ml);
    float lc = __uint_as_float((uint32_t)(ml >> 32));   // 0 past nch: the chunk drops out
    // chunk outputs 16 at a time; the first batch goes out with the loads above (peeled:
    // a loop header there made the compiler wait for those first)
    u64 ov[16];
    auto load_batch = [&](int c0) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        ov[j] = __builtin_bit_cast(u64, __builtin_amdgcn_raw_buffer_load_b64(
                                            prs, ((c0 + j) * kAttnPart + 4 + 2 * lane) * 4, 0, kPol));
    };
    float o0 = 0.f, o1 = 0.f;
    // the 16 weights in four 16-byte LDS reads; chunks at or past nch have weight 0 and
    // partials read as 0, so their products add +0 and the sums need no branch
    auto add_batch = [&](int c0) {
      const float4* wp = reinterpret_cast<const float4*>(&w_lds[wave][c0]);
      const float4 w4[4] = {wp[0], wp[1], wp[2], wp[3]};
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float4 q = w4[j >> 2];
        const float wj = (j & 3) == 0 ? q.x : (j & 3) == 1 ? q.y : (j & 3) == 2 ? q.z : q.w;
        o0 = fmaf(wj, __uint_as_float((uint32_t)ov[j]), o0);
        o1 = fmaf(wj, __uint_as_float((uint32_t)(ov[j] >> 32)), o1);
      }
    };
    load_batch(0);
    {
      const float M = VALU ? wave_max_valu(lc > 0.f ? mc : -INFINITY)
                           : wave_max(lc > 0.f ? mc : -INFINITY);
      const float wc = lc > 0.f ? expf(mc - M) : 0.f;
      w_lds[wave][lane] = wc;
      lc = VALU ? wave_sum_valu(wc * lc) : wave_sum(wc * lc);   // Ls from here on
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    add_batch(0);
    for (int c0 = 16; c0 < nch; c0 += 16) {
      load_batch(c0);
      add_batch(c0);
    }
    const float Ls = lc;
    const float r0 = Ls > 0.f ? o0 / Ls : 0.f, r1 = Ls > 0.f ? o1 / Ls : 0.f;
    const int2 oi = a.out_index ? make_int2((int)(uint32_t)oiv, (int)(uint32_t)(oiv >> 32))
                                : make_int2(i0, i0 + 1);
    a.out[oi.x] = (uint16_t)f32_to_bf16(r0);
    a.out[oi.y] = (uint16_t)f32_to_bf16(r1);
  }
}

template <bool FROM_PART>
__global__ void __launch_bounds__(256) attn_decode_kernel(AttnArgs a) {
  constexpr int D = 128;
  __shared__ u32x4 q_lds[kAttnMaxRep][16];
  __shared__ u32x4 kpos[16], vpos[16];
  __shared__ float e_lds[4][kAttnBlock];
  __shared__ __attribute__((aligned(16))) float w_lds[4][kAttnMaxChunks];
  __shared__ int last_flag;
  const int kvh = blockIdx.x, c = blockIdx.y;
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int n_rep = a.H / a.Hkv;
  // 0. The q|k|v partials of this wave's first q head (and, on waves 0/1, of this kv
  //    head's k or v) do not depend on the position: in flight before it is read.
  const int ncols = (a.H + 2 * a.Hkv) * D;
  HeadPart hq, hkv;
  if (FROM_PART && wave < n_rep)
    head_issue(a.qkv_part, a.splits, ncols, kvh * n_rep + wave, lane, hq);
  const uint16_t* kbase = a.kc + (size_t)kvh * a.max_seq * D;
  const uint16_t* vbase = a.vc + (size_t)kvh * a.max_seq * D;
  const int dg = lane & 15, ps = lane >> 4;           // value pass: dims 8dg.., positions ps+4i
  u32x4 kr[16], vr[16];
  // K rows and V slices of positions [base, base + 64) of this kv head, clamped to `last`
  // (a position in the cache)
  auto load_k = [&](int base, int last) {
    const int pk = base + lane < last ? base + lane : last;
    const u32x4* krow = reinterpret_cast<const u32x4*>(kbase + (size_t)pk * D);
#pragma unroll
    for (int i = 0; i < 16; ++i) kr[i] = krow[i];
  };
  auto load_v = [&](int base, int last) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int pv = base + ps + 4 * i < last ? base + ps + 4 * i : last;
      vr[i] = *reinterpret_cast<const u32x4*>(vbase + (size_t)pv * D + 8 * dg);
    }
  };
  // With max_seq <= 64 * 64 every chunk is the fixed block [64c, 64c + 64), so its K rows
  // load before the position is known (rows at or past the length are masked); V, needed
  // only after the scores, waits for the position (chunks past the length load nothing
  // more).
  const bool fixed = a.fixed_chunks;
  if (fixed) load_k(c * kAttnBlock, (int)a.max_seq - 1);
  const int64_t pos = *a.pos;
  int64_t L64 = pos + 1;
  if (L64 < 0) L64 = 0;
  if (L64 > a.max_seq) L64 = a.max_seq;
  const int L = (int)L64;
  int nch = (L + kAttnBlock - 1) / kAttnBlock;
  if (nch > kAttnMaxChunks) nch = kAttnMaxChunks;
  if (c >= nch) return;                               // uniform over the workgroup
  const int clen = fixed ? kAttnBlock : (L + nch - 1) / nch;
  const int p0 = c * clen;
  const int p1 = p0 + clen < L ? p0 + clen : L;       // p0 < p1 unless the chunk is empty
  const bool has_pos = pos >= p0 && pos < p1;

  // 1. The first block's V slices (and, unless fixed, K rows), before the q prologue.
  auto load_block = [&](int base) {
    load_k(base, p1 - 1 > 0 ? p1 - 1 : 0);
    load_v(base, p1 - 1 > 0 ? p1 - 1 : 0);
  };
  if (fixed) load_v(p0, p1 - 1 > 0 ? p1 - 1 : 0);
  else if (p0 < p1) load_block(p0);
  if (FROM_PART && has_pos && wave < 2)   // k (wave 0) or v (wave 1) of position pos
    head_issue(a.qkv_part, a.splits, ncols, (wave == 0 ? a.H : a.H + a.Hkv) + kvh, lane, hkv);

  // 2. Prologue: q heads into LDS; k/v of position pos (cache + LDS) where it is scored.
  const size_t prow = (size_t)(pos >= 0 && pos < a.max_seq ? pos : 0) * D;
  if (FROM_PART) {
    const uint16_t* cr = a.cos_tab + prow;
    const uint16_t* sr = a.sin_tab + prow;
    if (has_pos && wave < 2) {
      float x0, x1;
      head_sum(a.qkv_part, a.splits, ncols, (wave == 0 ? a.H : a.H + a.Hkv) + kvh, lane, hkv,
               x0, x1);
      if (wave == 0) norm_rope_pair(x0, x1, a.kn, cr, sr, lane, a.eps, x0, x1);
      const uint32_t b0 = f32_to_bf16(x0), b1 = f32_to_bf16(x1);
      uint16_t* dst = (wave == 0 ? a.kc : a.vc) + ((size_t)kvh * a.max_seq + pos) * D;
      dst[lane] = (uint16_t)b0;
      dst[lane + 64] = (uint16_t)b1;
      uint16_t* l16 = reinterpret_cast<uint16_t*>(wave == 0 ? kpos : vpos);
      l16[lane] = (uint16_t)b0;
      l16[lane + 64] = (uint16_t)b1;
    }
    for (int hr = wave; hr < n_rep; hr += 4) {
      float x0, x1;
      if (hr != wave) head_issue(a.qkv_part, a.splits, ncols, kvh * n_rep + hr, lane, hq);
      head_sum(a.qkv_part, a.splits, ncols, kvh * n_rep + hr, lane, hq, x0, x1);
      norm_rope_pair(x0, x1, a.qn, cr, sr, lane, a.eps, x0, x1);
      uint16_t* l16 = reinterpret_cast<uint16_t*>(q_lds[hr]);
      l16[lane] = (uint16_t)f32_to_bf16(x0);
      l16[lane + 64] = (uint16_t)f32_to_bf16(x1);
    }
  } else {
    for (int hr = wave; hr < n_rep; hr += 4)
      if (lane < 16)
        q_lds[hr][lane] =
            reinterpret_cast<const u32x4*>(a.q + (size_t)(kvh * n_rep + hr) * D)[lane];
    if (has_pos && wave < 2 && lane < 16)   // the cache already holds k/v of pos
      (wave == 0 ? kpos : vpos)[lane] =
          reinterpret_cast<const u32x4*>((wave == 0 ? kbase : vbase) + (size_t)pos * D)[lane];
  }
  __syncthreads();

  // 3. Scores, softmax and the value sum, one 64-position block at a time.
  for (int hr = wave; hr < n_rep; hr += 4) {
    const int h = kvh * n_rep + hr;
    float m = -INFINITY, l = 0.f;
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = 0.f;
    for (int base = p0; base < p1; base += kAttnBlock) {
      if (base != p0 || hr != wave) load_block(base);
      const int p = base + lane;
      float acc = 0.f;
      if (p == pos) {
#pragma unroll
        for (int i = 0; i < 16; ++i) kr[i] = kpos[i];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const u32x4 qq = q_lds[hr][i];
        acc = dot2_bf16(kr[i].x, qq.x, acc);
        acc = dot2_bf16(kr[i].y, qq.y, acc);
        acc = dot2_bf16(kr[i].z, qq.z, acc);
        acc = dot2_bf16(kr[i].w, qq.w, acc);
      }
      const float s = p < p1 ? acc * a.scale : -INFINITY;
      const float mn = fmaxf(m, wave_max(s));
      const float e = p < p1 ? expf(s - mn) : 0.f;
      const float corr = expf(m - mn);
      l = fmaf(l, corr, wave_sum(e));
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] *= corr;
      m = mn;
      // the value sum takes e rounded to bf16, the sum l the unrounded e: the form of
      // torch's fused SDPA on bf16 tensors (moss_tts_lite/model.py:183-189)
      e_lds[wave][(lane & 3) * 16 + (lane >> 2)] = round_bf16(e);   // position ps+4i at ps*16+i
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float ei = e_lds[wave][ps * 16 + i];
        const int pv = base + ps + 4 * i;
        const u32x4 v = pv == pos ? vpos[dg] : pv < p1 ? vr[i] : u32x4{0u, 0u, 0u, 0u};
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          o[2 * j] = fmaf(ei, lo_bf(w4[j]), o[2 * j]);
          o[2 * j + 1] = fmaf(ei, hi_bf(w4[j]), o[2 * j + 1]);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o[j] += __shfl_xor(o[j], 16);
      o[j] += __shfl_xor(o[j], 32);
    }
    // publish (m, l, o) with agent-scope stores: visible to the merging workgroup on
    // any XCD without a whole-L2 writeback
    float* ph = a.part + ((size_t)h * kAttnMaxChunks + c) * kAttnPart;
    if (lane == 0) {
      __hip_atomic_store(ph, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(ph + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (lane < 16) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        __hip_atomic_store(ph + 4 + 8 * dg + j, o[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // 4. The last workgroup of this kv head merges its q heads' chunks in chunk order.
  // The count is a release (every partial store of the workgroup happens before it, through
  // the barrier) and the workgroup that makes it complete takes an acquire fence before any
  // thread reads the partials: the hand-off is ordered by the memory model, not only by the
  // store acknowledgements.
  __builtin_amdgcn_s_waitcnt(0);      // every partial store acknowledged before the count
  __syncthreads();
  if (threadIdx.x == 0) {
    last_flag = __hip_atomic_fetch_add(&a.counters[kvh], 1u, __ATOMIC_RELEASE,
                                       __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(nch - 1);
    if (last_flag) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (!last_flag) return;
  if (threadIdx.x == 0)
    __hip_atomic_store(&a.counters[kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  attn_merge<false>(a, kvh, nch, n_rep, wave, lane, w_lds);
}

// ----------------------------------------------------------------------------------
// Tile form of the decode attention, for max_seq <= 64 * 64: chunk c is the fixed block
// [64c, 64c + 64) of positions.  The workgroup loads the chunk's K and V rows once, before
// the position is read, and stages them in LDS.  Wave w scores positions 16w .. 16w+15
// against every q head of the kv head with four v_mfma_f32_16x16x32_bf16 (A = K rows,
// B = the q heads as columns).  The chunk softmax max and sum meet across the 4 waves
// in LDS, and O^T = V^T E^T runs on MFMA with the V^T operand read from the V rows by
// ds_read_b64_tr_b16 (a wave per 32 dims, every q head at once).  Every cross-lane step of
// this kernel (q/k RMSNorm, softmax, the merge) runs on the VALU (permlane swaps and DPP,
// mtl_common.h) instead of ds_bpermute: the same bits, about 0.5 us less per launch in the
// decode step.  The published (m, l, o[128]) per q head and the merge are those of
// attn_decode_kernel.
// ----------------------------------------------------------------------------------
template <bool FROM_PART, bool LOCAL>
__global__ void __launch_bounds__(256) attn_tile_kernel(AttnArgs a) {
  constexpr int D = 128, P = kAttnBlock;
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef float f4 __attribute__((ext_vector_type(4)));
  // rows padded by one item: the MFMA operand reads take one item from each of 16 rows,
  // which a 256-byte row stride would put in the same four LDS banks
  __shared__ u32x4 k_lds[P][17];                // the chunk's K rows, 8 dims per item
  __shared__ u32x4 v_lds[P][17];
  __shared__ u32x4 q_lds[16][17];               // q heads (rows past n_rep zero)
  __shared__ __attribute__((aligned(16))) float e_lds[kAttnMaxRep][P];   // exp(s - m), bf16 values
  __shared__ float red_m[4][16], red_l[4][16];  // per-wave max / sum per q head
  __shared__ __attribute__((aligned(16))) float w_lds[4][kAttnMaxChunks];
  __shared__ int last_flag;
  const int kvh = blockIdx.x, c = blockIdx.y;
  const int t = threadIdx.x, wave = wave_id(), lane = t & 63;
  const int n_rep = a.H / a.Hkv;
  // 0. Loads that do not depend on the position: this wave's first q head partials and
  //    the chunk's K/V rows (thread t: items t + 256j = row item/16, dims 8*(item%16)).
  const int ncols = (a.H + 2 * a.Hkv) * D;
  HeadPart hq, hkv;
  if (FROM_PART && wave < n_rep)
    head_issue(a.qkv_part, a.splits, ncols, kvh * n_rep + wave, lane, hq);
  // k (wave 0) and v (wave 1) of this kv head at position pos, loaded by every workgroup
  // before pos is known: only the one holding pos uses them, but its prologue then needs
  // no second round trip after the position arrives
  if (FROM_PART && wave < 2)
    head_issue(a.qkv_part, a.splits, ncols, (wave == 0 ? a.H : a.H + a.Hkv) + kvh, lane, hkv);
  const uint16_t* kbase = a.kc + (size_t)kvh * a.max_seq * D;
  const uint16_t* vbase = a.vc + (size_t)kvh * a.max_seq * D;
  const int last_row = (int)a.max_seq - 1;
  u32x4 kv[4], vv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int item = t + 256 * j;
    int p = c * P + (item >> 4);
    p = p < last_row ? p : last_row;
    kv[j] = *reinterpret_cast<const u32x4*>(kbase + (size_t)p * D + 8 * (item & 15));
    vv[j] = *reinterpret_cast<const u32x4*>(vbase + (size_t)p * D + 8 * (item & 15));
  }
  const int64_t pos = *a.pos;
  int64_t L64 = pos + 1;
  if (L64 < 0) L64 = 0;
  if (L64 > a.max_seq) L64 = a.max_seq;
  const int L = (int)L64;
  const int nch = (L + P - 1) / P;
  if (c >= nch) return;                               // uniform over the workgroup
  const int p0 = c * P;
  const int p1 = p0 + P < L ? p0 + P : L;
  const bool has_pos = pos >= p0 && pos < p1;

  // 1. Prologue: q heads into LDS; k/v of position pos into the cache and the LDS tile.
  const size_t prow = (size_t)(pos >= 0 && pos < a.max_seq ? pos : 0) * D;
  if (FROM_PART) {
    const uint16_t* cr = a.cos_tab + prow;
    const uint16_t* sr = a.sin_tab + prow;
    if (has_pos && wave < 2) {
      float x0, x1;
      head_sum(a.qkv_part, a.splits, ncols, (wave == 0 ? a.H : a.H + a.Hkv) + kvh, lane, hkv,
               x0, x1);
      if (wave == 0)
        norm_rope_vals<true>(x0, x1, bf16_to_f32(a.kn[lane]), bf16_to_f32(a.kn[lane + 64]),
                             bf16_to_f32(cr[lane]), bf16_to_f32(cr[lane + 64]),
                             bf16_to_f32(sr[lane]), bf16_to_f32(sr[lane + 64]), a.eps, x0, x1);
      const uint32_t b0 = f32_to_bf16(x0), b1 = f32_to_bf16(x1);
      uint16_t* dst = (wave == 0 ? a.kc : a.vc) + ((size_t)kvh * a.max_seq + pos) * D;
      dst[lane] = (uint16_t)b0;
      dst[lane + 64] = (uint16_t)b1;
      uint16_t* l16 = reinterpret_cast<uint16_t*>((wave == 0 ? k_lds : v_lds)[pos - p0]);
      l16[lane] = (uint16_t)b0;
      l16[lane + 64] = (uint16_t)b1;
    }
    for (int hr = wave; hr < n_rep; hr += 4) {
      float x0, x1;
      if (hr != wave) head_issue(a.qkv_part, a.splits, ncols, kvh * n_rep + hr, lane, hq);
      head_sum(a.qkv_part, a.splits, ncols, kvh * n_rep + hr, lane, hq, x0, x1);
      norm_rope_vals<true>(x0, x1, bf16_to_f32(a.qn[lane]), bf16_to_f32(a.qn[lane + 64]),
                           bf16_to_f32(cr[lane]), bf16_to_f32(cr[lane + 64]),
                           bf16_to_f32(sr[lane]), bf16_to_f32(sr[lane + 64]), a.eps, x0, x1);
      uint16_t* l16 = reinterpret_cast<uint16_t*>(q_lds[hr]);
      l16[lane] = (uint16_t)f32_to_bf16(x0);
      l16[lane + 64] = (uint16_t)f32_to_bf16(x1);
    }
  } else {
    for (int hr = wave; hr < n_rep; hr += 4)
      if (lane < 16)
        q_lds[hr][lane] =
            reinterpret_cast<const u32x4*>(a.q + (size_t)(kvh * n_rep + hr) * D)[lane];
  }
  for (int i = n_rep * 16 + t; i < 16 * 16; i += 256) q_lds[i >> 4][i & 15] = u32x4{0u, 0u, 0u, 0u};
  // the chunk's rows; rows at or past the length are zero, and the row of pos comes from
  // the prologue when it computed k/v there
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int item = t + 256 * j;
    const int row = item >> 4, p = p0 + row;
    if (FROM_PART && p == pos) continue;
    const u32x4 z{0u, 0u, 0u, 0u};
    k_lds[row][item & 15] = p < p1 ? kv[j] : z;
    v_lds[row][item & 15] = p < p1 ? vv[j] : z;
  }
  __syncthreads();

  // 2. Scores s[p][h] = K[p] . q[h] on MFMA; lane l holds positions 16w + 4(l/16) + r of
  //    q head l%16.  Chunk softmax: max and sum per head across the 4 waves.
  f4 S = {0.f, 0.f, 0.f, 0.f};
  u32x4 ka[4], qb[4];                           // all 8 operand reads in flight at once
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    ka[k] = k_lds[16 * wave + (lane & 15)][4 * k + (lane >> 4)];
    qb[k] = q_lds[lane & 15][4 * k + (lane >> 4)];
  }
  __builtin_amdgcn_sched_barrier(0);            // keep the scheduler from re-pairing them
#pragma unroll
  for (int k = 0; k < 4; ++k)
    S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[k]),
                                                __builtin_bit_cast(bf16x8, qb[k]), S, 0, 0, 0);
  const int hd = lane & 15, g = lane >> 4;
  float sv[4], mloc = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int p = p0 + 16 * wave + 4 * g + r;
    sv[r] = p < p1 ? S[r] * a.scale : -INFINITY;
    mloc = fmaxf(mloc, sv[r]);
  }
  mloc = xor16_max(mloc);                       // cross-lane steps on the VALU
  mloc = xor32_max(mloc);
  if (g == 0) red_m[wave][hd] = mloc;
  __syncthreads();
  const float M = fmaxf(fmaxf(red_m[0][hd], red_m[1][hd]), fmaxf(red_m[2][hd], red_m[3][hd]));
  float lsum = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float e = expf(sv[r] - M);                  // 0 for masked positions
    // value sum over bf16(e), sum over e: torch's fused SDPA form (model.py:183-189)
    if (hd < n_rep) e_lds[hd][16 * wave + 4 * g + r] = round_bf16(e);
    lsum += e;
  }
  lsum = xor16_add(lsum);
  lsum = xor32_add(lsum);
  if (g == 0) red_l[wave][hd] = lsum;
  __syncthreads();

  // 3. O^T (dims x q heads) = V^T (dims x positions) E^T (positions x heads) on MFMA:
  //    wave w takes dims 32w .. 32w+31 (two 16-dim blocks) for every q head at once.  The
  //    A operand V^T comes straight from the V rows in LDS through ds_read_b64_tr_b16: in
  //    each 16-lane group, lane j reads 4 dims (4(j%4) ..) of position row j/4, and the
  //    transpose hands lane i dim i of those 4 rows; two reads give a lane its 8
  //    positions.  B = E^T: lane (g, hd) packs the bf16 probabilities (rounded above) of
  //    head hd at its 8 positions.  Then publish (m, l, o).
  {
    typedef short s4 __attribute__((ext_vector_type(4)));
    const int hd2 = lane & 15, g2 = lane >> 4;
    bf16x8 eb[2];                                  // B operands of the two 32-position steps
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const float* er = &e_lds[hd2 < n_rep ? hd2 : 0][32 * ks + 8 * g2];
      const float4 e0 = reinterpret_cast<const float4*>(er)[0];
      const float4 e1 = reinterpret_cast<const float4*>(er)[1];
      const float ev[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
      u32x4 w;
      uint32_t* wp = reinterpret_cast<uint32_t*>(&w);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        wp[i] = hd2 < n_rep ? (__float_as_uint(ev[2 * i]) >> 16) |
                                  (__float_as_uint(ev[2 * i + 1]) & 0xffff0000u)
                            : 0u;
      eb[ks] = __builtin_bit_cast(bf16x8, w);
    }
    // this lane's transpose-read addresses: row j/4 of its 8-row step, dims 4(j%4) ..
    const int jr = (lane & 15) >> 2, jc = 4 * (lane & 3);
    f4 acc[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int d0 = 32 * wave + 16 * mb + jc;     // first of this lane's 4 dims
      s4 rv[2][2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int row = 32 * ks + 8 * g2 + 4 * hf + jr;
          const uint16_t* src = reinterpret_cast<const uint16_t*>(v_lds[row]) + d0;
          rv[ks][hf] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (s4 __attribute__((address_space(3)))*)(src));
        }
      acc[mb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const s4 lo = rv[ks][0], hi = rv[ks][1];
        const bf16x8 A = __builtin_bit_cast(
            bf16x8, (short __attribute__((ext_vector_type(8)))){lo[0], lo[1], lo[2], lo[3],
                                                                 hi[0], hi[1], hi[2], hi[3]});
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, eb[ks], acc[mb], 0, 0, 0);
      }
    }
    // acc[mb][r]: dim 32w + 16mb + 4g2 + r of q head hd2
    if (hd2 < n_rep) {
      float* ph = a.part + ((size_t)(kvh * n_rep + hd2) * kAttnMaxChunks + c) * kAttnPart;
      if (wave == 0 && g2 == 0) {
        const float mh = fmaxf(fmaxf(red_m[0][hd2], red_m[1][hd2]), fmaxf(red_m[2][hd2], red_m[3][hd2]));
        const float lh = (red_l[0][hd2] + red_l[1][hd2]) + (red_l[2][hd2] + red_l[3][hd2]);
        if (LOCAL) {
          *reinterpret_cast<float2*>(ph) = make_float2(mh, lh);
        } else {
          __hip_atomic_store(ph, mh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(ph + 1, lh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        float* po = ph + 4 + 32 * wave + 16 * mb + 4 * g2;
        if (LOCAL) {
          // plain stores: they end in this XCD's L2, where the merging workgroup reads them
          *reinterpret_cast<float4*>(po) =
              make_float4(acc[mb][0], acc[mb][1], acc[mb][2], acc[mb][3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            __hip_atomic_store(po + r, acc[mb][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }

  // 4. The last workgroup of this kv head merges its q heads' chunks in chunk order.
  __builtin_amdgcn_s_waitcnt(0);      // every partial store acknowledged before the count
  __syncthreads();
  if (LOCAL) {
    // XCD-local hand-off.  Workgroups are dispatched to the 8 XCDs in turn by linear id
    // and the grid's x extent (the kv heads) is a multiple of 8, so every chunk of kv
    // head kvh (linear ids kvh + gridDim.x * c) runs on one XCD and shares its L2: the
    // partial stores above were acknowledged by that L2, and the count is an atomic
    // there, so the last workgroup reads the partials from the L2 without the agent-scope
    // write-back and invalidate.  Each workgroup adds 1 to the 7-bit field of its own XCD
    // (8 fields); the count is their sum, and a count spread over two fields means the
    // placement did not hold, which is recorded in the placement word.
    if (t == 0) {
      unsigned long long* cnt = reinterpret_cast<unsigned long long*>(a.counters) + kvh;
      const unsigned long long add = 1ull << (7 * xcc_id());
      const unsigned long long tot =
          __hip_atomic_fetch_add(cnt, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
      int n = 0, fields = 0;
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        const int f = (int)((tot >> (7 * x)) & 0x7full);
        n += f;
        fields += f != 0;
      }
      last_flag = n == nch;
      if (n == nch) {
        __hip_atomic_store(cnt, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (fields > 1)
          __hip_atomic_fetch_add(reinterpret_cast<uint32_t*>(
                                     reinterpret_cast<char*>(a.counters) + kAttnPlacementWord),
                                 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
    if (!last_flag) return;
    attn_merge<true, true>(a, kvh, nch, n_rep, wave, lane, w_lds);
    return;
  }
  // Agent-scope hand-off (release count, acquire fence of the completing workgroup, as in
  // attn_decode_kernel).
  if (t == 0) {
    last_flag = __hip_atomic_fetch_add(&a.counters[kvh], 1u, __ATOMIC_RELEASE,
                                       __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(nch - 1);
    if (last_flag) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (!last_flag) return;
  if (t == 0)
    __hip_atomic_store(&a.counters[kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  attn_merge<true>(a, kvh, nch, n_rep, wave, lane, w_lds);
}

// ----------------------------------------------------------------------------------
// bf16 head GEMV + argmax.  Each wave streams a contiguous band of rows (lane l reads
// 16 B at k = 8l + 512i, 1 KB contiguous per wave load), reduces each row across the
// wave, rounds the logit to bf16 and keeps the first maximum; waves then workgroups
// are merged in row order.
// ----------------------------------------------------------------------------------
constexpr int kHeadWGs = 1024;
constexpr int kHeadKitMax = 24;  // K <= 12288 (512 channels per item)

__device__ __forceinline__ bool better(float va, long long ia, float vb, long long ib) {
  if (ia < 0) return false;
  if (ib < 0) return true;
  const bool na = va != va, nb = vb != vb;
  if (na) return !nb || ia < ib;
  if (nb) return false;
  return va > vb || (va == vb && ia < ib);
}

template <int kHeadKit>
__global__ void __launch_bounds__(256) head_gemv_kernel(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ w,
                                                        int64_t N, int K,
                                                        uint16_t* __restrict__ logits,
                                                        float* __restrict__ part_v,
                                                        long long* __restrict__ part_i,
                                                        const uint16_t* __restrict__ norm_w,
                                                        const float* __restrict__ slots,
                                                        float eps, int64_t pad_period,
                                                        int64_t pad_index,
                                                        float* __restrict__ out_f32) {
  __shared__ float sv[4];
  __shared__ long long si[4];
  const int wave = wave_id(), lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * 4 + wave;
  const int64_t nwt = (int64_t)gridDim.x * 4;
  const int64_t r0 = N * gw / nwt, r1 = N * (gw + 1) / nwt;
  const int kit = (K + 511) / 512;
  u32x4 xv[kHeadKit];
#pragma unroll
  for (int i = 0; i < kHeadKit; ++i) {
    const int k = 512 * i + 8 * lane;
    xv[i] = (i < kit && k < K) ? *reinterpret_cast<const u32x4*>(x + k) : u32x4{0u, 0u, 0u, 0u};
  }
  if (norm_w) {   // x is the residual stream: apply the final RMSNorm here (model.py:34-40)
    const float r = rsqrtf(slot_total_valu(slots, K, lane) / (float)K + eps);
#pragma unroll
    for (int i = 0; i < kHeadKit; ++i) {
      const int k = 512 * i + 8 * lane;
      if (i < kit && k < K) {
        const u32x4 g = *reinterpret_cast<const u32x4*>(norm_w + k);
        const uint32_t hh[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
        const uint32_t ww[4] = {g.x, g.y, g.z, g.w};
        uint32_t o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t lo = f32_to_bf16(round_bf16(lo_bf(ww[c]) * round_bf16(lo_bf(hh[c]) * r)));
          const uint32_t hi = f32_to_bf16(round_bf16(hi_bf(ww[c]) * round_bf16(hi_bf(hh[c]) * r)));
          o[c] = lo | (hi << 16);
        }
        xv[i] = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
  }
  float best = 0.f;
  long long bidx = -1;
  constexpr int RB = kHeadKit <= 8 ? 2 : 1;   // rows per pass: their loads in flight together
  for (int64_t rb = r0; rb < r1; rb += RB) {
    u32x4 ww[RB][kHeadKit];
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int64_t r = rb + j < r1 ? rb + j : r1 - 1;
      const uint16_t* wr = w + r * K;
#pragma unroll
      for (int i = 0; i < kHeadKit; ++i) {
        const int k = 512 * i + 8 * lane;
        if (i < kit && k < K)
          ww[j][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + k));
      }
    }
    float acc[RB];
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      acc[j] = 0.f;
#pragma unroll
      for (int i = 0; i < kHeadKit; ++i) {
        const int k = 512 * i + 8 * lane;
        if (i < kit && k < K) {
          acc[j] = dot2_bf16(ww[j][i].x, xv[i].x, acc[j]);
          acc[j] = dot2_bf16(ww[j][i].y, xv[i].y, acc[j]);
          acc[j] = dot2_bf16(ww[j][i].z, xv[i].z, acc[j]);
          acc[j] = dot2_bf16(ww[j][i].w, xv[i].w, acc[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < RB; ++j) {
      const int64_t r = rb + j;
      if (r >= r1) break;
      const float sum = wave_sum_valu(acc[j]);   // cross-lane steps on the VALU
      uint32_t hb = f32_to_bf16(sum);
      if (pad_period > 0 && r % pad_period == pad_index) hb = 0xff80u;   // -inf
      if (logits && lane == 0) logits[r] = (uint16_t)hb;
      if (out_f32 && lane == 0) out_f32[r] = bf16_to_f32(hb);   // the bf16 value, for fp32 readers
      const float lv = bf16_to_f32(hb);
      if (better(lv, r, best, bidx)) {   // rows in ascending order: first maximum kept
        best = lv;
        bidx = r;
      }
    }
  }
  if (!part_v) return;   // logits only
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = bidx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    long long bi = si[0];
    for (int i = 1; i < 4; ++i)
      if (better(sv[i], si[i], b, bi)) {
        b = sv[i];
        bi = si[i];
      }
    part_v[blockIdx.x] = b;
    part_i[blockIdx.x] = bi;
  }
}

// Launch the head GEMV with x held in ceil(K/512) items of 8 channels per lane, on `wgs`
// workgroups (kHeadWGs when an argmax reads the per-workgroup partials).
template <typename... Args>
static void launch_head_on(int wgs, int64_t K, hipStream_t s, Args... args) {
  if (K <= 4096)
    hipLaunchKernelGGL(head_gemv_kernel<8>, dim3(wgs), dim3(256), 0, s, args...);
  else if (K <= 8192)
    hipLaunchKernelGGL(head_gemv_kernel<16>, dim3(wgs), dim3(256), 0, s, args...);
  else
    hipLaunchKernelGGL(head_gemv_kernel<24>, dim3(wgs), dim3(256), 0, s, args...);
}

template <typename... Args>
static void launch_head(int64_t K, hipStream_t s, Args... args) {
  launch_head_on(kHeadWGs, K, s, args...);
}

template <int kKit>
__global__ void __launch_bounds__(256) bf16_rows_norm_kernel(Bf16RowsArgs p) {
  bf16_rows_norm_body<kKit>(p, blockIdx.x);
}

static int g_dec_cus = 0;

static int decode_device_cus() {
  if (!g_dec_cus) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_dec_cus = n;
  }
  return g_dec_cus;
}

__global__ void __launch_bounds__(256) argmax_final_kernel(const float* __restrict__ part_v,
                                                           const long long* __restrict__ part_i,
                                                           int nparts, int64_t* token_out,
                                                           int64_t* pos) {
  __shared__ float sv[256];
  __shared__ long long si[256];
  float b = 0.f;
  long long bi = -1;
  for (int i = threadIdx.x; i < nparts; i += 256)   // ascending: ties keep the lower index
    if (better(part_v[i], part_i[i], b, bi)) {
      b = part_v[i];
      bi = part_i[i];
    }
  sv[threadIdx.x] = b;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s && better(sv[threadIdx.x + s], si[threadIdx.x + s], sv[threadIdx.x],
                                  si[threadIdx.x])) {
      sv[threadIdx.x] = sv[threadIdx.x + s];
      si[threadIdx.x] = si[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    token_out[0] = si[0] < 0 ? 0 : (int64_t)si[0];
    if (pos) pos[0] += 1;   // the step's last launch also advances the position
  }
}

__global__ void advance_position_kernel(int64_t* pos) {
  if (threadIdx.x == 0 && blockIdx.x == 0) pos[0] += 1;
}

// act[i] = bf16(silu(bf16 gate_i) * bf16 up_i) from fp32 projections (fast.py:170-171): the
// SwiGLU of a layer whose up_proj stays bf16 while gate_proj is int4, so the two come from
// separate GEMVs.
__global__ void silu_mul_f32_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                    uint16_t* __restrict__ act, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    act[i] = (uint16_t)silu_mul_bf16(gate[i], up[i]);
}

}  // namespace mtl

using namespace mtl;

extern "C" {

int mtl_rmsnorm(const void* x, const void* w, void* out, int64_t rows, int64_t n, float eps,
                void* stream) {
  if (!x || !w || !out) return MTL_ERR_INVALID_ARG;
  if (rows < 1 || n < 8 || n % 8 != 0 || rows > (1 << 30)) return MTL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w) || !aligned16(out)) return MTL_ERR_ALIGN;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                     static_cast<uint16_t*>(out), (int)n, eps);
  return launch_status();
}

int mtl_embed_sum(const int64_t* ids, int32_t n_tables, const void* const* tables,
                  const int64_t* vocabs, int64_t hidden, void* out, void* stream) {
  if (!ids || !tables || !vocabs || !out) return MTL_ERR_INVALID_ARG;
  if (n_tables < 1 || n_tables > kEmbedMaxTables || hidden < 1 || hidden * 2 >= ((int64_t)1 << 31))
    return MTL_ERR_SHAPE;
  const int blocks = (int)((hidden + 255) / 256);
  hipLaunchKernelGGL(embed_sum_kernel<false>, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     ids, n_tables, reinterpret_cast<const uint16_t* const*>(tables), vocabs,
                     hidden, static_cast<uint16_t*>(out), nullptr, nullptr, nullptr);
  return launch_status();
}

int mtl_embed_sum_stats(const int64_t* ids, int32_t n_tables, const void* const* tables,
                        const int64_t* vocabs, int64_t hidden, void* out, const int32_t* scatter,
                        void* h_ord, float* slots, void* stream) {
  if (!ids || !tables || !vocabs || !out || !slots) return MTL_ERR_INVALID_ARG;
  if (n_tables < 1 || n_tables > kEmbedMaxTables || hidden < 1 || hidden * 2 >= ((int64_t)1 << 31))
    return MTL_ERR_SHAPE;
  if (hidden % kResidCols != 0 || hidden > (int64_t)kSlotCols * kMaxSlots) return MTL_ERR_SHAPE;
  const int blocks = (int)(hidden / 256);
  hipLaunchKernelGGL(embed_sum_kernel<true>, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     ids, n_tables, reinterpret_cast<const uint16_t* const*>(tables), vocabs,
                     hidden, static_cast<uint16_t*>(out), scatter, static_cast<uint16_t*>(h_ord),
                     slots);
  return launch_status();
}

int mtl_qk_norm_rope_kv(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                        const void* cos_tab, const void* sin_tab, const int64_t* pos, void* q_out,
                        void* k_cache, void* v_cache, int32_t n_heads, int32_t n_kv_heads,
                        int32_t head_dim, int64_t max_seq, float eps, void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !pos || !q_out || !k_cache ||
      !v_cache)
    return MTL_ERR_INVALID_ARG;
  if (head_dim != 128) return MTL_ERR_UNSUPPORTED;
  if (n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads != 0 || max_seq < 1)
    return MTL_ERR_SHAPE;
  hipLaunchKernelGGL(qk_norm_rope_kv_kernel<false>, dim3(n_heads + 2 * n_kv_heads), dim3(64), 0,
                     (hipStream_t)stream, static_cast<const uint16_t*>(qkv), nullptr, 0, 0,
                     static_cast<const uint16_t*>(q_norm_w), static_cast<const uint16_t*>(k_norm_w),
                     static_cast<const uint16_t*>(cos_tab), static_cast<const uint16_t*>(sin_tab),
                     pos, static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache), n_heads, n_kv_heads, max_seq, eps);
  return launch_status();
}

int mtl_qk_norm_rope_kv_partials(const float* partials, int32_t splits, const void* q_norm_w,
                                 const void* k_norm_w, const void* cos_tab, const void* sin_tab,
                                 const int64_t* pos, void* q_out, void* k_cache, void* v_cache,
                                 int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                 int64_t max_seq, float eps, void* stream) {
  if (!partials || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !pos || !q_out || !k_cache ||
      !v_cache)
    return MTL_ERR_INVALID_ARG;
  if (head_dim != 128) return MTL_ERR_UNSUPPORTED;
  if (n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads != 0 || max_seq < 1 || splits < 1)
    return MTL_ERR_SHAPE;
  const int ncols = (n_heads + 2 * n_kv_heads) * head_dim;
  hipLaunchKernelGGL(qk_norm_rope_kv_kernel<true>, dim3(n_heads + 2 * n_kv_heads), dim3(64), 0,
                     (hipStream_t)stream, nullptr, partials, splits, ncols,
                     static_cast<const uint16_t*>(q_norm_w), static_cast<const uint16_t*>(k_norm_w),
                     static_cast<const uint16_t*>(cos_tab), static_cast<const uint16_t*>(sin_tab),
                     pos, static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache), n_heads, n_kv_heads, max_seq, eps);
  return launch_status();
}

int mtl_residual_rmsnorm(const float* partials, int32_t splits, const void* resid, void* h_out,
                         const void* w, void* x_out, const int32_t* gather, int64_t n, float eps,
                         void* stream) {
  if (!resid || !w || !x_out || (partials && !h_out)) return MTL_ERR_INVALID_ARG;
  if (n < 4 || n % 4 != 0 || n > 4 * kNormThreads * kNormMaxQuads) return MTL_ERR_SHAPE;
  if (partials && splits < 1) return MTL_ERR_SHAPE;
  if ((partials && !aligned16(partials)) || (reinterpret_cast<uintptr_t>(resid) & 7u) ||
      (reinterpret_cast<uintptr_t>(w) & 7u) || (h_out && (reinterpret_cast<uintptr_t>(h_out) & 7u)) ||
      (reinterpret_cast<uintptr_t>(x_out) & 7u))
    return MTL_ERR_ALIGN;
  hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(1), dim3(kNormThreads),
                     gather ? (size_t)n * 2 : 0, (hipStream_t)stream, partials, splits,
                     static_cast<const uint16_t*>(resid), static_cast<uint16_t*>(h_out),
                     static_cast<const uint16_t*>(w), static_cast<uint16_t*>(x_out), gather,
                     (int)n, eps);
  return launch_status();
}

int64_t mtl_decode_attention_workspace_bytes(int32_t n_heads, int32_t head_dim) {
  if (n_heads < 1 || head_dim != 128) return 0;
  return kAttnCounterBytes + (int64_t)n_heads * kAttnMaxChunks * kAttnPart * 4;
}

static int attn_check(int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int64_t max_seq,
                      void* workspace, int64_t ws_bytes, const void* k_cache,
                      const void* v_cache) {
  if (head_dim != 128) return MTL_ERR_UNSUPPORTED;
  if (n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads != 0 ||
      n_heads / n_kv_heads > kAttnMaxRep || n_kv_heads * 8 > kAttnPlacementWord ||
      max_seq < 1 || max_seq > (1 << 24))
    return MTL_ERR_SHAPE;
  if (!workspace || ws_bytes < mtl_decode_attention_workspace_bytes(n_heads, head_dim))
    return MTL_ERR_WORKSPACE;
  if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(workspace)) return MTL_ERR_ALIGN;
  return MTL_OK;
}

// Hand-off of the tile attention's chunk partials: XCD-local (1, the default) or
// agent-scope (0); mtl_decode_attention_set_handoff.
static int g_attn_local_handoff = 1;

int mtl_decode_attention_set_handoff(int32_t local) {
  if (local != 0 && local != 1) return MTL_ERR_INVALID_ARG;
  g_attn_local_handoff = local;
  return MTL_OK;
}

static void attn_launch(AttnArgs& a, void* workspace, bool from_part, hipStream_t s) {
  a.counters = static_cast<uint32_t*>(workspace);
  a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kAttnCounterBytes);
  a.fixed_chunks = a.max_seq <= kAttnBlock * kAttnMaxChunks;   // the tile kernel where it fits
  int64_t ch = (a.max_seq + kAttnBlock - 1) / kAttnBlock;
  if (ch > kAttnMaxChunks) ch = kAttnMaxChunks;
  const dim3 grid(a.Hkv, (unsigned)ch);
  // the XCD-local hand-off needs every chunk of a kv head on one XCD: kv heads a multiple
  // of 8, so linear ids kvh + Hkv * c agree modulo 8
  const bool local = g_attn_local_handoff && a.Hkv % 8 == 0 && a.Hkv <= kAttnMaxKvLocal;
  if (a.fixed_chunks) {
    if (from_part) {
      if (local) hipLaunchKernelGGL((attn_tile_kernel<true, true>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((attn_tile_kernel<true, false>), grid, dim3(256), 0, s, a);
    } else {
      if (local) hipLaunchKernelGGL((attn_tile_kernel<false, true>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((attn_tile_kernel<false, false>), grid, dim3(256), 0, s, a);
    }
  } else if (from_part) {
    hipLaunchKernelGGL(attn_decode_kernel<true>, grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(attn_decode_kernel<false>, grid, dim3(256), 0, s, a);
  }
}

int mtl_decode_attention(const void* q, const void* k_cache, const void* v_cache,
                         const int64_t* pos, void* out, const int32_t* out_index, int32_t n_heads,
                         int32_t n_kv_heads, int32_t head_dim, int64_t max_seq, float scale,
                         void* workspace, int64_t ws_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !pos || !out) return MTL_ERR_INVALID_ARG;
  const int st = attn_check(n_heads, n_kv_heads, head_dim, max_seq, workspace, ws_bytes, k_cache,
                            v_cache);
  if (st != MTL_OK) return st;
  if (!aligned16(q)) return MTL_ERR_ALIGN;
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.kc = const_cast<uint16_t*>(static_cast<const uint16_t*>(k_cache));
  a.vc = const_cast<uint16_t*>(static_cast<const uint16_t*>(v_cache));
  a.pos = pos;
  a.out = static_cast<uint16_t*>(out);
  a.out_index = out_index;
  a.H = n_heads;
  a.Hkv = n_kv_heads;
  a.max_seq = max_seq;
  a.scale = scale;
  attn_launch(a, workspace, false, (hipStream_t)stream);
  return launch_status();
}

int64_t mtl_head_workspace_bytes(int64_t N) {
  (void)N;
  return (int64_t)kHeadWGs * (4 + 8);
}

int mtl_bf16_gemv_argmax(const void* x, const void* w, int64_t N, int64_t K, void* logits,
                         int64_t* token_out, void* workspace, int64_t ws_bytes, void* stream) {
  if (!x || !w) return MTL_ERR_INVALID_ARG;
  if (N < 1 || K < 8 || K % 8 != 0 || K > 512 * kHeadKitMax) return MTL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w)) return MTL_ERR_ALIGN;
  if (!workspace || ws_bytes < mtl_head_workspace_bytes(N)) return MTL_ERR_WORKSPACE;
  if (!aligned16(workspace)) return MTL_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  float* pv = static_cast<float*>(workspace);
  long long* pi = reinterpret_cast<long long*>(static_cast<char*>(workspace) + kHeadWGs * 4);
  launch_head(K, s,
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), N, (int)K,
                     static_cast<uint16_t*>(logits), pv, pi, nullptr, nullptr, 0.f, 0, 0, nullptr);
  if (token_out)
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, s, pv, pi, kHeadWGs,
                       token_out, nullptr);
  return launch_status();
}

int mtl_residual_add(const float* partials, int32_t splits, void* h, const int32_t* scatter,
                     void* h_ord, float* slots, int64_t n, void* stream) {
  if (!h || !slots) return MTL_ERR_INVALID_ARG;
  if (n < 4 || n % 4 != 0 || n > kSlotCols * kMaxSlots) return MTL_ERR_SHAPE;
  if (partials && splits < 1) return MTL_ERR_SHAPE;
  if ((partials && !aligned16(partials)) || (reinterpret_cast<uintptr_t>(h) & 7u)) return MTL_ERR_ALIGN;
  hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)((n + kResidCols - 1) / kResidCols)),
                     dim3(64), 0, (hipStream_t)stream,
                     partials, splits, static_cast<uint16_t*>(h), scatter,
                     static_cast<uint16_t*>(h_ord), slots, (int)n);
  return launch_status();
}

int mtl_decode_attention_fused(const float* qkv_partials, int32_t splits, const void* q_norm_w,
                               const void* k_norm_w, const void* cos_tab, const void* sin_tab,
                               void* k_cache, void* v_cache, const int64_t* pos, void* out,
                               const int32_t* out_index, int32_t n_heads, int32_t n_kv_heads,
                               int32_t head_dim, int64_t max_seq, float scale, float eps,
                               void* workspace, int64_t ws_bytes, void* stream) {
  if (!qkv_partials || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !k_cache || !v_cache ||
      !pos || !out)
    return MTL_ERR_INVALID_ARG;
  const int st = attn_check(n_heads, n_kv_heads, head_dim, max_seq, workspace, ws_bytes, k_cache,
                            v_cache);
  if (st != MTL_OK) return st;
  if (splits < 1) return MTL_ERR_SHAPE;
  AttnArgs a{};
  a.qkv_part = qkv_partials;
  a.splits = splits;
  a.qn = static_cast<const uint16_t*>(q_norm_w);
  a.kn = static_cast<const uint16_t*>(k_norm_w);
  a.cos_tab = static_cast<const uint16_t*>(cos_tab);
  a.sin_tab = static_cast<const uint16_t*>(sin_tab);
  a.kc = static_cast<uint16_t*>(k_cache);
  a.vc = static_cast<uint16_t*>(v_cache);
  a.pos = pos;
  a.out = static_cast<uint16_t*>(out);
  a.out_index = out_index;
  a.H = n_heads;
  a.Hkv = n_kv_heads;
  a.max_seq = max_seq;
  a.scale = scale;
  a.eps = eps;
  attn_launch(a, workspace, true, (hipStream_t)stream);
  return launch_status();
}

static int argmax_norm(const void* h, const void* norm_w, const float* slots, float eps,
                       const void* w, int64_t N, int64_t K, void* logits, int64_t* token_out,
                       int64_t* pos, void* workspace, int64_t ws_bytes, void* stream) {
  if (!h || !norm_w || !slots || !w) return MTL_ERR_INVALID_ARG;
  if (N < 1 || K < 8 || K % 8 != 0 || K > 512 * kHeadKitMax) return MTL_ERR_SHAPE;
  if (!aligned16(h) || !aligned16(w) || !aligned16(norm_w) || !aligned16(slots))
    return MTL_ERR_ALIGN;
  if (!workspace || ws_bytes < mtl_head_workspace_bytes(N)) return MTL_ERR_WORKSPACE;
  if (!aligned16(workspace)) return MTL_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  float* pv = static_cast<float*>(workspace);
  long long* pi = reinterpret_cast<long long*>(static_cast<char*>(workspace) + kHeadWGs * 4);
  launch_head(K, s,
                     static_cast<const uint16_t*>(h), static_cast<const uint16_t*>(w), N, (int)K,
                     static_cast<uint16_t*>(logits), pv, pi, static_cast<const uint16_t*>(norm_w),
                     slots, eps, 0, 0, nullptr);
  if (token_out)
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, s, pv, pi, kHeadWGs,
                       token_out, pos);
  return launch_status();
}

int mtl_bf16_gemv_argmax_norm(const void* h, const void* norm_w, const float* slots, float eps,
                              const void* w, int64_t N, int64_t K, void* logits,
                              int64_t* token_out, void* workspace, int64_t ws_bytes,
                              void* stream) {
  return argmax_norm(h, norm_w, slots, eps, w, N, K, logits, token_out, nullptr, workspace,
                     ws_bytes, stream);
}

int mtl_bf16_gemv_argmax_norm_advance(const void* h, const void* norm_w, const float* slots,
                                      float eps, const void* w, int64_t N, int64_t K,
                                      void* logits, int64_t* token_out, int64_t* pos,
                                      void* workspace, int64_t ws_bytes, void* stream) {
  if (!token_out || !pos) return MTL_ERR_INVALID_ARG;
  return argmax_norm(h, norm_w, slots, eps, w, N, K, logits, token_out, pos, workspace,
                     ws_bytes, stream);
}

int mtl_bf16_gemv(const void* x, const void* w, int64_t N, int64_t K, void* out,
                  int64_t pad_period, int64_t pad_index, void* stream) {
  if (!x || !w || !out) return MTL_ERR_INVALID_ARG;
  if (N < 1 || K < 8 || K % 8 != 0 || K > 512 * kHeadKitMax) return MTL_ERR_SHAPE;
  if (pad_period < 0 || (pad_period > 0 && (pad_index < 0 || pad_index >= pad_period)))
    return MTL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w)) return MTL_ERR_ALIGN;
  launch_head(K, (hipStream_t)stream,
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), N, (int)K,
                     static_cast<uint16_t*>(out), nullptr, nullptr, nullptr, nullptr, 0.f,
                     pad_period, pad_index, nullptr);
  return launch_status();
}

int mtl_bf16_gemv_norm(const void* h, const void* norm_w, const float* slots, float eps,
                       const void* w, int64_t N, int64_t K, float* out, void* stream) {
  if (!h || !norm_w || !slots || !w || !out) return MTL_ERR_INVALID_ARG;
  if (N < 1 || K < 8 || K % 8 != 0 || K > 512 * kHeadKitMax) return MTL_ERR_SHAPE;
  if (!aligned16(h) || !aligned16(w) || !aligned16(norm_w) || !aligned16(slots))
    return MTL_ERR_ALIGN;
  if (K <= 4096) {   // x formed once per workgroup into LDS
    const int rpw = bf16_rows_per_wg(N, decode_device_cus());
    const int64_t wgs = (N + rpw - 1) / rpw;
    if (wgs >= ((int64_t)1 << 31) || (int64_t)rpw * K * 2 >= ((int64_t)1 << 31))
      return MTL_ERR_SHAPE;                     // a band's bytes address one buffer resource
    Bf16RowsArgs p{static_cast<const uint16_t*>(h), static_cast<const uint16_t*>(norm_w), slots,
                   eps, static_cast<const uint16_t*>(w), N, (int)K, rpw, out};
    hipLaunchKernelGGL(bf16_rows_norm_kernel<8>, dim3((unsigned)wgs), dim3(256), 0,
                       (hipStream_t)stream, p);
    return launch_status();
  }
  // longer rows: the head GEMV, one row per wave where N allows (every wave forms x)
  const int64_t wgs = (N + 3) / 4 < kHeadWGs ? (N + 3) / 4 : kHeadWGs;
  launch_head_on((int)wgs, K, (hipStream_t)stream, static_cast<const uint16_t*>(h),
                 static_cast<const uint16_t*>(w), N, (int)K, static_cast<uint16_t*>(nullptr),
                 static_cast<float*>(nullptr), static_cast<long long*>(nullptr),
                 static_cast<const uint16_t*>(norm_w), slots, eps, (int64_t)0, (int64_t)0, out);
  return launch_status();
}

int mtl_advance_position(int64_t* pos, void* stream) {
  if (!pos) return MTL_ERR_INVALID_ARG;
  hipLaunchKernelGGL(advance_position_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, pos);
  return launch_status();
}

int mtl_silu_mul_f32(const float* gate, const float* up, void* act, int64_t n, void* stream) {
  if (!gate || !up || !act) return MTL_ERR_INVALID_ARG;
  if (n < 1 || n >= ((int64_t)1 << 31)) return MTL_ERR_SHAPE;
  int blocks = (int)((n + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(silu_mul_f32_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, gate,
                     up, static_cast<uint16_t*>(act), n);
  return launch_status();
}

}  // extern "C"
