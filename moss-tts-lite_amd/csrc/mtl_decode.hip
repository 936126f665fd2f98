// Decode-step kernels around the int4 GEMV (gfx950): RMSNorm, embedding sum, q/k norm +
// RoPE + KV-cache write, GQA decode attention, bf16 head GEMV with greedy argmax.
//
// Rounding follows the reference's bf16 tensor ops step by step (every bf16 tensor op
// computes in fp32 and rounds to bf16); reductions run in a fixed order, so every
// launch is bitwise repeatable.
#include "mtl_common.h"
#include "mtl_decode.h"

namespace mtl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float lo_bf(uint32_t w) { return bf16_to_f32(w & 0xffffu); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return bf16_to_f32(w >> 16); }

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
// h = bf16(bf16(sum of split-K partials) + h) over 16 blocks of the hidden dim; each
// block publishes its sum of squares (slots[16]) and scatters h into the next GEMV's
// act-order input order (h_ord[scatter[i]] = h[i]).
// ----------------------------------------------------------------------------------
constexpr int kNormSlots = 16;

__global__ void __launch_bounds__(64) residual_add_kernel(
    const float* __restrict__ part, int splits, uint16_t* h, const int32_t* __restrict__ scatter,
    uint16_t* __restrict__ h_ord, float* __restrict__ slots, int n) {
  const int b = blockIdx.x, t = threadIdx.x;
  const int per = n / kNormSlots;
  float ss = 0.f;
  for (int q = t; q < per / 4; q += 64) {
    const int i = b * per + 4 * q;
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
  ss = wave_sum(ss);
  if (t == 0) slots[b] = ss;
}

// ----------------------------------------------------------------------------------
// Embedding sum (model.py:156-161): sequential bf16 adds of one row per table.
// ----------------------------------------------------------------------------------
__global__ void embed_sum_kernel(const int64_t* __restrict__ ids, int n_tables,
                                 const uint16_t* const* __restrict__ tables,
                                 const int64_t* __restrict__ vocabs, int64_t hidden,
                                 uint16_t* __restrict__ out) {
  for (int64_t d = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; d < hidden;
       d += (int64_t)gridDim.x * blockDim.x) {
    float h = 0.f;
    for (int i = 0; i < n_tables; ++i) {
      const int64_t id = ids[i];
      const float v = (id >= 0 && id < vocabs[i]) ? bf16_to_f32(tables[i][id * hidden + d]) : 0.f;
      h = (i == 0) ? v : round_bf16(h + v);
    }
    out[d] = (uint16_t)f32_to_bf16(h);
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
// GQA decode attention, split over the sequence.  Grid (kv head, chunk); wave w of a
// workgroup serves q head kvh*n_rep + w (+4, ...).  Scores are lane-per-position dot
// products against the wave-uniform q; the value sum is dims-per-lane.  Each chunk
// writes (max, sum, o[128]) and attn_combine_kernel merges chunks in order.
// ----------------------------------------------------------------------------------
constexpr int kAttnChunks = 16;
constexpr int kAttnPart = 132;   // m, l, 2 pad, o[128]

__global__ void __launch_bounds__(256) attn_partial_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int64_t* __restrict__ pos_ptr,
    float* __restrict__ part, int H, int Hkv, int64_t max_seq, float scale) {
  constexpr int D = 128;
  const int kvh = blockIdx.x, c = blockIdx.y;
  const int wave = wave_id(), lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const int n_rep = H / Hkv;
  int64_t L = *pos_ptr + 1;
  if (L < 0) L = 0;
  if (L > max_seq) L = max_seq;
  const int clen = (int)((L + kAttnChunks - 1) / kAttnChunks);
  const int p0 = c * clen;
  const int p1 = (int)(p0 + clen < L ? p0 + clen : L);
  const uint16_t* kbase = kc + (size_t)kvh * max_seq * D;
  const uint16_t* vbase = vc + (size_t)kvh * max_seq * D;
  for (int hr = wave; hr < n_rep; hr += nw) {
    const int h = kvh * n_rep + hr;
    const uint32_t* qh = reinterpret_cast<const uint32_t*>(q + (size_t)h * D);
    uint32_t qv[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) qv[i] = qh[i];
    float m = -INFINITY, l = 0.f, o0 = 0.f, o1 = 0.f;
    for (int base = p0; base < p1; base += 64) {
      const int p = base + lane;
      float s = -INFINITY;
      if (p < p1) {
        const u32x4* kr = reinterpret_cast<const u32x4*>(kbase + (size_t)p * D);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const u32x4 kk = kr[i];
          acc = dot2_bf16(kk.x, qv[4 * i + 0], acc);
          acc = dot2_bf16(kk.y, qv[4 * i + 1], acc);
          acc = dot2_bf16(kk.z, qv[4 * i + 2], acc);
          acc = dot2_bf16(kk.w, qv[4 * i + 3], acc);
        }
        s = acc * scale;
      }
      const float mn = fmaxf(m, wave_max(s));
      const float e = (p < p1) ? expf(s - mn) : 0.f;
      const float corr = expf(m - mn);
      l = fmaf(l, corr, wave_sum(e));
      o0 *= corr;
      o1 *= corr;
      const int cnt = p1 - base < 64 ? p1 - base : 64;
      const uint32_t* vr = reinterpret_cast<const uint32_t*>(vbase + (size_t)base * D) + lane;
#pragma unroll 16
      for (int j = 0; j < cnt; ++j) {
        const float ej = __shfl(e, j);
        const uint32_t vv = vr[(size_t)j * (D / 2)];
        o0 = fmaf(ej, lo_bf(vv), o0);
        o1 = fmaf(ej, hi_bf(vv), o1);
      }
      m = mn;
    }
    float* ph = part + ((size_t)h * kAttnChunks + c) * kAttnPart;
    if (lane == 0) {
      ph[0] = m;
      ph[1] = l;
    }
    ph[4 + 2 * lane] = o0;
    ph[5 + 2 * lane] = o1;
  }
}

// Same attention, with q/k RMSNorm + RoPE + the KV write of position pos folded in: each
// workgroup rebuilds its q heads from the q|k|v split-K partials; the workgroup whose
// chunk holds pos also builds k and v there, writes them to the cache and uses its LDS
// copy for that position (fast.py:134-162).
__device__ __forceinline__ void head_from_partials(const float* __restrict__ part, int splits,
                                                   int ncols, int head, int t, float& x0,
                                                   float& x1) {
  const float* p0 = part + (size_t)head * 128 + t;
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
}

__device__ __forceinline__ void norm_rope_pair(float x0, float x1, const uint16_t* w,
                                               const uint16_t* cr, const uint16_t* sr, int t,
                                               float eps, float& o0, float& o1) {
  float ss = fmaf(x0, x0, x1 * x1);
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / 128.f + eps);
  const float n0 = round_bf16(bf16_to_f32(w[t]) * round_bf16(x0 * r));
  const float n1 = round_bf16(bf16_to_f32(w[t + 64]) * round_bf16(x1 * r));
  o0 = round_bf16(round_bf16(n0 * bf16_to_f32(cr[t])) + round_bf16(-n1 * bf16_to_f32(sr[t])));
  o1 = round_bf16(round_bf16(n1 * bf16_to_f32(cr[t + 64])) + round_bf16(n0 * bf16_to_f32(sr[t + 64])));
}

__global__ void __launch_bounds__(256) attn_fused_kernel(
    const float* __restrict__ qkv_part, int splits, const uint16_t* __restrict__ qn,
    const uint16_t* __restrict__ kn, const uint16_t* __restrict__ cos_tab,
    const uint16_t* __restrict__ sin_tab, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    const int64_t* __restrict__ pos_ptr, float* __restrict__ part, int H, int Hkv,
    int64_t max_seq, float scale, float eps) {
  constexpr int D = 128;
  __shared__ uint32_t q_lds[4][D / 2];       // normed+rotated q heads (bf16 pairs)
  __shared__ uint32_t kpos[D / 2], vpos[D / 2];
  const int kvh = blockIdx.x, c = blockIdx.y;
  const int wave = wave_id(), lane = threadIdx.x & 63, nw = blockDim.x >> 6;
  const int n_rep = H / Hkv;
  const int ncols = (H + 2 * Hkv) * D;
  const int64_t pos = *pos_ptr;
  int64_t L = pos + 1;
  if (L < 0) L = 0;
  if (L > max_seq) L = max_seq;
  const int clen = (int)((L + kAttnChunks - 1) / kAttnChunks);
  const int p0 = c * clen;
  const int p1 = (int)(p0 + clen < L ? p0 + clen : L);
  const bool has_pos = pos >= p0 && pos < p1;
  const uint16_t* cr = cos_tab + (pos >= 0 && pos < max_seq ? pos : 0) * D;
  const uint16_t* sr = sin_tab + (pos >= 0 && pos < max_seq ? pos : 0) * D;
  uint16_t* kbase = kc + (size_t)kvh * max_seq * D;
  uint16_t* vbase = vc + (size_t)kvh * max_seq * D;
  // prologue: k and v of position pos (only the workgroup that scores it)
  if (has_pos && wave < 2) {
    float x0, x1;
    head_from_partials(qkv_part, splits, ncols, (wave == 0 ? H : H + Hkv) + kvh, lane, x0, x1);
    if (wave == 0) norm_rope_pair(x0, x1, kn, cr, sr, lane, eps, x0, x1);
    const uint32_t b0 = f32_to_bf16(x0), b1 = f32_to_bf16(x1);
    uint16_t* dst = (wave == 0 ? kbase : vbase) + (size_t)pos * D;
    dst[lane] = (uint16_t)b0;
    dst[lane + 64] = (uint16_t)b1;
    uint16_t* l16 = reinterpret_cast<uint16_t*>(wave == 0 ? kpos : vpos);
    l16[lane] = (uint16_t)b0;
    l16[lane + 64] = (uint16_t)b1;
  }
  for (int hr = wave; hr < n_rep; hr += nw) {
    const int h = kvh * n_rep + hr;
    float x0, x1;
    head_from_partials(qkv_part, splits, ncols, h, lane, x0, x1);
    norm_rope_pair(x0, x1, qn, cr, sr, lane, eps, x0, x1);
    uint16_t* l16 = reinterpret_cast<uint16_t*>(q_lds[hr & 3]);
    l16[lane] = (uint16_t)f32_to_bf16(x0);
    l16[lane + 64] = (uint16_t)f32_to_bf16(x1);
  }
  __syncthreads();
  for (int hr = wave; hr < n_rep; hr += nw) {
    const int h = kvh * n_rep + hr;
    uint32_t qv[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) qv[i] = q_lds[hr & 3][i];
    float m = -INFINITY, l = 0.f, o0 = 0.f, o1 = 0.f;
    for (int base = p0; base < p1; base += 64) {
      const int p = base + lane;
      float s = -INFINITY;
      if (p < p1) {
        float acc = 0.f;
        if (p == pos) {
#pragma unroll
          for (int i = 0; i < 64; ++i) acc = dot2_bf16(kpos[i], qv[i], acc);
        } else {
          const u32x4* kr = reinterpret_cast<const u32x4*>(kbase + (size_t)p * D);
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const u32x4 kk = kr[i];
            acc = dot2_bf16(kk.x, qv[4 * i + 0], acc);
            acc = dot2_bf16(kk.y, qv[4 * i + 1], acc);
            acc = dot2_bf16(kk.z, qv[4 * i + 2], acc);
            acc = dot2_bf16(kk.w, qv[4 * i + 3], acc);
          }
        }
        s = acc * scale;
      }
      const float mn = fmaxf(m, wave_max(s));
      const float e = (p < p1) ? expf(s - mn) : 0.f;
      const float corr = expf(m - mn);
      l = fmaf(l, corr, wave_sum(e));
      o0 *= corr;
      o1 *= corr;
      const int cnt = p1 - base < 64 ? p1 - base : 64;
      const uint32_t* vr = reinterpret_cast<const uint32_t*>(vbase + (size_t)base * D) + lane;
#pragma unroll 16
      for (int j = 0; j < cnt; ++j) {
        const float ej = __shfl(e, j);
        const uint32_t vv = (base + j == pos) ? vpos[lane] : vr[(size_t)j * (D / 2)];
        o0 = fmaf(ej, lo_bf(vv), o0);
        o1 = fmaf(ej, hi_bf(vv), o1);
      }
      m = mn;
    }
    float* ph = part + ((size_t)h * kAttnChunks + c) * kAttnPart;
    if (lane == 0) {
      ph[0] = m;
      ph[1] = l;
    }
    ph[4 + 2 * lane] = o0;
    ph[5 + 2 * lane] = o1;
  }
}

__global__ void __launch_bounds__(128) attn_combine_kernel(const float* __restrict__ part,
                                                           uint16_t* __restrict__ out,
                                                           const int32_t* __restrict__ out_index) {
  const int h = blockIdx.x, t = threadIdx.x;
  const float* ph = part + (size_t)h * kAttnChunks * kAttnPart;
  float mc[kAttnChunks], lc[kAttnChunks], oc[kAttnChunks];
#pragma unroll
  for (int c = 0; c < kAttnChunks; ++c) {   // every load issued before any use
    mc[c] = ph[c * kAttnPart];
    lc[c] = ph[c * kAttnPart + 1];
    oc[c] = ph[c * kAttnPart + 4 + t];
  }
  float M = -INFINITY;
#pragma unroll
  for (int c = 0; c < kAttnChunks; ++c)
    if (lc[c] > 0.f) M = fmaxf(M, mc[c]);
  float Ls = 0.f, o = 0.f;
#pragma unroll
  for (int c = 0; c < kAttnChunks; ++c)
    if (lc[c] > 0.f) {
      const float wgt = expf(mc[c] - M);
      Ls = fmaf(wgt, lc[c], Ls);
      o = fmaf(wgt, oc[c], o);
    }
  const int i = h * 128 + t;
  out[out_index ? out_index[i] : i] = (uint16_t)f32_to_bf16(Ls > 0.f ? o / Ls : 0.f);
}

// ----------------------------------------------------------------------------------
// bf16 head GEMV + argmax.  Each wave streams a contiguous band of rows (lane l reads
// 16 B at k = 8l + 512i, 1 KB contiguous per wave load), reduces each row across the
// wave, rounds the logit to bf16 and keeps the first maximum; waves then workgroups
// are merged in row order.
// ----------------------------------------------------------------------------------
constexpr int kHeadWGs = 1024;
constexpr int kHeadKit = 16;     // K <= 8192

__device__ __forceinline__ bool better(float va, long long ia, float vb, long long ib) {
  if (ia < 0) return false;
  if (ib < 0) return true;
  const bool na = va != va, nb = vb != vb;
  if (na) return !nb || ia < ib;
  if (nb) return false;
  return va > vb || (va == vb && ia < ib);
}

__global__ void __launch_bounds__(256) head_gemv_kernel(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ w,
                                                        int64_t N, int K,
                                                        uint16_t* __restrict__ logits,
                                                        float* __restrict__ part_v,
                                                        long long* __restrict__ part_i,
                                                        const uint16_t* __restrict__ norm_w,
                                                        const float* __restrict__ slots,
                                                        float eps) {
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
    float ssum = 0.f;
#pragma unroll
    for (int i = 0; i < kNormSlots; ++i) ssum += slots[i];
    const float r = rsqrtf(ssum / (float)K + eps);
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
  for (int64_t r = r0; r < r1; ++r) {
    const uint16_t* wr = w + r * K;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kHeadKit; ++i) {
      const int k = 512 * i + 8 * lane;
      if (i < kit && k < K) {
        const u32x4 ww = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr + k));
        acc = dot2_bf16(ww.x, xv[i].x, acc);
        acc = dot2_bf16(ww.y, xv[i].y, acc);
        acc = dot2_bf16(ww.z, xv[i].z, acc);
        acc = dot2_bf16(ww.w, xv[i].w, acc);
      }
    }
    acc = wave_sum(acc);
    const uint32_t hb = f32_to_bf16(acc);
    if (logits && lane == 0) logits[r] = (uint16_t)hb;
    const float lv = bf16_to_f32(hb);
    if (better(lv, r, best, bidx)) {
      best = lv;
      bidx = r;
    }
  }
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

__global__ void __launch_bounds__(256) argmax_final_kernel(const float* __restrict__ part_v,
                                                           const long long* __restrict__ part_i,
                                                           int nparts, int64_t* token_out) {
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
  if (threadIdx.x == 0) token_out[0] = si[0] < 0 ? 0 : (int64_t)si[0];
}

__global__ void advance_position_kernel(int64_t* pos) {
  if (threadIdx.x == 0 && blockIdx.x == 0) pos[0] += 1;
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
  if (n_tables < 1 || hidden < 1) return MTL_ERR_SHAPE;
  const int blocks = (int)((hidden + 255) / 256);
  hipLaunchKernelGGL(embed_sum_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, ids,
                     n_tables, reinterpret_cast<const uint16_t* const*>(tables), vocabs, hidden,
                     static_cast<uint16_t*>(out));
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
  return (int64_t)n_heads * kAttnChunks * kAttnPart * 4;
}

int mtl_decode_attention(const void* q, const void* k_cache, const void* v_cache,
                         const int64_t* pos, void* out, const int32_t* out_index, int32_t n_heads,
                         int32_t n_kv_heads, int32_t head_dim, int64_t max_seq, float scale,
                         void* workspace, int64_t ws_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !pos || !out) return MTL_ERR_INVALID_ARG;
  if (head_dim != 128) return MTL_ERR_UNSUPPORTED;
  if (n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads != 0 || max_seq < 1 ||
      max_seq > (1 << 24))
    return MTL_ERR_SHAPE;
  if (!workspace || ws_bytes < mtl_decode_attention_workspace_bytes(n_heads, head_dim))
    return MTL_ERR_WORKSPACE;
  if (!aligned16(k_cache) || !aligned16(v_cache) || !aligned16(q)) return MTL_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(attn_partial_kernel, dim3(n_kv_heads, kAttnChunks), dim3(256), 0, s,
                     static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k_cache),
                     static_cast<const uint16_t*>(v_cache), pos, static_cast<float*>(workspace),
                     n_heads, n_kv_heads, max_seq, scale);
  hipLaunchKernelGGL(attn_combine_kernel, dim3(n_heads), dim3(128), 0, s,
                     static_cast<const float*>(workspace), static_cast<uint16_t*>(out), out_index);
  return launch_status();
}

int64_t mtl_head_workspace_bytes(int64_t N) {
  (void)N;
  return (int64_t)kHeadWGs * (4 + 8);
}

int mtl_bf16_gemv_argmax(const void* x, const void* w, int64_t N, int64_t K, void* logits,
                         int64_t* token_out, void* workspace, int64_t ws_bytes, void* stream) {
  if (!x || !w) return MTL_ERR_INVALID_ARG;
  if (N < 1 || K < 8 || K % 8 != 0 || K > 512 * kHeadKit) return MTL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w)) return MTL_ERR_ALIGN;
  if (!workspace || ws_bytes < mtl_head_workspace_bytes(N)) return MTL_ERR_WORKSPACE;
  if (!aligned16(workspace)) return MTL_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  float* pv = static_cast<float*>(workspace);
  long long* pi = reinterpret_cast<long long*>(static_cast<char*>(workspace) + kHeadWGs * 4);
  hipLaunchKernelGGL(head_gemv_kernel, dim3(kHeadWGs), dim3(256), 0, s,
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), N, (int)K,
                     static_cast<uint16_t*>(logits), pv, pi, nullptr, nullptr, 0.f);
  if (token_out)
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, s, pv, pi, kHeadWGs,
                       token_out);
  return launch_status();
}

int mtl_residual_add(const float* partials, int32_t splits, void* h, const int32_t* scatter,
                     void* h_ord, float* slots, int64_t n, void* stream) {
  if (!h || !slots) return MTL_ERR_INVALID_ARG;
  if (n < 64 || n % 64 != 0 || n > (1 << 20)) return MTL_ERR_SHAPE;
  if (partials && splits < 1) return MTL_ERR_SHAPE;
  if ((partials && !aligned16(partials)) || (reinterpret_cast<uintptr_t>(h) & 7u)) return MTL_ERR_ALIGN;
  hipLaunchKernelGGL(residual_add_kernel, dim3(kNormSlots), dim3(64), 0, (hipStream_t)stream,
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
  if (head_dim != 128) return MTL_ERR_UNSUPPORTED;
  if (n_heads < 1 || n_kv_heads < 1 || n_heads % n_kv_heads != 0 || n_heads / n_kv_heads > 4 ||
      max_seq < 1 || max_seq > (1 << 24) || splits < 1)
    return MTL_ERR_SHAPE;
  if (!workspace || ws_bytes < mtl_decode_attention_workspace_bytes(n_heads, head_dim))
    return MTL_ERR_WORKSPACE;
  if (!aligned16(k_cache) || !aligned16(v_cache)) return MTL_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(attn_fused_kernel, dim3(n_kv_heads, kAttnChunks), dim3(256), 0, s,
                     qkv_partials, splits, static_cast<const uint16_t*>(q_norm_w),
                     static_cast<const uint16_t*>(k_norm_w), static_cast<const uint16_t*>(cos_tab),
                     static_cast<const uint16_t*>(sin_tab), static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache), pos, static_cast<float*>(workspace), n_heads,
                     n_kv_heads, max_seq, scale, eps);
  hipLaunchKernelGGL(attn_combine_kernel, dim3(n_heads), dim3(128), 0, s,
                     static_cast<const float*>(workspace), static_cast<uint16_t*>(out), out_index);
  return launch_status();
}

int mtl_bf16_gemv_argmax_norm(const void* h, const void* norm_w, const float* slots, float eps,
                              const void* w, int64_t N, int64_t K, void* logits,
                              int64_t* token_out, void* workspace, int64_t ws_bytes,
                              void* stream) {
  if (!h || !norm_w || !slots || !w) return MTL_ERR_INVALID_ARG;
  if (N < 1 || K < 8 || K % 8 != 0 || K > 512 * kHeadKit) return MTL_ERR_SHAPE;
  if (!aligned16(h) || !aligned16(w) || !aligned16(norm_w)) return MTL_ERR_ALIGN;
  if (!workspace || ws_bytes < mtl_head_workspace_bytes(N)) return MTL_ERR_WORKSPACE;
  if (!aligned16(workspace)) return MTL_ERR_ALIGN;
  hipStream_t s = (hipStream_t)stream;
  float* pv = static_cast<float*>(workspace);
  long long* pi = reinterpret_cast<long long*>(static_cast<char*>(workspace) + kHeadWGs * 4);
  hipLaunchKernelGGL(head_gemv_kernel, dim3(kHeadWGs), dim3(256), 0, s,
                     static_cast<const uint16_t*>(h), static_cast<const uint16_t*>(w), N, (int)K,
                     static_cast<uint16_t*>(logits), pv, pi, static_cast<const uint16_t*>(norm_w),
                     slots, eps);
  if (token_out)
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, s, pv, pi, kHeadWGs,
                       token_out);
  return launch_status();
}

int mtl_advance_position(int64_t* pos, void* stream) {
  if (!pos) return MTL_ERR_INVALID_ARG;
  hipLaunchKernelGGL(advance_position_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, pos);
  return launch_status();
}

}  // extern "C"
