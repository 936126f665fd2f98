// Prompt-length kernels of the prefill around the int4 GEMM (gfx950): the embedding sum,
// RMSNorm with the act-order gather, q/k RMSNorm + RoPE + KV write, and causal GQA
// attention, each over all prompt rows in one launch (moss_tts_lite/fast.py:210-270, the
// quantized prefill that runs every layer at t = prompt length).
//
// Rounding follows the reference's bf16 tensor ops as in the decode-step kernels: the
// norms and RoPE are bitwise the decode kernels' arithmetic on each row.  The attention
// computes scores and the value sum on MFMA (bf16 operands, fp32 accumulation) with an
// online softmax in fp32.
#include "mtl_common.h"
#include "mtl_decode.h"
#include "mtl_w4core.h"

namespace mtl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// ----------------------------------------------------------------------------------
// Embedding sum over rows (model.py:156-161, fast.py:210-216): row r of out is
// bf16(...bf16(T0[ids[r][0]] + T1[ids[r][1]]) + ...).
// ----------------------------------------------------------------------------------
__global__ void embed_rows_kernel(const int64_t* __restrict__ ids, int n_tables,
                                  const uint16_t* const* __restrict__ tables,
                                  const int64_t* __restrict__ vocabs, int64_t hidden,
                                  uint16_t* __restrict__ out) {
  const int64_t r = blockIdx.y;
  const int64_t* row_ids = ids + r * n_tables;
  for (int64_t d = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; d < hidden;
       d += (int64_t)gridDim.x * blockDim.x) {
    float h = 0.f;
    for (int i = 0; i < n_tables; ++i) {
      const int64_t id = row_ids[i];
      const float v = (id >= 0 && id < vocabs[i]) ? bf16_to_f32(tables[i][id * hidden + d]) : 0.f;
      h = (i == 0) ? v : round_bf16(h + v);
    }
    out[r * hidden + d] = (uint16_t)f32_to_bf16(h);
  }
}

// ----------------------------------------------------------------------------------
// RMSNorm of each row (model.py:34-40), summed in the order of mtl_rmsnorm, written as
// out[r][j] = x_norm[r][gather[j]] (the act-order input order of the next int4 GEMM) or
// unpermuted.  One 256-thread workgroup per row; the normalised row passes through LDS.
// ----------------------------------------------------------------------------------
constexpr int kRowNormMax = 16384;
constexpr int kRowNormChunks = kRowNormMax / 2048;   // 8-element chunks per thread
constexpr int kRowNormMaxSplits = 8;                 // K splits of a residual GEMM's partials

// With `part` (fp32 [splits][rows][n], the K-split sums of an o or down GEMM): first the
// residual add of prefill_reduce_kernel<MTL_EPI_RESIDUAL>, h = bf16(bf16(sum of the splits in
// split order) + h) written back to x in place, then the RMSNorm of that h: one launch for
// the split sum, the residual and the next GEMM's input.
// With `sums` the output is staged for the prompt-length GEMM (mtl_w4_gemm_prefill_staged):
// each 8-channel item of the output row in pair order, and sums[row][g] the sum of its
// 32-channel group g, formed as the GEMM's own staging forms it (a v_dot2 chain per item,
// then the butterfly over 4 items).
__global__ void __launch_bounds__(256) rmsnorm_gather_kernel(
    uint16_t* x, int64_t ldx, const uint16_t* __restrict__ w,
    const int32_t* __restrict__ gather, uint16_t* out, int64_t ldo, int n, float eps,
    const float* __restrict__ part, int splits, float* __restrict__ sums) {
  __shared__ uint16_t xs[kRowNormMax];
  __shared__ float red[4];
  uint16_t* xr = x + (size_t)blockIdx.x * ldx;
  uint16_t* orow = out + (size_t)blockIdx.x * ldo;
  const int t = threadIdx.x;
  const int nch = n / 2048 + (t * 8 < n % 2048 ? 1 : 0);   // this thread's chunks
  // every load of the row first: x and w chunks (8 elements at 8 t + 2048 c) and the
  // gather indices (j = t + 256 i)
  u32x4 xv[kRowNormChunks], wv[kRowNormChunks];
  int32_t gi[4 * kRowNormChunks];
  int4 gq[2 * kRowNormChunks];                  // staged: the gather indices of item t + 256 c
  float* srow = sums ? sums + (size_t)blockIdx.x * (n >> 5) : nullptr;
  // an output item (channels 8 q .. 8 q + 7, q = t + 256 c) in pair order, with the sum of
  // its 32-channel group (lanes 4k .. 4k + 3 hold one group: n % 32 == 0)
  auto staged_put = [&](const u32x4 v, int c) {
    float sum;
    const u32x4 pv = pair_order_dot(v, sum);
    sum = group_sum_valu<4>(sum);
    *reinterpret_cast<u32x4*>(orow + 8 * t + 2048 * c) = pv;
    if ((t & 3) == 0) srow[(t + 256 * c) >> 2] = sum;
  };
#pragma unroll
  for (int c = 0; c < kRowNormChunks; ++c) {
    if (c < nch) {
      xv[c] = *reinterpret_cast<const u32x4*>(xr + 8 * t + 2048 * c);
      wv[c] = *reinterpret_cast<const u32x4*>(w + 8 * t + 2048 * c);
    }
  }
  if (part) {
    const size_t plane = (size_t)gridDim.x * n;
    const float* prow = part + (size_t)blockIdx.x * n;
#pragma unroll
    for (int c = 0; c < kRowNormChunks; ++c) {
      if (c < nch) {
        // every split's loads of the chunk first (one round trip, not one per split),
        // then the sum in split order
        const float* pc = prow + 8 * t + 2048 * c;
        float4 pl[kRowNormMaxSplits], ph[kRowNormMaxSplits];
#pragma unroll
        for (int z = 0; z < kRowNormMaxSplits; ++z) {
          if (z < splits) {
            pl[z] = *reinterpret_cast<const float4*>(pc + z * plane);
            ph[z] = *reinterpret_cast<const float4*>(pc + z * plane + 4);
          }
        }
        float4 lo = pl[0], hi = ph[0];
#pragma unroll
        for (int z = 1; z < kRowNormMaxSplits; ++z) {
          if (z < splits) {
            lo.x += pl[z].x; lo.y += pl[z].y; lo.z += pl[z].z; lo.w += pl[z].w;
            hi.x += ph[z].x; hi.y += ph[z].y; hi.z += ph[z].z; hi.w += ph[z].w;
          }
        }
        const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        const uint32_t a[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t e0 = f32_to_bf16(round_bf16(v[2 * j]) + lo_bf(a[j]));
          const uint32_t e1 = f32_to_bf16(round_bf16(v[2 * j + 1]) + hi_bf(a[j]));
          o[j] = e0 | (e1 << 16);
        }
        xv[c] = u32x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<u32x4*>(xr + 8 * t + 2048 * c) = xv[c];
      }
    }
  }
  if (gather && sums) {
#pragma unroll
    for (int c = 0; c < kRowNormChunks; ++c) {
      if (c < nch) {
        gq[2 * c] = *reinterpret_cast<const int4*>(gather + 8 * t + 2048 * c);
        gq[2 * c + 1] = *reinterpret_cast<const int4*>(gather + 8 * t + 2048 * c + 4);
      }
    }
  } else if (gather) {
#pragma unroll
    for (int i = 0; i < 4 * kRowNormChunks; ++i)
      if (t + 256 * i < n) gi[i] = gather[t + 256 * i];
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < kRowNormChunks; ++c) {
    if (c < nch) {
      const uint32_t a[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float f0 = lo_bf(a[j]), f1 = hi_bf(a[j]);
        ss = fmaf(f0, f0, ss);
        ss = fmaf(f1, f1, ss);
      }
    }
  }
  ss = wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  const float total = (red[0] + red[1]) + (red[2] + red[3]);
  const float r = rsqrtf(total / (float)n + eps);
#pragma unroll
  for (int c = 0; c < kRowNormChunks; ++c) {
    if (c < nch) {
      const uint32_t a[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
      const uint32_t b[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float y0 = round_bf16(lo_bf(b[j]) * round_bf16(lo_bf(a[j]) * r));
        const float y1 = round_bf16(hi_bf(b[j]) * round_bf16(hi_bf(a[j]) * r));
        o[j] = f32_to_bf16(y0) | (f32_to_bf16(y1) << 16);
      }
      if (sums && !gather) {
        staged_put(u32x4{o[0], o[1], o[2], o[3]}, c);
      } else {
        uint16_t* dst = gather ? xs : orow;
        *reinterpret_cast<u32x4*>(dst + 8 * t + 2048 * c) = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
  }
  if (!gather) return;
  __syncthreads();
  if (sums) {
#pragma unroll
    for (int c = 0; c < kRowNormChunks; ++c) {
      if (c < nch) {
        const int4 g0 = gq[2 * c], g1 = gq[2 * c + 1];
        auto e = [&](int i) { return (uint32_t)xs[i]; };
        staged_put(u32x4{e(g0.x) | (e(g0.y) << 16), e(g0.z) | (e(g0.w) << 16),
                         e(g1.x) | (e(g1.y) << 16), e(g1.z) | (e(g1.w) << 16)}, c);
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4 * kRowNormChunks; ++i)
    if (t + 256 * i < n) orow[t + 256 * i] = xs[gi[i]];
}

// ----------------------------------------------------------------------------------
// q/k RMSNorm + RoPE + KV write for rows at positions pos0 + r (fast.py:226-237): one
// 64-lane workgroup per (head, row), the decode kernel's arithmetic per row.  With `part`
// (fp32 [splits][rows][part_cols], the q|k|v GEMM's K-split sums), the heads below
// part_cols take bf16(sum of the splits in split order), the bits the GEMM's split-sum
// launch writes to qkv; the other heads (a bf16-kept v_proj's) read qkv.
// ----------------------------------------------------------------------------------
__global__ void __launch_bounds__(64) qk_norm_rope_rows_kernel(
    const uint16_t* __restrict__ qkv, int64_t ldq, int64_t pos0,
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ kn,
    const uint16_t* __restrict__ cos_tab, const uint16_t* __restrict__ sin_tab,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int H,
    int Hkv, int64_t max_seq, float eps, const float* __restrict__ part, int splits,
    int64_t part_cols) {
  constexpr int D = 128;
  const int b = blockIdx.x, t = threadIdx.x;
  const int64_t r = blockIdx.y, pos = pos0 + r;
  float x0, x1;
  if (part && (int64_t)(b + 1) * D <= part_cols) {
    const size_t plane = (size_t)gridDim.y * part_cols;
    const float* pc = part + r * part_cols + (size_t)b * D;
    float p0[kRowNormMaxSplits], p1[kRowNormMaxSplits];
#pragma unroll
    for (int z = 0; z < kRowNormMaxSplits; ++z) {
      if (z < splits) {
        p0[z] = pc[z * plane + t];
        p1[z] = pc[z * plane + t + 64];
      }
    }
    float s0 = p0[0], s1 = p1[0];
#pragma unroll
    for (int z = 1; z < kRowNormMaxSplits; ++z) {
      if (z < splits) {
        s0 += p0[z];
        s1 += p1[z];
      }
    }
    x0 = bf16_to_f32((uint16_t)f32_to_bf16(s0));
    x1 = bf16_to_f32((uint16_t)f32_to_bf16(s1));
  } else {
    const uint16_t* src = qkv + r * ldq + (size_t)b * D;
    x0 = bf16_to_f32(src[t]);
    x1 = bf16_to_f32(src[t + 64]);
  }
  if (b >= H + Hkv) {   // v head: copied unchanged
    uint16_t* dst = vc + ((size_t)(b - H - Hkv) * max_seq + pos) * D;
    dst[t] = (uint16_t)f32_to_bf16(x0);
    dst[t + 64] = (uint16_t)f32_to_bf16(x1);
    return;
  }
  float o0, o1;
  norm_rope_pair(x0, x1, b < H ? qn : kn, cos_tab + pos * D, sin_tab + pos * D, t, eps, o0, o1);
  uint16_t* dst = b < H ? q_out + r * (H * D) + (size_t)b * D
                        : kc + ((size_t)(b - H) * max_seq + pos) * D;
  dst[t] = (uint16_t)f32_to_bf16(o0);
  dst[t + 64] = (uint16_t)f32_to_bf16(o1);
}

// ----------------------------------------------------------------------------------
// Causal GQA attention over the prompt rows (fast.py:238-242, SDPA with is_causal: row r
// at position pos0 + r attends to cache positions [0, pos0 + r]).
//
// Workgroup (kv head g, block of 16 rows); wave w serves q heads g * n_rep + w (+4).  Per
// tile of 32 cache positions, staged once in LDS for the workgroup (K and V rows as they
// are, 16-byte stores):
//   S^T (positions x rows) = K Q^T: v_mfma_f32_16x16x32_bf16 with A = K rows, B = Q^T;
//     lane (lg, lj) gets positions 16h + 4 lg + i of row lj, i = 0..3, h = 0, 1;
//   online softmax per row (the lane's own column) in fp32;
//   O^T (dims x rows) += V^T P^T: B = P^T is the lane's own 8 probabilities (bf16) with
//     k index 8 lg + e standing for position 4 lg + e (e < 4) or 16 + 4 lg + e - 4, and A
//     = V^T at the same positions, read from the V rows by ds_read_b64_tr_b16 (in each
//     16-lane group lane j reads dims 4 (j % 4) .. of row j / 4, and the transpose hands
//     lane i dim i of those 4 rows: two reads, positions 4 lg .. and 16 + 4 lg ..).
// So no operand crosses lanes.  O^T / l goes out as bf16, each value to
// out[r][out_index[c]] (the act-order input order of the o projection) or column c.
// ----------------------------------------------------------------------------------
constexpr int kPaRows = 16;
constexpr int kPaKeys = 32;

struct PrefillAttnArgs {
  const uint16_t* q;        // bf16 [rows, H * 128]
  const uint16_t* kc;       // bf16 [Hkv, max_seq, 128]
  const uint16_t* vc;
  uint16_t* out;            // bf16 [rows, ldo]
  const int32_t* out_index;
  int64_t ldo, pos0, max_seq;
  int rows, H, Hkv;
  float scale;
};

template <int HPW>   // q heads per wave: n_rep <= 4 * HPW
__global__ void __launch_bounds__(512) prefill_attn_kernel(PrefillAttnArgs a) {
  constexpr int D = 128;
  // Two wave groups of 4 take alternate tiles (group g2: tiles 2 it + g2), each with its
  // own LDS tile; their (m, l, O) meet in LDS at the end.  The raw buffer holds the two
  // K tiles ([32][16 items + 1 pad] u32x4 each), then the two V tiles (the same form), and
  // after the loop the merge exchange (4 x 32 x 64 + 4 x 2 x 64 floats: the same bytes).
  constexpr int kKItems = 2 * kPaKeys * 17;
  __shared__ u32x4 lds_raw[2 * kKItems];
  static_assert(2 * kKItems * 16 >= (4 * 32 * 64 + 4 * 2 * 64) * 4, "merge exchange");
  const int kvh = blockIdx.x, rb = blockIdx.y;
  const int t = threadIdx.x, wave = wave_id(), lane = t & 63;
  const int g2 = wave >> 2, hw = wave & 3, tg = t & 255;
  const int lg = lane >> 4, lj = lane & 15;
  u32x4* k_lds = lds_raw + g2 * kPaKeys * 17;                       // [32][17]
  u32x4* v_lds = lds_raw + kKItems + g2 * kPaKeys * 17;             // [32][17]
  const int n_rep = a.H / a.Hkv;
  const int r0 = rb * kPaRows;
  const int my_row = r0 + lj;                          // this lane's query row
  const bool row_ok = my_row < a.rows;
  const int64_t my_pos = a.pos0 + (row_ok ? my_row : a.rows - 1);
  const int last_row = (r0 + kPaRows < a.rows ? r0 + kPaRows : a.rows) - 1;
  const int64_t last_pos = a.pos0 + last_row;          // the block's last position
  const int ntiles = (int)(last_pos / kPaKeys) + 1;
  const int nit = (ntiles + 1) / 2;

  // Q^T operands of this wave's heads: lane (lg, lj) holds dims 32 c + 8 lg .. +7 of row lj
  u32x4 qb[HPW][4];
  floatx4 o[HPW][8];
  float m[HPW], l[HPW];
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    const int hr = hw + 4 * hi;
    const int hq = kvh * n_rep + (hr < n_rep ? hr : 0);
    const uint16_t* qrow = a.q + (size_t)(row_ok ? my_row : 0) * (a.H * D) + (size_t)hq * D;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qrow + 32 * c + 8 * lg);
      qb[hi][c] = row_ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int d = 0; d < 8; ++d) o[hi][d] = floatx4{0.f, 0.f, 0.f, 0.f};
    m[hi] = -INFINITY;
    l[hi] = 0.f;
  }

  const uint16_t* kbase = a.kc + (size_t)kvh * a.max_seq * D;
  const uint16_t* vbase = a.vc + (size_t)kvh * a.max_seq * D;
  // tile loads: the group's items tg and tg + 256 are (position item / 16, dims
  // 8 (item % 16) ..); the group's next tile is in flight while this one is multiplied
  u32x4 kv[2], vv[2];
  auto tile_load = [&](int kt) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int item = tg + 256 * j;
      const int64_t p = (int64_t)kt * kPaKeys + (item >> 4);
      const bool ok = p <= last_pos;
      const size_t off = (size_t)(ok ? p : 0) * D + 8 * (item & 15);
      kv[j] = *reinterpret_cast<const u32x4*>(kbase + off);
      vv[j] = *reinterpret_cast<const u32x4*>(vbase + off);
      if (!ok) { kv[j] = u32x4{0u, 0u, 0u, 0u}; vv[j] = kv[j]; }
    }
  };
  tile_load(g2);
  for (int it = 0; it < nit; ++it) {
    const int kt = 2 * it + g2;                        // past the last tile: all zero, skipped
    __syncthreads();                                   // the previous tiles are consumed
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int item = tg + 256 * j;
      const int kr = item >> 4, c8 = item & 15;
      k_lds[kr * 17 + c8] = kv[j];
      v_lds[kr * 17 + c8] = vv[j];
    }
    __syncthreads();
    if (kt + 2 < ntiles) tile_load(kt + 2);
    if (kt >= ntiles) continue;                        // uniform over the wave

#pragma unroll
    for (int hi = 0; hi < HPW; ++hi) {
      if (hw + 4 * hi >= n_rep) break;                 // uniform over the wave
      // S^T for positions kt*32 + [0, 16) and [16, 32)
      floatx4 s[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        s[h] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const bf16x8_t A = __builtin_bit_cast(bf16x8_t, k_lds[(16 * h + lj) * 17 + 4 * c + lg]);
          s[h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8_t, qb[hi][c]),
                                                         s[h], 0, 0, 0);
        }
      }
      float mx = -INFINITY;
      float sv[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t p = (int64_t)kt * kPaKeys + 16 * h + 4 * lg + i;
          sv[h][i] = p <= my_pos ? s[h][i] * a.scale : -INFINITY;
          mx = fmaxf(mx, sv[h][i]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // a row may have no position yet in the odd group's tiles: m stays -inf, l 0, O 0
      const float m_new = fmaxf(m[hi], mx);
      const bool none = m_new == -INFINITY;
      const float alpha = none ? 1.f : expf(m[hi] - m_new);
      float psum = 0.f;
      float pv[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pv[h][i] = none ? 0.f : expf(sv[h][i] - m_new);
          psum += pv[h][i];
        }
      psum += __shfl_xor(psum, 16);
      psum += __shfl_xor(psum, 32);
      l[hi] = l[hi] * alpha + psum;
      m[hi] = m_new;
      const u32x4 pw{cvt_pk_bf16(pv[0][0], pv[0][1]), cvt_pk_bf16(pv[0][2], pv[0][3]),
                     cvt_pk_bf16(pv[1][0], pv[1][1]), cvt_pk_bf16(pv[1][2], pv[1][3])};
      const bf16x8_t P = __builtin_bit_cast(bf16x8_t, pw);
      typedef short s4 __attribute__((ext_vector_type(4)));
      typedef short s8 __attribute__((ext_vector_type(8)));
      // this lane's transpose-read rows (4 lg + lj / 4, and 16 more) and first dim
      const uint16_t* vr0 = reinterpret_cast<const uint16_t*>(v_lds + (4 * lg + (lj >> 2)) * 17) +
                            4 * (lj & 3);
      const uint16_t* vr1 = vr0 + 16 * 17 * 8;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (s4 __attribute__((address_space(3)))*)(vr0 + 16 * d));
        const s4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (s4 __attribute__((address_space(3)))*)(vr1 + 16 * d));
        const bf16x8_t A = __builtin_bit_cast(
            bf16x8_t, s8{lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]});
        o[hi][d] = o[hi][d] * alpha;
        o[hi][d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, P, o[hi][d], 0, 0, 0);
      }
    }
  }

  // The odd group hands (m, l, O) to the even group through LDS, head by head; the even
  // group combines (its m is finite: position 0 is in tile 0) and writes
  // out[row][hq * 128 + 16 d + 4 lg + i] = bf16(O / l).
  float* mo = reinterpret_cast<float*>(lds_raw);        // [4 waves][32 values][64 lanes]
  float* ml = mo + 4 * 32 * 64;                         // [4 waves][2][64 lanes]
  uint16_t* orow = a.out + (size_t)(row_ok ? my_row : 0) * a.ldo;
#pragma unroll
  for (int hi = 0; hi < HPW; ++hi) {
    const int hr = hw + 4 * hi;
    __syncthreads();                                   // LDS free (tiles or previous head)
    if (g2 == 1 && hr < n_rep) {
#pragma unroll
      for (int d = 0; d < 8; ++d)
#pragma unroll
        for (int i = 0; i < 4; ++i) mo[(hw * 32 + 4 * d + i) * 64 + lane] = o[hi][d][i];
      ml[(hw * 2) * 64 + lane] = m[hi];
      ml[(hw * 2 + 1) * 64 + lane] = l[hi];
    }
    __syncthreads();
    if (g2 == 1 || hr >= n_rep || !row_ok) continue;
    const float m1 = ml[(hw * 2) * 64 + lane], l1 = ml[(hw * 2 + 1) * 64 + lane];
    const float mt = fmaxf(m[hi], m1);
    const float a0 = expf(m[hi] - mt), a1 = m1 == -INFINITY ? 0.f : expf(m1 - mt);
    const float inv = 1.f / (l[hi] * a0 + l1 * a1);
    const int hq = kvh * n_rep + hr;
#pragma unroll
    for (int d = 0; d < 8; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = o[hi][d][i] * a0 + mo[(hw * 32 + 4 * d + i) * 64 + lane] * a1;
        const int c = hq * D + 16 * d + 4 * lg + i;
        orow[a.out_index ? a.out_index[c] : c] = (uint16_t)f32_to_bf16(v * inv);
      }
  }
}

}  // namespace mtl

using namespace mtl;

extern "C" {

int mtl_embed_rows(const int64_t* ids, int64_t rows, int32_t n_tables, const void* const* tables,
                   const int64_t* vocabs, int64_t hidden, void* out, void* stream) {
  if (!ids || !tables || !vocabs || !out) return MTL_ERR_INVALID_ARG;
  if (rows < 1 || rows > 65535 || n_tables < 1 || hidden <= 0) return MTL_ERR_SHAPE;
  const int blocks = (int)((hidden + 255) / 256);
  hipLaunchKernelGGL(embed_rows_kernel, dim3(blocks < 64 ? blocks : 64, (unsigned)rows), dim3(256),
                     0, (hipStream_t)stream, ids, n_tables,
                     reinterpret_cast<const uint16_t* const*>(tables), vocabs, hidden,
                     static_cast<uint16_t*>(out));
  return launch_status();
}

int mtl_rmsnorm_gather(const void* x, int64_t ldx, const void* w, const int32_t* gather,
                       void* out, int64_t ldo, int64_t rows, int64_t n, float eps, void* stream) {
  if (!x || !w || !out) return MTL_ERR_INVALID_ARG;
  if (rows < 1 || rows > (int64_t)1 << 30 || n <= 0 || n % 8 != 0 || n > kRowNormMax ||
      ldx < n || ldo < n || ldx % 8 != 0 || ldo % 8 != 0)
    return MTL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w) || !aligned16(out)) return MTL_ERR_ALIGN;
  if (x == out && ldx != ldo) return MTL_ERR_INVALID_ARG;   // in place: the same row pitch
  hipLaunchKernelGGL(rmsnorm_gather_kernel, dim3((unsigned)rows), dim3(256), 0,
                     (hipStream_t)stream, const_cast<uint16_t*>(static_cast<const uint16_t*>(x)),
                     ldx, static_cast<const uint16_t*>(w), gather, static_cast<uint16_t*>(out),
                     ldo, (int)n, eps, nullptr, 0, nullptr);
  return launch_status();
}

int mtl_rmsnorm_gather_staged(const void* x, int64_t ldx, const void* w, const int32_t* gather,
                              void* out, int64_t ldo, float* sums, int64_t rows, int64_t n,
                              float eps, void* stream) {
  if (!x || !w || !out || !sums) return MTL_ERR_INVALID_ARG;
  if (rows < 1 || rows > (int64_t)1 << 30 || n <= 0 || n % 32 != 0 || n > kRowNormMax ||
      ldx < n || ldo < n || ldx % 8 != 0 || ldo % 8 != 0 || rows * (n / 32) * 4 >= ((int64_t)1 << 31))
    return MTL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(w) || !aligned16(out) || (gather && !aligned16(gather)) ||
      (reinterpret_cast<uintptr_t>(sums) & 3u))
    return MTL_ERR_ALIGN;
  if (x == out && ldx != ldo) return MTL_ERR_INVALID_ARG;   // in place: the same row pitch
  hipLaunchKernelGGL(rmsnorm_gather_kernel, dim3((unsigned)rows), dim3(256), 0,
                     (hipStream_t)stream, const_cast<uint16_t*>(static_cast<const uint16_t*>(x)),
                     ldx, static_cast<const uint16_t*>(w), gather, static_cast<uint16_t*>(out),
                     ldo, (int)n, eps, nullptr, 0, sums);
  return launch_status();
}

int mtl_residual_rmsnorm_gather(const float* partials, int32_t splits, int64_t partials_bytes,
                                void* h, int64_t ldh, const void* w, const int32_t* gather,
                                void* out, int64_t ldo, float* sums, int64_t rows, int64_t n,
                                float eps, void* stream) {
  if (!partials || !h || !w || !out) return MTL_ERR_INVALID_ARG;
  if (sums && (n % 32 != 0 || rows * (n / 32) * 4 >= ((int64_t)1 << 31))) return MTL_ERR_SHAPE;
  if (sums && ((gather && !aligned16(gather)) || (reinterpret_cast<uintptr_t>(sums) & 3u)))
    return MTL_ERR_ALIGN;
  if (splits < 1 || splits > kRowNormMaxSplits || rows < 1 || rows > (int64_t)1 << 30 || n <= 0 ||
      n % 8 != 0 || n > kRowNormMax || ldh < n || ldo < n || ldh % 8 != 0 || ldo % 8 != 0)
    return MTL_ERR_SHAPE;
  if (partials_bytes < (int64_t)splits * rows * n * 4) return MTL_ERR_WORKSPACE;
  if (!aligned16(partials) || !aligned16(h) || !aligned16(w) || !aligned16(out))
    return MTL_ERR_ALIGN;
  if (h == out) return MTL_ERR_INVALID_ARG;   // h is updated in place; out is the norm
  hipLaunchKernelGGL(rmsnorm_gather_kernel, dim3((unsigned)rows), dim3(256), 0,
                     (hipStream_t)stream, static_cast<uint16_t*>(h), ldh,
                     static_cast<const uint16_t*>(w), gather, static_cast<uint16_t*>(out), ldo,
                     (int)n, eps, partials, (int)splits, sums);
  return launch_status();
}

int mtl_qk_norm_rope_kv_rows(const void* qkv, int64_t ldq, int64_t rows, int64_t pos0,
                             const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                             const void* sin_tab, void* q_out, void* k_cache, void* v_cache,
                             int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                             int64_t max_seq, float eps, void* stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !q_out || !k_cache || !v_cache)
    return MTL_ERR_INVALID_ARG;
  if (head_dim != 128) return MTL_ERR_UNSUPPORTED;
  if (n_heads <= 0 || n_kv_heads <= 0 || rows < 1 || rows > 65535 || pos0 < 0 ||
      pos0 + rows > max_seq || ldq < (int64_t)(n_heads + 2 * n_kv_heads) * 128)
    return MTL_ERR_SHAPE;
  hipLaunchKernelGGL(qk_norm_rope_rows_kernel, dim3(n_heads + 2 * n_kv_heads, (unsigned)rows),
                     dim3(64), 0, (hipStream_t)stream, static_cast<const uint16_t*>(qkv), ldq,
                     pos0, static_cast<const uint16_t*>(q_norm_w),
                     static_cast<const uint16_t*>(k_norm_w), static_cast<const uint16_t*>(cos_tab),
                     static_cast<const uint16_t*>(sin_tab), static_cast<uint16_t*>(q_out),
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), n_heads,
                     n_kv_heads, max_seq, eps, nullptr, 0, 0);
  return launch_status();
}

int mtl_qk_norm_rope_kv_rows_partials(const float* partials, int32_t splits,
                                      int64_t partials_bytes, int64_t part_cols,
                                      const void* qkv, int64_t ldq, int64_t rows, int64_t pos0,
                                      const void* q_norm_w, const void* k_norm_w,
                                      const void* cos_tab, const void* sin_tab, void* q_out,
                                      void* k_cache, void* v_cache, int32_t n_heads,
                                      int32_t n_kv_heads, int32_t head_dim, int64_t max_seq,
                                      float eps, void* stream) {
  if (!partials || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !q_out || !k_cache ||
      !v_cache)
    return MTL_ERR_INVALID_ARG;
  if (head_dim != 128) return MTL_ERR_UNSUPPORTED;
  const int64_t cols = (int64_t)(n_heads + 2 * n_kv_heads) * 128;
  if (n_heads <= 0 || n_kv_heads <= 0 || rows < 1 || rows > 65535 || pos0 < 0 ||
      pos0 + rows > max_seq || splits < 1 || splits > kRowNormMaxSplits || part_cols < 128 ||
      part_cols % 128 != 0 || part_cols > cols)
    return MTL_ERR_SHAPE;
  if (part_cols < cols && (!qkv || ldq < cols)) return qkv ? MTL_ERR_SHAPE : MTL_ERR_INVALID_ARG;
  if (partials_bytes < (int64_t)splits * rows * part_cols * 4) return MTL_ERR_WORKSPACE;
  if (!aligned16(partials)) return MTL_ERR_ALIGN;
  hipLaunchKernelGGL(qk_norm_rope_rows_kernel, dim3(n_heads + 2 * n_kv_heads, (unsigned)rows),
                     dim3(64), 0, (hipStream_t)stream, static_cast<const uint16_t*>(qkv), ldq,
                     pos0, static_cast<const uint16_t*>(q_norm_w),
                     static_cast<const uint16_t*>(k_norm_w), static_cast<const uint16_t*>(cos_tab),
                     static_cast<const uint16_t*>(sin_tab), static_cast<uint16_t*>(q_out),
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), n_heads,
                     n_kv_heads, max_seq, eps, partials, (int)splits, part_cols);
  return launch_status();
}

int mtl_prefill_attention(const void* q, const void* k_cache, const void* v_cache, int64_t rows,
                          int64_t pos0, void* out, int64_t ldo, const int32_t* out_index,
                          int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, int64_t max_seq,
                          float scale, void* stream) {
  if (!q || !k_cache || !v_cache || !out) return MTL_ERR_INVALID_ARG;
  if (head_dim != 128) return MTL_ERR_UNSUPPORTED;
  if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads / n_kv_heads > 8 ||
      rows < 1 || pos0 < 0 || pos0 + rows > max_seq || (rows + kPaRows - 1) / kPaRows > 65535 ||
      ldo < (int64_t)n_heads * 128)
    return MTL_ERR_SHAPE;
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache)) return MTL_ERR_ALIGN;
  PrefillAttnArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.out = static_cast<uint16_t*>(out);
  a.out_index = out_index;
  a.ldo = ldo;
  a.pos0 = pos0;
  a.max_seq = max_seq;
  a.rows = (int)rows;
  a.H = n_heads;
  a.Hkv = n_kv_heads;
  a.scale = scale;
  const dim3 grid(n_kv_heads, (unsigned)((rows + kPaRows - 1) / kPaRows));
  if (n_heads / n_kv_heads <= 4)
    hipLaunchKernelGGL(prefill_attn_kernel<1>, grid, dim3(512), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(prefill_attn_kernel<2>, grid, dim3(512), 0, (hipStream_t)stream, a);
  return launch_status();
}

}  // extern "C"
