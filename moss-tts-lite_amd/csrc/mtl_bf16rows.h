// bf16 GEMV with RMSNorm staging for the kept (unquantised) projections of the decode step,
// as a workgroup body: the kernel of mtl_bf16_gemv_norm runs it alone, and the strip GEMV's
// combined launch runs it beside the int4 q|k GEMV that reads the same h.
#pragma once
#include "mtl_common.h"

namespace mtl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // as in the other kernels

// bf16 GEMV with RMSNorm staging for a kept projection (few rows per wave: v_proj is
// 1024 x 4096).  The workgroup forms x = RMSNorm(h) once into LDS (each thread a share
// of the 8-channel items) while its waves' first weight rows are already in flight; each
// wave then holds x in registers in the head GEMV's lane layout (k = 512 i + 8 lane) and
// streams rows wave, wave + 4, ... of the workgroup's band, two rows per pass.  Products,
// their order and the roundings are the head GEMV's, so the results are the same bits;
// the head GEMV forms x in every wave, which costs more than the row itself here.
struct Bf16RowsArgs {
  const uint16_t* h;          // bf16 [K] residual stream
  const uint16_t* norm_w;     // bf16 [K] RMSNorm weight
  const float* slots;         // sums of squares of h per 16 columns
  float eps;
  const uint16_t* w;          // bf16 [N, K] rows
  int64_t N;
  int K, rows_per_wg;
  float* out;                 // [N]: the bf16 products as fp32
};

// The body of one workgroup (256 threads, 4 waves) over band `bid`: the rows
// bid * rows_per_wg .. of w.
template <int kKit>
__device__ __forceinline__ void bf16_rows_norm_body(const Bf16RowsArgs& p, int bid) {
  const uint16_t* __restrict__ h = p.h;
  const uint16_t* __restrict__ norm_w = p.norm_w;
  const float* __restrict__ slots = p.slots;
  const float eps = p.eps;
  const uint16_t* __restrict__ w = p.w;
  const int64_t N = p.N;
  const int K = p.K, rows_per_wg = p.rows_per_wg;
  float* __restrict__ out = p.out;
  __shared__ u32x4 xs[kKit * 64];               // x items: item j holds channels 8j .. 8j+7
  const int t = threadIdx.x, wave = wave_id(), lane = t & 63;
  const int64_t b0 = (int64_t)bid * rows_per_wg;
  const int nrows = (int)((b0 + rows_per_wg < N ? b0 + rows_per_wg : N) - b0);
  // Every load goes through a bounds-checked buffer resource (the band's rows, h, norm_w,
  // the slots): a row past the band or a channel past K reads 0, so no load sits under a
  // branch (a branch around a load made the compiler wait for all loads in flight), and a
  // zero weight against a zero x item adds nothing (the sums cannot be -0).
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(w + b0 * K), (short)0, nrows * K * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t hrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(h), (short)0, K * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t grs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(norm_w), (short)0, K * 2, 0x00020000);
  const int ns = (K + kSlotCols - 1) / kSlotCols;
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(slots), (short)0, ns * 4, 0x00020000);
  const int wbytes = nrows * K * 2;
  // x = bf16(norm_w * bf16(h * r)), r from h's sums of squares (every wave sums them).
  // Its inputs (shared by every workgroup, so mostly L2 hits) are loaded before the weight
  // rows: loads complete in issue order, so x is formed while the rows stream in.
  float4 sv[kMaxSlots / 256];
#pragma unroll
  for (int it = 0; it < kMaxSlots / 256; ++it)
    sv[it] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                            srs, (4 * lane + 256 * it) * 4, 0, 0));
  const int items = K / 8;
  constexpr int kStage = (kKit * 64 + 255) / 256;   // items staged per thread
  u32x4 hv[kStage], gv[kStage];
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int j = t + 256 * u;
    hv[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(hrs, 16 * j, 0, 0));
    gv[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(grs, 16 * j, 0, 0));
  }
  // rows rl and rl + 4 of the band (a wave's rows in one pass), non-temporal
  u32x4 ww[2][kKit];
  auto issue = [&](int rl) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r = rl + 4 * j;
#pragma unroll
      for (int i = 0; i < kKit; ++i) {
        const int k = 512 * i + 8 * lane;
        const int off = r < nrows && k < K ? (r * K + k) * 2 : wbytes;
        ww[j][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, off, 0, 2));
      }
    }
  };
  __builtin_amdgcn_sched_barrier(0);
  issue(wave);
  __builtin_amdgcn_sched_barrier(0);
  float ss = 0.f;
#pragma unroll
  for (int it = 0; it < kMaxSlots / 256; ++it) {
    const int bs = 4 * lane + 256 * it;
    const float4 v = sv[it];
    ss += ((bs < ns ? v.x : 0.f) + (bs + 1 < ns ? v.y : 0.f)) +
          ((bs + 2 < ns ? v.z : 0.f) + (bs + 3 < ns ? v.w : 0.f));
  }
  const float r = rsqrtf(wave_sum_valu(ss) / (float)K + eps);
#pragma unroll
  for (int u = 0; u < kStage; ++u) {
    const int j = t + 256 * u;
    if (j < items) {
      const uint32_t hh[4] = {hv[u].x, hv[u].y, hv[u].z, hv[u].w};
      const uint32_t gg[4] = {gv[u].x, gv[u].y, gv[u].z, gv[u].w};
      uint32_t o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t lo = f32_to_bf16(round_bf16(lo_bf(gg[c]) * round_bf16(lo_bf(hh[c]) * r)));
        const uint32_t hi = f32_to_bf16(round_bf16(hi_bf(gg[c]) * round_bf16(hi_bf(hh[c]) * r)));
        o[c] = lo | (hi << 16);
      }
      xs[j] = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
  __syncthreads();
  u32x4 xv[kKit];
#pragma unroll
  for (int i = 0; i < kKit; ++i) {
    const int j = 64 * i + lane;                 // channels 512 i + 8 lane
    xv[i] = 8 * j < K ? xs[j] : u32x4{0u, 0u, 0u, 0u};
  }
  for (int rb = wave; rb < nrows; rb += 8) {
    float acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      acc[j] = 0.f;
#pragma unroll
      for (int i = 0; i < kKit; ++i) {
        acc[j] = dot2_bf16(ww[j][i].x, xv[i].x, acc[j]);
        acc[j] = dot2_bf16(ww[j][i].y, xv[i].y, acc[j]);
        acc[j] = dot2_bf16(ww[j][i].z, xv[i].z, acc[j]);
        acc[j] = dot2_bf16(ww[j][i].w, xv[i].w, acc[j]);
      }
    }
    issue(rb + 8);                               // the next pass's rows (past the band: 0)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int row = rb + 4 * j;
      const float sum = wave_sum_valu(acc[j]);
      if (row < nrows && lane == 0) out[b0 + row] = bf16_to_f32(f32_to_bf16(sum));
    }
  }
}

// Rows per workgroup of bf16_rows_norm_kernel and of the bf16 half of the combined launch:
// 8 (two rows per wave and pass), or 16 where that still leaves 3 workgroups per CU.
// Measured on the MOSS step's kept linears (v_proj 1024 rows, up_proj 12288 rows beside
// their int4 partners): 526 -> 541 steps/s against a band spreading the rows over the CUs
// (4 and 48 rows); 16 rows for v_proj or 8 / 12 for up_proj measured the same or slower.
inline int bf16_rows_per_wg(int64_t N, int cus) {
  return N / 16 >= 3 * (int64_t)cus ? 16 : 8;
}


}  // namespace mtl
