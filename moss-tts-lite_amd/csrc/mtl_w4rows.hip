// Skinny-batch int4 GEMM over full-K column strips for gfx950: y[M, N] = x[M, K] @ W, with
// 2 <= M <= 16 rows (prefill chunks, batched decode), AutoGPTQ metadata, g = 128 or 256.
//
// The weights are the strip layout of the M = 1 strip GEMV (mtl_w4strip.hip): 1 KB block
// (s * K/128 + b) holds columns 16s..16s+15 over input channels 128b..128b+127, lane l's 16
// bytes being the B operands of four v_mfma_f32_16x16x32_bf16.  Here the 16 A rows are the
// 16 x rows (rows >= M read as zero), so one MFMA does the work of 16 GEMVs and the code
// unpack is shared by every row.  A workgroup owns CT strips over all of K, so no split-K
// partial ever leaves it: the split-K GEMM writes and re-reads splits * M * N * 4 bytes of
// partials, which at M = 16 on the 4096 x 24576 projection is 12.6 MB per launch.
//
// x of all M rows over all of K is staged once per workgroup in LDS as [M][K/8 + 1] items
// in pair order (one item of padding per row against bank conflicts) (up to 16 * K * 2 bytes: K <= 4096), plus one zero row that the A operands of
// rows >= M read, with its per-group sums as [group][16 rows]
// (rows >= M zero), so every workgroup (one per CU) reads x once from L2 and a lane reads
// the sums of its four result rows with one LDS load.
#include "mtl_w4core.h"

namespace mtl {

constexpr int kStripCols = 16;         // output columns per strip
constexpr int kRowsMax = 16;
constexpr int kRowsMaxK = 4096;       // 16 rows of x and a zero row in LDS (140 KB)
constexpr int kRowsMaxWaves = 16;
// Waves per workgroup: 16 (128 VGPRs each), 12 (168 VGPRs) at 16 blocks per wave.
constexpr int rows_max_waves(int nb) { return nb >= 16 ? 12 : kRowsMaxWaves; }
constexpr int kRowsAux = 2;           // weight stream: non-temporal (read once)

struct RowsArgs {
  const u32x4* w;             // strip layout
  const uint16_t* scales;     // fp16 [G, N]
  const uint32_t* qzeros;     // int32 [G, N/8]
  const uint16_t* x;          // bf16 [M, K], rows ldx apart
  void* y;                    // [M, N], rows ldy apart, bf16 or f32
  int64_t ldx, ldy;
  int M, K, N, group, zero_offset, out_f32, kblocks, xcd_order;
};

// Wave w serves strip w % CT over K slice w / CT (KW slices of NB blocks); WIN blocks of the
// weight stream in flight per wave, as in the M = 1 strip GEMV.
template <int GR, int NB, int CT, int WIN>
__global__ void __launch_bounds__(64 * rows_max_waves(NB), 1) w4_rows_kernel(RowsArgs a) {
  constexpr int NGW = 4 * NB / GR;             // quantisation groups per slice
  constexpr int GI = 4 * GR;                   // x items per group
  constexpr int MB = GR <= 4 ? 4 / GR : 1;     // groups starting in one block
  static_assert((4 * NB) % GR == 0 && 64 % GI == 0, "whole groups per slice and per wave");
  static_assert(NB % WIN == 0 && (GR != 8 || WIN % 2 == 0), "ring window");
  extern __shared__ u32x4 smem[];
  const int nw = blockDim.x >> 6;
  const int kw = nw / CT;                      // K slices
  const int K8 = a.K >> 3;                     // x items per row
  const int ngrp = a.K / a.group;
  // rows XS = K8 + 1 items apart: the 16 rows an MFMA's A operand reads then start 16
  // bytes apart in the LDS banks instead of all on the same banks
  const int XS = K8 + 1;
  u32x4* xa = smem;                                                   // [M + 1][XS]
  float* xg = reinterpret_cast<float*>(smem + (size_t)(a.M + 1) * XS);  // [ngrp][16]
  float* ytile = xg + 16 * ngrp;                                      // [nw][16][16]

  const int wave = wave_id();
  const int lane = threadIdx.x & 63;
  const int lg = lane >> 4, lj = lane & 15;
  const int cs = wave % CT, ks = wave / CT;
  const int G = gridDim.x;
  const int wg = a.xcd_order ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int s = wg * CT + cs;
  const int N = a.N;
  const int col = s * kStripCols + lj;
  const int rq0 = ks * 4 * NB;                 // first row quad (32 channels) of the slice

  // 1. The weight ring and its group metadata go out first (they do not depend on x).
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4*>(a.w), (short)0, (int)((int64_t)(N / kStripCols) * a.kblocks * 1024),
      0x00020000);
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.scales), (short)0, ngrp * N * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t zrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(a.qzeros), (short)0, ngrp * (N >> 3) * 4, 0x00020000);
  const int blk0 = s * a.kblocks + ks * NB;
  const int grp0 = rq0 / GR;
  u32x4 wq[WIN];
  uint32_t ms[WIN][MB], mz[WIN][MB];
  auto issue = [&](int r, int b) {             // block b into ring slot r (r = b % WIN)
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      if (GR <= 4 || (r & 1) == 0) {           // g = 256: one group per block pair
        const int g = grp0 + (GR <= 4 ? b * MB + m : b >> 1);
        ms[r][m] = __builtin_amdgcn_raw_buffer_load_b16(srsrc, col * 2, g * N * 2, 0);
        mz[r][m] = __builtin_amdgcn_raw_buffer_load_b32(zrsrc, (col >> 3) * 4, g * (N >> 3) * 4, 0);
      }
    }
    wq[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          wrsrc, lane * 16, (blk0 + b) * 1024, kRowsAux));
  };
#pragma unroll
  for (int b = 0; b < WIN; ++b) issue(b, b);
  __builtin_amdgcn_sched_barrier(0);

  // 2. x of all M rows into LDS in pair order, with per-group sums.  Flat item f = m*K8 + i:
  //    a wave covers 64 consecutive items, whose groups of GI items (GI divides 64 and K8)
  //    sit in GI consecutive lanes of one row.  Loads of a batch are all issued first.
  {
    const int nthr = blockDim.x;
    const int total = a.M * K8;
    for (int z = threadIdx.x; z < ngrp * 16; z += nthr)        // group sums of rows >= M
      if ((z & 15) >= a.M) xg[z] = 0.f;
    for (int z = threadIdx.x; z < K8; z += nthr)               // row M: the zero A row
      xa[a.M * XS + z] = u32x4{0u, 0u, 0u, 0u};
    // loads per thread in flight: 16 rows of K = 4096 in one batch (12 at 12 waves, 8 at 16)
    constexpr int BATCH = rows_max_waves(NB) == 12 ? 12 : 8;
    for (int f0 = 0; f0 < total; f0 += BATCH * nthr) {
      u32x4 v[BATCH];
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int f = f0 + u * nthr + threadIdx.x;
        const int m = f / K8, i = f - m * K8;
        v[u] = f < total ? *reinterpret_cast<const u32x4*>(a.x + m * a.ldx + (int64_t)i * 8)
                         : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int fb = f0 + u * nthr + wave * 64;        // wave-uniform
        if (fb >= total) break;
        const int f = fb + lane;
        float sum;
        const u32x4 pv = pair_order(v[u], sum);
#pragma unroll
        for (int o = 1; o < GI; o <<= 1) sum += __shfl_xor(sum, o);
        if (f < total) {                                 // M * K8 need not fill the wave
          const int m = f / K8, i = f - m * K8;
          xa[m * XS + i] = pv;
          if ((i & (GI - 1)) == 0) xg[(i / GI) * 16 + m] = sum;
        }
      }
    }
  }
  __syncthreads();

  // 3. MFMA over the slice's row quads as the ring delivers them.  Lane l supplies A row
  //    l%16 (x row m = l%16, the zero row when m >= M) and holds results D[4*(l/16) + r][l%16],
  //    r = 0..3; per group y[m] += s * (A[m] - (128 + z) * X[m]).
  const uint32_t kMagic = vgpr_const(0x43004300u);
  const uint32_t kLo = vgpr_const(0x000F000Fu);
  const u32x4* xrow = xa + (lj < a.M ? lj : a.M) * XS;       // rows >= M read the zero row
  float tot[4] = {0.f, 0.f, 0.f, 0.f};
  float cur_s = 0.f, cur_z = 0.f;
  floatx4 acc;
  auto turn = [&](const int b0, const bool refill) {
#pragma unroll
    for (int r = 0; r < WIN; ++r) {
      const int b = b0 + r;
      const u32x4 w4 = wq[r];
      float gs[MB], gz[MB];
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        gs[m] = f16_to_f32(ms[r][m] & 0xffffu);
        gz[m] = (float)(128 + (int)((mz[r][m] >> ((col & 7) * 4)) & 0xfu) + a.zero_offset);
      }
      if (GR == 8 && (r & 1) == 0) { cur_s = gs[0]; cur_z = gz[0]; }
      asm volatile("" ::: "memory");
      if (refill) issue(r, b + WIN);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int rq = rq0 + 4 * b + j;
        const int q = (4 * r + j) % GR;
        if (q == 0) acc = floatx4{0.f, 0.f, 0.f, 0.f};
        const uint32_t w = j == 0 ? w4.x : j == 1 ? w4.y : j == 2 ? w4.z : w4.w;
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xrow[4 * rq + lg]),
                                                      unpack_codes8(w, kLo, kMagic), acc, 0, 0, 0);
        if (q == GR - 1) {
          const float sc = GR == 8 ? cur_s : gs[j / GR];
          const float cz = GR == 8 ? cur_z : gz[j / GR];
          const float4 X = *reinterpret_cast<const float4*>(xg + (rq / GR) * 16 + 4 * lg);
          tot[0] = fmaf(sc, fmaf(-cz, X.x, acc[0]), tot[0]);
          tot[1] = fmaf(sc, fmaf(-cz, X.y, acc[1]), tot[1]);
          tot[2] = fmaf(sc, fmaf(-cz, X.z, acc[2]), tot[2]);
          tot[3] = fmaf(sc, fmaf(-cz, X.w, acc[3]), tot[3]);
        }
      }
    }
  };
#pragma unroll
  for (int b0 = 0; b0 < NB - WIN; b0 += WIN) turn(b0, true);
  turn(NB - WIN, false);

  // 4. Per-slice results meet in LDS and are added in slice order (bitwise repeatable).
#pragma unroll
  for (int e = 0; e < 4; ++e) ytile[(wave * 16 + 4 * lg + e) * 16 + lj] = tot[e];
  __syncthreads();
  for (int idx = threadIdx.x; idx < CT * 256; idx += blockDim.x) {
    const int c = idx >> 8, m = (idx >> 4) & 15, n = idx & 15;
    if (m >= a.M) continue;
    float v = 0.f;
    for (int k = 0; k < kw; ++k) v += ytile[((k * CT + c) * 16 + m) * 16 + n];
    const int64_t o = m * a.ldy + (int64_t)(wg * CT + c) * kStripCols + n;
    if (a.out_f32) static_cast<float*>(a.y)[o] = v;
    else static_cast<uint16_t*>(a.y)[o] = (uint16_t)f32_to_bf16(v);
  }
}

// Launch geometry: CT strips per workgroup so that the grid fits one workgroup per CU
// (x takes up to 128 KB of LDS), then the most waves (up to 16) that split K evenly with
// NB blocks of 16, 8, 4 or 2.
struct RowsGeom {
  int ct, nb, kw;
};

static RowsGeom rows_geometry(int64_t K, int64_t N, int cus) {
  const int64_t strips = N / kStripCols;
  const int64_t kb = K / 128;
  RowsGeom g{0, 0, 0};
  for (const int ct : {1, 2, 3, 4, 6, 8, 12, 16}) {
    if (strips % ct == 0 && strips / ct <= cus) { g.ct = ct; break; }
  }
  if (!g.ct) return g;
  for (const int nb : {2, 4, 8, 16}) {
    if (kb % nb == 0 && (kb / nb) * g.ct <= rows_max_waves(nb)) {
      g.nb = nb;
      g.kw = (int)(kb / nb);
      break;
    }
  }
  return g;
}

// Dynamic LDS above 64 KB is granted per kernel (once per instantiation, before its first
// launch; not a stream operation, so it is safe during graph capture).
template <typename Kern>
static void rows_launch(Kern kern, dim3 grid, dim3 block, size_t lds, hipStream_t st,
                        const RowsArgs& a, bool& opted) {
  if (!opted) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    opted = true;
  }
  hipLaunchKernelGGL(kern, grid, block, lds, st, a);
}

template <int GR, int CT>
static void rows_nb(const RowsArgs& a, const RowsGeom& g, size_t lds, hipStream_t st) {
  const dim3 grid(a.N / (kStripCols * CT)), block(64 * CT * g.kw);
  static bool opted[4] = {false, false, false, false};
  switch (g.nb) {
    case 2: rows_launch(w4_rows_kernel<GR, 2, CT, 2>, grid, block, lds, st, a, opted[0]); break;
    case 4: rows_launch(w4_rows_kernel<GR, 4, CT, 4>, grid, block, lds, st, a, opted[1]); break;
    case 8: rows_launch(w4_rows_kernel<GR, 8, CT, 4>, grid, block, lds, st, a, opted[2]); break;
    default: rows_launch(w4_rows_kernel<GR, 16, CT, 4>, grid, block, lds, st, a, opted[3]); break;
  }
}

template <int GR>
static void rows_ct(const RowsArgs& a, const RowsGeom& g, size_t lds, hipStream_t st) {
  switch (g.ct) {
    case 1: rows_nb<GR, 1>(a, g, lds, st); break;
    case 2: rows_nb<GR, 2>(a, g, lds, st); break;
    case 3: rows_nb<GR, 3>(a, g, lds, st); break;
    case 4: rows_nb<GR, 4>(a, g, lds, st); break;
    case 6: rows_nb<GR, 6>(a, g, lds, st); break;
    case 8: rows_nb<GR, 8>(a, g, lds, st); break;
    case 12: rows_nb<GR, 12>(a, g, lds, st); break;
    default: rows_nb<GR, 16>(a, g, lds, st); break;
  }
}

static int g_rows_cus = 0;

static int device_cus() {
  if (!g_rows_cus) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_rows_cus = n;
  }
  return g_rows_cus;
}

}  // namespace mtl

using namespace mtl;

extern "C" {

int mtl_w4_gemm_strip_rows(const void* x, int64_t M, int64_t ldx, int64_t K,
                           const int32_t* strip_weight, const void* scales,
                           const int32_t* qzeros, int64_t N, int32_t group_size,
                           int32_t zero_offset, void* y, int64_t ldy, int32_t out_dtype,
                           void* stream) {
  if (!x || !strip_weight || !scales || !qzeros || !y) return MTL_ERR_INVALID_ARG;
  if (out_dtype != MTL_OUT_BF16 && out_dtype != MTL_OUT_F32) return MTL_ERR_INVALID_ARG;
  if (group_size != 32 && group_size != 64 && group_size != 128 && group_size != 256)
    return MTL_ERR_GROUP;
  // g = 32 and 64 bring 2 to 4 groups per block, whose metadata and corrections do not
  // fit the register budget of 16 rows: the split-K GEMM serves them
  if (group_size < 128) return MTL_ERR_UNSUPPORTED;
  if (M < 1 || M > kRowsMax || K <= 0 || N <= 0 || K % 256 != 0 || K > kRowsMaxK ||
      N % kStripCols != 0 || K % group_size != 0 || ldx < K || ldy < N ||
      ldx * (M - 1) + K >= ((int64_t)1 << 31) || ldy * (M - 1) + N >= ((int64_t)1 << 31))
    return MTL_ERR_SHAPE;
  if (!aligned16(x) || ldx % 8 != 0 || !aligned16(strip_weight) || !aligned16(scales) ||
      (reinterpret_cast<uintptr_t>(qzeros) & 7u) ||
      (reinterpret_cast<uintptr_t>(y) & (out_dtype == MTL_OUT_F32 ? 3u : 1u)))
    return MTL_ERR_ALIGN;
  const RowsGeom g = rows_geometry(K, N, device_cus());
  if (!g.ct || !g.nb) return MTL_ERR_SHAPE;
  RowsArgs a;
  a.w = reinterpret_cast<const u32x4*>(strip_weight);
  a.scales = static_cast<const uint16_t*>(scales);
  a.qzeros = reinterpret_cast<const uint32_t*>(qzeros);
  a.x = static_cast<const uint16_t*>(x);
  a.y = y;
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = (int)M; a.K = (int)K; a.N = (int)N;
  a.group = group_size;
  a.zero_offset = zero_offset;
  a.out_f32 = out_dtype == MTL_OUT_F32;
  a.kblocks = (int)(K / 128);
  const int64_t G = N / (kStripCols * g.ct);
  a.xcd_order = G % 8 == 0;
  const size_t lds = (size_t)(M + 1) * (K / 8 + 1) * 16 + (size_t)16 * (K / group_size) * 4 +
                     (size_t)g.ct * g.kw * 256 * 4;
  hipStream_t st = (hipStream_t)stream;
  if (group_size == 128) rows_ct<4>(a, g, lds, st);
  else rows_ct<8>(a, g, lds, st);
  return launch_status();
}

}  // extern "C"
