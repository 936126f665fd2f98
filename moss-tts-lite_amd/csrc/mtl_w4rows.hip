// Skinny-batch int4 GEMM over full-K column strips for gfx950: y[M, N] = x[M, K] @ W, with
// 1 <= M <= 16 rows (prefill chunks, batched decode), g = 32 to 256, AutoGPTQ metadata or
// the reference's qsz pairs, x optionally gathered through an act-order index.
//
// The weights are the strip layout of the M = 1 strip GEMV (mtl_w4strip.hip): 1 KB block
// (s * K/128 + b) holds columns 16s..16s+15 over input channels 128b..128b+127, lane l's 16
// bytes being the B operands of four v_mfma_f32_16x16x32_bf16.  Here the 16 A rows are the
// 16 x rows (rows >= M read as zero), so one MFMA does the work of 16 GEMVs and the code
// unpack is shared by every row.  A workgroup owns CT strips over all of K, so no split-K
// partial ever leaves it: the split-K GEMM writes and re-reads splits * M * N * 4 bytes of
// partials, which at M = 16 on the 4096 x 24576 projection is 12.6 MB per launch.
//
// x of all M rows sits in LDS as [M + 1][KP/8 + 1] items in pair order (one item of padding
// per row against bank conflicts), plus one zero row that the A operands of rows >= M read,
// with its per-group sums as [group][16 rows] (rows >= M zero), so a lane reads the sums of
// its four result rows with one LDS load.  K runs in phases of KP input channels, as many
// as 16 rows fit the 160 KB of LDS (all of K at once up to K = 4096): each phase stages
// its x, every wave multiplies its blocks of that phase, and the weight ring runs on across
// the phase boundary (the last ring turn of a phase issues the next phase's first blocks).
#include "mtl_w4core.h"

namespace mtl {

constexpr int kStripCols = 16;         // output columns per strip
constexpr int kRowsMax = 16;
constexpr size_t kRowsMaxLds = 160 * 1024;
constexpr int kRowsMaxWaves = 16;
// Waves per workgroup: 16 (128 VGPRs each), 12 (168 VGPRs) at 16 blocks per wave.
constexpr int rows_max_waves(int nb) { return nb >= 16 ? 12 : kRowsMaxWaves; }
// Weight blocks in flight per wave: 4, or 2 at g <= 64 (whose 2 to 4 groups per block bring
// as many metadata registers) and at 2 blocks per wave.
constexpr int rows_ring(int gr, int nb) { return nb == 2 || gr <= 2 ? 2 : 4; }
constexpr int kRowsAux = 2;           // weight stream: non-temporal (read once)

struct RowsArgs {
  const u32x4* w;             // strip layout
  const uint16_t* scales;     // fp16 [G, N] (GPTQ), or the qsz bf16 pairs [G, N, 2]
  const uint32_t* qzeros;     // int32 [G, N/8] (GPTQ metadata)
  const uint16_t* x;          // bf16 [M, K], rows ldx apart
  const int32_t* perm;        // input row k of the weight is x channel perm[k]; NULL: k
  void* y;                    // [M, N], rows ldy apart, bf16 or f32
  int64_t ldx, ldy;
  int M, K, N, group, zero_offset, out_f32, kblocks, xcd_order;
  int kp;                     // input channels per phase (a multiple of 256 dividing K)
  int ct;                     // strips per workgroup
  int xraw;                   // act-order: x's M rows sit in LDS past the slice tiles
};

// Wave w serves strip w % CT over K slice w / CT (KW slices of NB blocks per phase, CT =
// a.ct); WIN blocks of the weight stream in flight per wave, as in the M = 1 strip GEMV.
template <int GR, int NB, int FMT, bool PERM>
__global__ void __launch_bounds__(64 * rows_max_waves(NB), 1) w4_rows_kernel(RowsArgs a) {
  constexpr int WIN = rows_ring(GR, NB);
  constexpr int GI = 4 * GR;                   // x items per group
  constexpr int MB = GR <= 4 ? 4 / GR : 1;     // groups starting in one block
  static_assert((4 * NB) % GR == 0 && 64 % GI == 0, "whole groups per slice and per wave");
  static_assert(NB % WIN == 0 && (GR != 8 || WIN % 2 == 0), "ring window");
  constexpr bool kQsz = FMT == STRIP_META_QSZ;
  extern __shared__ u32x4 smem[];
  const int nw = blockDim.x >> 6;
  const int K8 = a.kp >> 3;                    // x items per row and phase
  const int ngrp = a.K / a.group;              // groups over all of K (metadata bounds)
  const int pgrp = a.kp / a.group;             // groups per phase (LDS sums)
  const int kbp = a.kp >> 7;                   // blocks per phase
  const int nphase = a.K / a.kp;
  // x item f of a phase is row f / K8, item f % K8: a shift and a mask where K8 is a power
  // of two (every phase of the decode shapes), instead of the integer division's ~40 VALU
  const bool k8p2 = (K8 & (K8 - 1)) == 0;
  const int k8s = 31 - __builtin_clz(K8);
  auto row_of = [&](int f) { return k8p2 ? f >> k8s : f / K8; };
  const int kr8 = a.K >> 3;                    // x items per row over all of K
  const bool kr8p2 = (kr8 & (kr8 - 1)) == 0;
  const int kr8s = 31 - __builtin_clz(kr8);
  // rows XS = K8 + 1 items apart: the 16 rows an MFMA's A operand reads then start 16
  // bytes apart in the LDS banks instead of all on the same banks
  const int XS = K8 + 1;
  u32x4* xa = smem;                                                   // [M + 1][XS]
  float* xg = reinterpret_cast<float*>(smem + (size_t)(a.M + 1) * XS);  // [pgrp][16]
  float* ytile = xg + 16 * pgrp;                                      // [nw][16][16]
  uint16_t* xr = reinterpret_cast<uint16_t*>(ytile + nw * 256);       // xraw: [M][K]

  const int wave = wave_id();
  const int lane = threadIdx.x & 63;
  const int lg = lane >> 4, lj = lane & 15;
  const int CT = a.ct;
  const int cs = wave % CT, ks = wave / CT;
  const int G = gridDim.x;
  const int wg = a.xcd_order ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int s = wg * CT + cs;
  const int N = a.N;
  const int col = s * kStripCols + lj;
  const int rq0 = ks * 4 * NB;                 // the slice's first row quad (32 channels) in a phase

  const int xbytes = (int)(((int64_t)(a.M - 1) * a.ldx + a.K) * 2);
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x), (short)0, xbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(a.perm), (short)0, PERM ? a.K * 4 : 0, 0x00020000);
  // Act-order with x resident (a.xraw): x's M rows go to LDS once, in 16-byte loads that
  // a few cycles of the texture unit serve per wave instead of a cycle per gathered
  // channel, and every phase gathers from there.  The first batch of those loads goes out
  // ahead of the weight stream, so it does not queue behind it.
  const int xr_items = PERM && a.xraw ? a.M * (a.K >> 3) : 0;
  u32x4 rv[4];
  auto raw_load = [&](int f0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int f = f0 + u * (int)blockDim.x + threadIdx.x;
      const int m = kr8p2 ? f >> kr8s : f / kr8, i = f - m * kr8;
      const int xo = f < xr_items ? (m * (int)a.ldx + 8 * i) * 2 : xbytes;
      rv[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, xo, 0, 0));
    }
  };
  auto raw_store = [&](int f0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int f = f0 + u * (int)blockDim.x + threadIdx.x;
      if (f < xr_items) reinterpret_cast<u32x4*>(xr)[f] = rv[u];   // item m * K/8 + i
    }
  };
  if (xr_items) raw_load(0);
  // x without the gather: the BATCH items per thread of phase items f0 + u * threads,
  // through the bounds-checked resource (items past the M rows read 0)
  constexpr int BATCH = 4;   // items per thread in flight (more spill the MFMA loop's registers)
  auto x_batch = [&](int c0, int f0, u32x4 (&v)[BATCH]) {
    const int nthr = blockDim.x;
    const int total = a.M * K8;
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int f = f0 + u * nthr + threadIdx.x;
      const int m = row_of(f), i = f - m * K8;
      const int xo = f < total ? (m * (int)a.ldx + c0 + 8 * i) * 2 : xbytes;
      v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, xo, 0, 0));
    }
  };
  // phase 0's first batch goes out ahead of the weight stream: loads return in issue order,
  // so behind the ring it would wait for the ring's blocks
  u32x4 xv0[BATCH];
  if constexpr (!PERM) x_batch(0, 0, xv0);

  // 1. The weight ring and its group metadata go out next (they do not depend on x).
  //    Block i of this wave's sequence (i = phase * NB + b) is K block phase * kbp + ks * NB + b.
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4*>(a.w), (short)0, (int)((int64_t)(N / kStripCols) * a.kblocks * 1024),
      0x00020000);
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.scales), (short)0, ngrp * N * (kQsz ? 4 : 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t zrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(a.qzeros), (short)0, kQsz ? 0 : ngrp * (N >> 3) * 4, 0x00020000);
  const int wblk0 = s * a.kblocks;
  u32x4 wq[WIN];
  uint32_t ms[WIN][MB], mz[kQsz ? 1 : WIN][MB];
  auto issue = [&](int r, int i) {             // block i into ring slot r (r = i % WIN)
    const int kb = (i / NB) * kbp + ks * NB + i % NB;
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      if (GR <= 4 || (r & 1) == 0) {           // g = 256: one group per block pair
        const int g = GR <= 4 ? kb * MB + m : kb >> 1;
        if constexpr (kQsz) {
          ms[r][m] = qsz_load(srsrc, col, g, N);
        } else {
          ms[r][m] = __builtin_amdgcn_raw_buffer_load_b16(srsrc, col * 2, g * N * 2, 0);
          mz[r][m] = __builtin_amdgcn_raw_buffer_load_b32(zrsrc, (col >> 3) * 4, g * (N >> 3) * 4, 0);
        }
      }
    }
    wq[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          wrsrc, lane * 16, (wblk0 + kb) * 1024, kRowsAux));
  };
#pragma unroll
  for (int b = 0; b < WIN; ++b) issue(b, b);
  __builtin_amdgcn_sched_barrier(0);

  // 2. Per phase: x of all M rows over the phase's channels into LDS in pair order, with
  //    per-group sums.  Flat item f = m*K8 + i: a wave covers 64 consecutive items, whose
  //    groups of GI items (GI divides 64 and K8) sit in GI consecutive lanes of one row.
  //    Loads of a batch are all issued first.  Row M (the zero A row) and the sums of rows
  //    >= M are written once; staging never touches them.
  for (int z = threadIdx.x; z < pgrp * 16; z += blockDim.x)
    if ((z & 15) >= a.M) xg[z] = 0.f;
  for (int z = threadIdx.x; z < K8; z += blockDim.x) xa[a.M * XS + z] = u32x4{0u, 0u, 0u, 0u};
  // x comes through bounds-checked buffer resources over the M rows (and the act-order
  // index): an item past the last row reads 0, so a batch's loads carry no branch and go
  // out together (a branch per load made the compiler wait for each before the next)
  // a staged batch into LDS in pair order, with its per-group sums
  auto put = [&](int f0, const u32x4 (&v)[BATCH]) {
    const int nthr = blockDim.x;
    const int total = a.M * K8;
#pragma unroll
    for (int u = 0; u < BATCH; ++u) {
      const int fb = f0 + u * nthr + wave * 64;        // wave-uniform
      if (fb >= total) break;
      const int f = fb + lane;
      float sum;
      // v_perm and a v_dot2 chain: about 8 VALU per item against pair_order's 20 (the sums
      // round in another order than the M = 1 strip GEMV's tree: within fp32 rounding);
      // with the index arithmetic above, gate|up at M = 16 went from 15.8 to 14.6 us and
      // down from 21.0 to 15.4
      const u32x4 pv = pair_order_dot(v[u], sum);
      sum = group_sum_valu<GI>(sum);           // every lane of the wave active here
      if (f < total) {                                 // M * K8 need not fill the wave
        const int m = row_of(f), i = f - m * K8;
        xa[m * XS + i] = pv;
        if ((i & (GI - 1)) == 0) xg[(i / GI) * 16 + m] = sum;
      }
    }
  };
  // phase p's items from item f_start on (phase 0 without the gather: its first batch went
  // out ahead of the weight stream and is put before the first call)
  auto stage = [&](int p, int f_start) {
    const int nthr = blockDim.x;
    const int total = a.M * K8;
    const int c0 = p * a.kp;                   // the phase's first input row
    for (int f0 = f_start; f0 < total; f0 += BATCH * nthr) {
      u32x4 v[BATCH];
      if (PERM && a.xraw) {                    // act-order, x resident in LDS
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
          const int f = f0 + u * nthr + threadIdx.x;
          const int i = f - row_of(f) * K8;
          const int po = f < total ? (c0 + 8 * i) * 4 : a.K * 4;   // past the end: 0
          const int4 p0 = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(prs, po, 0, 0));
          const int4 p1 = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(prs, po + 16, 0, 0));
          const int mr = row_of(f) < a.M ? row_of(f) : a.M - 1;          // items past the end: unused
          const uint16_t* xm = xr + mr * a.K;
          v[u] = u32x4{xm[p0.x] | ((uint32_t)xm[p0.y] << 16), xm[p0.z] | ((uint32_t)xm[p0.w] << 16),
                       xm[p1.x] | ((uint32_t)xm[p1.y] << 16), xm[p1.z] | ((uint32_t)xm[p1.w] << 16)};
        }
      } else if constexpr (PERM) {             // act-order: 8 channels through the index
        constexpr int HB = 1;                  // items per index batch (register budget)
#pragma unroll
        for (int u0 = 0; u0 < BATCH; u0 += HB) {
          int4 pi[HB][2];
#pragma unroll
          for (int u = 0; u < HB; ++u) {
            const int f = f0 + (u0 + u) * nthr + threadIdx.x;
            const int i = f - row_of(f) * K8;
            const int po = f < total ? (c0 + 8 * i) * 4 : a.K * 4;   // past the end: 0
            pi[u][0] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(prs, po, 0, 0));
            pi[u][1] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(prs, po + 16, 0, 0));
          }
#pragma unroll
          for (int u = 0; u < HB; ++u) {
            const int f = f0 + (u0 + u) * nthr + threadIdx.x;
            const int ro = (f < total ? row_of(f) * (int)a.ldx : xbytes) * 2;
            auto e = [&](int c) {
              return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(xrs, ro + 2 * c, 0, 0);
            };
            v[u0 + u] = u32x4{e(pi[u][0].x) | (e(pi[u][0].y) << 16), e(pi[u][0].z) | (e(pi[u][0].w) << 16),
                              e(pi[u][1].x) | (e(pi[u][1].y) << 16), e(pi[u][1].z) | (e(pi[u][1].w) << 16)};
          }
        }
      } else {
        x_batch(c0, f0, v);
      }
      put(f0, v);
    }
  };

  if (xr_items) {
    raw_store(0);
    for (int f0 = 4 * (int)blockDim.x; f0 < xr_items; f0 += 4 * (int)blockDim.x) {
      raw_load(f0);
      raw_store(f0);
    }
    __syncthreads();
  }

  // 3. MFMA over the slice's row quads as the ring delivers them.  Lane l supplies A row
  //    l%16 (x row m = l%16, the zero row when m >= M) and holds results D[4*(l/16) + r][l%16],
  //    r = 0..3; per group y[m] += s * (A[m] - c * X[m]) + d * X[m] (as qsz_decode states).
  const uint32_t kMagic = vgpr_const(0x43004300u);
  const uint32_t kLo = vgpr_const(0x000F000Fu);
  const u32x4* xrow = xa + (lj < a.M ? lj : a.M) * XS;       // rows >= M read the zero row
  float tot[4] = {0.f, 0.f, 0.f, 0.f};
  float cur_s = 0.f, cur_z = 0.f, cur_d = 0.f;
  floatx4 acc;
  // One ring turn over blocks b0 .. b0 + WIN - 1 of phase p; refills issue the blocks WIN
  // later in the wave's sequence (from a phase's last turn, the next phase's first blocks).
  auto turn = [&](const int p, const int b0, const bool refill) {
#pragma unroll
    for (int r = 0; r < WIN; ++r) {
      const int b = b0 + r;
      const u32x4 w4 = wq[r];
      float gs[MB], gz[MB], gd[MB];
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        if constexpr (kQsz) {
          qsz_decode(ms[r][m], gs[m], gz[m], gd[m]);
        } else {
          gs[m] = f16_to_f32(ms[r][m] & 0xffffu);
          gz[m] = (float)(128 + (int)((mz[r][m] >> ((col & 7) * 4)) & 0xfu) + a.zero_offset);
          gd[m] = 0.f;
        }
      }
      if (GR == 8 && (r & 1) == 0) { cur_s = gs[0]; cur_z = gz[0]; cur_d = gd[0]; }
      asm volatile("" ::: "memory");
      if (refill) issue(r, p * NB + b + WIN);
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
          if constexpr (kQsz) {
            const float dz = GR == 8 ? cur_d : gd[j / GR];
            tot[0] = fmaf(dz, X.x, tot[0]);
            tot[1] = fmaf(dz, X.y, tot[1]);
            tot[2] = fmaf(dz, X.z, tot[2]);
            tot[3] = fmaf(dz, X.w, tot[3]);
          }
        }
      }
    }
  };
  // Every phase but the last refills in every turn (its last turn issues the next phase's
  // first blocks); the last phase peels its last turn, which issues nothing, so every
  // refill is unconditional inside a turn and the load waits stay exact.
  if constexpr (!PERM) put(0, xv0);            // phase 0's first batch, loaded early
  const int f_first = PERM ? 0 : BATCH * (int)blockDim.x;
  for (int p = 0; p < nphase - 1; ++p) {
    if (p > 0) __syncthreads();                // every wave is done with the last phase's x
    stage(p, p == 0 ? f_first : 0);
    __syncthreads();
#pragma unroll
    for (int b0 = 0; b0 < NB; b0 += WIN) turn(p, b0, true);
  }
  {
    const int p = nphase - 1;
    if (p > 0) __syncthreads();
    stage(p, p == 0 ? f_first : 0);
    __syncthreads();
#pragma unroll
    for (int b0 = 0; b0 < NB - WIN; b0 += WIN) turn(p, b0, true);
    turn(p, NB - WIN, false);
  }

  // 4. Per-slice results meet in LDS and are added in slice order (bitwise repeatable).
  //    ytile lies past the x tile and its sums, so no wave still reading x is disturbed.
#pragma unroll
  for (int e = 0; e < 4; ++e) ytile[(wave * 16 + 4 * lg + e) * 16 + lj] = tot[e];
  __syncthreads();
  const int kw = nw / CT;
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
// (x takes up to 140 KB of LDS), then the most waves (up to 16) that split a phase's kb
// blocks evenly with NB blocks of 2, 4, 8 or 16 per wave.
struct RowsGeom {
  int ct, nb, kw;
};

static RowsGeom rows_geometry(int64_t kb, int64_t N, int cus) {
  const int64_t strips = N / kStripCols;
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

static size_t rows_lds(int64_t M, int64_t kp, int group, const RowsGeom& g) {
  return (size_t)(M + 1) * (kp / 8 + 1) * 16 + (size_t)16 * (kp / group) * 4 +
         (size_t)g.ct * g.kw * 256 * 4;
}

// The phase length: the largest multiple of 256 dividing K whose x tile of 16 rows, group
// sums and slice tiles fit the LDS with a launch geometry; 0 if none does.  It does not
// depend on M, so a row's result does not depend on the rows batched with it (the same
// phases, slices and summation order at every M).
static int64_t rows_phase(int64_t K, int64_t N, int group, int cus, RowsGeom& geom) {
  for (int64_t parts = 1; parts <= K / 256; ++parts) {
    if (K % parts || (K / parts) % 256) continue;
    const int64_t kp = K / parts;
    const RowsGeom g = rows_geometry(kp / 128, N, cus);
    if (g.ct && g.nb && rows_lds(kRowsMax, kp, group, g) <= kRowsMaxLds) {
      geom = g;
      return kp;
    }
  }
  return 0;
}

// Dynamic LDS above 64 KB is granted per kernel (once per instantiation, before its first
// launch; not a stream operation, so it is safe during graph capture).
template <typename Kern>
static void rows_launch(Kern kern, dim3 grid, dim3 block, size_t lds, hipStream_t st,
                        const RowsArgs& a, bool& opted) {
  if (!opted) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kRowsMaxLds);
    opted = true;
  }
  hipLaunchKernelGGL(kern, grid, block, lds, st, a);
}

template <int GR, int FMT, bool PERM>
static void rows_nb(const RowsArgs& a, const RowsGeom& g, size_t lds, hipStream_t st) {
  const dim3 grid(a.N / (kStripCols * g.ct)), block(64 * g.ct * g.kw);
  static bool opted[4] = {false, false, false, false};
  switch (g.nb) {
    case 2: rows_launch(w4_rows_kernel<GR, 2, FMT, PERM>, grid, block, lds, st, a, opted[0]); break;
    case 4: rows_launch(w4_rows_kernel<GR, 4, FMT, PERM>, grid, block, lds, st, a, opted[1]); break;
    case 8: rows_launch(w4_rows_kernel<GR, 8, FMT, PERM>, grid, block, lds, st, a, opted[2]); break;
    default: rows_launch(w4_rows_kernel<GR, 16, FMT, PERM>, grid, block, lds, st, a, opted[3]); break;
  }
}

// act-order inputs (GPTQ metadata only) run the PERM variants, whose staging gathers x
template <int FMT, bool PERM>
static void rows_group(const RowsArgs& a, const RowsGeom& g, size_t lds, hipStream_t st) {
  switch (a.group) {
    case 32: rows_nb<1, FMT, PERM>(a, g, lds, st); break;
    case 64: rows_nb<2, FMT, PERM>(a, g, lds, st); break;
    case 128: rows_nb<4, FMT, PERM>(a, g, lds, st); break;
    default: rows_nb<8, FMT, PERM>(a, g, lds, st); break;
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

// Shared by the entry points (and mtl_int4pack_mm): shapes and alignment, then the launch.
int strip_rows(const void* x, int64_t M, int64_t ldx, int64_t K, const int32_t* perm,
               const int32_t* strip_weight, const void* meta, const int32_t* qzeros, int64_t N,
               int32_t group_size, int32_t zero_offset, int fmt, void* y, int64_t ldy,
               int32_t out_dtype, void* stream) {
  if (!x || !strip_weight || !meta || (fmt == STRIP_META_GPTQ && !qzeros) || !y)
    return MTL_ERR_INVALID_ARG;
  if (out_dtype != MTL_OUT_BF16 && out_dtype != MTL_OUT_F32) return MTL_ERR_INVALID_ARG;
  if (group_size != 32 && group_size != 64 && group_size != 128 && group_size != 256)
    return MTL_ERR_GROUP;
  if (M < 1 || M > kRowsMax || K <= 0 || N <= 0 || K % 256 != 0 || N % kStripCols != 0 ||
      K % group_size != 0 || ldx < K || ldy < N || N * K / 2 >= ((int64_t)1 << 31) ||
      (ldx * (M - 1) + K) * 2 >= ((int64_t)1 << 31) || ldy * (M - 1) + N >= ((int64_t)1 << 31))
    return MTL_ERR_SHAPE;
  if (!aligned16(x) || ldx % 8 != 0 || !aligned16(strip_weight) || (perm && !aligned16(perm)) ||
      (reinterpret_cast<uintptr_t>(meta) & (fmt == STRIP_META_QSZ ? 3u : 1u)) ||
      (reinterpret_cast<uintptr_t>(qzeros) & 3u) ||
      (reinterpret_cast<uintptr_t>(y) & (out_dtype == MTL_OUT_F32 ? 3u : 1u)))
    return MTL_ERR_ALIGN;
  RowsGeom g;
  const int64_t kp = rows_phase(K, N, group_size, device_cus(), g);
  if (!kp) return MTL_ERR_SHAPE;
  RowsArgs a;
  a.w = reinterpret_cast<const u32x4*>(strip_weight);
  a.scales = static_cast<const uint16_t*>(meta);
  a.qzeros = reinterpret_cast<const uint32_t*>(qzeros);
  a.x = static_cast<const uint16_t*>(x);
  a.perm = perm;
  a.y = y;
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = (int)M; a.K = (int)K; a.N = (int)N;
  a.group = group_size;
  a.zero_offset = zero_offset;
  a.out_f32 = out_dtype == MTL_OUT_F32;
  a.kblocks = (int)(K / 128);
  a.kp = (int)kp;
  a.ct = g.ct;
  const int64_t G = N / (kStripCols * g.ct);
  a.xcd_order = G % 8 == 0;
  size_t lds = rows_lds(M, kp, group_size, g);
  // act-order: x's rows resident in LDS when they fit beside the tile (M * K bf16)
  a.xraw = perm && lds + (size_t)M * K * 2 <= kRowsMaxLds;
  if (a.xraw) lds += (size_t)M * K * 2;
  hipStream_t st = (hipStream_t)stream;
  if (fmt == STRIP_META_QSZ) rows_group<STRIP_META_QSZ, false>(a, g, lds, st);
  else if (perm) rows_group<STRIP_META_GPTQ, true>(a, g, lds, st);
  else rows_group<STRIP_META_GPTQ, false>(a, g, lds, st);
  return launch_status();
}

}  // namespace mtl

using namespace mtl;

extern "C" {

int mtl_w4_gemm_strip_rows(const void* x, int64_t M, int64_t ldx, int64_t K,
                           const int32_t* strip_weight, const void* scales,
                           const int32_t* qzeros, int64_t N, int32_t group_size,
                           int32_t zero_offset, void* y, int64_t ldy, int32_t out_dtype,
                           void* stream) {
  return strip_rows(x, M, ldx, K, nullptr, strip_weight, scales, qzeros, N, group_size,
                    zero_offset, STRIP_META_GPTQ, y, ldy, out_dtype, stream);
}

int mtl_w4_gemm_strip_rows_ex(const void* x, int64_t M, int64_t ldx, int64_t K,
                              const int32_t* perm, const int32_t* strip_weight, const void* meta,
                              const int32_t* qzeros, int64_t N, int32_t group_size,
                              int32_t zero_offset, int32_t meta_format, void* y, int64_t ldy,
                              int32_t out_dtype, void* stream) {
  if (meta_format != MTL_META_GPTQ && meta_format != MTL_META_QSZ) return MTL_ERR_INVALID_ARG;
  if (meta_format == MTL_META_QSZ && (perm || zero_offset)) return MTL_ERR_INVALID_ARG;
  return strip_rows(x, M, ldx, K, perm, strip_weight, meta, qzeros, N, group_size, zero_offset,
                    meta_format == MTL_META_QSZ ? STRIP_META_QSZ : STRIP_META_GPTQ, y, ldy,
                    out_dtype, stream);
}

}  // extern "C"
