// int4 GEMM over full-K column strips at prompt length for gfx950: y[M, N] = x[M, K] @ W
// for any M (the prefill's projections, moss_tts_lite/fast.py:218-270, where every linear
// runs at M = prompt length).
//
// Weights are the strip layout of the decode GEMV (mtl_w4strip.hip): 1 KB block
// (s * K/128 + b) holds columns 16s..16s+15 over input channels 128b..128b+127, lane l's
// 16 bytes being the B operands (codes as bf16 128 + q) of four v_mfma_f32_16x16x32_bf16
// over the block's four 32-channel chunks.  Group metadata is in the strip order of
// mtl_w4_strip_meta.  Per quantisation group the MFMA sums A = sum x * (128 + q) exactly in
// fp32 and the group adds s * (A - (128 + z) * X) with X the group's sum of x, as in the
// decode GEMV; on the reference's qsz records, s * A + (d - 136 s) * X, two FMAs per output
// with d - 136 s formed once per group and column (g = 32 folds every 32 channels).
//
// A workgroup (4 waves) owns a tile of 64 x rows by 8 strips (128 columns); wave w serves
// strips 2w and 2w+1 for all 64 rows (4 MFMA row tiles), so one unpacked B operand feeds 4
// MFMAs and one A operand read from LDS feeds 2.  The K loop walks 128-channel blocks:
// the x tile of block b + 1 (64 rows x 128 channels, in the pair order the code unpack
// produces, with its per-group sums) is loaded while block b is multiplied and goes to
// the other of two LDS buffers, one barrier per block; each wave keeps D blocks of its
// two strips' weights and metadata in flight in a register ring.  The grid is (N / 128)
// x (M / 64): with N / 128 a multiple of 8, the row tiles of one column tile run on one
// XCD, so its weights are fetched into one L2.
#include "mtl_w4core.h"

namespace mtl {

constexpr int kPfRows = 64;                      // x rows per workgroup
constexpr int kPfWaves = 4;
constexpr int kPfStrips = 2 * kPfWaves;          // 128 columns per workgroup
constexpr int kPfCols = 16 * kPfStrips;
constexpr int kPfPitch = 17;                     // LDS items per x row: 16 + 1 (banks)
constexpr int kPfWavesPerEU = 3;                 // 168 VGPRs: 3 workgroups per CU
constexpr int kPfRing = 2;                       // weight blocks in flight per wave
constexpr int kPfMaxSplits = 8;
constexpr int kEpiPartials = -1;                 // host-side mode of prefill_gemm

struct PrefillArgs {
  const uint16_t* x;          // bf16 [M, K], rows ldx apart, in the weight's input order
  const u32x4* w;             // strip layout
  const uint16_t* scales;     // strip-ordered fp16 scales, or the reference's qsz pairs
  const uint32_t* qzeros;     // strip-ordered zero nibbles (GPTQ metadata)
  void* y;                    // see the epilogues
  float* part;                // splits > 1: fp32 partial sums [splits][M][N]
  const float* xsum;          // staged x: fp32 sums per 32 channels [M][K/32], rows ldsum apart
  int64_t ldx, ldy, ldsum;
  int M, K, N, group, zero_offset, kblocks, out_f32;
  int splits, kps;            // K splits (blockIdx.z) of kps blocks each
};

// Sums over aligned groups of 4, 8 or 16 lanes: group_sum_valu (mtl_common.h).

// PRE: x arrives staged by its producer (mtl_rmsnorm_gather_staged and the residual form):
// each 8-channel item already in pair order, with fp32 sums per 32 channels, so the staging
// copies items into LDS and forms the group sums from the 32-channel sums: (S0 + S1) +
// (S2 + S3) is the order of group_sum_valu's butterfly, so the sums are the bits the
// in-kernel staging computes.
template <int GR, int EPI, int FMT, bool PRE = false>
__global__ void __launch_bounds__(64 * kPfWaves) __attribute__((amdgpu_waves_per_eu(kPfWavesPerEU)))
w4_prefill_kernel(PrefillArgs a) {
  constexpr int MB = GR <= 4 ? 4 / GR : 1;       // groups starting in one block
  constexpr int GI = GR <= 4 ? 4 * GR : 16;      // x items per staged sum
  constexpr int D = kPfRing;
  static_assert(D % 2 == 0, "ring turns hold whole block pairs (g = 256)");
  __shared__ u32x4 xa[2][kPfRows * kPfPitch];    // x tile: [row][item] in pair order
  __shared__ float xs[2][MB][kPfRows];           // its group sums (g = 256: block sums)

  const int t = threadIdx.x, lane = t & 63, wave = wave_id();
  const int lg = lane >> 4, lj = lane & 15;
  const int row0 = blockIdx.y * kPfRows;
  const int kb = a.kblocks;
  const int kb0 = blockIdx.z * a.kps, kb1 = kb0 + a.kps;   // this split's blocks (kps even)
  const int N = a.N;
  const int sA = blockIdx.x * kPfStrips + 2 * wave;   // this wave's strips sA, sA + 1

  // x staging: thread t stages items t + 256 r (r = 0..3) of the tile: row (t >> 4) + 16 r,
  // item t & 15 (channels 8 (t & 15) .. +7 of the block), through a bounds-checked buffer
  // resource over the M rows, so rows at or past M stage zeros.
  const int srow = t >> 4, sitem = t & 15;
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x + (size_t)row0 * a.ldx), (short)0,
      (int)(((int64_t)(a.M - row0) - 1) * a.ldx * 2 + (int64_t)a.K * 2), 0x00020000);
  const int xoff = (int)(srow * a.ldx * 2) + 16 * sitem;
  const int xrstep = (int)(16 * a.ldx * 2);      // 16 rows, a uniform offset
  u32x4 xv[4];
  // PRE: the four 32-channel sums of the block for each of the thread's rows (every thread
  // of a row loads them; the row's item-0 thread writes the group sums)
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(PRE ? a.xsum + (size_t)row0 * a.ldsum : nullptr), (short)0,
      PRE ? (int)((((int64_t)(a.M - row0) - 1) * a.ldsum + (a.K >> 5)) * 4) : 0, 0x00020000);
  const int soff = PRE ? (int)(srow * a.ldsum * 4) : 0;
  const int srstep = PRE ? (int)(16 * a.ldsum * 4) : 0;
  float4 sv[PRE ? 4 : 1];
  auto x_load = [&](int b) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      xv[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                            xrsrc, xoff, r * xrstep + b * 256, 0));
    if constexpr (PRE) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sv[r] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                               srs, soff, r * srstep + b * 16, 0));
    }
  };
  auto x_store_part = [&](int buf, int r) {     // item set r: rows srow + 16 r
    if constexpr (PRE) {
      xa[buf][(srow + 16 * r) * kPfPitch + sitem] = xv[r];
      if (sitem == 0) {
        const float4 q = sv[r];
        const int row = srow + 16 * r;
        if (GR == 1) {
          xs[buf][0][row] = q.x; xs[buf][MB > 1 ? 1 : 0][row] = q.y;
          xs[buf][MB > 2 ? 2 : 0][row] = q.z; xs[buf][MB > 3 ? 3 : 0][row] = q.w;
        } else if (GR == 2) {
          xs[buf][0][row] = q.x + q.y; xs[buf][MB > 1 ? 1 : 0][row] = q.z + q.w;
        } else {
          xs[buf][0][row] = (q.x + q.y) + (q.z + q.w);
        }
      }
    } else {
      float sum;
      const u32x4 pv = pair_order_dot(xv[r], sum);
      sum = group_sum_valu<GI>(sum);
      xa[buf][(srow + 16 * r) * kPfPitch + sitem] = pv;
      if ((sitem & (GI - 1)) == 0) xs[buf][sitem / GI][srow + 16 * r] = sum;
    }
  };
  auto x_store = [&](int buf) {
#pragma unroll
    for (int r = 0; r < 4; ++r) x_store_part(buf, r);
  };

  // Weight ring: block b of both strips and the metadata records it starts go to slot
  // b % D; a slot is refilled as soon as its block is unpacked.
  const int ngroups = a.K / a.group;
  const int krec = GR == 8 ? kb >> 1 : kb;       // metadata records per strip
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4*>(a.w), (short)0, (int)((int64_t)(N / 16) * kb * 1024), 0x00020000);
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.scales), (short)0,
      FMT == STRIP_META_QSZ ? ngroups * N * 4 : ngroups * N * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t zrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(a.qzeros), (short)0,
      FMT == STRIP_META_QSZ ? 0 : ngroups * (N >> 1), 0x00020000);
  u32x4 wq[D][2];
  StripMeta<MB> mt[FMT == STRIP_META_GPTQ ? D : 1][2];
  uint32_t mq[FMT == STRIP_META_QSZ ? D : 1][2][MB];   // the reference's (scale, zero) pairs
  auto issue = [&](int r, int b) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int strip = sA + s;
      if (GR <= 4 || (r & 1) == 0) {
        if constexpr (FMT == STRIP_META_GPTQ) {
          strip_meta_load<MB>(srsrc, zrsrc, lj, strip * krec + (GR == 8 ? b >> 1 : b), mt[r][s]);
        } else {
#pragma unroll
          for (int m = 0; m < MB; ++m)
            mq[r][s][m] = qsz_load(srsrc, 16 * strip + lj, GR == 8 ? b >> 1 : b * MB + m, N);
        }
      }
      wq[r][s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                               wrsrc, lane * 16, (strip * kb + b) * 1024, 0));
    }
  };
#pragma unroll
  for (int r = 0; r < D; ++r) issue(r, kb0 + r);
  x_load(kb0);
  x_store(0);
  x_load(kb0 + 1);
  __syncthreads();

  const uint32_t kMagic = vgpr_const(0x43004300u);   // bf16 (128, 128)
  const uint32_t kLo = vgpr_const(0x000F000Fu);
  const floatx4 zero4{0.f, 0.f, 0.f, 0.f};
  floatx4 tot[4][2];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) { tot[tt][0] = zero4; tot[tt][1] = zero4; }
  // Chunks per correction: a group (g <= 128), or a block at g = 256, whose group's two
  // blocks are folded one after the other with the pair's scale and zero.
  constexpr int GC = GR <= 4 ? GR : 4;
  float gs[2][MB], gz[2][MB], gd[2][MB];

  for (int b0 = kb0; b0 < kb1; b0 += D) {
#pragma unroll
    for (int r = 0; r < D; ++r) {
      const int b = b0 + r;
      const int buf = r & 1;                     // b0 - kb0 and kb0 are even
      if (GR <= 4 || (r & 1) == 0) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          if constexpr (FMT == STRIP_META_GPTQ) {
            strip_meta_decode<MB>(mt[r][s], lj, a.zero_offset, gs[s], gz[s]);
          } else {
#pragma unroll
            for (int m = 0; m < MB; ++m) {
              qsz_decode(mq[r][s][m], gs[s][m], gz[s][m], gd[s][m]);
              gd[s][m] = fmaf(-gs[s][m], gz[s][m], gd[s][m]);   // d - s * c
            }
          }
        }
      }
      bf16x8_t B[2][4];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4 w = wq[r][s];
        B[s][0] = unpack_codes8(w.x, kLo, kMagic);
        B[s][1] = unpack_codes8(w.y, kLo, kMagic);
        B[s][2] = unpack_codes8(w.z, kLo, kMagic);
        B[s][3] = unpack_codes8(w.w, kLo, kMagic);
      }
      // keep the refill below the unpack (IR and machine scheduling)
      asm volatile("" ::: "memory");
      issue(r, b + D < kb1 ? b + D : kb1 - 1);   // unconditional refill (clamped)
      __builtin_amdgcn_sched_barrier(0);
      if (GR >= 4) {
        // One group per block (or a block of a g = 256 pair): the row tiles run as a
        // pipeline.  The MFMAs of tile tt are issued before the group correction of tile
        // tt - 1 and a quarter of the next block's staging, so that VALU work overlaps the
        // MFMAs in flight; two accumulator pairs are live.
        floatx4 acc[2][2];
        auto mm = [&](int tt) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bf16x8_t A =
                __builtin_bit_cast(bf16x8_t, xa[buf][(16 * tt + lj) * kPfPitch + 4 * j + lg]);
            acc[tt & 1][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B[0][j], j == 0 ? zero4 : acc[tt & 1][0], 0, 0, 0);
            acc[tt & 1][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B[1][j], j == 0 ? zero4 : acc[tt & 1][1], 0, 0, 0);
          }
        };
        auto fold = [&](int tt) {
          const float4 X4 = *reinterpret_cast<const float4*>(&xs[buf][0][16 * tt + 4 * lg]);
          const float X[4] = {X4.x, X4.y, X4.z, X4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (FMT == STRIP_META_QSZ) {   // s * acc + (d - s * c) * X: two FMAs
              tot[tt][0][i] = fmaf(gd[0][0], X[i], fmaf(gs[0][0], acc[tt & 1][0][i], tot[tt][0][i]));
              tot[tt][1][i] = fmaf(gd[1][0], X[i], fmaf(gs[1][0], acc[tt & 1][1][i], tot[tt][1][i]));
            } else {
              tot[tt][0][i] = fmaf(gs[0][0], fmaf(-gz[0][0], X[i], acc[tt & 1][0][i]), tot[tt][0][i]);
              tot[tt][1][i] = fmaf(gs[1][0], fmaf(-gz[1][0], X[i], acc[tt & 1][1][i]), tot[tt][1][i]);
            }
          }
          x_store_part(buf ^ 1, tt);             // block b + 1, loaded during block b - 1
          asm volatile("" ::"v"(tot[tt][0]), "v"(tot[tt][1]) : "memory");
        };
        mm(0);
#pragma unroll
        for (int tt = 1; tt < 4; ++tt) {
          mm(tt);
          fold(tt - 1);
        }
        fold(3);
        __builtin_amdgcn_sched_barrier(0);
        x_load(b + 2 < kb1 ? b + 2 : kb1 - 1);
        __syncthreads();
        continue;
      }
      // Row tile by row tile, so one accumulator pair is live at a time.
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        floatx4 acc0, acc1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int q = j % GC;
          const bf16x8_t A =
              __builtin_bit_cast(bf16x8_t, xa[buf][(16 * tt + lj) * kPfPitch + 4 * j + lg]);
          acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B[0][j], q == 0 ? zero4 : acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B[1][j], q == 0 ? zero4 : acc1, 0, 0, 0);
          if (q == GC - 1) {                     // fold the group into tot
            const int m = GR <= 4 ? j / GR : 0;
            const float4 X4 = *reinterpret_cast<const float4*>(&xs[buf][m][16 * tt + 4 * lg]);
            const float X[4] = {X4.x, X4.y, X4.z, X4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if constexpr (FMT == STRIP_META_QSZ) { // s * acc + (d - s * c) * X: two FMAs
                tot[tt][0][i] = fmaf(gd[0][m], X[i], fmaf(gs[0][m], acc0[i], tot[tt][0][i]));
                tot[tt][1][i] = fmaf(gd[1][m], X[i], fmaf(gs[1][m], acc1[i], tot[tt][1][i]));
              } else {
                tot[tt][0][i] = fmaf(gs[0][m], fmaf(-gz[0][m], X[i], acc0[i]), tot[tt][0][i]);
                tot[tt][1][i] = fmaf(gs[1][m], fmaf(-gz[1][m], X[i], acc1[i]), tot[tt][1][i]);
              }
            }
          }
        }
        // pin the tile's corrections here: the next tile's LDS reads (and so its MFMAs)
        // cannot move above a volatile asm that reads tot and clobbers memory
        asm volatile("" ::"v"(tot[tt][0]), "v"(tot[tt][1]) : "memory");
      }
      // block b + 1 (loaded during block b - 1) into the other buffer, then block b + 2
      // into registers (the last blocks reload the last block, unused)
      __builtin_amdgcn_sched_barrier(0);
      x_store(buf ^ 1);
      x_load(b + 2 < kb1 ? b + 2 : kb1 - 1);
      __syncthreads();
    }
  }

  // Epilogue: tot[tt][s][i] is row row0 + 16 tt + 4 lg + i, column 16 (sA + s) + lj.
  if (a.splits > 1) {                            // partial sums; prefill_reduce_kernel finishes
    float* pz = a.part + (size_t)blockIdx.z * a.M * N;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + 16 * tt + 4 * lg + i;
          if (row < a.M) pz[(size_t)row * N + 16 * (sA + s) + lj] = tot[tt][s][i];
        }
    return;
  }
  if (EPI == MTL_EPI_SILU_MUL) {
    // Strips 8c .. 8c+7 are two 64-column gate|up blocks (32 gate | 32 up columns each):
    // waves 0 and 2 hold gate strips, waves 1 and 3 their up partners.  The up values
    // meet the gate values in LDS (the x buffers, free after the last barrier).
    float* ut = reinterpret_cast<float*>(&xa[0][0]);    // [2][2][4][4][64]
    const int pair = wave >> 1;
    if (wave & 1) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i) ut[(((pair * 2 + s) * 4 + tt) * 4 + i) * 64 + lane] = tot[tt][s][i];
    }
    __syncthreads();
    if (wave & 1) return;
    uint16_t* act = static_cast<uint16_t*>(a.y);
    const int jb = 2 * blockIdx.x + pair;                // 32-column SwiGLU output block
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + 16 * tt + 4 * lg + i;
          const float u = ut[(((pair * 2 + s) * 4 + tt) * 4 + i) * 64 + lane];
          if (row < a.M)
            act[(size_t)row * a.ldy + 32 * jb + 16 * s + lj] = (uint16_t)silu_mul_bf16(tot[tt][s][i], u);
        }
    return;
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int col = 16 * (sA + s) + lj;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = row0 + 16 * tt + 4 * lg + i;
        if (row >= a.M) continue;
        const size_t o = (size_t)row * a.ldy + col;
        const float v = tot[tt][s][i];
        if (EPI == MTL_EPI_RESIDUAL) {
          uint16_t* h = static_cast<uint16_t*>(a.y);
          // h = bf16(bf16(acc) + h) (fast.py:168-171 on prompt rows)
          h[o] = (uint16_t)f32_to_bf16(round_bf16(v) + bf16_to_f32(h[o]));
        } else if (a.out_f32) {
          static_cast<float*>(a.y)[o] = v;
        } else {
          static_cast<uint16_t*>(a.y)[o] = (uint16_t)f32_to_bf16(v);
        }
      }
  }
}

// Sums the K-split partials in split order and applies the epilogue; thread t handles 4
// consecutive output columns of one row (SiLU*up: 4 SwiGLU columns, from their gate and up
// partials 32 columns apart).
template <int EPI>
__global__ void __launch_bounds__(256) prefill_reduce_kernel(PrefillArgs a) {
  const int N = a.N;
  const int ncols = EPI == MTL_EPI_SILU_MUL ? N / 2 : N;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = idx / (ncols / 4);
  if (row >= a.M) return;
  const int c = (int)(idx % (ncols / 4)) * 4;      // first output column
  const size_t plane = (size_t)a.M * N;
  const float* base = a.part + (size_t)row * N;
  if (EPI == MTL_EPI_SILU_MUL) {
    const int g = 64 * (c >> 5) + (c & 31);          // gate column; up is 32 to the right
    float4 gs = *reinterpret_cast<const float4*>(base + g);
    float4 us = *reinterpret_cast<const float4*>(base + g + 32);
    for (int z = 1; z < a.splits; ++z) {
      const float4 gv = *reinterpret_cast<const float4*>(base + z * plane + g);
      const float4 uv = *reinterpret_cast<const float4*>(base + z * plane + g + 32);
      gs.x += gv.x; gs.y += gv.y; gs.z += gv.z; gs.w += gv.w;
      us.x += uv.x; us.y += uv.y; us.z += uv.z; us.w += uv.w;
    }
    uint16_t* act = static_cast<uint16_t*>(a.y) + (size_t)row * a.ldy + c;
    act[0] = (uint16_t)silu_mul_bf16(gs.x, us.x);
    act[1] = (uint16_t)silu_mul_bf16(gs.y, us.y);
    act[2] = (uint16_t)silu_mul_bf16(gs.z, us.z);
    act[3] = (uint16_t)silu_mul_bf16(gs.w, us.w);
    return;
  }
  float4 v = *reinterpret_cast<const float4*>(base + c);
  for (int z = 1; z < a.splits; ++z) {
    const float4 p = *reinterpret_cast<const float4*>(base + z * plane + c);
    v.x += p.x; v.y += p.y; v.z += p.z; v.w += p.w;
  }
  const float y[4] = {v.x, v.y, v.z, v.w};
  const size_t o = (size_t)row * a.ldy + c;
  for (int e = 0; e < 4; ++e) {
    if (EPI == MTL_EPI_RESIDUAL) {
      uint16_t* h = static_cast<uint16_t*>(a.y);
      h[o + e] = (uint16_t)f32_to_bf16(round_bf16(y[e]) + bf16_to_f32(h[o + e]));
    } else if (a.out_f32) {
      static_cast<float*>(a.y)[o + e] = y[e];
    } else {
      static_cast<uint16_t*>(a.y)[o + e] = (uint16_t)f32_to_bf16(y[e]);
    }
  }
}

// K splits for a launch of `tiles` workgroups over kb blocks: enough splits for about three
// workgroups per CU (the 3 that fit), each split a whole number of ring turns (kPfRing
// blocks), at most kPfMaxSplits.  At 256 prompt rows this gives q|k|v 4 splits and down 6
// (2 and 4 for two workgroups per CU: the prompt 7.71 -> 7.67 ms, min 7.65 -> 7.55, same
// box; one per CU 7.75 against 7.30; four, which splits gate|up too, 8.29).
static int prefill_splits(int64_t tiles, int64_t kb, int cus) {
  int s = 1;
  while (s < kPfMaxSplits && tiles * s < 3 * cus) ++s;
  while (s > 1 && kb % ((int64_t)s * kPfRing) != 0) --s;
  return s;
}

static int g_pf_cus = 0;

static int pf_device_cus() {
  if (!g_pf_cus) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_pf_cus = n;
  }
  return g_pf_cus;
}

template <int GR, int EPI, int FMT, bool PRE = false>
static void prefill_launch(const PrefillArgs& a, hipStream_t st, bool reduce = true) {
  const dim3 grid(a.N / kPfCols, (a.M + kPfRows - 1) / kPfRows, a.splits), block(64 * kPfWaves);
  hipLaunchKernelGGL((w4_prefill_kernel<GR, EPI, FMT, PRE>), grid, block, 0, st, a);
  if (a.splits > 1 && reduce) {
    const int64_t ncols = EPI == MTL_EPI_SILU_MUL ? a.N / 2 : a.N;
    const int64_t threads = (int64_t)a.M * (ncols / 4);
    hipLaunchKernelGGL(prefill_reduce_kernel<EPI>, dim3((unsigned)((threads + 255) / 256)),
                       dim3(256), 0, st, a);
  }
}

// Staged x (a.xsum) comes with the plain and SiLU*up epilogues only.
template <int GR, int FMT>
static void prefill_epi(const PrefillArgs& a, int epilogue, hipStream_t st) {
  if (a.xsum) {
    if (epilogue == MTL_EPI_SILU_MUL) prefill_launch<GR, MTL_EPI_SILU_MUL, FMT, true>(a, st);
    else prefill_launch<GR, MTL_EPI_NONE, FMT, true>(a, st);
    return;
  }
  if (epilogue == MTL_EPI_RESIDUAL) prefill_launch<GR, MTL_EPI_RESIDUAL, FMT>(a, st);
  else if (epilogue == MTL_EPI_SILU_MUL) prefill_launch<GR, MTL_EPI_SILU_MUL, FMT>(a, st);
  else prefill_launch<GR, MTL_EPI_NONE, FMT>(a, st);
}

template <int GR, int FMT>
static void prefill_partials_launch(const PrefillArgs& a, hipStream_t st) {
  if (a.xsum) prefill_launch<GR, MTL_EPI_NONE, FMT, true>(a, st, false);
  else prefill_launch<GR, MTL_EPI_NONE, FMT>(a, st, false);
}

// The K-split partial sums only (no reduce launch): fp32 [splits][M][N] in a.part, or with
// one split the fp32 sums written there as y.
template <int FMT>
static void prefill_group_partials(const PrefillArgs& a, hipStream_t st) {
  switch (a.group) {
    case 32: prefill_partials_launch<1, FMT>(a, st); break;
    case 64: prefill_partials_launch<2, FMT>(a, st); break;
    case 128: prefill_partials_launch<4, FMT>(a, st); break;
    default: prefill_partials_launch<8, FMT>(a, st); break;
  }
}

template <int FMT>
static void prefill_group(const PrefillArgs& a, int epilogue, hipStream_t st) {
  switch (a.group) {
    case 32: prefill_epi<1, FMT>(a, epilogue, st); break;
    case 64: prefill_epi<2, FMT>(a, epilogue, st); break;
    case 128: prefill_epi<4, FMT>(a, epilogue, st); break;
    default: prefill_epi<8, FMT>(a, epilogue, st); break;
  }
}

// Both metadata contracts (fmt: STRIP_META_*); with STRIP_META_QSZ, scales is the
// reference's qsz bf16 [K/g, N, 2] and zeros is unused.
static int prefill_gemm(const void* x, int64_t M, int64_t ldx, int64_t K,
                        const int32_t* strip_weight, const void* scales, const int32_t* zeros,
                        int64_t N, int32_t group_size, int32_t zero_offset, int32_t epilogue,
                        int32_t out_dtype, void* y, int64_t ldy, float* workspace,
                        int64_t ws_bytes, int fmt, hipStream_t st,
                        const float* xsum = nullptr);

static int prefill_gemm(const void* x, int64_t M, int64_t ldx, int64_t K,
                             const int32_t* strip_weight, const void* scales,
                             const int32_t* zeros, int64_t N, int32_t group_size,
                             int32_t zero_offset, int32_t epilogue, int32_t out_dtype, void* y,
                             int64_t ldy, float* workspace, int64_t ws_bytes, int fmt,
                             hipStream_t st, const float* xsum) {
  if (!x || !strip_weight || !scales || (!y && epilogue != kEpiPartials))
    return MTL_ERR_INVALID_ARG;
  // staged x: the plain, SiLU*up and partials epilogues; its 32-channel sums 16-byte rows
  if (xsum && epilogue == MTL_EPI_RESIDUAL) return MTL_ERR_INVALID_ARG;
  if (xsum && (!aligned16(xsum) || M * (K / 32) * 4 >= ((int64_t)1 << 31))) {
    if (!aligned16(xsum)) return MTL_ERR_ALIGN;
    return MTL_ERR_SHAPE;
  }
  if (epilogue != MTL_EPI_NONE && epilogue != MTL_EPI_RESIDUAL && epilogue != MTL_EPI_SILU_MUL &&
      epilogue != kEpiPartials)
    return MTL_ERR_INVALID_ARG;
  if (epilogue == kEpiPartials) {   // y unused: its checks read the partials' pitch
    out_dtype = MTL_OUT_F32;
    y = workspace;
    ldy = N;
  }
  if (out_dtype != MTL_OUT_BF16 && out_dtype != MTL_OUT_F32) return MTL_ERR_INVALID_ARG;
  if (epilogue != MTL_EPI_NONE && epilogue != kEpiPartials && out_dtype != MTL_OUT_BF16)
    return MTL_ERR_INVALID_ARG;
  if (group_size != 32 && group_size != 64 && group_size != 128 && group_size != 256)
    return MTL_ERR_GROUP;
  const int64_t ncols = epilogue == MTL_EPI_SILU_MUL ? N / 2 : N;
  const int64_t meta_bytes = fmt == STRIP_META_QSZ ? 4 : 2;
  if (M < 1 || M > (int64_t)kPfRows * 65535 || K <= 0 || N <= 0 || K % 256 != 0 ||
      K > 65536 || N % kPfCols != 0 || K % group_size != 0 || ldx < K || ldy < ncols ||
      (N / 16) * (K / 128) * 1024 >= ((int64_t)1 << 31) || M * ldx * 2 >= ((int64_t)1 << 31) ||
      (K / group_size) * N * meta_bytes >= ((int64_t)1 << 31))
    return MTL_ERR_SHAPE;
  const bool meta_ok = fmt == STRIP_META_QSZ ? (reinterpret_cast<uintptr_t>(scales) & 3u) == 0
                                             : aligned16(scales);
  if (!aligned16(x) || ldx % 8 != 0 || !aligned16(strip_weight) || !meta_ok ||
      (workspace && !aligned16(workspace)) ||
      (reinterpret_cast<uintptr_t>(y) & (out_dtype == MTL_OUT_F32 ? 3u : 1u)))
    return MTL_ERR_ALIGN;
  PrefillArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.w = reinterpret_cast<const u32x4*>(strip_weight);
  a.scales = static_cast<const uint16_t*>(scales);
  a.qzeros = reinterpret_cast<const uint32_t*>(zeros);
  a.y = y;
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = (int)M; a.K = (int)K; a.N = (int)N;
  a.group = group_size;
  a.zero_offset = zero_offset;
  a.kblocks = (int)(K / 128);
  a.out_f32 = out_dtype == MTL_OUT_F32;
  // K splits when the workspace holds their partial sums, else one pass
  const int64_t need = mtl_w4_gemm_prefill_workspace_bytes(M, K, N);
  a.splits = need > 0 && workspace && ws_bytes >= need ? (int)(need / (M * N * 4)) : 1;
  a.kps = a.kblocks / a.splits;
  a.part = workspace;
  a.xsum = xsum;
  a.ldsum = K / 32;
  if (epilogue == kEpiPartials) {
    // the caller sums the splits (mtl_residual_rmsnorm_gather): as many splits as the
    // shape takes, into `workspace`; with one split the sums go there as fp32 y
    const int s = prefill_splits((N / kPfCols) * ((M + kPfRows - 1) / kPfRows), K / 128,
                                 pf_device_cus());
    if (!workspace || ws_bytes < (int64_t)s * M * N * 4) return MTL_ERR_WORKSPACE;
    a.splits = s;
    a.kps = a.kblocks / s;
    if (s == 1) {
      a.y = workspace;
      a.ldy = N;
      a.out_f32 = 1;
    }
    if (fmt == STRIP_META_QSZ) prefill_group_partials<STRIP_META_QSZ>(a, st);
    else prefill_group_partials<STRIP_META_GPTQ>(a, st);
    return launch_status();
  }
  if (fmt == STRIP_META_QSZ) prefill_group<STRIP_META_QSZ>(a, epilogue, st);
  else prefill_group<STRIP_META_GPTQ>(a, epilogue, st);
  return launch_status();
}

}  // namespace mtl

using namespace mtl;

extern "C" {

int64_t mtl_w4_gemm_prefill_workspace_bytes(int64_t M, int64_t K, int64_t N) {
  if (M < 1 || K < 256 || K % 256 != 0 || N < kPfCols || N % kPfCols != 0) return 0;
  const int s = prefill_splits((N / kPfCols) * ((M + kPfRows - 1) / kPfRows), K / 128,
                               pf_device_cus());
  return s > 1 ? (int64_t)s * M * N * 4 : 0;
}

int mtl_w4_gemm_prefill(const void* x, int64_t M, int64_t ldx, int64_t K,
                        const int32_t* strip_weight, const void* strip_scales,
                        const int32_t* strip_zeros, int64_t N, int32_t group_size,
                        int32_t zero_offset, int32_t epilogue, int32_t out_dtype, void* y,
                        int64_t ldy, float* workspace, int64_t ws_bytes, void* stream) {
  if (!strip_zeros) return MTL_ERR_INVALID_ARG;
  if (!aligned16(strip_zeros)) return MTL_ERR_ALIGN;
  return prefill_gemm(x, M, ldx, K, strip_weight, strip_scales, strip_zeros, N, group_size,
                      zero_offset, epilogue, out_dtype, y, ldy, workspace, ws_bytes,
                      STRIP_META_GPTQ, (hipStream_t)stream);
}

int64_t mtl_w4_gemm_prefill_partials_bytes(int64_t M, int64_t K, int64_t N) {
  if (M < 1 || K < 256 || K % 256 != 0 || N < kPfCols || N % kPfCols != 0) return 0;
  const int s = prefill_splits((N / kPfCols) * ((M + kPfRows - 1) / kPfRows), K / 128,
                               pf_device_cus());
  return (int64_t)s * M * N * 4;
}

int mtl_w4_gemm_prefill_partials(const void* x, const float* x_sums, int64_t M, int64_t ldx,
                                 int64_t K, const int32_t* strip_weight, const void* meta,
                                 const int32_t* strip_zeros, int64_t N, int32_t group_size,
                                 int32_t zero_offset, int32_t meta_format, float* partials,
                                 int64_t partials_bytes, void* stream) {
  if (meta_format != MTL_META_GPTQ && meta_format != MTL_META_QSZ) return MTL_ERR_INVALID_ARG;
  if (meta_format == MTL_META_GPTQ && !strip_zeros) return MTL_ERR_INVALID_ARG;
  if (meta_format == MTL_META_GPTQ && !aligned16(strip_zeros)) return MTL_ERR_ALIGN;
  if (!partials) return MTL_ERR_INVALID_ARG;
  return prefill_gemm(x, M, ldx, K, strip_weight, meta,
                      meta_format == MTL_META_GPTQ ? strip_zeros : nullptr, N, group_size,
                      meta_format == MTL_META_GPTQ ? zero_offset : 0, kEpiPartials,
                      MTL_OUT_F32, partials, N, partials, partials_bytes,
                      meta_format == MTL_META_QSZ ? STRIP_META_QSZ : STRIP_META_GPTQ,
                      (hipStream_t)stream, x_sums);
}

int mtl_w4_gemm_prefill_staged(const void* x, const float* x_sums, int64_t M, int64_t ldx,
                               int64_t K, const int32_t* strip_weight, const void* meta,
                               const int32_t* strip_zeros, int64_t N, int32_t group_size,
                               int32_t zero_offset, int32_t meta_format, int32_t epilogue,
                               int32_t out_dtype, void* y, int64_t ldy, float* workspace,
                               int64_t ws_bytes, void* stream) {
  if (meta_format != MTL_META_GPTQ && meta_format != MTL_META_QSZ) return MTL_ERR_INVALID_ARG;
  if (meta_format == MTL_META_GPTQ && !strip_zeros) return MTL_ERR_INVALID_ARG;
  if (meta_format == MTL_META_GPTQ && !aligned16(strip_zeros)) return MTL_ERR_ALIGN;
  if (!x_sums || (epilogue != MTL_EPI_NONE && epilogue != MTL_EPI_SILU_MUL))
    return MTL_ERR_INVALID_ARG;
  return prefill_gemm(x, M, ldx, K, strip_weight, meta,
                      meta_format == MTL_META_GPTQ ? strip_zeros : nullptr, N, group_size,
                      meta_format == MTL_META_GPTQ ? zero_offset : 0, epilogue, out_dtype, y,
                      ldy, workspace, ws_bytes,
                      meta_format == MTL_META_QSZ ? STRIP_META_QSZ : STRIP_META_GPTQ,
                      (hipStream_t)stream, x_sums);
}

int mtl_w4_gemm_prefill_qsz(const void* x, int64_t M, int64_t ldx, int64_t K,
                            const int32_t* strip_weight, const void* qsz, int64_t N,
                            int32_t group_size, int32_t epilogue, int32_t out_dtype, void* y,
                            int64_t ldy, float* workspace, int64_t ws_bytes, void* stream) {
  return prefill_gemm(x, M, ldx, K, strip_weight, qsz, nullptr, N, group_size, 0, epilogue,
                      out_dtype, y, ldy, workspace, ws_bytes, STRIP_META_QSZ,
                      (hipStream_t)stream);
}

// Whether mtl_int4pack_mm runs M > 1 rows on the prompt-length GEMM (else on the skinny
// strip GEMM, in 16-row launches when N is not a multiple of its 128-column tiles).
static bool int4pack_prefill(int64_t M, int64_t N) {
  return N % kPfCols == 0 && !strip_rows_pays(M, N);
}

int64_t mtl_int4pack_mm_workspace_bytes(int64_t M, int64_t K, int64_t N) {
  return M > 1 && int4pack_prefill(M, N) ? mtl_w4_gemm_prefill_workspace_bytes(M, K, N) : 0;
}

// The drop-in for torch._weight_int4pack_mm: M = 1 on the full-K strip GEMV, 2 to 16 rows on
// the skinny strip GEMM (strip_rows_pays), more on the prompt-length GEMM (or, when N is not
// a multiple of 128, the skinny GEMM 16 rows at a time).
int mtl_int4pack_mm(const void* x, int64_t M, int64_t K, const int32_t* packed,
                    int32_t group_size, const void* qsz, int64_t N, void* y, void* workspace,
                    int64_t ws_bytes, void* stream) {
  if (!x || !packed || !qsz || !y) return MTL_ERR_INVALID_ARG;
  if (group_size != 32 && group_size != 64 && group_size != 128 && group_size != 256)
    return MTL_ERR_GROUP;
  if (M < 1 || K <= 0 || N <= 0 || K % 256 != 0 || N % 16 != 0 || K % group_size != 0 ||
      (N / 16) * (K / 128) * 1024 >= ((int64_t)1 << 31) || M * K >= ((int64_t)1 << 31) ||
      (K / group_size) * N * 4 >= ((int64_t)1 << 31))
    return MTL_ERR_SHAPE;
  if (!aligned16(x) || !aligned16(packed) || (reinterpret_cast<uintptr_t>(qsz) & 3u) ||
      (reinterpret_cast<uintptr_t>(y) & 7u))
    return MTL_ERR_ALIGN;
  hipStream_t st = (hipStream_t)stream;
  const bool strip_ok = K <= 16384 && strip_blocks_per_wave(K, 1, group_size) > 0;
  StripArgs sa = {};
  sa.w = reinterpret_cast<const u32x4*>(packed);
  sa.scales = static_cast<const uint16_t*>(qsz);
  sa.K = (int)K;
  sa.N = (int)N;
  sa.group = group_size;
  sa.fmt = STRIP_META_QSZ;
  if (M == 1 && strip_ok) {
    sa.x = static_cast<const uint16_t*>(x);
    sa.y16 = static_cast<uint16_t*>(y);
    return strip_launch(sa, st);
  }
  if (int4pack_prefill(M, N))
    return prefill_gemm(x, M, K, K, packed, qsz, nullptr, N, group_size, 0, MTL_EPI_NONE,
                        MTL_OUT_BF16, y, N, static_cast<float*>(workspace), ws_bytes,
                        STRIP_META_QSZ, st);
  for (int64_t r0 = 0; r0 < M; r0 += 16) {
    const int64_t rows = M - r0 < 16 ? M - r0 : 16;
    if (const int status = strip_rows(static_cast<const uint16_t*>(x) + r0 * K, rows, K, K,
                                      nullptr, packed, qsz, nullptr, N, group_size, 0,
                                      STRIP_META_QSZ, static_cast<uint16_t*>(y) + r0 * N, N,
                                      MTL_OUT_BF16, stream))
      return status;
  }
  return MTL_OK;
}

}  // extern "C"
