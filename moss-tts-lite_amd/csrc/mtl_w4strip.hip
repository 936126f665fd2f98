// int4 GEMV over full-K column strips for gfx950 (M = 1, AutoGPTQ meta).
//
// A workgroup owns CT strips of 16 output columns over the whole input dimension K, so
// no split-K partial leaves the workgroup: the epilogue holds final sums and applies the
// decode step's residual add (publishing the RMSNorm statistics and the act-order copy
// of h), SiLU(gate)*up of an interleaved gate|up projection, or hands the fp32 results
// to the next kernel as a single "split".  This removes the cross-workgroup reduction (a
// kernel boundary, or a last-workgroup hand-off) from every int4 GEMV of the step.
//
// Weight layout (mtl_w4_strip): 1 KB block (s * K/128 + b) holds columns 16s..16s+15 over
// input channels 128b..128b+127.  Its 16-byte word l holds the qweight words
// (k-octet 16b + 4j + l/16, column 16s + l%16), j = 0..3.  Word j of lane l is the B
// operand of v_mfma_f32_16x16x32_bf16 number j over channels 128b + 32j .. +31 (lane l
// supplies rows 8(l/16) .. +7 of column l%16), so one 1 KB load per wave feeds four
// MFMAs, and a strip's K/128 blocks are consecutive in memory.
//
// Wave w of a workgroup serves strip w % CT over K slice w / CT (KW slices of NB blocks,
// KW * NB = K/128).  The CT waves of a slice stage its x once into LDS; the KW per-slice
// column sums of a strip meet in LDS and are added in slice order, so results are
// bitwise repeatable.
#include "mtl_w4core.h"
#include "mtl_bf16rows.h"

namespace mtl {

constexpr int kStripCols = 16;
constexpr int kStripBlockK = 128;     // input channels per 1 KB block
constexpr int kStripMaxWaves = 16;
// Blocks in flight per wave (the load ring, a divisor of NB) when fewer waves are resident:
// 4 (all of them for NB of 2 and 4, and for NB = 6 at g >= 128; 2 at g <= 64, whose 2 or 4
// groups per block bring as many metadata registers).  The launch geometry picks 2 at NB = 8
// when many waves are resident, and the deep rings of 8 and 16 are launch-shape options.
constexpr int strip_ring(int gr, int nb) { return nb == 6 ? (gr <= 2 ? 2 : 6) : nb < 4 ? nb : 4; }
// Waves per workgroup allowed (GR = g / 32, NB blocks per wave, WIN in flight): 16 (128
// VGPRs each); 12 (168 VGPRs) at NB = 16; 8 at g = 32 from NB = 8 on, whose metadata needs
// more than 128 VGPRs.
constexpr int strip_max_waves(int gr, int nb, int win) {
  return gr == 1 && nb >= 8 ? 8 : nb >= 16 ? 12 : kStripMaxWaves;
}
constexpr int kStripAux = 2;          // weight stream: non-temporal (read once per step)
// Strips per workgroup of the act-order gather (x copied into LDS and gathered there): the
// whole of x is staged per workgroup, so fewer, wider workgroups stage less, as long as
// they stay about as many as the CUs.  Two strips where that leaves at least 192
// workgroups (measured, GPTQ module at one row: q|k|v 6144 columns 4.99 -> 4.6 us, gate|up
// 24576 columns 11.7 -> 10.3 us; o and down, 4096 columns, are slower with 128 workgroups:
// 4.04 -> 4.4 and 7.95 -> 9.4 us; four strips are slower on every shape).
constexpr int kGatherCT = 2;
constexpr int kGatherMinWGs = 192;

// The body of one workgroup: `bid` of a launch of G strip workgroups (the kernel's own
// grid, or the first G workgroups of the combined launch below).
template <int GR, int XSRC, int EPI, int NB, int CT, int WIN, int FMT>
__device__ __forceinline__ void strip_body(const StripArgs& a, const int bid, const int G) {
  constexpr int ITEMS = 16 * NB;               // x items (8 channels) per K slice
  constexpr int STAGERS = 64 * CT;             // threads that stage one slice
  constexpr int ROUNDS = (ITEMS + STAGERS - 1) / STAGERS;
  constexpr int NGW = 4 * NB / GR;             // quantisation groups per slice
  constexpr int GI = 4 * GR;                   // x items per group
  static_assert((4 * NB) % GR == 0, "a slice must cover whole quantisation groups");
  static_assert(64 % GI == 0 && ITEMS % GI == 0, "a wave must stage whole groups");
  static_assert(EPI != STRIP_EPI_SILU || CT % 2 == 0, "SiLU*up pairs gate strips with up strips");
  static_assert(WIN >= 1 && WIN <= NB && NB % WIN == 0, "ring window");
  extern __shared__ u32x4 xa_all[];            // [KW][ITEMS] x items in pair order
  __shared__ float xg[kStripMaxWaves][NGW];    // per-slice group sums of x
  __shared__ float ytile[kStripMaxWaves][kStripCols];   // [slice * CT + strip][column]

  const int wave = wave_id();
  const int kw = (blockDim.x >> 6) / CT;       // K slices
  const int lane = threadIdx.x & 63;
  const int lg = lane >> 4, lj = lane & 15;
  const int cs = wave % CT, ks = wave / CT;    // this wave's strip and slice
  // Workgroups go to the 8 XCDs round robin; with xcd_order, XCD x runs the contiguous
  // workgroups x*G/8 .. (x+1)*G/8 - 1, so the cache lines of scales and zeros that
  // neighbouring strips share are fetched into one L2 only.
  const int wg = a.xcd_order ? (bid & 7) * (G >> 3) + (bid >> 3) : bid;
  // SiLU*up: the workgroup holds P = CT/2 (gate, up) strip pairs; pair p is the gate strip
  // 4*(p/2) + p%2 and its up partner two strips (32 columns) to the right, in the gate|up
  // interleave of 32-column blocks.  Waves cs < P serve the gate strips of pairs
  // P*wg + cs, waves cs >= P their up strips.  Otherwise CT consecutive strips.
  constexpr int P = CT / 2;
  const int s0 = EPI == STRIP_EPI_SILU ? 0 : wg * CT;
  int s = s0 + cs;
  if (EPI == STRIP_EPI_SILU) {
    const int p = P * wg + cs % P;
    s = 4 * (p >> 1) + (p & 1) + (cs >= P ? 2 : 0);
  }
  const int N = a.N;
  const int col = s * kStripCols + lj;
  const int item0 = ks * ITEMS;                // first x item of the slice
  u32x4* xa = xa_all + ks * ITEMS;

  // 1. Activation loads of this thread's items of the slice (raw; transformed once the
  //    weights are in flight).  Every item index is below K/8: K = 128 * KW * NB.
  const int tt = cs * 64 + lane;               // thread index among the slice's stagers
  // XSRC_PERM: the workgroup copies all of x (K/8 items, XR per thread) into LDS behind
  // the slices' tile, and each stager gathers its items' 8 channels from there through
  // perm (loaded with x, so the gather costs one round trip, like the other sources)
  constexpr int XR = XSRC == XSRC_PERM ? (NB + 4 * CT - 1) / (4 * CT) : 1;
  u32x4 xr[XR];
  u32x4 pv[XSRC == XSRC_PERM ? ROUNDS : 1];    // the items' 8 gather indices (uint16)
  if (XSRC == XSRC_PERM) {
    const int nitems = a.K >> 3;
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const int i = r * (int)blockDim.x + (int)threadIdx.x;
      xr[r] = *reinterpret_cast<const u32x4*>(a.x + (size_t)(i < nitems ? i : 0) * 8);
    }
  }
  u32x4 xv[ROUNDS], wv[XSRC == XSRC_RMSNORM ? ROUNDS : 1];
  float4 sg[XSRC == XSRC_SILU_PART ? ROUNDS : 1][2], su[XSRC == XSRC_SILU_PART ? ROUNDS : 1][2];
  const float* sbase[XSRC == XSRC_SILU_PART ? ROUNDS : 1];
  bool iok[ROUNDS];
#pragma unroll
  for (int r = 0; r < ROUNDS; ++r) {
    const int i = r * STAGERS + tt;
    iok[r] = i < ITEMS;
    const int it = item0 + (iok[r] ? i : 0);
    if (XSRC == XSRC_BF16) {
      xv[r] = *reinterpret_cast<const u32x4*>(a.x + (size_t)it * 8);
    } else if (XSRC == XSRC_PERM) {
      xv[r] = u32x4{0u, 0u, 0u, 0u};
      pv[r] = *reinterpret_cast<const u32x4*>(a.perm + (size_t)it * 8);
    } else if (XSRC == XSRC_RMSNORM) {
      xv[r] = *reinterpret_cast<const u32x4*>(a.hn + (size_t)it * 8);
      wv[r] = *reinterpret_cast<const u32x4*>(a.wn + (size_t)it * 8);
    } else {
      // channels 8it..8it+7 sit in one 32-column block of the gate|up interleave:
      // gate columns 64*(j/32) + j%32, their up partners 32 columns to the right; or
      // (xhalves) gate column j, its up partner K columns to the right
      xv[r] = u32x4{0u, 0u, 0u, 0u};
      const int j0 = it * 8;
      sbase[r] = a.xhalves ? a.xpart + j0 : a.xpart + 64 * (j0 >> 5) + (j0 & 31);
      const int uo = a.xhalves ? a.K : 32;
      sg[r][0] = ld_f4(sbase[r]);
      sg[r][1] = ld_f4(sbase[r] + 4);
      su[r][0] = ld_f4(sbase[r] + uo);
      su[r][1] = ld_f4(sbase[r] + uo + 4);
    }
  }
  const bool stages = cs * 64 < ITEMS;         // wave-uniform: this wave stages items
  SlotLoad slot_l;
  // RMSNorm: wave 0 alone loads the sums-of-squares slots and shares r through LDS (every
  // staging wave loading all of them cost 1 KB per wave: q|k|v 4.72 -> 4.56 us)
  if (XSRC == XSRC_RMSNORM && wave == 0) slot_issue(a.slots, a.K, lane, slot_l);
  // residual epilogue inputs of wave 0's column owners, read ahead of everything else
  u32x2 h_pre{0u, 0u};
  int32_t sc_pre[4] = {0, 0, 0, 0};
  const int c_own = (EPI == STRIP_EPI_SILU ? 0 : s0 * kStripCols) + 4 * (lane % (4 * CT));
  if (EPI == STRIP_EPI_RESID && wave == 0) {
    h_pre = *reinterpret_cast<const u32x2*>(a.h + c_own);
    if (a.h_ord && a.scatter) {
      const int4 p4 = *reinterpret_cast<const int4*>(a.scatter + c_own);
      sc_pre[0] = p4.x; sc_pre[1] = p4.y; sc_pre[2] = p4.z; sc_pre[3] = p4.w;
    }
  }

  // 2-3. The weight stream and its group metadata, WIN blocks in flight per wave: block b
  //      and the scales/zeros of the groups starting in it go to ring slot b % WIN, and
  //      block b + WIN is issued into that slot as soon as block b's operands are out.
  //      Loads complete in issue order, so waiting for block b never waits for a later
  //      one, and the unpack and MFMA work overlaps the rest of the stream.
  constexpr int MB = GR <= 4 ? 4 / GR : 1;     // groups starting in one block
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4*>(a.w), (short)0, (int)((int64_t)(N / kStripCols) * a.kblocks * 1024),
      0x00020000);
  const int blk0 = s * a.kblocks + ks * NB;
  // Metadata in the strip order of mtl_w4_strip_meta: record (s * KR + i) per block
  // (per block pair at g = 256) holds the MB scales of each of the strip's 16 columns
  // contiguously (fp16) and their zero nibbles, so a lane loads its column's metadata
  // of a block with one scale load and one zero load (a uniform record offset and one
  // per-lane offset).
  // The reference's qsz (STRIP_META_QSZ) instead: one (scale, zero) pair per group and
  // column, read in place at (group * N + column) * 4.
  const int ngroups = a.K / a.group;
  const int krec = GR == 8 ? a.kblocks >> 1 : a.kblocks;     // records per strip
  const int rec0 = s * krec + (GR == 8 ? (ks * NB) >> 1 : ks * NB);
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.scales), (short)0,
      FMT == STRIP_META_QSZ ? ngroups * N * 4 : ngroups * N * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t zrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(a.qzeros), (short)0,
      FMT == STRIP_META_QSZ ? 0 : ngroups * (N >> 1), 0x00020000);
  u32x4 wq[WIN];
  StripMeta<MB> mt[FMT == STRIP_META_GPTQ ? WIN : 1];
  uint32_t mq[FMT == STRIP_META_QSZ ? WIN : 1][MB];
  const int kbs = ks * NB;                     // the slice's first block within K
  // block b into ring slot r (r = b % WIN, a compile-time index at every call)
  auto issue = [&](int r, int b) {
    if (GR <= 4 || (r & 1) == 0) {             // g = 256: one record per block pair (b, r alike in parity)
      if constexpr (FMT == STRIP_META_GPTQ) {
        strip_meta_load<MB>(srsrc, zrsrc, lj, rec0 + (GR == 8 ? b >> 1 : b), mt[r]);
      } else {
#pragma unroll
        for (int m = 0; m < MB; ++m)
          mq[r][m] = qsz_load(srsrc, col, GR == 8 ? (kbs + b) >> 1 : (kbs + b) * MB + m, N);
      }
    }
    wq[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          wrsrc, lane * 16, (blk0 + b) * 1024, kStripAux));
  };
#pragma unroll
  for (int b = 0; b < WIN; ++b) issue(b, b);
  __builtin_amdgcn_sched_barrier(0);

  // 4. x into LDS in pair order, with per-group sums (fixed butterfly order).
  if (XSRC == XSRC_PERM) {
    u32x4* xs = xa_all + kw * ITEMS;           // x in the checkpoint's order
    const int nitems = a.K >> 3;
#pragma unroll
    for (int r = 0; r < XR; ++r) {
      const int i = r * (int)blockDim.x + (int)threadIdx.x;
      if (i < nitems) xs[i] = xr[r];
    }
    __syncthreads();
    if (stages) {
      const uint16_t* xs16 = reinterpret_cast<const uint16_t*>(xs);
#pragma unroll
      for (int r = 0; r < ROUNDS; ++r) {
        const uint32_t p[8] = {pv[r].x & 0xffffu, pv[r].x >> 16, pv[r].y & 0xffffu,
                               pv[r].y >> 16, pv[r].z & 0xffffu, pv[r].z >> 16,
                               pv[r].w & 0xffffu, pv[r].w >> 16};
        uint32_t e[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) e[c] = xs16[p[c]];
        xv[r] = u32x4{e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                      e[6] | (e[7] << 16)};
      }
    }
  }
  __shared__ float norm_sh;
  if (XSRC == XSRC_RMSNORM) {
    if (wave == 0) {
      const float t = rsqrtf(wave_sum_valu(slot_finish(slot_l, a.K, lane)) / (float)a.K + a.eps);
      if (lane == 0) norm_sh = t;
    }
    __syncthreads();
  }
  if (stages) {
    float norm_r = 0.f;
    if (XSRC == XSRC_RMSNORM) norm_r = norm_sh;
#pragma unroll
    for (int r = 0; r < ROUNDS; ++r) {
      u32x4 v = xv[r];
      if (XSRC == XSRC_RMSNORM) {
        v = rmsnorm8(v, wv[r], norm_r);
      } else if (XSRC == XSRC_SILU_PART) {
        float g[8] = {sg[r][0].x, sg[r][0].y, sg[r][0].z, sg[r][0].w,
                      sg[r][1].x, sg[r][1].y, sg[r][1].z, sg[r][1].w};
        float u[8] = {su[r][0].x, su[r][0].y, su[r][0].z, su[r][0].w,
                      su[r][1].x, su[r][1].y, su[r][1].z, su[r][1].w};
        for (int sp = 1; sp < a.xsplits; ++sp) {     // further splits, summed in split order
          const float* p = sbase[r] + (size_t)sp * a.xpart_ld;
          const int uo = a.xhalves ? a.K : 32;
          const float4 g0 = ld_f4(p), g1 = ld_f4(p + 4), u0 = ld_f4(p + uo), u1 = ld_f4(p + uo + 4);
          g[0] += g0.x; g[1] += g0.y; g[2] += g0.z; g[3] += g0.w;
          g[4] += g1.x; g[5] += g1.y; g[6] += g1.z; g[7] += g1.w;
          u[0] += u0.x; u[1] += u0.y; u[2] += u0.z; u[3] += u0.w;
          u[4] += u1.x; u[5] += u1.y; u[6] += u1.z; u[7] += u1.w;
        }
        v = u32x4{silu_mul_bf16(g[0], u[0]) | (silu_mul_bf16(g[1], u[1]) << 16),
                  silu_mul_bf16(g[2], u[2]) | (silu_mul_bf16(g[3], u[3]) << 16),
                  silu_mul_bf16(g[4], u[4]) | (silu_mul_bf16(g[5], u[5]) << 16),
                  silu_mul_bf16(g[6], u[6]) | (silu_mul_bf16(g[7], u[7]) << 16)};
      }
      float sum;
      const u32x4 pv = pair_order(v, sum);
      sum = group_sum_valu<GI>(sum);            // every lane of the wave active here
      const int i = r * STAGERS + tt;
      if (iok[r]) {
        xa[i] = pv;
        if ((i & (GI - 1)) == 0) xg[ks][i / GI] = sum;
      }
    }
  }
  __syncthreads();

  // 5. MFMA over the slice's row quads, block by block as the ring delivers them; per
  //    quantisation group y += s * (A - (128 + z) * X).  All 16 A rows are x, so every
  //    accumulator row holds the lane's column.  One accumulator chains the MFMAs of a
  //    group (the other waves of the SIMD cover the dependency): fewer registers, so every
  //    workgroup of the launch is resident at once (measured 7 % faster than four).
  const uint32_t kMagic = vgpr_const(0x43004300u);   // bf16 (128, 128)
  const uint32_t kLo = vgpr_const(0x000F000Fu);
  float tot = 0.f;
  float cur_s = 0.f, cur_z = 0.f, cur_d = 0.f;  // g = 256: the group of this block pair
  floatx4 acc;
  // Ring turns with the WIN ring slots unrolled inside, so ring indexes stay compile-time.
  // The turns are unrolled too (measured faster than a loop, whose ring registers need
  // copies at the back edge), except at g = 32 from 6 blocks on, whose four groups per
  // block would not fit in registers unrolled.  The last turn is
  // peeled: it issues no refills, so inside the loop every refill is unconditional and the
  // waits stay exact (a refill under a run-time branch makes the compiler wait for every
  // outstanding load).  Groups never straddle a turn: 4 * WIN row quads hold whole groups
  // (WIN even for g = 256), so q and the group of a block are fixed
  // per slot.
  static_assert(GR != 8 || WIN % 2 == 0, "g = 256 pairs blocks within a ring turn");
  auto turn = [&](const int b0, const bool refill) {
#pragma unroll
    for (int r = 0; r < WIN; ++r) {
      const int b = b0 + r;
      const u32x4 w4 = wq[r];
      float gs[MB], gz[MB], gd[MB];             // (s, c, d) of the block's groups (qsz_decode)
      if (GR <= 4 || (r & 1) == 0) {
        if constexpr (FMT == STRIP_META_GPTQ) {
          strip_meta_decode<MB>(mt[r], lj, a.zero_offset, gs, gz);
#pragma unroll
          for (int m = 0; m < MB; ++m) gd[m] = 0.f;
        } else {
#pragma unroll
          for (int m = 0; m < MB; ++m) qsz_decode(mq[r][m], gs[m], gz[m], gd[m]);
        }
      }
      if (GR == 8 && (r & 1) == 0) { cur_s = gs[0]; cur_z = gz[0]; cur_d = gd[0]; }
      // keep the compiler from hoisting later ring loads (and their registers) above here:
      // an empty asm with a memory clobber orders the loads at the IR level, the
      // scheduling barrier in the machine scheduler
      asm volatile("" ::: "memory");
      if (refill) issue(r, b + WIN);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int rq = 4 * b + j;               // row quad within the slice
        const int q = (4 * r + j) % GR;         // == rq % GR: 4 * b0 is a multiple of GR
        if (q == 0) acc = floatx4{0.f, 0.f, 0.f, 0.f};
        const uint32_t w = j == 0 ? w4.x : j == 1 ? w4.y : j == 2 ? w4.z : w4.w;
        const bf16x8_t A = __builtin_bit_cast(bf16x8_t, xa[4 * rq + lg]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, unpack_codes8(w, kLo, kMagic), acc, 0, 0, 0);
        if (q == GR - 1) {
          const float Asum = acc[0];
          const float sc = GR == 8 ? cur_s : gs[j / GR];
          const float cz = GR == 8 ? cur_z : gz[j / GR];
          const float X = xg[ks][rq / GR];
          tot = fmaf(sc, fmaf(-cz, X, Asum), tot);
          if constexpr (FMT == STRIP_META_QSZ) tot = fmaf(GR == 8 ? cur_d : gd[j / GR], X, tot);
        }
      }
    }
  };
  constexpr int kTurnUnroll = GR == 1 && NB >= 6 ? 1 : NB / WIN;
#pragma unroll kTurnUnroll
  for (int b0 = 0; b0 < NB - WIN; b0 += WIN) turn(b0, true);
  turn(NB - WIN, false);

  // 6. Per-slice column sums meet in LDS; wave 0 adds them in slice order, four columns
  //    per lane (lanes 0 .. 4*CT-1 own columns s0*16 + 4*lane .. +3).
  if (lg == 0) ytile[wave][lj] = tot;
  __syncthreads();
  if (wave != 0) return;
  const int q4 = lane % (4 * CT);                // CT need not be a power of two
  const int ec = q4 >> 2;                        // strip of these columns
  if (EPI == STRIP_EPI_SILU) {
    // lanes 0..4P-1 sum the gate columns 4*(lane%4)..+3 of pair P*wg + lane/4 and their up
    // partners (strip ec + P) straight from LDS, both in slice order: no cross-lane step
    // between the sums and SiLU on the launch's tail.  Column i of pair p's gate strip is
    // SwiGLU output 16*p + i (64-column blocks of 32 gate | 32 up), so lane l writes
    // 16*P*wg + 4*l .. +3.
    if (lane >= 4 * P) return;
    float g[4] = {0.f, 0.f, 0.f, 0.f}, u[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < kw; ++k) {
      const float4 g4 = *reinterpret_cast<const float4*>(&ytile[k * CT + ec][4 * (q4 & 3)]);
      const float4 u4 = *reinterpret_cast<const float4*>(&ytile[k * CT + ec + P][4 * (q4 & 3)]);
      g[0] += g4.x; g[1] += g4.y; g[2] += g4.z; g[3] += g4.w;
      u[0] += u4.x; u[1] += u4.y; u[2] += u4.z; u[3] += u4.w;
    }
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = silu_mul_bf16(g[e], u[e]);
    *reinterpret_cast<u32x2*>(a.act + (size_t)wg * 16 * P + 4 * lane) =
        u32x2{o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
    return;
  }
  float y[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < kw; ++k) {
    const float4 t4 = *reinterpret_cast<const float4*>(&ytile[k * CT + ec][4 * (q4 & 3)]);
    y[0] += t4.x; y[1] += t4.y; y[2] += t4.z; y[3] += t4.w;
  }
  const int c0 = s0 * kStripCols + 4 * q4;
  const bool owner = lane < 4 * CT;
  if (EPI == STRIP_EPI_STORE) {
    if (owner) {
      if (a.y16)
        *reinterpret_cast<u32x2*>(a.y16 + c0) =
            u32x2{f32_to_bf16(y[0]) | (f32_to_bf16(y[1]) << 16),
                  f32_to_bf16(y[2]) | (f32_to_bf16(y[3]) << 16)};
      else
        *reinterpret_cast<float4*>(a.y + c0) = make_float4(y[0], y[1], y[2], y[3]);
    }
    return;
  }
  // 7. Residual epilogue (fast.py:168-171): h = bf16(bf16(y) + h) in place, h scattered to
  //    the next GEMV's input order, and each strip's sum of squares as one slot.
  const u32x2 rr = h_pre;
  float hv[4] = {bf16_to_f32(rr.x & 0xffffu), bf16_to_f32(rr.x >> 16),
                 bf16_to_f32(rr.y & 0xffffu), bf16_to_f32(rr.y >> 16)};
  float ss = residual4(y, hv);
  ss = slot_combine_valu(ss);
  if (owner) {
    *reinterpret_cast<u32x2*>(a.h + c0) =
        u32x2{f32_to_bf16(hv[0]) | (f32_to_bf16(hv[1]) << 16),
              f32_to_bf16(hv[2]) | (f32_to_bf16(hv[3]) << 16)};
    if (a.h_ord) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        a.h_ord[a.scatter ? sc_pre[c] : c0 + c] = (uint16_t)f32_to_bf16(hv[c]);
    }
    if ((lane & 3) == 0) a.slots_out[s0 + ec] = ss;
  }
}

// Launch geometry: CT strips per workgroup, NB blocks per wave, WIN blocks in flight per
// wave.  A workgroup has (K/128 / NB) * CT waves within strip_max_waves.
struct StripGeom {
  int ct, nb, win;
};

static bool nb_fits(int64_t kb, int nb, int ct, int gr) {
  return nb > 0 && kb % nb == 0 && (kb / nb) * ct <= strip_max_waves(gr, nb, 0);
}

// Blocks per wave for K/128 = kb blocks: even NB (whole groups up to g = 256), 8 where it
// fits (measured fastest on the decode shapes; 4 and 16 are slower), else the first of 4,
// 6, 2, 16 that fits.
static int blocks_per_wave(int64_t K, int ct, int group) {
  if (K <= 0 || K % (2 * kStripBlockK) != 0) return 0;
  const int64_t kb = K / kStripBlockK;
  for (const int nb : {8, 4, 6, 2, 16})
    if (nb_fits(kb, nb, ct, group / 32)) return nb;
  return 0;
}

// Blocks per wave of the strip GEMV with ct strips per workgroup at this group size (0: the
// shape does not fit); group sizes other than 32, 64, 128, 256 are checked as 32.
int strip_blocks_per_wave(int64_t K, int ct, int group) {
  const bool known = group == 32 || group == 64 || group == 128 || group == 256;
  return blocks_per_wave(K, ct, known ? group : 32);
}

// The load ring: 2 blocks in flight per wave at NB = 8 when the launch keeps at least 12
// waves per CU of a 256-CU chip (gate|up: 24, down: 12), else the ring of strip_ring.  A
// CU accepts only about 20 KB of loads into its memory pipeline at a time; a wave whose
// next load does not fit stalls at that instruction, so a deeper ring than the waves
// together need only delays their other work (measured: gate|up 11.15 -> 10.83 us, down
// 7.09 -> 6.85 us with the ring of 2; o, at 4 waves per CU, is slower with it: 4.1 -> 4.6).
static int default_ring(int gr, int nb, int64_t waves) {
  return nb == 8 && waves >= 12 * 256 ? 2 : strip_ring(gr, nb);
}

// Rings each NB is built with (deep rings of 8 and 16: g >= 128, GPTQ metadata).
static bool ring_built(int gr, int nb, int win, int fmt) {
  const bool deep = gr >= 4 && fmt == STRIP_META_GPTQ;
  switch (nb) {
    case 2: return win == 2;
    case 4: return win == 4;
    case 6: return win == strip_ring(gr, 6);
    case 8: return win == 2 || win == 4 || (win == 8 && deep);
    case 16: return win == 4 || ((win == 8 || win == 16) && deep);
    default: return false;
  }
}

template <int GR, int XSRC, int EPI, int NB, int CT, int WIN, int FMT>
__global__ void __launch_bounds__(64 * strip_max_waves(GR, NB, WIN), 1)
w4_strip_kernel(StripArgs a) {
  strip_body<GR, XSRC, EPI, NB, CT, WIN, FMT>(a, blockIdx.x, gridDim.x);
}

// The RMSNorm-staged GEMV (one strip per workgroup, 4 waves) and a bf16 kept projection
// over the same h in one launch: workgroups below ga run the strip GEMV, the others the
// bf16 rows (mtl_bf16rows.h).  Two dependent launches become one, and the two products
// stream at once (the kept v_proj beside the int4 q|k of the MOSS step).
template <int GR, int NB, int WIN, int FMT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
w4_strip_bf16_kernel(StripArgs a, Bf16RowsArgs b, int ga) {
  if ((int)blockIdx.x < ga)
    strip_body<GR, XSRC_RMSNORM, STRIP_EPI_STORE, NB, 1, WIN, FMT>(a, blockIdx.x, ga);
  else
    bf16_rows_norm_body<8>(b, (int)blockIdx.x - ga);
}

// Resolve the launch shape of a: the requested geometry, automatic where a field is 0.
// Strips per workgroup: SiLU*up 2 (one gate|up pair) or 6 (three pairs); the RMSNorm-staged
// store 1, 2 or 4; the others 1.  The reference's qsz metadata takes the automatic CT.
static int strip_geometry(const StripArgs& a, StripGeom& g) {
  const int gr = a.group / 32;
  const mtl_strip_geometry& r = a.geom;
  const bool gather = a.perm && !a.h && !a.xpart && !a.hn;
  const int auto_ct = a.act ? 2
                     : gather && a.N % (kStripCols * kGatherCT) == 0 &&
                               a.N / (kStripCols * kGatherCT) >= kGatherMinWGs &&
                               blocks_per_wave(a.K, kGatherCT, a.group) ? kGatherCT : 1;
  g.ct = r.strips_per_wg ? r.strips_per_wg : auto_ct;
  if (a.act) {
    if (g.ct != 2 && g.ct != 6) return MTL_ERR_UNSUPPORTED;
  } else if ((a.hn && !a.h) || gather) {
    if (g.ct != 1 && g.ct != 2 && g.ct != 4) return MTL_ERR_UNSUPPORTED;
  } else if (g.ct != 1) {
    return MTL_ERR_UNSUPPORTED;
  }
  if (a.fmt == STRIP_META_QSZ && g.ct != auto_ct) return MTL_ERR_UNSUPPORTED;
  if (a.N % (kStripCols * g.ct) != 0 || a.K % (2 * kStripBlockK) != 0) return MTL_ERR_SHAPE;
  const int64_t kb = a.K / kStripBlockK;
  g.nb = r.blocks_per_wave ? r.blocks_per_wave : blocks_per_wave(a.K, g.ct, a.group);
  if (!nb_fits(kb, g.nb, g.ct, gr)) return MTL_ERR_SHAPE;
  const int64_t wgs = a.N / (kStripCols * g.ct);
  g.win = r.ring ? r.ring : default_ring(gr, g.nb, wgs * (kb / g.nb) * g.ct);
  if (!ring_built(gr, g.nb, g.win, a.fmt)) return MTL_ERR_UNSUPPORTED;
  if (r.xcd_order < -1 || r.xcd_order > 1) return MTL_ERR_INVALID_ARG;
  return MTL_OK;
}

template <int GR, int XSRC, int EPI, int CT, int FMT>
static void strip_nb(const StripArgs& a, const StripGeom& g, hipStream_t st) {
  const dim3 grid(a.N / (kStripCols * CT));
  const dim3 block(64 * CT * (a.kblocks / g.nb));
  // the slices' x tile, and for the act-order gather all of x behind it
  const size_t lds = (size_t)(a.kblocks / g.nb) * 16 * g.nb * sizeof(u32x4) +
                     (XSRC == XSRC_PERM ? (size_t)a.K * 2 : 0);
  constexpr bool kDeep = GR >= 4 && FMT == STRIP_META_GPTQ;
#define MTL_STRIP_LAUNCH(NB_, WIN_) \
  hipLaunchKernelGGL((w4_strip_kernel<GR, XSRC, EPI, NB_, CT, WIN_, FMT>), grid, block, lds, st, a)
  switch (g.nb) {
    case 2: MTL_STRIP_LAUNCH(2, 2); break;
    case 4: MTL_STRIP_LAUNCH(4, 4); break;
    case 6: MTL_STRIP_LAUNCH(6, strip_ring(GR, 6)); break;
    case 8:
      if (g.win == 2) {
        MTL_STRIP_LAUNCH(8, 2);
      } else if constexpr (kDeep) {
        if (g.win == 8) MTL_STRIP_LAUNCH(8, 8); else MTL_STRIP_LAUNCH(8, 4);
      } else {
        MTL_STRIP_LAUNCH(8, 4);
      }
      break;
    default:
      if constexpr (kDeep) {
        if (g.win == 16) MTL_STRIP_LAUNCH(16, 16);
        else if (g.win == 8) MTL_STRIP_LAUNCH(16, 8);
        else MTL_STRIP_LAUNCH(16, 4);
      } else {
        MTL_STRIP_LAUNCH(16, 4);
      }
      break;
  }
#undef MTL_STRIP_LAUNCH
}

template <int GR, int FMT>
static void strip_variant(const StripArgs& a, const StripGeom& g, hipStream_t st) {
  if (a.act) {
    if (FMT == STRIP_META_GPTQ && g.ct == 6) strip_nb<GR, XSRC_RMSNORM, STRIP_EPI_SILU, 6, FMT>(a, g, st);
    else strip_nb<GR, XSRC_RMSNORM, STRIP_EPI_SILU, 2, FMT>(a, g, st);
  } else if (a.h) {
    if (a.xpart) strip_nb<GR, XSRC_SILU_PART, STRIP_EPI_RESID, 1, FMT>(a, g, st);
    else strip_nb<GR, XSRC_BF16, STRIP_EPI_RESID, 1, FMT>(a, g, st);
  } else if (a.hn) {
    if (FMT == STRIP_META_GPTQ && g.ct == 4) strip_nb<GR, XSRC_RMSNORM, STRIP_EPI_STORE, 4, FMT>(a, g, st);
    else if (FMT == STRIP_META_GPTQ && g.ct == 2) strip_nb<GR, XSRC_RMSNORM, STRIP_EPI_STORE, 2, FMT>(a, g, st);
    else strip_nb<GR, XSRC_RMSNORM, STRIP_EPI_STORE, 1, FMT>(a, g, st);
  } else if (a.xpart) {
    strip_nb<GR, XSRC_SILU_PART, STRIP_EPI_STORE, 1, FMT>(a, g, st);
  } else if (FMT == STRIP_META_GPTQ && a.perm) {
    if (g.ct == 4) strip_nb<GR, XSRC_PERM, STRIP_EPI_STORE, 4, FMT>(a, g, st);
    else if (g.ct == 2) strip_nb<GR, XSRC_PERM, STRIP_EPI_STORE, 2, FMT>(a, g, st);
    else strip_nb<GR, XSRC_PERM, STRIP_EPI_STORE, 1, FMT>(a, g, st);
  } else {
    strip_nb<GR, XSRC_BF16, STRIP_EPI_STORE, 1, FMT>(a, g, st);
  }
}

template <int FMT>
static void strip_group(const StripArgs& a, const StripGeom& g, hipStream_t st) {
  switch (a.group) {
    case 32: strip_variant<1, FMT>(a, g, st); break;
    case 64: strip_variant<2, FMT>(a, g, st); break;
    case 128: strip_variant<4, FMT>(a, g, st); break;
    default: strip_variant<8, FMT>(a, g, st); break;
  }
}

// Shapes, pointers and alignment are checked by the entry points.
int strip_launch(const StripArgs& args, hipStream_t st) {
  StripArgs a = args;
  StripGeom g;
  if (const int status = strip_geometry(a, g)) return status;
  a.kblocks = a.K / kStripBlockK;
  a.xcd_order = a.geom.xcd_order != -1 && (a.N / (kStripCols * g.ct)) % 8 == 0;
  if (a.fmt == STRIP_META_QSZ) strip_group<STRIP_META_QSZ>(a, g, st);
  else strip_group<STRIP_META_GPTQ>(a, g, st);
  return launch_status();
}

// The combined launch of an RMSNorm-staged strip GEMV (XSRC_RMSNORM, store epilogue) and
// a bf16 kept projection; MTL_ERR_UNSUPPORTED where its shape does not apply (the caller
// then issues the two launches): one strip per workgroup in 4 waves, K <= 4096.
template <int GR, int FMT>
static int strip_bf16_group(const StripArgs& a, const StripGeom& g, const Bf16RowsArgs& b,
                            int gb, hipStream_t st) {
  const int ga = a.N / kStripCols;
  const dim3 grid(ga + gb), block(256);
  const size_t lds = (size_t)(a.kblocks / g.nb) * 16 * g.nb * sizeof(u32x4);
#define MTL_STRIP_BF16(NB_, WIN_) \
  hipLaunchKernelGGL((w4_strip_bf16_kernel<GR, NB_, WIN_, FMT>), grid, block, lds, st, a, b, ga)
  if (g.nb == 8 && g.win == 4) MTL_STRIP_BF16(8, 4);
  else if (g.nb == 8 && g.win == 2) MTL_STRIP_BF16(8, 2);
  else return MTL_ERR_UNSUPPORTED;
#undef MTL_STRIP_BF16
  return MTL_OK;
}

int strip_launch_bf16(const StripArgs& args, const Bf16RowsArgs& b, int gb, hipStream_t st) {
  StripArgs a = args;
  StripGeom g;
  if (!a.hn || a.h || a.act || a.xpart) return MTL_ERR_UNSUPPORTED;
  if (const int status = strip_geometry(a, g)) return status;
  a.kblocks = a.K / kStripBlockK;
  if (g.ct != 1 || 64 * (a.kblocks / g.nb) != 256 || a.K > 4096 || b.K != a.K)
    return MTL_ERR_UNSUPPORTED;
  a.xcd_order = a.geom.xcd_order != -1 && (a.N / kStripCols) % 8 == 0;
  int st_code = MTL_ERR_UNSUPPORTED;
  switch (a.group) {
    case 32: st_code = a.fmt == STRIP_META_QSZ ? strip_bf16_group<1, STRIP_META_QSZ>(a, g, b, gb, st)
                                               : strip_bf16_group<1, STRIP_META_GPTQ>(a, g, b, gb, st); break;
    case 64: st_code = a.fmt == STRIP_META_QSZ ? strip_bf16_group<2, STRIP_META_QSZ>(a, g, b, gb, st)
                                               : strip_bf16_group<2, STRIP_META_GPTQ>(a, g, b, gb, st); break;
    case 128: st_code = a.fmt == STRIP_META_QSZ ? strip_bf16_group<4, STRIP_META_QSZ>(a, g, b, gb, st)
                                                : strip_bf16_group<4, STRIP_META_GPTQ>(a, g, b, gb, st); break;
    default: st_code = a.fmt == STRIP_META_QSZ ? strip_bf16_group<8, STRIP_META_QSZ>(a, g, b, gb, st)
                                               : strip_bf16_group<8, STRIP_META_GPTQ>(a, g, b, gb, st); break;
  }
  return st_code ? st_code : launch_status();
}

// Strip layout (see the top of this file); rows past K/8 never occur (K % 256 == 0).
__global__ void strip_weights_kernel(const uint32_t* __restrict__ qw, int64_t K, int64_t N,
                                     uint4* __restrict__ out) {
  const int64_t kb = K / kStripBlockK;
  const int64_t total = (N / kStripCols) * kb * 64;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t l = t & 63, blk = t >> 6;
    const int64_t b = blk % kb, s = blk / kb;
    const int64_t col = kStripCols * s + (l & 15);
    const int64_t row = 16 * b + (l >> 4);
    out[t] = make_uint4(qw[(row + 0) * N + col], qw[(row + 4) * N + col],
                        qw[(row + 8) * N + col], qw[(row + 12) * N + col]);
  }
}

// Strip metadata (see the strip GEMV): thread t handles record rec = t / 8 (block, or block
// pair at g = 256, of strip s = rec / KR) and columns 2*(t%8), +1 of the strip.
__global__ void strip_meta_kernel(const uint16_t* __restrict__ scales,
                                  const uint32_t* __restrict__ qzeros, int64_t N, int64_t krec,
                                  int64_t nrec, int mb, int pair, uint16_t* __restrict__ sc_out,
                                  uint8_t* __restrict__ z_out) {
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < nrec * 8;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t rec = t >> 3, cp = t & 7;
    const int64_t s = rec / krec, i = rec % krec;
    uint32_t zbits[2] = {0u, 0u};
    for (int h = 0; h < 2; ++h) {
      const int64_t c = 2 * cp + h, n = kStripCols * s + c;
      for (int m = 0; m < mb; ++m) {
        const int64_t g = pair ? i : i * mb + m;
        sc_out[(rec * kStripCols + c) * mb + m] = scales[g * N + n];
        const uint32_t z = (qzeros[g * (N >> 3) + (n >> 3)] >> (4 * (n & 7))) & 0xfu;
        zbits[h] |= z << (4 * m);
      }
    }
    if (mb == 4) {
      reinterpret_cast<uint16_t*>(z_out)[rec * 16 + 2 * cp] = (uint16_t)zbits[0];
      reinterpret_cast<uint16_t*>(z_out)[rec * 16 + 2 * cp + 1] = (uint16_t)zbits[1];
    } else if (mb == 2) {
      z_out[rec * 16 + 2 * cp] = (uint8_t)zbits[0];
      z_out[rec * 16 + 2 * cp + 1] = (uint8_t)zbits[1];
    } else {
      z_out[rec * 8 + cp] = (uint8_t)(zbits[0] | (zbits[1] << 4));
    }
  }
}

}  // namespace mtl

using namespace mtl;

extern "C" {

int mtl_w4_strip_meta(const void* scales, const int32_t* qzeros, int64_t K, int64_t N,
                      int32_t group_size, void* strip_scales, int32_t* strip_zeros,
                      void* stream) {
  if (!scales || !qzeros || !strip_scales || !strip_zeros) return MTL_ERR_INVALID_ARG;
  if (group_size != 32 && group_size != 64 && group_size != 128 && group_size != 256)
    return MTL_ERR_GROUP;
  if (!mtl_w4_strip_bytes(K, N) || K % group_size != 0) return MTL_ERR_SHAPE;
  if (!aligned16(strip_scales) || !aligned16(strip_zeros)) return MTL_ERR_ALIGN;
  const int pair = group_size == 256;
  const int mb = pair ? 1 : 128 / group_size;
  const int64_t krec = pair ? K / 256 : K / 128;
  const int64_t nrec = (N / kStripCols) * krec;
  int blocks = (int)((nrec * 8 + 255) / 256);
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(strip_meta_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(scales),
                     reinterpret_cast<const uint32_t*>(qzeros), N, krec, nrec, mb, pair,
                     static_cast<uint16_t*>(strip_scales),
                     reinterpret_cast<uint8_t*>(strip_zeros));
  return launch_status();
}

int64_t mtl_w4_strip_bytes(int64_t K, int64_t N) {
  if (K <= 0 || N <= 0 || N % kStripCols != 0 || K % (2 * kStripBlockK) != 0) return 0;
  return N * K / 2;
}

int mtl_w4_strip(const int32_t* qweight, int64_t K, int64_t N, int32_t* strip,
                 int64_t strip_bytes, void* stream) {
  if (!qweight || !strip) return MTL_ERR_INVALID_ARG;
  const int64_t need = mtl_w4_strip_bytes(K, N);
  if (!need || need >= ((int64_t)1 << 31)) return MTL_ERR_SHAPE;
  if (strip_bytes < need) return MTL_ERR_WORKSPACE;
  if (!aligned16(strip) || !aligned16(qweight)) return MTL_ERR_ALIGN;
  const int64_t total = need / 16;
  int blocks = (int)((total + 255) / 256);
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(strip_weights_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const uint32_t*>(qweight), K, N,
                     reinterpret_cast<uint4*>(strip));
  return launch_status();
}

}  // extern "C"
