// int4 weight GEMV / skinny GEMM for gfx950 (M = 1..16), fp32 accumulation.
//
// One kernel serves both weight contracts of the hot path:
//   * AutoGPTQ meta (scales fp16 [G,N], qzeros int4 [G,N/8]):  w = (q - z) * s
//   * the reference's qsz meta (bf16 [G,N,2] = scale, zero):    w = (q - 8) * s + zero
//     (moss_tts_lite/gptq.py:87-97; the op it replaces is torch._weight_int4pack_mm at
//      fast.py:118, gptq.py:582, fast_native.py:169)
// written as w = (q - c) * s + d.  Since (q - c) * s is exact in fp32, both equal the
// exact dequantised weight.
//
// Work decomposition (deterministic, no atomics on the data):
//   * a workgroup owns a 256-column tile and one split of 512 input channels; its 4
//     waves sit side by side along N (64 columns each) and share the LDS copy of x;
//   * per 32-channel row quad, lane l issues one 16-byte buffer load: qweight row
//     4q + l/16, columns 4*(l%16)..+3 -- exactly the B operand of
//     v_mfma_f32_16x16x32_bf16 for those 4 columns.  All 16 loads of a lane are in
//     flight before the first wait;
//   * blockIdx.y splits K; each workgroup publishes an fp32 partial tile and the last
//     workgroup of the tile (agent-scope counter) sums the splits in split order,
//     applies the epilogue and resets the counter, so results (and graph replays) are
//     bitwise repeatable and the next launch needs no memset.  Fused consumers may
//     instead read the partial tiles themselves.
//
// Inner loop: a qweight word holds 8 codes; OR-ing nibble pairs into 0x4300 gives the
// bf16 pair (128 + q_j, 128 + q_{j+4}) (one v_and_or_b32 each), so one word is the 8-value
// B fragment of an MFMA whose A fragment is x staged in LDS in the same pair order (all
// 16 A rows = x for M = 1, one row per x row otherwise).  Per group (g/32 quads) the
// accumulated sum A = sum x*(128+q) and X = sum x give
//     sum x*w = s * (A - (128 + c) * X) + d * X.
#include "mtl_w4core.h"
#include "mtl_bf16rows.h"
#include "mtl_decode.h"

namespace mtl {

static int g_gemm_cus = 0;

static int gemm_device_cus() {
  if (!g_gemm_cus) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    g_gemm_cus = n;
  }
  return g_gemm_cus;
}

constexpr int kTileN = 256;        // output columns per workgroup (4 waves)
constexpr int kWaveN = 64;         // output columns per wave (16 lanes x 4)
constexpr int kRowQuads = 16;      // qweight row quads (4 rows = 32 channels) per split
constexpr int kRowsPerWG = 4 * kRowQuads;   // qweight rows per split: 512 input channels
constexpr int kMaxM = 16;
// Cache policy of the weight stream (read once per step): non-temporal.
constexpr int kStreamAux = 2;

struct W4Args {
  const uint16_t* x;        // bf16 [M, K]
  const u32x4* qweight;     // int32 [K/8, N] viewed as [K/8, N/4] x 16 B
  const uint16_t* meta0;    // GPTQ: fp16 scales [G, N]; QSZ: bf16 qsz [G, N, 2]
  const uint32_t* qzeros;   // GPTQ: [G, N/8]
  const int32_t* perm;      // optional act-order gather index [K]
  const float* xpart;       // XSRC_SILU_PART: gate|up partials [xsplits, M, xpart_ld]
  int xsplits, xpart_ld;
  const uint16_t* hn;       // XSRC_RMSNORM: residual stream h [K] (act-order order)
  const uint16_t* wn;       //               norm weight [K] (same order)
  const float* slots;       //               sums of squares of h, one per 16 columns
  float eps;
  uint16_t* h_ord;          // EPI_RESIDUAL_SLOTS: h scattered into the next GEMV's order
  const int32_t* scatter;   //   h_ord[scatter[n]] = h[n] (NULL: h_ord[n] = h[n])
  float* slots_out;         //   one sum of h^2 per 16 columns
  int tiled;                // qweight in the wave-contiguous layout of mtl_w4_tile
  const uint16_t* resid;    // RESIDUAL epilogue input [M, N]
  void* y;
  float* partial;           // [splits, M, N]
  unsigned* counters;       // [col_tiles], zero between launches
  int inkernel_reduce;      // 1: last workgroup reduces; 0: w4_reduce_kernel does
  int partials_only;        // 1: always publish [splits, M, N] partials, no epilogue
  int M, K, N, group, zero_offset, splits, epilogue, out_f32;
};

// Internal epilogue of mtl_w4_gemm_residual: h = bf16(bf16(acc) + h) in place, h scattered
// to h_ord, sums of squares of h per 16 columns to slots_out (M = 1, reduced in the kernel).
constexpr int kEpiResidualSlots = 3;

// The int4 GEMV / skinny GEMM.  Workgroup = 4 waves side by side along N (64 columns
// each: lane l owns columns 4*(l%16)..+3) over one split of 512 input channels (64
// qweight rows = 16 row quads).  Per row quad, lane l loads the 16-byte word group of
// qweight row 4q + l/16, i.e. exactly the B operand of v_mfma_f32_16x16x32_bf16 for
// its 4 columns; the A operand is x (row m = l%16, or row 0 broadcast when MR = 1).
// GR = row quads per quantisation group (group / 32).
// KW = waves stacked along K (1, 2 or 4): wave w covers columns (w % 4) * 64 of the
// tile and row quads (w / 4) * 16/KW .. +16/KW of the split; the KW partial tiles are
// summed through LDS in fixed order.  KW > 1 serves M = 1.
template <int MR, int GR, int FMT, int XSRC, int KW>
__global__ void __launch_bounds__(256 * KW) w4_gemm_kernel(W4Args a) {
  constexpr bool LATE_X = XSRC == XSRC_PERM;  // the gather needs perm: x after the weights
  constexpr int NG = kRowQuads / GR;          // groups per split
  constexpr int RQW = kRowQuads / KW;         // row quads per wave
  constexpr int NGW = RQW / GR;               // groups per wave
  static_assert(RQW % GR == 0, "a wave must cover whole quantisation groups");
  static_assert(MR == 1 || KW == 1, "K-stacked waves serve M = 1");
  constexpr int GI = 4 * GR;                  // x items (8 channels) per group
  constexpr int XPT = MR == 1 ? 1 : 4;        // staging items per thread
  __shared__ u32x4 xa[MR][kRowsPerWG];        // x in pair order, one item per qweight row
  __shared__ float xg[MR][NG];                // per-group sums of x
  __shared__ float ytile[KW][MR][kTileN];     // per-K-slice results, for the epilogue mapping
  __shared__ uint32_t xn[XSRC == XSRC_SILU_PART ? kRowsPerWG : 1][4];   // SiLU*up items

  const int wave = wave_id();
  const int wn = wave & 3, wk = wave >> 2;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int lg = lane >> 4, lj = lane & 15;
  const int tile = blockIdx.x, split = blockIdx.y;
  const int N = a.N, M = a.M;
  const int rows_total = a.K >> 3;
  const int row0 = split * kRowsPerWG;
  const int col = tile * kTileN + wn * kWaveN + 4 * lj;
  const bool col_ok = col < N;

  // 1. x items this thread stages: (m, i) = (t/64 + 4j, t%64) for MR = 16, (0, t) for
  //    MR = 1 (threads 0..63).  Raw values now; transformed once the loads are back.
  u32x4 xv[XPT], wv[XSRC == XSRC_RMSNORM ? XPT : 1];
  bool xok[XPT];
  SlotLoad slot_l;                            // XSRC_RMSNORM: the sums of squares of h
  const bool stager = MR > 1 || t < kRowsPerWG;
  auto load_x = [&]() {
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int m = MR == 1 ? 0 : (t >> 6) + 4 * j;
      const int i = MR == 1 ? t : (t & 63);
      const int row = row0 + (i < kRowsPerWG ? i : 0);
      xok[j] = stager && m < M && row < rows_total;
      const int rc = row < rows_total ? row : rows_total - 1;
      const int mc = m < M ? m : M - 1;
      const size_t xoff = (size_t)mc * a.K;
      u32x4 v{0u, 0u, 0u, 0u};
      if (!stager) {
      } else if (XSRC == XSRC_PERM) {
        const u32x4 p0 = *reinterpret_cast<const u32x4*>(a.perm + rc * 8);
        const u32x4 p1 = *reinterpret_cast<const u32x4*>(a.perm + rc * 8 + 4);
        const uint32_t e0 = a.x[xoff + p0.x], e1 = a.x[xoff + p0.y];
        const uint32_t e2 = a.x[xoff + p0.z], e3 = a.x[xoff + p0.w];
        const uint32_t e4 = a.x[xoff + p1.x], e5 = a.x[xoff + p1.y];
        const uint32_t e6 = a.x[xoff + p1.z], e7 = a.x[xoff + p1.w];
        v = u32x4{e0 | (e1 << 16), e2 | (e3 << 16), e4 | (e5 << 16), e6 | (e7 << 16)};
      } else if (XSRC == XSRC_SILU_PART) {
        // staged four threads per item below
      } else if (XSRC == XSRC_RMSNORM) {
        v = *reinterpret_cast<const u32x4*>(a.hn + rc * 8);
        wv[j] = *reinterpret_cast<const u32x4*>(a.wn + rc * 8);
      } else {
        v = *reinterpret_cast<const u32x4*>(a.x + xoff + rc * 8);
      }
      xv[j] = v;
    }
  };
  if (!LATE_X) load_x();
  // SiLU(gate)*up staging (M = 1): thread t computes channels 2*(t%4), +1 of item t/4
  // from the gate|up split-K partials (gate columns contiguous in the 32-column
  // interleave, up columns 32 to the right), summing the splits in order.  The first 8
  // splits are loaded here, ahead of the weight stream.
  const int s_row = row0 + (t >> 2);
  const float* s_pb = nullptr;
  float2 sG[XSRC == XSRC_SILU_PART ? 8 : 1], sU[XSRC == XSRC_SILU_PART ? 8 : 1];
  auto silu_batch = [&](int s0) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int sp = s0 + q < a.xsplits ? s0 + q : a.xsplits - 1;
      sG[q] = *reinterpret_cast<const float2*>(s_pb + (size_t)sp * a.xpart_ld);
      sU[q] = *reinterpret_cast<const float2*>(s_pb + (size_t)sp * a.xpart_ld + 32);
    }
  };
  if (XSRC == XSRC_SILU_PART && t < 4 * kRowsPerWG) {
    const int j0 = (s_row < rows_total ? s_row : rows_total - 1) * 8;
    s_pb = a.xpart + 64 * (j0 >> 5) + (j0 & 31) + 2 * (t & 3);
    silu_batch(0);
  }
  if (XSRC == XSRC_RMSNORM && stager) slot_issue(a.slots, a.K, lane, slot_l);

  // 2. Group metadata of the lane's 4 columns, one entry per group of the split.
  const int colc = col_ok ? col : N - 4;
  const int ngroups = a.K / a.group;
  u32x4 meta[NGW];
#pragma unroll
  for (int g = 0; g < NGW; ++g) {
    int grp = (row0 * 8) / (32 * GR) + wk * NGW + g;
    grp = grp < ngroups ? grp : ngroups - 1;
    if (FMT == MTL_META_QSZ) {
      meta[g] = *reinterpret_cast<const u32x4*>(a.meta0 + ((size_t)grp * N + colc) * 2);
    } else {
      const u32x2 s = *reinterpret_cast<const u32x2*>(a.meta0 + (size_t)grp * N + colc);
      const uint32_t zw = a.qzeros[(size_t)grp * (N >> 3) + (colc >> 3)];
      meta[g] = u32x4{s.x, s.y, zw >> ((colc & 7) * 4), 0u};
    }
  }

  // 3. The weight stream: 16 independent 16-byte buffer loads per lane, uniform row
  //    offset per quad; rows past K/8 and columns past N read 0 through the range check.
  const int splits_total = (rows_total + kRowsPerWG - 1) / kRowsPerWG;
  const __amdgpu_buffer_rsrc_t qrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4*>(a.qweight), (short)0,
      (int)(a.tiled ? (int64_t)splits_total * N * 4 * kRowsPerWG : (int64_t)rows_total * N * 4),
      0x00020000);
  // tiled: the wave's 16 row quads are 16 consecutive 1 KB blocks
  const int tblk = (split * (N / kWaveN) + tile * (kTileN / kWaveN) + wn) * kRowQuads;
  u32x4 wq[RQW];
#pragma unroll
  for (int q = 0; q < RQW; ++q) {
    const int gq = wk * RQW + q;              // row quad within the split
    const int row = row0 + 4 * gq + lg;
    int voff, soff;
    if (a.tiled) {
      voff = col_ok ? lane * 16 : 0x7ffffff0;
      soff = (tblk + gq) * 1024;
    } else {
      voff = (col_ok && row < rows_total) ? (lg * N + col) * 4 : 0x7ffffff0;
      soff = (row0 + 4 * gq) * N * 4;
    }
    wq[q] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qrsrc, voff, soff,
                                                                            kStreamAux));
  }

  if (LATE_X) load_x();
  // Keep the scheduler from hoisting the uses of x above the weight stream: every load
  // of the wave is in flight before the first wait.
  __builtin_amdgcn_sched_barrier(0);

  // 4. x into LDS in pair order, with per-group sums (fixed butterfly order).
  if (XSRC == XSRC_SILU_PART) {
    if (t < 4 * kRowsPerWG) {
      float g0 = 0.f, g1 = 0.f, u0 = 0.f, u1 = 0.f;
      for (int s0 = 0; s0 < a.xsplits; s0 += 8) {
        if (s0 > 0) silu_batch(s0);
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (s0 + q < a.xsplits) {
            g0 += sG[q].x; g1 += sG[q].y;
            u0 += sU[q].x; u1 += sU[q].y;
          }
      }
      xn[t >> 2][t & 3] =
          s_row < rows_total ? silu_mul_bf16(g0, u0) | (silu_mul_bf16(g1, u1) << 16) : 0u;
    }
    __syncthreads();
    if (stager) xv[0] = u32x4{xn[t][0], xn[t][1], xn[t][2], xn[t][3]};
  }
  if (stager) {
    float norm_r = 0.f;
    if (XSRC == XSRC_RMSNORM)     // rsqrt(mean(h^2) + eps) from the slots (one wave)
      norm_r = rsqrtf(wave_sum_valu(slot_finish(slot_l, a.K, lane)) / (float)a.K + a.eps);
#pragma unroll
    for (int j = 0; j < XPT; ++j) {
      const int m = MR == 1 ? 0 : (t >> 6) + 4 * j;
      const int i = MR == 1 ? t : (t & 63);
      u32x4 v = xv[j];
      if (XSRC == XSRC_RMSNORM) v = rmsnorm8(v, wv[j], norm_r);
      if (!xok[j]) v = u32x4{0u, 0u, 0u, 0u};
      float s;
      xa[m][i] = pair_order(v, s);
      s = group_sum_valu<GI>(s);                // every lane of the staging waves active here
      if ((i & (GI - 1)) == 0) xg[m][i / GI] = s;
    }
  }
  __syncthreads();

  // 5. MFMA over the row quads, one quantisation group at a time; per group
  //    y += s * (A - (128 + c) * X) (+ d * X for the qsz contract).
  const uint32_t kMagic = vgpr_const(0x43004300u);   // bf16 (128, 128)
  const uint32_t kLo = vgpr_const(0x000F000Fu);
  constexpr int NR = MR == 1 ? 1 : 4;         // result rows held per lane
  float tot[4][NR];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int r = 0; r < NR; ++r) tot[c][r] = 0.f;
  const int am = MR == 1 ? 0 : lj;            // A operand row of this lane
#pragma unroll
  for (int g = 0; g < NGW; ++g) {
    floatx4 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < GR; ++q) {
      const int rq = g * GR + q;
      const bf16x8_t A = __builtin_bit_cast(bf16x8_t, xa[am][4 * (wk * RQW + rq) + lg]);
      const uint32_t w[4] = {wq[rq].x, wq[rq].y, wq[rq].z, wq[rq].w};
#pragma unroll
      for (int c = 0; c < 4; ++c)
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, unpack_codes8(w[c], kLo, kMagic),
                                                         acc[c], 0, 0, 0);
    }
    float sc[4], cz[4], dz[4];
    if (FMT == MTL_META_QSZ) {
      const uint32_t mw[4] = {meta[g].x, meta[g].y, meta[g].z, meta[g].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        sc[c] = bf16_to_f32(mw[c] & 0xffffu);
        dz[c] = bf16_to_f32(mw[c] >> 16);
        cz[c] = 136.f;   // 128 (bf16 magic) + 8 (offset-binary centre)
      }
    } else {
      sc[0] = f16_to_f32(meta[g].x & 0xffffu);
      sc[1] = f16_to_f32(meta[g].x >> 16);
      sc[2] = f16_to_f32(meta[g].y & 0xffffu);
      sc[3] = f16_to_f32(meta[g].y >> 16);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        cz[c] = (float)(128 + (int)((meta[g].z >> (4 * c)) & 0xfu) + a.zero_offset);
        dz[c] = 0.f;
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const float X = xg[MR == 1 ? 0 : 4 * lg + r][wk * NGW + g];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float tt = fmaf(-cz[c], X, acc[c][r]);
        float v = fmaf(sc[c], tt, tot[c][r]);
        if (FMT == MTL_META_QSZ) v = fmaf(dz[c], X, v);
        tot[c][r] = v;
      }
    }
  }

  // 6. Result tile to LDS, then re-read as 4 consecutive columns per thread: thread t
  //    owns columns tile*256 + 4*(t%64) of rows t/64, t/64 + 4, ...
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int m = MR == 1 ? 0 : 4 * lg + r;
    if ((MR == 1 && lg == 0) || (MR > 1 && m < M))
      *reinterpret_cast<float4*>(&ytile[wk][m][wn * kWaveN + 4 * lj]) =
          make_float4(tot[0][r], tot[1][r], tot[2][r], tot[3][r]);
  }
  __syncthreads();
  constexpr int RPT = MR == 1 ? 1 : 4;        // rows per thread in the epilogue mapping
  const int ecol = tile * kTileN + 4 * lane;
  const bool ecol_ok = ecol < N;
  float v[RPT][4];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int m = wave + 4 * j;
    v[j][0] = v[j][1] = v[j][2] = v[j][3] = 0.f;
    if (m < MR) {
#pragma unroll
      for (int k = 0; k < KW; ++k) {           // K slices summed in order
        const float4 y4 = *reinterpret_cast<const float4*>(&ytile[k][m][4 * lane]);
        v[j][0] += y4.x; v[j][1] += y4.y; v[j][2] += y4.z; v[j][3] += y4.w;
      }
    }
  }
  // MR = 1: wave 0 carries row 0; threads past 255 (KW > 1) only join the barriers
  const bool active = (MR == 1 ? wave == 0 : true) && t < kTileN;

  // 7. Split-K.  Every workgroup publishes its fp32 partial tile.  With an in-kernel
  //    reduction (the residual GEMV with published sums of squares, whose epilogue the
  //    reduce kernel lacks) the partials travel as agent-scope atomic stores, a per-tile
  //    release count names the last workgroup, which acquires and sums all splits in
  //    split order (one column per thread, up to 32 loads in flight) and resets the
  //    counter.  Otherwise w4_reduce_kernel (or a fused consumer) sums them.
  if (a.splits > 1 || a.partials_only) {
    float* pbase = a.partial + (size_t)split * M * N + ecol;
    if (!a.inkernel_reduce || a.partials_only) {
      if (active && ecol_ok) {
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
          const int m = wave + 4 * j;
          if (m < M)
            *reinterpret_cast<float4*>(pbase + (size_t)m * N) =
                make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
        }
      }
      return;
    }
    // publish and reduce one column per thread (threads 0..255), all split loads of a
    // row in flight together; the sums then go through LDS to the epilogue mapping
    const int pc = t & (kTileN - 1);
    const int pcol = tile * kTileN + pc;
    const bool pub = t < kTileN && pcol < N;
    const int mrows = MR < M ? MR : M;
    if (pub) {
      for (int m = 0; m < mrows; ++m) {
        float val = 0.f;
#pragma unroll
        for (int k = 0; k < KW; ++k) val += ytile[k][m][pc];   // as the epilogue mapping sums
        __hip_atomic_store(a.partial + ((size_t)split * M + m) * N + pcol, val, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // release count / acquire fence of the completing workgroup (as in the decode attention)
    __builtin_amdgcn_s_waitcnt(0);   // every partial store acknowledged before the count
    __syncthreads();
    __shared__ int last_flag;
    if (t == 0) {
      last_flag = __hip_atomic_fetch_add(&a.counters[tile], 1u, __ATOMIC_RELEASE,
                                         __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(a.splits - 1);
      if (last_flag) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (!last_flag) return;
    if (t == 0)
      __hip_atomic_store(&a.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int S = a.splits;
    if (pub) {
      for (int m = 0; m < mrows; ++m) {
        const float* q = a.partial + (size_t)m * N + pcol;
        float sum = 0.f;
        for (int s0 = 0; s0 < S; s0 += 32) {
          float pv[32];
#pragma unroll
          for (int jj = 0; jj < 32; ++jj) {
            const int sp = s0 + jj < S ? s0 + jj : S - 1;
            pv[jj] = __hip_atomic_load(q + (size_t)sp * M * N, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
          }
#pragma unroll
          for (int jj = 0; jj < 32; ++jj)
            if (s0 + jj < S) sum += pv[jj];                  // split order
        }
        ytile[0][m][pc] = sum;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int m = wave + 4 * j;
      if (m < MR) {
        const float4 y4 = *reinterpret_cast<const float4*>(&ytile[0][m][4 * lane]);
        v[j][0] = y4.x; v[j][1] = y4.y; v[j][2] = y4.z; v[j][3] = y4.w;
      }
    }
  }
  if (!active) return;

  // 8. Epilogue, 4 consecutive columns per thread.
  if (MR == 1 && a.epilogue == kEpiResidualSlots) {
    // the residual add of fast.py:168-171, publishing what the next RMSNorm needs
    float ss = 0.f;
    if (ecol_ok) {
      const u32x2 rr = *reinterpret_cast<const u32x2*>(a.resid + ecol);
      float hv[4] = {bf16_to_f32(rr.x & 0xffffu), bf16_to_f32(rr.x >> 16),
                     bf16_to_f32(rr.y & 0xffffu), bf16_to_f32(rr.y >> 16)};
#pragma unroll
      for (int c = 0; c < 4; ++c) hv[c] = round_bf16(round_bf16(v[0][c]) + hv[c]);
      *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.y) + ecol) =
          u32x2{f32_to_bf16(hv[0]) | (f32_to_bf16(hv[1]) << 16),
                f32_to_bf16(hv[2]) | (f32_to_bf16(hv[3]) << 16)};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        ss = fmaf(hv[c], hv[c], ss);
        if (a.h_ord)
          a.h_ord[a.scatter ? a.scatter[ecol + c] : ecol + c] = (uint16_t)f32_to_bf16(hv[c]);
      }
    }
    ss = slot_combine(ss);
    if ((lane & 3) == 0 && ecol_ok) a.slots_out[ecol / kSlotCols] = ss;
    return;
  }
  if (a.epilogue == MTL_EPI_SILU_MUL) {
    // Fused columns come in blocks of 64 = 32 gate | 32 up; lane l (l%16 < 8) holds
    // gate columns whose up partners sit 8 lanes higher.
    const int no = N >> 1;
    const int lb = lane & 15;
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int m = wave + 4 * j;
      float u[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) u[c] = __shfl_down(v[j][c], 8);
      if (m < M && ecol_ok && lb < 8) {
        const int o = tile * (kTileN / 2) + (lane >> 4) * 32 + lb * 4;
        uint32_t h[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) h[c] = silu_mul_bf16(v[j][c], u[c]);
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.y) + (size_t)m * no + o) =
            u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
      }
    }
  } else if (ecol_ok) {
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
      const int m = wave + 4 * j;
      if (m >= M) continue;
      const size_t o = (size_t)m * N + ecol;
      float y[4] = {v[j][0], v[j][1], v[j][2], v[j][3]};
      if (a.epilogue == MTL_EPI_RESIDUAL) {
        const u32x2 rr = *reinterpret_cast<const u32x2*>(a.resid + o);
        y[0] = round_bf16(y[0]) + bf16_to_f32(rr.x & 0xffffu);
        y[1] = round_bf16(y[1]) + bf16_to_f32(rr.x >> 16);
        y[2] = round_bf16(y[2]) + bf16_to_f32(rr.y & 0xffffu);
        y[3] = round_bf16(y[3]) + bf16_to_f32(rr.y >> 16);
      }
      if (a.out_f32) {
        *reinterpret_cast<float4*>(static_cast<float*>(a.y) + o) = make_float4(y[0], y[1], y[2], y[3]);
      } else {
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.y) + o) =
            u32x2{f32_to_bf16(y[0]) | (f32_to_bf16(y[1]) << 16),
                  f32_to_bf16(y[2]) | (f32_to_bf16(y[3]) << 16)};
      }
    }
  }
}

// Sum the split-K partial tiles in split order and apply the epilogue.  One thread
// per 4 consecutive output columns of one row (for SILU_MUL: 4 gate columns and their
// 4 up partners 32 columns to the right).
__global__ void __launch_bounds__(256) w4_reduce_kernel(W4Args a) {
  const int N = a.N, M = a.M;
  const int S = a.splits;
  const int quads = (a.epilogue == MTL_EPI_SILU_MUL) ? N / 8 : N / 4;
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= M * quads) return;
  const int m = t / quads;
  const int q = t - m * quads;
  if (a.epilogue == MTL_EPI_SILU_MUL) {
    // quad q covers gate columns 64*(q/8) + 4*(q%8) .. +3, up columns +32
    const int col = 64 * (q >> 3) + 4 * (q & 7);
    float g[4] = {0.f, 0.f, 0.f, 0.f}, u[4] = {0.f, 0.f, 0.f, 0.f};
    const float* base = a.partial + (size_t)m * N + col;
    const size_t stride = (size_t)M * N;
    for (int s0 = 0; s0 < S; s0 += 8) {   // 8 independent loads in flight, summed in order
      float4 vg[8], vu[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int sp = s0 + j < S ? s0 + j : S - 1;
        vg[j] = ld_f4(base + sp * stride);
        vu[j] = ld_f4(base + sp * stride + 32);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < S) {
          g[0] += vg[j].x; g[1] += vg[j].y; g[2] += vg[j].z; g[3] += vg[j].w;
          u[0] += vu[j].x; u[1] += vu[j].y; u[2] += vu[j].z; u[3] += vu[j].w;
        }
    }
    const int o = 32 * (q >> 3) + 4 * (q & 7);
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.y) + (size_t)m * (N / 2) + o) =
        u32x2{silu_mul_bf16(g[0], u[0]) | (silu_mul_bf16(g[1], u[1]) << 16),
              silu_mul_bf16(g[2], u[2]) | (silu_mul_bf16(g[3], u[3]) << 16)};
    return;
  }
  const int col = 4 * q;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  const float* base = a.partial + (size_t)m * N + col;
  const size_t stride = (size_t)M * N;
  for (int s0 = 0; s0 < S; s0 += 8) {   // 8 independent loads in flight, summed in order
    float4 p[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) p[j] = ld_f4(base + (s0 + j < S ? s0 + j : S - 1) * stride);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (s0 + j < S) { v[0] += p[j].x; v[1] += p[j].y; v[2] += p[j].z; v[3] += p[j].w; }
  }
  const size_t o = (size_t)m * N + col;
  if (a.epilogue == MTL_EPI_RESIDUAL) {
    const u32x2 rr = *reinterpret_cast<const u32x2*>(a.resid + o);
    v[0] = round_bf16(v[0]) + bf16_to_f32(rr.x & 0xffffu);
    v[1] = round_bf16(v[1]) + bf16_to_f32(rr.x >> 16);
    v[2] = round_bf16(v[2]) + bf16_to_f32(rr.y & 0xffffu);
    v[3] = round_bf16(v[3]) + bf16_to_f32(rr.y >> 16);
  }
  if (a.out_f32) {
    *reinterpret_cast<float4*>(static_cast<float*>(a.y) + o) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.y) + o) =
        u32x2{f32_to_bf16(v[0]) | (f32_to_bf16(v[1]) << 16),
              f32_to_bf16(v[2]) | (f32_to_bf16(v[3]) << 16)};
  }
}

// ----------------------------------------------------------------------------
// Launch planning
// ----------------------------------------------------------------------------

struct Plan {
  int splits, col_tiles, kw;
};

// kw > 1 (waves stacked along K) for M = 1, so small shapes still put about 2 waves on
// every SIMD; a wave must cover whole groups.  Every M = 1 launch of a shape (partials
// only or reduced in the kernel) uses the same kw, so their sums agree bit for bit.
static Plan plan_for(int64_t K, int64_t N, int64_t M = 1, int group = 128) {
  Plan p;
  const int rows = (int)(K / 8);
  p.splits = (rows + kRowsPerWG - 1) / kRowsPerWG;
  p.col_tiles = (int)((N + kTileN - 1) / kTileN);
  p.kw = 1;
  const int64_t waves = (int64_t)p.splits * p.col_tiles * 4;
  if (M == 1 && waves < 1536) {   // measured: stacking does not pay from 1536 waves up
    const int gr = group / 32;
    while (p.kw < 4 && waves * p.kw < 2048 && (kRowQuads / (2 * p.kw)) % gr == 0) p.kw *= 2;
  }
  return p;
}

// Workspace = a fixed tile-counter region (so partial tiles of one shape never land on
// another shape's counters) followed by the fp32 partial tiles [splits, M, N].
constexpr int64_t kCounterBytes = 16384;   // 4096 column tiles: N <= 1M

template <int MR, int GR, int KW>
static void launch_fmt(const W4Args& a, int fmt, dim3 grid, hipStream_t s) {
  const dim3 block(256 * KW);
  if (fmt == MTL_META_QSZ)
    hipLaunchKernelGGL((w4_gemm_kernel<MR, GR, MTL_META_QSZ, XSRC_BF16, KW>), grid, block, 0, s, a);
  else if (a.xpart)
    hipLaunchKernelGGL((w4_gemm_kernel<1, GR, MTL_META_GPTQ, XSRC_SILU_PART, KW>), grid, block, 0, s, a);
  else if (a.hn)
    hipLaunchKernelGGL((w4_gemm_kernel<1, GR, MTL_META_GPTQ, XSRC_RMSNORM, KW>), grid, block, 0, s, a);
  else if (a.perm)
    hipLaunchKernelGGL((w4_gemm_kernel<MR, GR, MTL_META_GPTQ, XSRC_PERM, KW>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((w4_gemm_kernel<MR, GR, MTL_META_GPTQ, XSRC_BF16, KW>), grid, block, 0, s, a);
}

template <int MR, int GR>
static void launch_kw(const W4Args& a, int fmt, int kw, dim3 grid, hipStream_t s) {
  if constexpr (MR == 1) {
    if (kw == 4) {
      if constexpr (kRowQuads / 4 % GR == 0) { launch_fmt<MR, GR, 4>(a, fmt, grid, s); return; }
    } else if (kw == 2) {
      if constexpr (kRowQuads / 2 % GR == 0) { launch_fmt<MR, GR, 2>(a, fmt, grid, s); return; }
    }
  }
  launch_fmt<MR, GR, 1>(a, fmt, grid, s);
}

// Row quads per quantisation group: group / 32.
template <int MR>
static void launch_gr(const W4Args& a, int fmt, int kw, dim3 grid, hipStream_t s) {
  switch (a.group) {
    case 32: launch_kw<MR, 1>(a, fmt, kw, grid, s); break;
    case 64: launch_kw<MR, 2>(a, fmt, kw, grid, s); break;
    case 128: launch_kw<MR, 4>(a, fmt, kw, grid, s); break;
    default: launch_kw<MR, 8>(a, fmt, kw, grid, s); break;
  }
}

static void launch_w4(const W4Args& a, int fmt, const Plan& p, hipStream_t s) {
  const dim3 grid(p.col_tiles, p.splits);
  if (a.M == 1) launch_gr<1>(a, fmt, p.kw, grid, s);
  else launch_gr<16>(a, fmt, 1, grid, s);
}

// The buffer descriptor's size and offsets are 32-bit: the weight rows of the last
// split (up to 64 past K/8) must stay addressable.
static bool weight_fits(int64_t K, int64_t N) {
  return (K / 8 + kRowsPerWG) * N * 4 < ((int64_t)1 << 31);
}

static W4Args blank_args() {
  W4Args a;
  a.x = nullptr;
  a.qweight = nullptr;
  a.meta0 = nullptr;
  a.qzeros = nullptr;
  a.perm = nullptr;
  a.xpart = nullptr;
  a.xsplits = 0;
  a.xpart_ld = 0;
  a.hn = nullptr;
  a.wn = nullptr;
  a.slots = nullptr;
  a.eps = 0.f;
  a.h_ord = nullptr;
  a.scatter = nullptr;
  a.slots_out = nullptr;
  a.tiled = 0;
  a.resid = nullptr;
  a.y = nullptr;
  a.partial = nullptr;
  a.counters = nullptr;
  a.inkernel_reduce = 0;
  a.partials_only = 0;
  a.M = a.K = a.N = a.group = a.zero_offset = a.splits = a.epilogue = a.out_f32 = 0;
  return a;
}

static int w4_gemm(const void* x, int64_t M, int64_t K, const int32_t* qweight, int fmt,
                   const void* meta0, const int32_t* qzeros, const int32_t* perm, int64_t N,
                   int group, int zero_offset, int epilogue, const void* resid, void* y,
                   int out_dtype, void* workspace, int64_t ws_bytes, hipStream_t stream) {
  if (!x || !qweight || !meta0 || !y) return MTL_ERR_INVALID_ARG;
  if (fmt != MTL_META_GPTQ && fmt != MTL_META_QSZ) return MTL_ERR_INVALID_ARG;
  if (fmt == MTL_META_GPTQ && !qzeros) return MTL_ERR_INVALID_ARG;
  if (epilogue < MTL_EPI_NONE || epilogue > MTL_EPI_SILU_MUL) return MTL_ERR_INVALID_ARG;
  if (out_dtype != MTL_OUT_BF16 && out_dtype != MTL_OUT_F32) return MTL_ERR_INVALID_ARG;
  if (epilogue == MTL_EPI_RESIDUAL && !resid) return MTL_ERR_INVALID_ARG;
  if (epilogue != MTL_EPI_NONE && out_dtype != MTL_OUT_BF16) return MTL_ERR_INVALID_ARG;
  if (group != 32 && group != 64 && group != 128 && group != 256) return MTL_ERR_GROUP;
  if (M < 1 || M > kMaxM || K <= 0 || N <= 0) return MTL_ERR_SHAPE;
  if (K % group != 0 || N % 8 != 0) return MTL_ERR_SHAPE;
  if (epilogue == MTL_EPI_SILU_MUL && N % 64 != 0) return MTL_ERR_SHAPE;
  if ((N + kTileN - 1) / kTileN > kCounterBytes / 4) return MTL_ERR_SHAPE;
  if (!weight_fits(K, N) || M * K >= ((int64_t)1 << 31)) return MTL_ERR_SHAPE;
  if (!aligned16(qweight) || !aligned16(x) || (perm && !aligned16(perm))) return MTL_ERR_ALIGN;
  if (perm && fmt != MTL_META_GPTQ) return MTL_ERR_INVALID_ARG;
  if (fmt == MTL_META_QSZ && !aligned16(meta0)) return MTL_ERR_ALIGN;
  if (fmt == MTL_META_GPTQ && (reinterpret_cast<uintptr_t>(meta0) & 7u)) return MTL_ERR_ALIGN;

  const Plan p = plan_for(K, N, M, group);
  W4Args a = blank_args();
  a.x = static_cast<const uint16_t*>(x);
  a.qweight = reinterpret_cast<const u32x4*>(qweight);
  a.meta0 = static_cast<const uint16_t*>(meta0);
  a.qzeros = reinterpret_cast<const uint32_t*>(qzeros);
  a.perm = perm;
  a.resid = static_cast<const uint16_t*>(resid);
  a.y = y;
  a.M = (int)M; a.K = (int)K; a.N = (int)N;
  a.group = group; a.zero_offset = zero_offset;
  a.splits = p.splits;
  a.epilogue = epilogue;
  a.out_f32 = out_dtype == MTL_OUT_F32;
  // Split-K partials are summed by w4_reduce_kernel, a second launch: the kernel boundary
  // makes them visible without an agent-scope release (an L2 write-back) in each of the
  // hundreds of workgroups, which made the last-workgroup reduction 2.4x slower at M = 1 on
  // gate|up (34.6 against 14.4 us) and 2x at M = 16 (46.0 against 22.4 us).
  a.inkernel_reduce = 0;
  if (p.splits > 1) {
    const int64_t need = kCounterBytes + (int64_t)p.splits * M * N * 4;
    if (!workspace || ws_bytes < need) return MTL_ERR_WORKSPACE;
    if (!aligned16(workspace)) return MTL_ERR_ALIGN;
    a.counters = static_cast<unsigned*>(workspace);
    a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  }
  launch_w4(a, fmt, p, stream);
  if (p.splits > 1 && !a.inkernel_reduce) {
    const int quads = (int)(M * (epilogue == MTL_EPI_SILU_MUL ? N / 8 : N / 4));
    hipLaunchKernelGGL(w4_reduce_kernel, dim3((quads + 255) / 256), dim3(256), 0, stream, a);
  }
  return launch_status();
}

// Partials-only launch for fused consumers: writes fp32 [splits, M, N] into `partials`
// (splits = w4_splits(K)); x comes from `x` (bf16, optionally through `perm`) or, when
// `xpart` is set, from the gate|up partials of the previous GEMV (SiLU*up, M = 1).
static bool is_strip(int layout) {
  return layout == MTL_LAYOUT_STRIP || layout == MTL_LAYOUT_STRIP_QSZ;
}

static int check_layout(int layout, int64_t M, int64_t K, int64_t N, const int32_t* perm,
                        int group) {
  if (layout != MTL_LAYOUT_ROWS && layout != MTL_LAYOUT_TILED && !is_strip(layout))
    return MTL_ERR_INVALID_ARG;
  if (layout == MTL_LAYOUT_TILED && (N % kWaveN != 0 || M != 1 || perm)) return MTL_ERR_SHAPE;
  if (is_strip(layout) &&
      (M != 1 || perm || N <= 0 || N % 16 != 0 || K > 16384 ||
       !strip_blocks_per_wave(K, 1, group) ||
       N * K / 2 >= ((int64_t)1 << 31)))
    return MTL_ERR_SHAPE;
  return MTL_OK;
}

// The strip GEMV reads 16 scales (32 B) and 16 zero nibbles (8 B) of a strip at a time
// (GPTQ metadata), or one 4-byte (scale, zero) pair per lane (the reference's qsz).
static bool strip_meta_aligned(int layout, const void* scales, const int32_t* qzeros) {
  if (layout == MTL_LAYOUT_STRIP_QSZ) return (reinterpret_cast<uintptr_t>(scales) & 3u) == 0;
  return aligned16(scales) && (reinterpret_cast<uintptr_t>(qzeros) & 7u) == 0;
}

// The metadata pointers a layout needs: qzeros is unused with the reference's qsz.
static bool meta_given(int layout, const void* meta0, const int32_t* qzeros) {
  return meta0 && (qzeros || layout == MTL_LAYOUT_STRIP_QSZ);
}

// The strip GEMV's arguments common to every entry point.
static StripArgs strip_args(int64_t K, const int32_t* w, const void* scales,
                            const int32_t* qzeros, int64_t N, int group, int zero_offset,
                            int layout = MTL_LAYOUT_STRIP) {
  StripArgs a;
  a.fmt = layout == MTL_LAYOUT_STRIP_QSZ ? STRIP_META_QSZ : STRIP_META_GPTQ;
  a.y16 = nullptr;
  a.w = reinterpret_cast<const u32x4*>(w);
  a.scales = static_cast<const uint16_t*>(scales);
  a.qzeros = reinterpret_cast<const uint32_t*>(qzeros);
  a.x = nullptr;
  a.perm = nullptr;
  a.xpart = nullptr;
  a.xhalves = 0;
  a.xsplits = 0;
  a.xpart_ld = 0;
  a.hn = a.wn = nullptr;
  a.slots = nullptr;
  a.eps = 0.f;
  a.y = nullptr;
  a.h = nullptr;
  a.scatter = nullptr;
  a.h_ord = nullptr;
  a.slots_out = nullptr;
  a.act = nullptr;
  a.K = (int)K; a.N = (int)N;
  a.group = group; a.zero_offset = zero_offset;
  a.kblocks = 0;
  a.xcd_order = 0;
  a.geom = mtl_strip_geometry{0, 0, 0, 0};
  return a;
}

static int w4_gemm_partials(const void* x, const float* xpart, int xsplits, int64_t xpart_ld,
                            int64_t M, int64_t K, const int32_t* qweight, const void* meta0,
                            const int32_t* qzeros, const int32_t* perm, int64_t N, int group,
                            int zero_offset, int layout, float* partials, int64_t partials_bytes,
                            hipStream_t stream, const mtl_strip_geometry* geom = nullptr) {
  if (const int st = check_layout(layout, M, K, N, perm, group)) return st;
  if ((!x && !xpart) || (x && xpart) || !qweight || !meta_given(layout, meta0, qzeros) ||
      !partials)
    return MTL_ERR_INVALID_ARG;
  if (group != 32 && group != 64 && group != 128 && group != 256) return MTL_ERR_GROUP;
  if (M < 1 || M > kMaxM || K <= 0 || N <= 0 || K % group != 0 || N % 8 != 0)
    return MTL_ERR_SHAPE;
  if (!weight_fits(K, N) || M * K >= ((int64_t)1 << 31)) return MTL_ERR_SHAPE;
  if (xpart) {
    if (M != 1) return MTL_ERR_UNSUPPORTED;
    if (perm) return MTL_ERR_INVALID_ARG;
    if (xsplits < 1 || xpart_ld != 2 * K) return MTL_ERR_SHAPE;
    if (!aligned16(xpart)) return MTL_ERR_ALIGN;
  } else if (!aligned16(x)) {
    return MTL_ERR_ALIGN;
  }
  if (!aligned16(qweight) || !aligned16(partials) || (perm && !aligned16(perm)))
    return MTL_ERR_ALIGN;
  if (is_strip(layout)) {   // full-K strips: the final sums, as one split
    if (partials_bytes < N * 4) return MTL_ERR_WORKSPACE;
    if (!strip_meta_aligned(layout, meta0, qzeros)) return MTL_ERR_ALIGN;
    StripArgs sa = strip_args(K, qweight, meta0, qzeros, N, group, zero_offset, layout);
    sa.x = static_cast<const uint16_t*>(x);
    sa.xpart = xpart;
    sa.xsplits = xsplits;
    sa.xpart_ld = (int)xpart_ld;
    sa.y = partials;
    if (geom) sa.geom = *geom;
    return strip_launch(sa, stream);
  }
  if (reinterpret_cast<uintptr_t>(meta0) & 7u) return MTL_ERR_ALIGN;
  const Plan p = plan_for(K, N, M, group);
  if (partials_bytes < (int64_t)p.splits * M * N * 4) return MTL_ERR_WORKSPACE;
  W4Args a = blank_args();
  a.x = static_cast<const uint16_t*>(x);
  a.qweight = reinterpret_cast<const u32x4*>(qweight);
  a.meta0 = static_cast<const uint16_t*>(meta0);
  a.qzeros = reinterpret_cast<const uint32_t*>(qzeros);
  a.perm = perm;
  a.xpart = xpart;
  a.xsplits = xsplits;
  a.xpart_ld = (int)xpart_ld;
  a.partial = partials;
  a.tiled = layout == MTL_LAYOUT_TILED;
  a.M = (int)M; a.K = (int)K; a.N = (int)N;
  a.group = group; a.zero_offset = zero_offset;
  a.splits = p.splits;
  a.epilogue = MTL_EPI_NONE;
  a.out_f32 = 1;
  a.partials_only = 1;
  launch_w4(a, MTL_META_GPTQ, p, stream);
  return launch_status();
}

// Partials-only launch whose input is RMSNorm(h) computed while staging (M = 1).
// Arguments of the RMSNorm-staged GEMV; for the strip layout also its launch arguments.
static int norm_partials_check(const void* h_ord, const void* w_ord, const float* slots,
                               float eps, int64_t K, const int32_t* qweight, const void* meta0,
                               const int32_t* qzeros, int64_t N, int group, int zero_offset,
                               int layout, float* partials, int64_t partials_bytes,
                               StripArgs* sa) {
  if (const int st = check_layout(layout, 1, K, N, nullptr, group)) return st;
  if (!h_ord || !w_ord || !slots || !qweight || !meta_given(layout, meta0, qzeros) || !partials)
    return MTL_ERR_INVALID_ARG;
  if (group != 32 && group != 64 && group != 128 && group != 256) return MTL_ERR_GROUP;
  if (K <= 0 || N <= 0 || K % group != 0 || N % 8 != 0) return MTL_ERR_SHAPE;
  if (!aligned16(slots)) return MTL_ERR_ALIGN;
  if (!weight_fits(K, N) || K > (int64_t)kSlotCols * kMaxSlots) return MTL_ERR_SHAPE;
  if (!aligned16(h_ord) || !aligned16(w_ord) || !aligned16(qweight) || !aligned16(partials))
    return MTL_ERR_ALIGN;
  if (is_strip(layout)) {   // full-K strips: the final sums, as one split
    if (partials_bytes < N * 4) return MTL_ERR_WORKSPACE;
    if (!strip_meta_aligned(layout, meta0, qzeros)) return MTL_ERR_ALIGN;
    *sa = strip_args(K, qweight, meta0, qzeros, N, group, zero_offset, layout);
    sa->hn = static_cast<const uint16_t*>(h_ord);
    sa->wn = static_cast<const uint16_t*>(w_ord);
    sa->slots = slots;
    sa->eps = eps;
    sa->y = partials;
  }
  return MTL_OK;
}

static int w4_gemm_norm_partials(const void* h_ord, const void* w_ord, const float* slots,
                                 float eps, int64_t K, const int32_t* qweight,
                                 const void* meta0, const int32_t* qzeros, int64_t N, int group,
                                 int zero_offset, int layout, float* partials,
                                 int64_t partials_bytes, hipStream_t stream,
                                 const mtl_strip_geometry* geom = nullptr) {
  StripArgs sa;
  if (const int st = norm_partials_check(h_ord, w_ord, slots, eps, K, qweight, meta0, qzeros, N,
                                         group, zero_offset, layout, partials, partials_bytes,
                                         &sa))
    return st;
  if (is_strip(layout)) {
    if (geom) sa.geom = *geom;
    return strip_launch(sa, stream);
  }
  if (reinterpret_cast<uintptr_t>(meta0) & 7u) return MTL_ERR_ALIGN;
  const Plan p = plan_for(K, N, 1, group);
  if (partials_bytes < (int64_t)p.splits * N * 4) return MTL_ERR_WORKSPACE;
  W4Args a = blank_args();
  a.qweight = reinterpret_cast<const u32x4*>(qweight);
  a.meta0 = static_cast<const uint16_t*>(meta0);
  a.qzeros = reinterpret_cast<const uint32_t*>(qzeros);
  a.hn = static_cast<const uint16_t*>(h_ord);
  a.wn = static_cast<const uint16_t*>(w_ord);
  a.slots = slots;
  a.eps = eps;
  a.partial = partials;
  a.tiled = layout == MTL_LAYOUT_TILED;
  a.M = 1; a.K = (int)K; a.N = (int)N;
  a.group = group; a.zero_offset = zero_offset;
  a.splits = p.splits;
  a.epilogue = MTL_EPI_NONE;
  a.out_f32 = 1;
  a.partials_only = 1;
  launch_w4(a, MTL_META_GPTQ, p, stream);
  return launch_status();
}

// M = 1 GEMV whose epilogue is the decode step's residual add (reduced in the kernel):
// h = bf16(bf16(x @ W) + h); h_ord[scatter[n]] = h[n]; slots[b] = sum of h^2 over columns
// 16b..16b+15.  x from `x` (bf16) or the gate|up partials (`xpart`, SiLU*up).  With the
// strip layout the full-K strip GEMV runs instead: no workspace, no split-K.
static int w4_gemm_residual(const void* x, const float* xpart, int xsplits, int64_t xpart_ld,
                            int64_t K, const int32_t* qweight, const void* meta0,
                            const int32_t* qzeros, int64_t N, int group, int zero_offset,
                            int layout, void* h, const int32_t* scatter, void* h_ord,
                            float* slots, void* workspace, int64_t ws_bytes,
                            hipStream_t stream, const mtl_strip_geometry* geom = nullptr) {
  if ((!x && !xpart) || (x && xpart) || !qweight || !meta_given(layout, meta0, qzeros) || !h ||
      !slots)
    return MTL_ERR_INVALID_ARG;
  const bool halves = xpart && (xsplits & MTL_XPART_HALVES);
  if (xpart) xsplits &= ~MTL_XPART_HALVES;
  if (halves && !is_strip(layout)) return MTL_ERR_UNSUPPORTED;
  if (const int st = check_layout(layout, 1, K, N, nullptr, group)) return st;
  if (group != 32 && group != 64 && group != 128 && group != 256) return MTL_ERR_GROUP;
  if (K <= 0 || N <= 0 || K % group != 0 || N % 8 != 0) return MTL_ERR_SHAPE;
  if (N > (int64_t)kSlotCols * kMaxSlots) return MTL_ERR_SHAPE;
  if (!weight_fits(K, N)) return MTL_ERR_SHAPE;
  if (xpart) {
    if (xsplits < 1 || xpart_ld != 2 * K) return MTL_ERR_SHAPE;
    if (!aligned16(xpart)) return MTL_ERR_ALIGN;
  } else if (!aligned16(x)) {
    return MTL_ERR_ALIGN;
  }
  if (!aligned16(qweight) || (reinterpret_cast<uintptr_t>(h) & 7u)) return MTL_ERR_ALIGN;
  if (is_strip(layout)) {
    if (!aligned16(slots) || (scatter && !aligned16(scatter)) ||
        !strip_meta_aligned(layout, meta0, qzeros))
      return MTL_ERR_ALIGN;
    StripArgs sa = strip_args(K, qweight, meta0, qzeros, N, group, zero_offset, layout);
    sa.x = static_cast<const uint16_t*>(x);
    sa.xpart = xpart;
    sa.xsplits = xsplits;
    sa.xpart_ld = (int)xpart_ld;
    sa.xhalves = halves;
    sa.h = static_cast<uint16_t*>(h);
    sa.scatter = scatter;
    sa.h_ord = static_cast<uint16_t*>(h_ord);
    sa.slots_out = slots;
    if (geom) sa.geom = *geom;
    return strip_launch(sa, stream);
  }
  if (reinterpret_cast<uintptr_t>(meta0) & 7u) return MTL_ERR_ALIGN;
  const Plan p = plan_for(K, N, 1, group);
  W4Args a = blank_args();
  if (p.splits > 1) {
    const int64_t need = kCounterBytes + (int64_t)p.splits * N * 4;
    if (!workspace || ws_bytes < need) return MTL_ERR_WORKSPACE;
    if (!aligned16(workspace)) return MTL_ERR_ALIGN;
    a.counters = static_cast<unsigned*>(workspace);
    a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  }
  a.x = static_cast<const uint16_t*>(x);
  a.qweight = reinterpret_cast<const u32x4*>(qweight);
  a.meta0 = static_cast<const uint16_t*>(meta0);
  a.qzeros = reinterpret_cast<const uint32_t*>(qzeros);
  a.xpart = xpart;
  a.xsplits = xsplits;
  a.xpart_ld = (int)xpart_ld;
  a.resid = static_cast<const uint16_t*>(h);
  a.y = h;
  a.h_ord = static_cast<uint16_t*>(h_ord);
  a.scatter = scatter;
  a.slots_out = slots;
  a.tiled = layout == MTL_LAYOUT_TILED;
  a.M = 1; a.K = (int)K; a.N = (int)N;
  a.group = group; a.zero_offset = zero_offset;
  a.splits = p.splits;
  a.epilogue = kEpiResidualSlots;
  a.out_f32 = 0;
  a.inkernel_reduce = 1;
  launch_w4(a, MTL_META_GPTQ, p, stream);
  return launch_status();
}

// M = 1 gate|up GEMV with RMSNorm staging whose epilogue is SiLU(gate)*up (strip layout
// only): act[j] = bf16(silu(bf16 gate_j) * bf16 up_j), columns in 32-column gate|up blocks.
static int w4_gemm_norm_silu(const void* h_ord, const void* w_ord, const float* slots, float eps,
                             int64_t K, const int32_t* qweight, const void* meta0,
                             const int32_t* qzeros, int64_t N, int group, int zero_offset,
                             int layout, void* act, hipStream_t stream,
                             const mtl_strip_geometry* geom = nullptr) {
  if (!h_ord || !w_ord || !slots || !qweight || !meta_given(layout, meta0, qzeros) || !act)
    return MTL_ERR_INVALID_ARG;
  if (!is_strip(layout)) return MTL_ERR_UNSUPPORTED;
  if (group != 32 && group != 64 && group != 128 && group != 256) return MTL_ERR_GROUP;
  if (K <= 0 || N <= 0 || K % group != 0 || N % 64 != 0 || K > 16384 ||
      (!geom && !strip_blocks_per_wave(K, 2, group)) ||
      N * K / 2 >= ((int64_t)1 << 31) || K > (int64_t)kSlotCols * kMaxSlots)
    return MTL_ERR_SHAPE;
  if (!aligned16(slots) || !aligned16(h_ord) || !aligned16(w_ord) || !aligned16(qweight) ||
      (reinterpret_cast<uintptr_t>(act) & 7u) || !strip_meta_aligned(layout, meta0, qzeros))
    return MTL_ERR_ALIGN;
  StripArgs sa = strip_args(K, qweight, meta0, qzeros, N, group, zero_offset, layout);
  sa.hn = static_cast<const uint16_t*>(h_ord);
  sa.wn = static_cast<const uint16_t*>(w_ord);
  sa.slots = slots;
  sa.eps = eps;
  sa.act = static_cast<uint16_t*>(act);
  if (geom) sa.geom = *geom;
  return strip_launch(sa, stream);
}

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

}  // namespace mtl

using namespace mtl;

extern "C" {

const char* mtl_status_string(int status) {
  switch (status) {
    case MTL_OK: return "ok";
    case MTL_ERR_INVALID_ARG: return "invalid argument";
    case MTL_ERR_SHAPE: return "invalid shape";
    case MTL_ERR_GROUP: return "unsupported group size";
    case MTL_ERR_ALIGN: return "misaligned pointer";
    case MTL_ERR_WORKSPACE: return "workspace missing or too small";
    case MTL_ERR_LAUNCH: return "HIP launch failure";
    case MTL_ERR_UNSUPPORTED: return "unsupported request";
    default: return "unknown status";
  }
}

int mtl_abi_version(void) { return 1; }

int64_t mtl_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int32_t group_size) {
  if (M < 1 || M > kMaxM || K <= 0 || N <= 0 || K % 8 != 0) return 0;
  (void)group_size;
  const int64_t splits = (K / 8 + kRowsPerWG - 1) / kRowsPerWG;
  return kCounterBytes + splits * M * N * 4;
}

int mtl_workspace_init(void* workspace, int64_t ws_bytes, void* stream) {
  if (!workspace || ws_bytes <= 0 || (ws_bytes & 3)) return MTL_ERR_INVALID_ARG;
  const int64_t n = ws_bytes / 4;
  int blocks = (int)((n + 255) / 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     static_cast<uint32_t*>(workspace), n, 0u);
  return launch_status();
}

int32_t mtl_w4_gemm_splits(int64_t K, int64_t N) {
  if (K <= 0 || N <= 0 || K % 8 != 0) return 0;
  return plan_for(K, N).splits;
}

int mtl_w4_gemv_strip(const void* x, int64_t K, const uint16_t* perm,
                      const int32_t* strip_weight, const void* strip_scales,
                      const int32_t* strip_zeros, int64_t N, int32_t group_size,
                      int32_t zero_offset, int32_t out_dtype, void* y, void* stream) {
  if (!x || !strip_weight || !strip_scales || !strip_zeros || !y) return MTL_ERR_INVALID_ARG;
  if (out_dtype != MTL_OUT_BF16 && out_dtype != MTL_OUT_F32) return MTL_ERR_INVALID_ARG;
  if (group_size != 32 && group_size != 64 && group_size != 128 && group_size != 256)
    return MTL_ERR_GROUP;
  if (K <= 0 || N <= 0 || K % 256 != 0 || N % 16 != 0 || K % group_size != 0 ||
      K > (perm ? 12288 : 16384) || N * K / 2 >= ((int64_t)1 << 31) ||
      !strip_blocks_per_wave(K, 1, group_size))
    return MTL_ERR_SHAPE;
  if (!aligned16(x) || (perm && !aligned16(perm)) || !aligned16(strip_weight) ||
      !strip_meta_aligned(MTL_LAYOUT_STRIP, strip_scales, strip_zeros) ||
      (reinterpret_cast<uintptr_t>(y) & (out_dtype == MTL_OUT_F32 ? 15u : 7u)))
    return MTL_ERR_ALIGN;
  StripArgs sa = strip_args(K, strip_weight, strip_scales, strip_zeros, N, group_size,
                            zero_offset);
  sa.x = static_cast<const uint16_t*>(x);
  sa.perm = perm;
  if (out_dtype == MTL_OUT_F32) sa.y = static_cast<float*>(y);
  else sa.y16 = static_cast<uint16_t*>(y);
  return strip_launch(sa, (hipStream_t)stream);
}

int mtl_w4_gemm_partials(const void* x, const float* xpart, int32_t xsplits, int64_t xpart_ld,
                         int64_t M, int64_t K, const int32_t* qweight, const void* scales,
                         const int32_t* qzeros, const int32_t* perm, int64_t N, int32_t group_size,
                         int32_t zero_offset, int32_t layout, float* partials,
                         int64_t partials_bytes, void* stream) {
  return w4_gemm_partials(x, xpart, xsplits, xpart_ld, M, K, qweight, scales, qzeros, perm, N,
                          group_size, zero_offset, layout, partials, partials_bytes,
                          (hipStream_t)stream);
}

int mtl_w4_gemm_norm_partials(const void* h, const void* w, const float* slots, float eps,
                              int64_t K, const int32_t* qweight, const void* scales,
                              const int32_t* qzeros, int64_t N, int32_t group_size,
                              int32_t zero_offset, int32_t layout, float* partials,
                              int64_t partials_bytes, void* stream) {
  return w4_gemm_norm_partials(h, w, slots, eps, K, qweight, scales, qzeros, N,
                               group_size, zero_offset, layout, partials, partials_bytes,
                               (hipStream_t)stream);
}

int mtl_w4_gemm_norm_partials_bf16(const void* h, const void* w, const float* slots, float eps,
                                   int64_t K, const int32_t* qweight, const void* scales,
                                   const int32_t* qzeros, int64_t N, int32_t group_size,
                                   int32_t zero_offset, int32_t layout, float* partials,
                                   int64_t partials_bytes, const void* bh, const void* bnorm_w,
                                   const void* bweight, int64_t bn, float* bout, void* stream) {
  if (!bh || !bnorm_w || !bweight || !bout) return MTL_ERR_INVALID_ARG;
  if (bn < 1 || K % 8 != 0) return MTL_ERR_SHAPE;
  if (!aligned16(bh) || !aligned16(bnorm_w) || !aligned16(bweight)) return MTL_ERR_ALIGN;
  StripArgs sa;
  if (const int st = norm_partials_check(h, w, slots, eps, K, qweight, scales, qzeros, N,
                                         group_size, zero_offset, layout, partials,
                                         partials_bytes, &sa))
    return st;
  if (is_strip(layout) && K <= 4096) {   // one launch where its shape applies
    const int rpw = bf16_rows_per_wg(bn, gemm_device_cus());
    const int64_t gb = (bn + rpw - 1) / rpw;
    if (gb + N / 16 < ((int64_t)1 << 31) && (int64_t)rpw * K * 2 < ((int64_t)1 << 31)) {
      const Bf16RowsArgs b{static_cast<const uint16_t*>(bh), static_cast<const uint16_t*>(bnorm_w),
                           slots, eps, static_cast<const uint16_t*>(bweight), bn, (int)K, rpw,
                           bout};
      const int st = strip_launch_bf16(sa, b, (int)gb, (hipStream_t)stream);
      if (st != MTL_ERR_UNSUPPORTED) return st;
    }
  }
  if (const int st = w4_gemm_norm_partials(h, w, slots, eps, K, qweight, scales, qzeros, N,
                                           group_size, zero_offset, layout, partials,
                                           partials_bytes, (hipStream_t)stream))
    return st;
  return mtl_bf16_gemv_norm(bh, bnorm_w, slots, eps, bweight, bn, K, bout, stream);
}

int mtl_w4_gemm_residual(const void* x, const float* xpart, int32_t xsplits, int64_t xpart_ld,
                         int64_t K, const int32_t* qweight, const void* scales,
                         const int32_t* qzeros, int64_t N, int32_t group_size, int32_t zero_offset,
                         int32_t layout, void* h, const int32_t* scatter, void* h_ord,
                         float* slots, void* workspace, int64_t ws_bytes, void* stream) {
  return w4_gemm_residual(x, xpart, xsplits, xpart_ld, K, qweight, scales, qzeros, N, group_size,
                          zero_offset, layout, h, scatter, h_ord, slots, workspace, ws_bytes,
                          (hipStream_t)stream);
}

int mtl_w4_gemm_norm_silu(const void* h, const void* w, const float* slots, float eps, int64_t K,
                          const int32_t* qweight, const void* scales, const int32_t* qzeros,
                          int64_t N, int32_t group_size, int32_t zero_offset, int32_t layout,
                          void* act, void* stream) {
  return w4_gemm_norm_silu(h, w, slots, eps, K, qweight, scales, qzeros, N, group_size,
                           zero_offset, layout, act, (hipStream_t)stream);
}

int mtl_gptq_gemm(const void* x, int64_t M, int64_t K, const int32_t* qweight,
                  const int32_t* qzeros, const void* scales, const int32_t* perm, int64_t N,
                  int32_t group_size, int32_t zero_offset, void* y, int32_t out_dtype,
                  void* workspace, int64_t ws_bytes, void* stream) {
  return w4_gemm(x, M, K, qweight, MTL_META_GPTQ, scales, qzeros, perm, N, group_size,
                 zero_offset, MTL_EPI_NONE, nullptr, y, out_dtype, workspace, ws_bytes,
                 (hipStream_t)stream);
}

int mtl_w4_gemm_fused(const void* x, int64_t M, int64_t K, const int32_t* qweight,
                      int32_t meta_format, const void* meta0, const int32_t* qzeros,
                      const int32_t* perm, int64_t N, int32_t group_size, int32_t zero_offset,
                      int32_t epilogue, const void* resid, void* y, int32_t out_dtype,
                      void* workspace, int64_t ws_bytes, void* stream) {
  return w4_gemm(x, M, K, qweight, meta_format, meta0, qzeros, perm, N, group_size,
                 zero_offset, epilogue, resid, y, out_dtype, workspace, ws_bytes,
                 (hipStream_t)stream);
}

int mtl_w4_gemm_partials_geom(const void* x, const float* xpart, int32_t xsplits,
                              int64_t xpart_ld, int64_t M, int64_t K, const int32_t* qweight,
                              const void* scales, const int32_t* qzeros, const int32_t* perm,
                              int64_t N, int32_t group_size, int32_t zero_offset, int32_t layout,
                              float* partials, int64_t partials_bytes,
                              const mtl_strip_geometry* geom, void* stream) {
  if (geom && !is_strip(layout)) return MTL_ERR_UNSUPPORTED;
  return w4_gemm_partials(x, xpart, xsplits, xpart_ld, M, K, qweight, scales, qzeros, perm, N,
                          group_size, zero_offset, layout, partials, partials_bytes,
                          (hipStream_t)stream, geom);
}

int mtl_w4_gemm_norm_partials_geom(const void* h, const void* w, const float* slots, float eps,
                                   int64_t K, const int32_t* qweight, const void* scales,
                                   const int32_t* qzeros, int64_t N, int32_t group_size,
                                   int32_t zero_offset, int32_t layout, float* partials,
                                   int64_t partials_bytes, const mtl_strip_geometry* geom,
                                   void* stream) {
  if (geom && !is_strip(layout)) return MTL_ERR_UNSUPPORTED;
  return w4_gemm_norm_partials(h, w, slots, eps, K, qweight, scales, qzeros, N, group_size,
                               zero_offset, layout, partials, partials_bytes,
                               (hipStream_t)stream, geom);
}

int mtl_w4_gemm_residual_geom(const void* x, const float* xpart, int32_t xsplits,
                              int64_t xpart_ld, int64_t K, const int32_t* qweight,
                              const void* scales, const int32_t* qzeros, int64_t N,
                              int32_t group_size, int32_t zero_offset, int32_t layout, void* h,
                              const int32_t* scatter, void* h_ord, float* slots, void* workspace,
                              int64_t ws_bytes, const mtl_strip_geometry* geom, void* stream) {
  if (geom && !is_strip(layout)) return MTL_ERR_UNSUPPORTED;
  return w4_gemm_residual(x, xpart, xsplits, xpart_ld, K, qweight, scales, qzeros, N, group_size,
                          zero_offset, layout, h, scatter, h_ord, slots, workspace, ws_bytes,
                          (hipStream_t)stream, geom);
}

int mtl_w4_gemm_norm_silu_geom(const void* h, const void* w, const float* slots, float eps,
                               int64_t K, const int32_t* qweight, const void* scales,
                               const int32_t* qzeros, int64_t N, int32_t group_size,
                               int32_t zero_offset, int32_t layout, void* act,
                               const mtl_strip_geometry* geom, void* stream) {
  return w4_gemm_norm_silu(h, w, slots, eps, K, qweight, scales, qzeros, N, group_size,
                           zero_offset, layout, act, (hipStream_t)stream, geom);
}



}  // extern "C"
