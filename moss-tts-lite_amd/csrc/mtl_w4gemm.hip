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
// Work decomposition (deterministic, no atomics):
//   * a wave owns a 256-column tile (64 lanes x 4 columns = one 16-byte qweight load per
//     lane per row, 1 KB contiguous per wave) and 16 qweight rows (128 input channels);
//     it issues all 16 loads up front, so the whole weight slice of the chip is in flight;
//   * a workgroup stacks 1, 2 or 4 waves along K and reduces them through LDS;
//   * blockIdx.y splits K further; each workgroup publishes an fp32 partial tile and
//     the last workgroup of the tile (agent-scope counter) sums the splits in split
//     order, applies the epilogue and resets the counter, so results (and graph
//     replays) are bitwise repeatable and the next launch needs no memset.
//
// Inner loop: a qweight word holds 8 codes; OR-ing nibble pairs into 0x4300 gives the
// bf16 pair (128 + q_j, 128 + q_{j+4}), and x is staged in LDS in the same pair order,
// so 7 integer ops + 4 v_dot2c_f32_bf16 handle 8 MACs.  Per group (g/8 rows) the
// accumulated sum A = sum x*(128+q) and X = sum x give
//     sum x*w = s * (A - (128 + c) * X) + d * X.
#include "mtl_common.h"

namespace mtl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kTileN = 256;        // output columns per wave tile
constexpr int kRowsPerWave = 16;   // qweight rows (x 8 input channels) per wave
constexpr int kMaxWaves = 4;       // waves stacked along K in one workgroup
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
  const float* slots;       //               per-block sums of squares of h [nslots]
  float eps;
  const uint16_t* resid;    // RESIDUAL epilogue input [M, N]
  void* y;
  float* partial;           // [splits, M, N]
  unsigned* counters;       // [col_tiles], zero between launches
  int inkernel_reduce;      // 1: last workgroup reduces; 0: w4_reduce_kernel does
  int partials_only;        // 1: always publish [splits, M, N] partials, no epilogue
  int M, K, N, group, zero_offset, splits, epilogue, out_f32;
};

// (a & m) | o in one VALU op; the constants live in registers because gfx9 VOP3
// encodings take no literal.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(o));
  return r;
}

__device__ __forceinline__ float4 ld_f4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}

// bf16(silu(bf16 g) * bf16 u): F.silu on a bf16 tensor then a bf16 product (fast.py:170-171).
__device__ __forceinline__ uint32_t silu_mul_bf16(float g, float u) {
  g = round_bf16(g);
  const float sg = round_bf16(g / (1.0f + expf(-g)));
  return f32_to_bf16(sg * round_bf16(u));
}

// Where the kernel reads its activation row from.
enum : int {
  XSRC_BF16 = 0,      // x bf16 [M, K]
  XSRC_PERM = 1,      // x bf16 [M, K] read through the act-order index: x[:, perm[k]]
  XSRC_SILU_PART = 2, // x = SiLU(gate) * up from the fp32 split-K partials of an
                      // interleaved gate|up GEMV (the down projection's input)
  XSRC_RMSNORM = 3    // x = bf16(w * bf16(h * r)): RMSNorm applied while staging, from the
                      // residual stream h and norm weight w (both already in the weight's
                      // act-order input order) and r = rsqrt(sum(slots)/K + eps)
};

constexpr int kNormSlots = 16;   // sums of squares published by the residual kernel

template <int MR, int RPG, int FMT, int XSRC>
__global__ void __launch_bounds__(256) w4_gemm_kernel(W4Args a) {
  constexpr bool PERM = XSRC == XSRC_PERM || XSRC == XSRC_SILU_PART;   // x staged after weights
  constexpr int RB = kRowsPerWave;
  constexpr int NCH = RB / RPG;            // metadata chunks per wave
  constexpr int XIT = (MR * RB + 63) / 64; // x staging items per lane
  __shared__ u32x4 xs[kMaxWaves][MR][RB];
  __shared__ float xsum[kMaxWaves][MR][RB];
  __shared__ float4 red[kMaxWaves][MR][64];

  const int nw = blockDim.x >> 6;
  const int wave = wave_id();
  const int lane = threadIdx.x & 63;
  const int tile = blockIdx.x;
  const int split = blockIdx.y;
  const int N = a.N;
  const int M = a.M;
  const int rows_total = a.K >> 3;
  const int wrow0 = __builtin_amdgcn_readfirstlane((split * nw + wave) * RB);
  const int col0 = tile * kTileN + lane * 4;
  const bool col_ok = col0 < N;

  // Loads below are branch-free so the waitcnt pass can count them exactly: rows past
  // K/8 are clamped to the last row (their x is staged as 0, so they add exactly 0) and
  // columns past N read 0 through the buffer range check.
  const int rows_last = rows_total - 1;

  // 1. x for this wave's rows.  Without act-order these loads go first, so the LDS
  //    staging waits only on them; with act-order the gather needs the index first, so
  //    it is issued after the weight stream and overlaps it instead.
  u32x4 xv[XIT];
  bool xok[XIT];
  u32x4 wv[XSRC == XSRC_RMSNORM ? XIT : 1];
  float4 slot4[XSRC == XSRC_RMSNORM ? kNormSlots / 4 : 1];
  auto load_x = [&]() {
#pragma unroll
    for (int it = 0; it < XIT; ++it) {
      const int item = lane + 64 * it;
      const int m = item / RB;
      const int row = wrow0 + (item % RB);
      const bool ok = item < MR * RB && m < M && row < rows_total;
      const size_t xoff = (size_t)(m < M ? m : M - 1) * a.K;
      const int rc = row < rows_total ? row : rows_last;
      u32x4 v;
      if (XSRC == XSRC_PERM) {
        const u32x4 p0 = *reinterpret_cast<const u32x4*>(a.perm + rc * 8);
        const u32x4 p1 = *reinterpret_cast<const u32x4*>(a.perm + rc * 8 + 4);
        const uint32_t e0 = a.x[xoff + p0.x], e1 = a.x[xoff + p0.y];
        const uint32_t e2 = a.x[xoff + p0.z], e3 = a.x[xoff + p0.w];
        const uint32_t e4 = a.x[xoff + p1.x], e5 = a.x[xoff + p1.y];
        const uint32_t e6 = a.x[xoff + p1.z], e7 = a.x[xoff + p1.w];
        v = u32x4{e0 | (e1 << 16), e2 | (e3 << 16), e4 | (e5 << 16), e6 | (e7 << 16)};
      } else if (XSRC == XSRC_SILU_PART) {
        // channels 8rc..8rc+7 of the intermediate; their gate columns are contiguous in
        // the 32-column interleave and the up columns sit 32 to the right.
        const int j0 = rc * 8;
        const float* pb = a.xpart + (size_t)(m < M ? m : M - 1) * a.xpart_ld +
                          64 * (j0 >> 5) + (j0 & 31);
        const size_t ss = (size_t)M * a.xpart_ld;
        float g[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float u[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < a.xsplits; s0 += 8) {   // 32 loads in flight, summed in order
          float4 G[8][2], U[8][2];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int sp = s0 + j < a.xsplits ? s0 + j : a.xsplits - 1;
            const float* q = pb + sp * ss;
            G[j][0] = ld_f4(q); G[j][1] = ld_f4(q + 4);
            U[j][0] = ld_f4(q + 32); U[j][1] = ld_f4(q + 36);
          }
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (s0 + j < a.xsplits) {
              g[0] += G[j][0].x; g[1] += G[j][0].y; g[2] += G[j][0].z; g[3] += G[j][0].w;
              g[4] += G[j][1].x; g[5] += G[j][1].y; g[6] += G[j][1].z; g[7] += G[j][1].w;
              u[0] += U[j][0].x; u[1] += U[j][0].y; u[2] += U[j][0].z; u[3] += U[j][0].w;
              u[4] += U[j][1].x; u[5] += U[j][1].y; u[6] += U[j][1].z; u[7] += U[j][1].w;
            }
        }
        v = u32x4{silu_mul_bf16(g[0], u[0]) | (silu_mul_bf16(g[1], u[1]) << 16),
                  silu_mul_bf16(g[2], u[2]) | (silu_mul_bf16(g[3], u[3]) << 16),
                  silu_mul_bf16(g[4], u[4]) | (silu_mul_bf16(g[5], u[5]) << 16),
                  silu_mul_bf16(g[6], u[6]) | (silu_mul_bf16(g[7], u[7]) << 16)};
      } else if (XSRC == XSRC_RMSNORM) {   // raw h now, normalised once the scale is known
        v = *reinterpret_cast<const u32x4*>(a.hn + rc * 8);
        wv[it] = *reinterpret_cast<const u32x4*>(a.wn + rc * 8);
      } else {
        v = *reinterpret_cast<const u32x4*>(a.x + xoff + rc * 8);
      }
      xv[it] = v;     // masked after the weight stream is issued (step 4)
      xok[it] = ok;
    }
  };
  if (!PERM) load_x();
  if (XSRC == XSRC_RMSNORM) {
#pragma unroll
    for (int i = 0; i < kNormSlots / 4; ++i) slot4[i] = ld_f4(a.slots + 4 * i);
  }

  // 2. Group metadata of the lane's 4 columns, one entry per RPG-row chunk.
  const int colc = col_ok ? col0 : N - 4;
  u32x4 meta[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int row = wrow0 + c * RPG;
    const int grp = ((row < rows_total ? row : rows_last) * 8) / a.group;
    if (FMT == MTL_META_QSZ) {
      meta[c] = *reinterpret_cast<const u32x4*>(a.meta0 + ((size_t)grp * N + colc) * 2);
    } else {
      const u32x2 s = *reinterpret_cast<const u32x2*>(a.meta0 + (size_t)grp * N + colc);
      const uint32_t zw = a.qzeros[(size_t)grp * (N >> 3) + (colc >> 3)];
      meta[c] = u32x4{s.x, s.y, zw >> ((colc & 7) * 4), 0u};
    }
  }

  // 3. Stream the weight slice: RB independent 16-byte buffer loads per lane with a
  //    scalar row offset.
  const __amdgpu_buffer_rsrc_t qrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<u32x4*>(a.qweight), (short)0, (int)((int64_t)rows_total * N * 4), 0x00020000);
  const int voff = col_ok ? col0 * 4 : 0x7ffffff0;
  u32x4 wq[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int row = wrow0 + r < rows_total ? wrow0 + r : rows_last;
    wq[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          qrsrc, voff, row * N * 4, kStreamAux));
  }

  if (PERM) load_x();
  // Keep the scheduler from hoisting the uses of x above the weight stream: every load
  // of the wave is in flight before the first wait.
  __builtin_amdgcn_sched_barrier(0);

  // 4. x into LDS in pair order (x0,x4),(x1,x5),(x2,x6),(x3,x7) with row sums.
  float norm_r = 0.f;
  if (XSRC == XSRC_RMSNORM) {   // RMSNorm scale: rsqrt(mean(h^2) + eps), slots summed in order
    float ssum = 0.f;
#pragma unroll
    for (int i = 0; i < kNormSlots / 4; ++i)
      ssum += ((slot4[i].x + slot4[i].y) + (slot4[i].z + slot4[i].w));
    norm_r = rsqrtf(ssum / (float)a.K + a.eps);
  }
#pragma unroll
  for (int it = 0; it < XIT; ++it) {
    const int item = lane + 64 * it;
    if (item < MR * RB) {
      u32x4 v = xv[it];
      if (XSRC == XSRC_RMSNORM) {   // x = bf16(w * bf16(h * r)), model.py:34-40
        const uint32_t hh[4] = {v.x, v.y, v.z, v.w};
        const uint32_t ww[4] = {wv[it].x, wv[it].y, wv[it].z, wv[it].w};
        uint32_t o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t lo = f32_to_bf16(round_bf16(
              bf16_to_f32(ww[c] & 0xffffu) * round_bf16(bf16_to_f32(hh[c] & 0xffffu) * norm_r)));
          const uint32_t hi = f32_to_bf16(round_bf16(
              bf16_to_f32(ww[c] >> 16) * round_bf16(bf16_to_f32(hh[c] >> 16) * norm_r)));
          o[c] = lo | (hi << 16);
        }
        v = u32x4{o[0], o[1], o[2], o[3]};
      }
      if (!xok[it]) v = u32x4{0u, 0u, 0u, 0u};
      const uint32_t e0 = v.x & 0xffffu, e1 = v.x >> 16, e2 = v.y & 0xffffu, e3 = v.y >> 16;
      const uint32_t e4 = v.z & 0xffffu, e5 = v.z >> 16, e6 = v.w & 0xffffu, e7 = v.w >> 16;
      xs[wave][item / RB][item % RB] =
          u32x4{e0 | (e4 << 16), e1 | (e5 << 16), e2 | (e6 << 16), e3 | (e7 << 16)};
      xsum[wave][item / RB][item % RB] =
          ((bf16_to_f32(e0) + bf16_to_f32(e1)) + (bf16_to_f32(e2) + bf16_to_f32(e3))) +
          ((bf16_to_f32(e4) + bf16_to_f32(e5)) + (bf16_to_f32(e6) + bf16_to_f32(e7)));
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // 5. Dot products, one group chunk at a time.
  float tot[MR][4];
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int c = 0; c < 4; ++c) tot[m][c] = 0.f;

  const uint32_t kMagic = __builtin_amdgcn_readfirstlane(0x43004300u);  // bf16 (128, 128)
  const uint32_t kLo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    float acc[MR][4];
    float X[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      X[m] = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[m][c] = 0.f;
    }
#pragma unroll
    for (int rr = 0; rr < RPG; ++rr) {
      const int r = ch * RPG + rr;
      const uint32_t w[4] = {wq[r].x, wq[r].y, wq[r].z, wq[r].w};
      uint32_t p[4][4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        p[c][0] = and_or(w[c], kLo, kMagic);
        p[c][1] = and_or(w[c] >> 4, kLo, kMagic);
        p[c][2] = and_or(w[c] >> 8, kLo, kMagic);
        p[c][3] = and_or(w[c] >> 12, kLo, kMagic);
      }
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const u32x4 xp = xs[wave][m][r];
        X[m] += xsum[wave][m][r];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float t = acc[m][c];
          t = dot2_bf16(p[c][0], xp.x, t);
          t = dot2_bf16(p[c][1], xp.y, t);
          t = dot2_bf16(p[c][2], xp.z, t);
          t = dot2_bf16(p[c][3], xp.w, t);
          acc[m][c] = t;
        }
      }
    }
    float sc[4], cz[4], dz[4];
    if (FMT == MTL_META_QSZ) {
      const uint32_t mw[4] = {meta[ch].x, meta[ch].y, meta[ch].z, meta[ch].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        sc[c] = bf16_to_f32(mw[c] & 0xffffu);
        dz[c] = bf16_to_f32(mw[c] >> 16);
        cz[c] = 136.f;   // 128 (bf16 magic) + 8 (offset-binary centre)
      }
    } else {
      sc[0] = f16_to_f32(meta[ch].x & 0xffffu);
      sc[1] = f16_to_f32(meta[ch].x >> 16);
      sc[2] = f16_to_f32(meta[ch].y & 0xffffu);
      sc[3] = f16_to_f32(meta[ch].y >> 16);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        cz[c] = (float)(128 + (int)((meta[ch].z >> (4 * c)) & 0xfu) + a.zero_offset);
        dz[c] = 0.f;
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float t = fmaf(-cz[c], X[m], acc[m][c]);
        float v = fmaf(sc[c], t, tot[m][c]);
        if (FMT == MTL_META_QSZ) v = fmaf(dz[c], X[m], v);
        tot[m][c] = v;
      }
  }

  // 6. Reduce the waves of the workgroup into wave 0 (fixed order 0, 1, 2, 3).
  if (nw > 1) {
    if (wave > 0) {
#pragma unroll
      for (int m = 0; m < MR; ++m)
        red[wave][m][lane] = make_float4(tot[m][0], tot[m][1], tot[m][2], tot[m][3]);
    }
    __syncthreads();
    if (wave > 0) return;
    for (int w2 = 1; w2 < nw; ++w2) {
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const float4 v = red[w2][m][lane];
        tot[m][0] += v.x; tot[m][1] += v.y; tot[m][2] += v.z; tot[m][3] += v.w;
      }
    }
  }

  // 7. Split-K.  Every workgroup publishes its fp32 partial tile.  With an in-kernel
  //    reduction the partials travel as relaxed agent-scope atomics (coherent across
  //    XCDs without a whole-L2 writeback), a per-tile counter names the last workgroup,
  //    and that one sums all splits in split order (loads batched 8 deep) and resets
  //    the counter.  Otherwise w4_reduce_kernel (or a fused consumer) sums them.
  if (a.splits > 1 || a.partials_only) {
    float* pbase = a.partial + (size_t)split * M * N + col0;
    if (!a.inkernel_reduce || a.partials_only) {
      if (col_ok) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
          if (m < M)
            *reinterpret_cast<float4*>(pbase + (size_t)m * N) =
                make_float4(tot[m][0], tot[m][1], tot[m][2], tot[m][3]);
      }
      return;
    }
    if (col_ok) {
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            __hip_atomic_store(pbase + (size_t)m * N + c, tot[m][c], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);   // every partial store acknowledged before the count
    int last = 0;
    if (lane == 0)
      last = __hip_atomic_fetch_add(&a.counters[tile], 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(a.splits - 1);
    last = __builtin_amdgcn_readfirstlane(__shfl(last, 0));
    if (!last) return;
    const int S = a.splits;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float s4[4] = {0.f, 0.f, 0.f, 0.f};
      if (col_ok && m < M) {
        const float* q = a.partial + (size_t)m * N + col0;
        const size_t stride = (size_t)M * N;
        for (int s0 = 0; s0 < S; s0 += 8) {
          float v[8][4];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int sp = s0 + j < S ? s0 + j : S - 1;
#pragma unroll
            for (int c = 0; c < 4; ++c)
              v[j][c] = __hip_atomic_load(q + sp * stride + c, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
          }
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (s0 + j < S) {
#pragma unroll
              for (int c = 0; c < 4; ++c) s4[c] += v[j][c];
            }
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) tot[m][c] = s4[c];
    }
    if (lane == 0)
      __hip_atomic_store(&a.counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // 8. Epilogue, 4 consecutive columns per lane.
  if (a.epilogue == MTL_EPI_SILU_MUL) {
    // Fused columns come in blocks of 64 = 32 gate | 32 up; lane l (l%16 < 8) holds
    // gate columns whose up partners sit 8 lanes higher.
    const int no = N >> 1;
    const int lb = lane & 15;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      float u[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) u[c] = __shfl_down(tot[m][c], 8);
      if (m < M && col_ok && lb < 8) {
        const int o = tile * (kTileN / 2) + (lane >> 4) * 32 + lb * 4;
        uint32_t h[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float g = round_bf16(tot[m][c]);
          const float sg = round_bf16(g / (1.0f + expf(-g)));
          h[c] = f32_to_bf16(sg * round_bf16(u[c]));
        }
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.y) + (size_t)m * no + o) =
            u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
      }
    }
  } else if (col_ok) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (m >= M) continue;
      const size_t o = (size_t)m * N + col0;
      float v[4] = {tot[m][0], tot[m][1], tot[m][2], tot[m][3]};
      if (a.epilogue == MTL_EPI_RESIDUAL) {
        const u32x2 rr = *reinterpret_cast<const u32x2*>(a.resid + o);
        v[0] = round_bf16(v[0]) + bf16_to_f32(rr.x & 0xffffu);
        v[1] = round_bf16(v[1]) + bf16_to_f32(rr.x >> 16);
        v[2] = round_bf16(v[2]) + bf16_to_f32(rr.y & 0xffffu);
        v[3] = round_bf16(v[3]) + bf16_to_f32(rr.y >> 16);
      }
      if (a.out_f32) {
        *reinterpret_cast<float4*>(static_cast<float*>(a.y) + o) =
            make_float4(v[0], v[1], v[2], v[3]);
      } else {
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.y) + o) =
            u32x2{f32_to_bf16(v[0]) | (f32_to_bf16(v[1]) << 16),
                  f32_to_bf16(v[2]) | (f32_to_bf16(v[3]) << 16)};
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

static int g_tune_waves = 0;   // 0: heuristic; 1, 2, 4: forced waves per workgroup

struct Plan {
  int waves, splits, col_tiles, row_blocks;
};

static Plan plan_for(int64_t K, int64_t N) {
  Plan p;
  const int rows = (int)(K / 8);
  p.row_blocks = (rows + kRowsPerWave - 1) / kRowsPerWave;
  p.col_tiles = (int)((N + kTileN - 1) / kTileN);
  int w = 1;
  if (g_tune_waves == 1 || g_tune_waves == 2 || g_tune_waves == 4) {
    w = g_tune_waves;
  } else {
    // Four waves per workgroup measured best on every decode shape (fewest splits,
    // so the least split-K traffic and counter work).
    w = 4;
  }
  while (w > 1 && w > p.row_blocks) w >>= 1;
  p.waves = w;
  p.splits = (p.row_blocks + w - 1) / w;
  return p;
}

// Workspace = a fixed tile-counter region (so partial tiles of one shape never land on
// another shape's counters) followed by the fp32 partial tiles [splits, M, N].
constexpr int64_t kCounterBytes = 16384;   // 4096 column tiles: N <= 1M
static int g_inkernel_reduce = 1;

template <int MR, int RPG>
static void launch_fmt(const W4Args& a, int fmt, dim3 grid, dim3 block, hipStream_t s) {
  if (fmt == MTL_META_QSZ)
    hipLaunchKernelGGL((w4_gemm_kernel<MR, RPG, MTL_META_QSZ, XSRC_BF16>), grid, block, 0, s, a);
  else if (a.xpart)
    hipLaunchKernelGGL((w4_gemm_kernel<1, RPG, MTL_META_GPTQ, XSRC_SILU_PART>), grid, block, 0, s, a);
  else if (a.hn)
    hipLaunchKernelGGL((w4_gemm_kernel<1, RPG, MTL_META_GPTQ, XSRC_RMSNORM>), grid, block, 0, s, a);
  else if (a.perm)
    hipLaunchKernelGGL((w4_gemm_kernel<MR, RPG, MTL_META_GPTQ, XSRC_PERM>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((w4_gemm_kernel<MR, RPG, MTL_META_GPTQ, XSRC_BF16>), grid, block, 0, s, a);
}

template <int MR>
static void launch_rpg(const W4Args& a, int fmt, dim3 grid, dim3 block, hipStream_t s) {
  const int rpg = a.group / 8 < kRowsPerWave ? a.group / 8 : kRowsPerWave;
  if (rpg == 4) launch_fmt<MR, 4>(a, fmt, grid, block, s);
  else if (rpg == 8) launch_fmt<MR, 8>(a, fmt, grid, block, s);
  else launch_fmt<MR, 16>(a, fmt, grid, block, s);
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
  // The weight buffer's byte size and row offsets are 32-bit in the buffer descriptor.
  if (K * N / 2 >= ((int64_t)1 << 31) || M * K >= ((int64_t)1 << 31)) return MTL_ERR_SHAPE;
  if (!aligned16(qweight) || !aligned16(x) || (perm && !aligned16(perm))) return MTL_ERR_ALIGN;
  if (perm && fmt != MTL_META_GPTQ) return MTL_ERR_INVALID_ARG;
  if (fmt == MTL_META_QSZ && !aligned16(meta0)) return MTL_ERR_ALIGN;
  if (fmt == MTL_META_GPTQ && (reinterpret_cast<uintptr_t>(meta0) & 7u)) return MTL_ERR_ALIGN;

  const Plan p = plan_for(K, N);
  W4Args a;
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
  a.partial = nullptr;
  a.counters = nullptr;
  a.xpart = nullptr;
  a.xsplits = 0;
  a.xpart_ld = 0;
  a.hn = nullptr;
  a.wn = nullptr;
  a.slots = nullptr;
  a.eps = 0.f;
  a.partials_only = 0;
  a.inkernel_reduce = g_inkernel_reduce;
  if (p.splits > 1) {
    const int64_t need = kCounterBytes + (int64_t)p.splits * M * N * 4;
    if (!workspace || ws_bytes < need) return MTL_ERR_WORKSPACE;
    if (!aligned16(workspace)) return MTL_ERR_ALIGN;
    a.counters = static_cast<unsigned*>(workspace);
    a.partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  }
  const dim3 grid(p.col_tiles, p.splits);
  const dim3 block(64 * p.waves);
  const int mr = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16;
  switch (mr) {
    case 1: launch_rpg<1>(a, fmt, grid, block, stream); break;
    case 2: launch_rpg<2>(a, fmt, grid, block, stream); break;
    case 4: launch_rpg<4>(a, fmt, grid, block, stream); break;
    case 8: launch_rpg<8>(a, fmt, grid, block, stream); break;
    default: launch_rpg<16>(a, fmt, grid, block, stream); break;
  }
  if (p.splits > 1 && !a.inkernel_reduce) {
    const int quads = (int)(M * (epilogue == MTL_EPI_SILU_MUL ? N / 8 : N / 4));
    hipLaunchKernelGGL(w4_reduce_kernel, dim3((quads + 255) / 256), dim3(256), 0, stream, a);
  }
  return launch_status();
}

// Partials-only launch for fused consumers: writes fp32 [splits, M, N] into `partials`
// (splits = w4_splits(K)); x comes from `x` (bf16, optionally through `perm`) or, when
// `xpart` is set, from the gate|up partials of the previous GEMV (SiLU*up, M = 1).
static int w4_gemm_partials(const void* x, const float* xpart, int xsplits, int64_t xpart_ld,
                            int64_t M, int64_t K, const int32_t* qweight, const void* meta0,
                            const int32_t* qzeros, const int32_t* perm, int64_t N, int group,
                            int zero_offset, float* partials, int64_t partials_bytes,
                            hipStream_t stream) {
  if ((!x && !xpart) || (x && xpart) || !qweight || !meta0 || !qzeros || !partials)
    return MTL_ERR_INVALID_ARG;
  if (group != 32 && group != 64 && group != 128 && group != 256) return MTL_ERR_GROUP;
  if (M < 1 || M > kMaxM || K <= 0 || N <= 0 || K % group != 0 || N % 8 != 0)
    return MTL_ERR_SHAPE;
  if (K * N / 2 >= ((int64_t)1 << 31) || M * K >= ((int64_t)1 << 31)) return MTL_ERR_SHAPE;
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
  if (reinterpret_cast<uintptr_t>(meta0) & 7u) return MTL_ERR_ALIGN;
  const Plan p = plan_for(K, N);
  if (partials_bytes < (int64_t)p.splits * M * N * 4) return MTL_ERR_WORKSPACE;
  W4Args a;
  a.x = static_cast<const uint16_t*>(x);
  a.qweight = reinterpret_cast<const u32x4*>(qweight);
  a.meta0 = static_cast<const uint16_t*>(meta0);
  a.qzeros = reinterpret_cast<const uint32_t*>(qzeros);
  a.perm = perm;
  a.xpart = xpart;
  a.xsplits = xsplits;
  a.xpart_ld = (int)xpart_ld;
  a.hn = nullptr;
  a.wn = nullptr;
  a.slots = nullptr;
  a.eps = 0.f;
  a.resid = nullptr;
  a.y = nullptr;
  a.partial = partials;
  a.counters = nullptr;
  a.M = (int)M; a.K = (int)K; a.N = (int)N;
  a.group = group; a.zero_offset = zero_offset;
  a.splits = p.splits;
  a.epilogue = MTL_EPI_NONE;
  a.out_f32 = 1;
  a.inkernel_reduce = 0;
  a.partials_only = 1;
  const dim3 grid(p.col_tiles, p.splits);
  const dim3 block(64 * p.waves);
  const int mr = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16;
  switch (mr) {
    case 1: launch_rpg<1>(a, MTL_META_GPTQ, grid, block, stream); break;
    case 2: launch_rpg<2>(a, MTL_META_GPTQ, grid, block, stream); break;
    case 4: launch_rpg<4>(a, MTL_META_GPTQ, grid, block, stream); break;
    case 8: launch_rpg<8>(a, MTL_META_GPTQ, grid, block, stream); break;
    default: launch_rpg<16>(a, MTL_META_GPTQ, grid, block, stream); break;
  }
  return launch_status();
}

// Partials-only launch whose input is RMSNorm(h) computed while staging (M = 1).
static int w4_gemm_norm_partials(const void* h_ord, const void* w_ord, const float* slots,
                                 float eps, int64_t K, const int32_t* qweight,
                                 const void* meta0, const int32_t* qzeros, int64_t N, int group,
                                 int zero_offset, float* partials, int64_t partials_bytes,
                                 hipStream_t stream) {
  if (!h_ord || !w_ord || !slots || !qweight || !meta0 || !qzeros || !partials)
    return MTL_ERR_INVALID_ARG;
  if (group != 32 && group != 64 && group != 128 && group != 256) return MTL_ERR_GROUP;
  if (K <= 0 || N <= 0 || K % group != 0 || N % 8 != 0) return MTL_ERR_SHAPE;
  if (!aligned16(slots)) return MTL_ERR_ALIGN;
  if (K * N / 2 >= ((int64_t)1 << 31)) return MTL_ERR_SHAPE;
  if (!aligned16(h_ord) || !aligned16(w_ord) || !aligned16(qweight) || !aligned16(partials))
    return MTL_ERR_ALIGN;
  if (reinterpret_cast<uintptr_t>(meta0) & 7u) return MTL_ERR_ALIGN;
  const Plan p = plan_for(K, N);
  if (partials_bytes < (int64_t)p.splits * N * 4) return MTL_ERR_WORKSPACE;
  W4Args a;
  a.x = nullptr;
  a.qweight = reinterpret_cast<const u32x4*>(qweight);
  a.meta0 = static_cast<const uint16_t*>(meta0);
  a.qzeros = reinterpret_cast<const uint32_t*>(qzeros);
  a.perm = nullptr;
  a.xpart = nullptr;
  a.xsplits = 0;
  a.xpart_ld = 0;
  a.hn = static_cast<const uint16_t*>(h_ord);
  a.wn = static_cast<const uint16_t*>(w_ord);
  a.slots = slots;
  a.eps = eps;
  a.resid = nullptr;
  a.y = nullptr;
  a.partial = partials;
  a.counters = nullptr;
  a.M = 1; a.K = (int)K; a.N = (int)N;
  a.group = group; a.zero_offset = zero_offset;
  a.splits = p.splits;
  a.epilogue = MTL_EPI_NONE;
  a.out_f32 = 1;
  a.inkernel_reduce = 0;
  a.partials_only = 1;
  launch_rpg<1>(a, MTL_META_GPTQ, dim3(p.col_tiles, p.splits), dim3(64 * p.waves), stream);
  return launch_status();
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
  const int64_t row_blocks = (K / 8 + kRowsPerWave - 1) / kRowsPerWave;
  // Sized for the deepest split (one wave per workgroup), so any plan fits.
  return kCounterBytes + row_blocks * M * N * 4;
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

int mtl_w4_gemm_partials(const void* x, const float* xpart, int32_t xsplits, int64_t xpart_ld,
                         int64_t M, int64_t K, const int32_t* qweight, const void* scales,
                         const int32_t* qzeros, const int32_t* perm, int64_t N, int32_t group_size,
                         int32_t zero_offset, float* partials, int64_t partials_bytes,
                         void* stream) {
  return w4_gemm_partials(x, xpart, xsplits, xpart_ld, M, K, qweight, scales, qzeros, perm, N,
                          group_size, zero_offset, partials, partials_bytes, (hipStream_t)stream);
}

int mtl_w4_gemm_norm_partials(const void* h, const void* w, const float* slots, float eps,
                              int64_t K, const int32_t* qweight, const void* scales,
                              const int32_t* qzeros, int64_t N, int32_t group_size,
                              int32_t zero_offset, float* partials, int64_t partials_bytes,
                              void* stream) {
  return w4_gemm_norm_partials(h, w, slots, eps, K, qweight, scales, qzeros, N,
                               group_size, zero_offset, partials, partials_bytes,
                               (hipStream_t)stream);
}

int mtl_gptq_gemm(const void* x, int64_t M, int64_t K, const int32_t* qweight,
                  const int32_t* qzeros, const void* scales, const int32_t* perm, int64_t N,
                  int32_t group_size, int32_t zero_offset, void* y, int32_t out_dtype,
                  void* workspace, int64_t ws_bytes, void* stream) {
  return w4_gemm(x, M, K, qweight, MTL_META_GPTQ, scales, qzeros, perm, N, group_size,
                 zero_offset, MTL_EPI_NONE, nullptr, y, out_dtype, workspace, ws_bytes,
                 (hipStream_t)stream);
}

int mtl_int4pack_mm(const void* x, int64_t M, int64_t K, const int32_t* packed,
                    int32_t group_size, const void* qsz, int64_t N, void* y, void* workspace,
                    int64_t ws_bytes, void* stream) {
  return w4_gemm(x, M, K, packed, MTL_META_QSZ, qsz, nullptr, nullptr, N, group_size, 0,
                 MTL_EPI_NONE, nullptr, y, MTL_OUT_BF16, workspace, ws_bytes,
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

// Tuning knob for launch-shape sweeps: force 1, 2 or 4 waves per workgroup (0 restores
// the heuristic).  Process-wide; not for concurrent use.
// Split-K reduction: 1 = in-kernel (last workgroup of a tile), 0 = separate kernel.
int mtl_tune_set_reduce(int32_t inkernel) {
  if (inkernel != 0 && inkernel != 1) return MTL_ERR_INVALID_ARG;
  g_inkernel_reduce = inkernel;
  return MTL_OK;
}

int mtl_tune_set_waves(int32_t waves) {
  if (waves != 0 && waves != 1 && waves != 2 && waves != 4) return MTL_ERR_INVALID_ARG;
  g_tune_waves = waves;
  return MTL_OK;
}

}  // extern "C"
