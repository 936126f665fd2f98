// Load-time layout utilities of the int4 path: the reference-contract packer, code
// unpacking, exact dequantisation and the act-order (g_idx) reorder.
#include "mtl_common.h"

namespace mtl {

// The strip layout (mtl_w4strip.hip) as 32-bit words: word (r, n) of a qweight [K/8, N]
// (channels 8r .. 8r+7 of column n) is word j = (r / 4) % 4 of 16-byte word
// l = 16 (r % 4) + n % 16 of 1 KB block (n / 16) * K/128 + r / 16.  Output index t of the
// layout maps back to (r, n) here.
__device__ __forceinline__ void strip_word_rn(int64_t t, int64_t kb, int64_t& r, int64_t& n) {
  const int64_t j = t & 3, l = (t >> 2) & 63, blk = t >> 8;
  const int64_t b = blk % kb, s = blk / kb;
  n = 16 * s + (l & 15);
  r = 16 * b + (l >> 4) + 4 * j;
}

__device__ __forceinline__ int64_t strip_word_index(int64_t r, int64_t n, int64_t kb) {
  return (((n >> 4) * kb + (r >> 4)) * 64 + 16 * (r & 3) + (n & 15)) * 4 + ((r >> 2) & 3);
}

// prepacked uint8 [N, K/2] (byte i of row n = q[n,2i] << 4 | q[n,2i+1]) -> the strip
// layout, whose word (r, n) holds the code of k = 8r + j in bits [4j, 4j+4).
__global__ void int4pack_convert_kernel(const uint8_t* __restrict__ pre, int64_t N, int64_t K,
                                        uint32_t* __restrict__ out) {
  const int64_t total = (K / 8) * N;
  const int64_t kb = K / 128;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    int64_t r, n;
    strip_word_rn(t, kb, r, n);
    const uint32_t b4 = *reinterpret_cast<const uint32_t*>(pre + n * (K / 2) + r * 4);
    uint32_t w = 0;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const uint32_t byte = (b4 >> (8 * jj)) & 0xffu;
      w |= (byte >> 4) << (4 * (2 * jj));          // even k: high nibble
      w |= (byte & 0xfu) << (4 * (2 * jj + 1));    // odd k: low nibble
    }
    out[t] = w;
  }
}

// torch's tiled int4 tensor (ROCm layout of aten._convert_weight_to_int4pack, inner_k_tiles
// T, half = T/2) -> qweight int32 [K/8, N].  torch stores 512-word blocks, one per
// (16 columns, 256 channels), the channel block the faster index.  Within a block, code
// (n, k) with r = k % 32, chunk j = (k % 256) / 32 and bits r4..r0 of r sits in word
// (b * 32 + c) * half + d, nibble e, where b = 2 * (j / half) + r3, d = j % half,
// c = 16 * r2 + n % 16 and e = r1 | r4 << 1 | r0 << 2.  Output word (q8, n) holds channels
// 8q8 .. 8q8+7: r3 and r4 come from q8, r2 splits them between two torch words
// (c = n % 16 for the first four, +16 for the last four).  Written in the strip layout.
__global__ void int4pack_from_torch_kernel(const uint32_t* __restrict__ tiles, int64_t N,
                                           int64_t K, int half, uint32_t* __restrict__ out) {
  const int64_t rows = K / 8;
  const int64_t total = rows * N;
  const int64_t kb = K / 256;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    int64_t q8, n;
    strip_word_rn(t, K / 128, q8, n);
    const int j = (int)(q8 >> 2) & 7;
    const int r3 = (int)q8 & 1, r4 = (int)(q8 >> 1) & 1;
    const int b = 2 * (j / half) + r3, d = j % half;
    const int64_t base = ((n >> 4) * kb + (q8 >> 5)) * 512;
    const uint32_t wa = tiles[base + (int64_t)(b * 32 + (int)(n & 15)) * half + d];
    const uint32_t wb = tiles[base + (int64_t)(b * 32 + 16 + (int)(n & 15)) * half + d];
    uint32_t w = 0;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const uint32_t src = jj < 4 ? wa : wb;
      const int e = ((jj >> 1) & 1) | (r4 << 1) | ((jj & 1) << 2);
      w |= ((src >> (4 * e)) & 0xfu) << (4 * jj);
    }
    out[t] = w;
  }
}

__global__ void unpack_codes_kernel(const uint32_t* __restrict__ qw, int64_t K, int64_t N,
                                    uint8_t* __restrict__ codes) {
  const int64_t total = (K / 8) * N;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / N;
    const int64_t n = t - r * N;
    const uint32_t w = qw[t];
#pragma unroll
    for (int j = 0; j < 8; ++j) codes[(r * 8 + j) * N + n] = (uint8_t)((w >> (4 * j)) & 0xfu);
  }
}

// Wave-contiguous layout of the GEMV weight stream: 16-byte word l of 1 KB block
// ((s * N/64 + cg) * 16 + q) holds qweight row 64s + 4q + l/16, columns 64cg + 4(l%16)..+3
// (rows past K/8 are zero).  One GEMV wave then reads 16 consecutive blocks.
__global__ void tile_weights_kernel(const uint4* __restrict__ qw, int64_t rows, int64_t N,
                                    int64_t splits, uint4* __restrict__ out) {
  const int64_t ncg = N / 64;
  const int64_t total = splits * ncg * 16 * 64;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t l = t & 63, blk = t >> 6;
    const int64_t q = blk & 15, sc = blk >> 4;
    const int64_t cg = sc % ncg, s = sc / ncg;
    const int64_t row = 64 * s + 4 * q + (l >> 4);
    const int64_t col = 64 * cg + 4 * (l & 15);
    out[t] = row < rows ? qw[(row * N + col) >> 2] : make_uint4(0u, 0u, 0u, 0u);
  }
}

// fp32 W[K, N]; fmt GPTQ: (q - (z + zero_offset)) * s over a qweight [K/8, N];
// QSZ: (q - 8) * scale + zero over the strip layout of mtl_int4pack_convert.
template <int FMT>
__global__ void dequant_kernel(const uint32_t* __restrict__ qw, const uint16_t* __restrict__ meta0,
                               const uint32_t* __restrict__ qzeros, int64_t K, int64_t N,
                               int group, int zero_offset, float* __restrict__ out) {
  const int64_t total = (K / 8) * N;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / N;
    const int64_t n = t - r * N;
    const uint32_t w = FMT == MTL_META_QSZ ? qw[strip_word_index(r, n, K / 128)] : qw[t];
    const int64_t grp = (r * 8) / group;
    float s, c, d;
    if (FMT == MTL_META_QSZ) {
      const uint16_t* q2 = meta0 + (grp * N + n) * 2;
      s = bf16_to_f32(q2[0]);
      d = bf16_to_f32(q2[1]);
      c = 8.f;
    } else {
      s = f16_to_f32(meta0[grp * N + n]);
      const uint32_t z = (qzeros[grp * (N / 8) + n / 8] >> (4 * (n & 7))) & 0xfu;
      c = (float)((int)z + zero_offset);
      d = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float q = (float)((w >> (4 * j)) & 0xfu);
      // (q - c) * s is exact in fp32, so this equals the unfused closed form.
      out[(r * 8 + j) * N + n] = fmaf(q - c, s, d);
    }
  }
}

// Stable counting sort of channels by group: one thread per group walks g_idx in order.
// err[0] is set when a group does not own exactly `group` channels or g_idx is out of range.
__global__ void actorder_perm_kernel(const int32_t* __restrict__ g_idx, int64_t K, int group,
                                     int32_t* __restrict__ perm, int32_t* __restrict__ err) {
  const int ngroups = (int)(K / group);
  for (int g = blockIdx.x * blockDim.x + threadIdx.x; g < ngroups; g += gridDim.x * blockDim.x) {
    int cnt = 0;
    for (int64_t k = 0; k < K; ++k) {
      const int gk = g_idx[k];
      if (gk < 0 || gk >= ngroups) { err[0] = 1; continue; }
      if (gk == g) {
        if (cnt < group) perm[(int64_t)g * group + cnt] = (int32_t)k;
        ++cnt;
      }
    }
    if (cnt != group) err[0] = 1;
  }
}

// qweight_sorted[r, n] nibble j = code of channel perm[8r + j] in the original layout.
__global__ void actorder_gather_kernel(const uint32_t* __restrict__ qw, const int32_t* __restrict__ perm,
                                       int64_t K, int64_t N, uint32_t* __restrict__ out) {
  const int64_t total = (K / 8) * N;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / N;
    const int64_t n = t - r * N;
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k = perm[r * 8 + j];
      const uint32_t src = qw[(k >> 3) * N + n];
      w |= ((src >> (4 * (k & 7))) & 0xfu) << (4 * j);
    }
    out[t] = w;
  }
}

__global__ void fill_u32_kernel_pack(uint32_t* p, int64_t n, uint32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

static int grid_for(int64_t total) {
  int64_t b = (total + 255) / 256;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return (int)b;
}

static bool valid_group(int g) { return g == 32 || g == 64 || g == 128 || g == 256; }

}  // namespace mtl

using namespace mtl;

extern "C" {

int mtl_int4pack_convert(const uint8_t* prepacked, int64_t N, int64_t K, int32_t inner_k_tiles,
                         int32_t* packed, void* stream) {
  if (!prepacked || !packed) return MTL_ERR_INVALID_ARG;
  if (inner_k_tiles != 2 && inner_k_tiles != 4 && inner_k_tiles != 8) return MTL_ERR_INVALID_ARG;
  if (N <= 0 || K <= 0 || K % 256 != 0 || N % 16 != 0) return MTL_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(prepacked) & 3u) || (reinterpret_cast<uintptr_t>(packed) & 3u))
    return MTL_ERR_ALIGN;
  const int64_t total = (K / 8) * N;
  hipLaunchKernelGGL(int4pack_convert_kernel, dim3(grid_for(total)), dim3(256), 0,
                     (hipStream_t)stream, prepacked, N, K, reinterpret_cast<uint32_t*>(packed));
  return launch_status();
}

int mtl_int4pack_from_torch_tiles(const int32_t* tiles, int64_t N, int64_t K,
                                  int32_t inner_k_tiles, int32_t* packed, void* stream) {
  if (!tiles || !packed) return MTL_ERR_INVALID_ARG;
  if (inner_k_tiles != 2 && inner_k_tiles != 4 && inner_k_tiles != 8) return MTL_ERR_INVALID_ARG;
  if (N <= 0 || K <= 0 || N % 16 != 0 || K % 256 != 0) return MTL_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(tiles) & 3u) || (reinterpret_cast<uintptr_t>(packed) & 3u))
    return MTL_ERR_ALIGN;
  const int64_t total = (K / 8) * N;
  hipLaunchKernelGGL(int4pack_from_torch_kernel, dim3(grid_for(total)), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint32_t*>(tiles), N, K,
                     inner_k_tiles / 2, reinterpret_cast<uint32_t*>(packed));
  return launch_status();
}

int64_t mtl_w4_tiled_bytes(int64_t K, int64_t N) {
  if (K <= 0 || N <= 0 || K % 8 != 0 || N % 64 != 0) return 0;
  const int64_t splits = (K / 8 + 63) / 64;
  return splits * (N / 64) * 16 * 1024;
}

int mtl_w4_tile(const int32_t* qweight, int64_t K, int64_t N, int32_t* tiled, int64_t tiled_bytes,
                void* stream) {
  if (!qweight || !tiled) return MTL_ERR_INVALID_ARG;
  if (K <= 0 || N <= 0 || K % 8 != 0 || N % 64 != 0) return MTL_ERR_SHAPE;
  const int64_t need = mtl_w4_tiled_bytes(K, N);
  if (tiled_bytes < need) return MTL_ERR_WORKSPACE;
  if ((reinterpret_cast<uintptr_t>(qweight) & 15u) || (reinterpret_cast<uintptr_t>(tiled) & 15u))
    return MTL_ERR_ALIGN;
  hipLaunchKernelGGL(tile_weights_kernel, dim3(grid_for(need / 16)), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint4*>(qweight), K / 8, N,
                     (K / 8 + 63) / 64, reinterpret_cast<uint4*>(tiled));
  return launch_status();
}

int mtl_unpack_codes(const int32_t* qweight, int64_t K, int64_t N, uint8_t* codes, void* stream) {
  if (!qweight || !codes) return MTL_ERR_INVALID_ARG;
  if (N <= 0 || K <= 0 || K % 8 != 0) return MTL_ERR_SHAPE;
  const int64_t total = (K / 8) * N;
  hipLaunchKernelGGL(unpack_codes_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const uint32_t*>(qweight), K, N, codes);
  return launch_status();
}

int mtl_gptq_dequant(const int32_t* qweight, const int32_t* qzeros, const void* scales, int64_t K,
                     int64_t N, int32_t group_size, int32_t zero_offset, float* w_out,
                     void* stream) {
  if (!qweight || !qzeros || !scales || !w_out) return MTL_ERR_INVALID_ARG;
  if (!valid_group(group_size)) return MTL_ERR_GROUP;
  if (N <= 0 || K <= 0 || K % group_size != 0 || N % 8 != 0) return MTL_ERR_SHAPE;
  const int64_t total = (K / 8) * N;
  hipLaunchKernelGGL((dequant_kernel<MTL_META_GPTQ>), dim3(grid_for(total)), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint32_t*>(qweight),
                     static_cast<const uint16_t*>(scales), reinterpret_cast<const uint32_t*>(qzeros),
                     K, N, group_size, zero_offset, w_out);
  return launch_status();
}

int mtl_qsz_dequant(const int32_t* packed, const void* qsz, int64_t K, int64_t N, int32_t group_size,
                    float* w_out, void* stream) {
  if (!packed || !qsz || !w_out) return MTL_ERR_INVALID_ARG;
  if (!valid_group(group_size)) return MTL_ERR_GROUP;
  if (N <= 0 || K <= 0 || K % group_size != 0 || K % 256 != 0 || N % 16 != 0)
    return MTL_ERR_SHAPE;
  const int64_t total = (K / 8) * N;
  hipLaunchKernelGGL((dequant_kernel<MTL_META_QSZ>), dim3(grid_for(total)), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const uint32_t*>(packed),
                     static_cast<const uint16_t*>(qsz), nullptr, K, N, group_size, 0, w_out);
  return launch_status();
}

int64_t mtl_actorder_scratch_bytes(int64_t K) {
  (void)K;
  return 256;
}

int mtl_gptq_actorder_prepare(const int32_t* qweight, const int32_t* g_idx, int64_t K, int64_t N,
                              int32_t group_size, int32_t* qweight_sorted, int32_t* perm,
                              void* scratch, int64_t scratch_bytes, void* stream) {
  if (!qweight || !g_idx || !qweight_sorted || !perm || !scratch) return MTL_ERR_INVALID_ARG;
  if (qweight == qweight_sorted) return MTL_ERR_INVALID_ARG;
  if (scratch_bytes < mtl_actorder_scratch_bytes(K)) return MTL_ERR_WORKSPACE;
  if (!valid_group(group_size)) return MTL_ERR_GROUP;
  if (N <= 0 || K <= 0 || K % group_size != 0 || N % 8 != 0) return MTL_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  int32_t* err = static_cast<int32_t*>(scratch);
  hipLaunchKernelGGL(fill_u32_kernel_pack, dim3(1), dim3(64), 0, s,
                     reinterpret_cast<uint32_t*>(err), (int64_t)1, 0u);
  const int ngroups = (int)(K / group_size);
  hipLaunchKernelGGL(actorder_perm_kernel, dim3((ngroups + 63) / 64), dim3(64), 0, s, g_idx, K,
                     group_size, perm, err);
  if (launch_status() != MTL_OK) return MTL_ERR_LAUNCH;
  // Load-time step: the group check needs the result on the host.
  int32_t h_err = 0;
  if (hipMemcpyAsync(&h_err, err, sizeof(int32_t), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return MTL_ERR_LAUNCH;
  if (h_err) return MTL_ERR_GROUP;
  const int64_t total = (K / 8) * N;
  hipLaunchKernelGGL(actorder_gather_kernel, dim3(grid_for(total)), dim3(256), 0, s,
                     reinterpret_cast<const uint32_t*>(qweight), perm, K, N,
                     reinterpret_cast<uint32_t*>(qweight_sorted));
  return launch_status();
}

}  // extern "C"
