// mtl_gptq_gemm_noalloc: the AutoGPTQ-layout int4 GEMM of mtl_gptq_gemm for callers that
// cannot allocate device memory (code under graph capture, tight serving loops).
//
// The split-K GEMM needs a workspace: a block of tile counters that must be zero when a
// launch starts (every launch leaves them zero again) followed by the fp32 partial tiles.
// Here that workspace is `scratch`, a file-scope device array of kScratchBytes. Each GPU
// the library runs on holds its own copy until the process ends. Host code never passes
// the array's name to a kernel or a copy: at the first call on a device (with that device
// current) hipGetSymbolAddress gives the device address, which is kept per device and
// used from then on. The same first call zero-fills the array with a kernel on the
// caller's stream.
//
// Every call on one GPU shares that GPU's array, so calls that overlap on one GPU (two
// streams, or two host threads) race; the caller orders them.
#include <hip/hip_runtime.h>

#include <mutex>

#include "mtl_common.h"
#include "mtl_gptq.h"

namespace {

constexpr int64_t kScratchBytes = MTL_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

std::mutex g_setup;
void* g_scratch[kMaxDevices] = {};

__global__ void zero_u32_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of this GPU's scratch array (set up once per device), or nullptr.
static void* device_scratch(hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_setup);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
      return nullptr;
    hipLaunchKernelGGL(zero_u32_kernel, dim3(1024), dim3(256), 0, stream,
                       static_cast<uint32_t*>(ptr), kScratchBytes / 4);
    if (hipGetLastError() != hipSuccess) return nullptr;
    g_scratch[dev] = ptr;
  }
  return g_scratch[dev];
}

extern "C" int mtl_gptq_gemm_noalloc(const void* x, int64_t M, int64_t K,
                                     const int32_t* qweight, const int32_t* qzeros,
                                     const void* scales, const int32_t* perm, int64_t N,
                                     int32_t group_size, int32_t zero_offset, void* y,
                                     int32_t out_dtype, void* stream) {
  const int64_t need = mtl_gemm_workspace_bytes(M, K, N, group_size);
  if (need > kScratchBytes) return MTL_ERR_WORKSPACE;
  void* ws = device_scratch(static_cast<hipStream_t>(stream));
  if (ws == nullptr) return MTL_ERR_LAUNCH;
  return mtl_gptq_gemm(x, M, K, qweight, qzeros, scales, perm, N, group_size, zero_offset, y,
                       out_dtype, ws, kScratchBytes, stream);
}
