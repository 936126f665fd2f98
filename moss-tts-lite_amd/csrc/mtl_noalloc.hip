// mtl_gptq_gemm_noalloc: the AutoGPTQ-layout int4 GEMM of mtl_gptq_gemm for callers that
// cannot allocate device memory (code under graph capture, tight serving loops).
//
// The split-K GEMM needs a workspace: a 16 KB block of tile counters followed by the fp32
// partial tiles.  mtl_gptq_gemm sums the partials in a second launch and reads no counter,
// and every partial it reads was written by the same call, so nothing in the workspace has
// to start at any value: the array is never cleared.  Here that workspace is `scratch`, a
// file-scope device array of kScratchBytes.  Each GPU the library runs on holds its own copy
// until the process ends.  Host code never passes the array's name to a kernel or a copy:
// at the first call on a device (with that device current) hipGetSymbolAddress gives the
// device address, which is kept per device and used from then on.  That lookup is not a
// stream operation, so a first call under graph capture records only the GEMM's launches.
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

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of this GPU's scratch array (looked up once per device), or nullptr.
static void* device_scratch() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_setup);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
      return nullptr;
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
  void* ws = device_scratch();
  if (ws == nullptr) return MTL_ERR_LAUNCH;
  return mtl_gptq_gemm(x, M, K, qweight, qzeros, scales, perm, N, group_size, zero_offset, y,
                       out_dtype, ws, kScratchBytes, stream);
}
