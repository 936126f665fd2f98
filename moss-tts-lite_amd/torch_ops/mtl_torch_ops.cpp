// torch dispatcher operators over the C ABI of libmtl_hip.so: mtl::weight_int4pack_mm and
// mtl::convert_weight_to_int4pack, the drop-ins for torch._weight_int4pack_mm and
// torch.ops.aten._convert_weight_to_int4pack that the reference calls eagerly
// (moss_tts_lite/fast.py:97-99, 118; gptq.py:75-76, 582; fast_native.py:169).
//
// Host code only: each operator checks its tensors, allocates the output (and the split-K
// workspace) from torch's caching allocator, and calls the C entry on torch's current
// stream of the input's device, so eager calls skip the Python and ctypes layers and a
// graph capture records the kernels like any torch operator.  Meta kernels give the output
// shapes to tracing.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "mtl_gptq.h"

namespace {

void check_status(int status, const char* what) {
  TORCH_CHECK(status == 0, what, ": ", mtl_status_string(status), " (status ", status, ")");
}

void check_pack_args(const at::Tensor& x, const at::Tensor& packed, int64_t g,
                     const at::Tensor& qsz, int64_t& K, int64_t& N) {
  TORCH_CHECK(x.dim() == 2, "x must be 2-D [M, K], got ", x.sizes());
  TORCH_CHECK(x.scalar_type() == at::kBFloat16, "expected x to be bfloat16, got ",
              x.scalar_type());
  TORCH_CHECK(qsz.scalar_type() == at::kBFloat16 && qsz.dim() == 3 && qsz.size(2) == 2,
              "qScaleAndZeros must be bfloat16 [K/g, N, 2]");
  TORCH_CHECK(g == 32 || g == 64 || g == 128 || g == 256,
              "qGroupSize must be 32, 64, 128 or 256, got ", g);
  K = qsz.size(0) * g;
  N = qsz.size(1);
  TORCH_CHECK(x.size(1) == K, "x has K=", x.size(1), ", weight expects K=", K);
  TORCH_CHECK(packed.scalar_type() == at::kInt && packed.dim() == 4 && packed.size(0) * 8 == N &&
                  packed.numel() * 8 == N * K,
              "packed weight must be int32 [N/8, K/(16*T), 32, T/2] for N=", N, ", K=", K);
}

at::Tensor weight_int4pack_mm(const at::Tensor& x, const at::Tensor& packed, int64_t g,
                              const at::Tensor& qsz) {
  int64_t K = 0, N = 0;
  check_pack_args(x, packed, g, qsz, K, N);
  TORCH_CHECK(x.is_cuda() && packed.device() == x.device() && qsz.device() == x.device(),
              "x, packed and qScaleAndZeros must be on one HIP device");
  const c10::DeviceGuard guard(x.device());
  const at::Tensor x2 = x.contiguous();
  const at::Tensor w = packed.contiguous();
  const at::Tensor q = qsz.contiguous();
  const int64_t M = x2.size(0);
  at::Tensor y = at::empty({M, N}, x2.options());
  if (M == 0) return y;
  const int64_t ws = mtl_int4pack_mm_workspace_bytes(M, K, N);
  at::Tensor wsb;
  if (ws > 0) wsb = at::empty({(ws + 3) / 4}, x2.options().dtype(at::kFloat));
  const hipStream_t stream = c10::hip::getCurrentHIPStream(x2.device().index()).stream();
  check_status(mtl_int4pack_mm(x2.data_ptr(), M, K, w.data_ptr<int32_t>(), (int32_t)g,
                               q.data_ptr(), N, y.data_ptr(), ws > 0 ? wsb.data_ptr() : nullptr,
                               ws > 0 ? wsb.numel() * 4 : 0, stream),
               "mtl_int4pack_mm");
  return y;
}

at::Tensor weight_int4pack_mm_meta(const at::Tensor& x, const at::Tensor& packed, int64_t g,
                                   const at::Tensor& qsz) {
  int64_t K = 0, N = 0;
  check_pack_args(x, packed, g, qsz, K, N);
  return at::empty({x.size(0), N}, x.options());
}

std::vector<int64_t> int4pack_shape(const at::Tensor& pre, int64_t tiles) {
  TORCH_CHECK(pre.scalar_type() == at::kByte && pre.dim() == 2, "expected a uint8 [N, K/2] tensor");
  TORCH_CHECK(tiles == 2 || tiles == 4 || tiles == 8, "innerKTiles must be 2, 4 or 8");
  const int64_t n = pre.size(0), k = pre.size(1) * 2;
  TORCH_CHECK(k % 256 == 0 && n % 16 == 0, "K=", k, " must be a multiple of 256 and N=", n,
              " a multiple of 16");
  return {n / 8, k / (16 * tiles), 32, tiles / 2};
}

at::Tensor convert_weight_to_int4pack(const at::Tensor& pre, int64_t tiles) {
  const auto shape = int4pack_shape(pre, tiles);
  TORCH_CHECK(pre.is_cuda(), "the int4 packer runs on a HIP device");
  const c10::DeviceGuard guard(pre.device());
  const at::Tensor src = pre.contiguous();
  at::Tensor out = at::empty(shape, src.options().dtype(at::kInt));
  const hipStream_t stream = c10::hip::getCurrentHIPStream(src.device().index()).stream();
  check_status(mtl_int4pack_convert(src.data_ptr<uint8_t>(), src.size(0), src.size(1) * 2,
                                    (int32_t)tiles, out.data_ptr<int32_t>(), stream),
               "mtl_int4pack_convert");
  return out;
}

at::Tensor convert_weight_to_int4pack_meta(const at::Tensor& pre, int64_t tiles) {
  return at::empty(int4pack_shape(pre, tiles), pre.options().dtype(at::kInt));
}

}  // namespace

TORCH_LIBRARY(mtl, m) {
  m.def("weight_int4pack_mm(Tensor x, Tensor packed, int q_group_size, "
        "Tensor q_scale_and_zeros) -> Tensor");
  m.def("convert_weight_to_int4pack(Tensor prepacked, int inner_k_tiles) -> Tensor");
}

TORCH_LIBRARY_IMPL(mtl, CUDA, m) {
  m.impl("weight_int4pack_mm", &weight_int4pack_mm);
  m.impl("convert_weight_to_int4pack", &convert_weight_to_int4pack);
}

TORCH_LIBRARY_IMPL(mtl, Meta, m) {
  m.impl("weight_int4pack_mm", &weight_int4pack_mm_meta);
  m.impl("convert_weight_to_int4pack", &convert_weight_to_int4pack_meta);
}
