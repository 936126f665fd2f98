// torch dispatcher operators over the C ABI of libmtl_hip.so: mtl::weight_int4pack_mm and
// mtl::convert_weight_to_int4pack, the drop-ins for torch._weight_int4pack_mm and
// torch.ops.aten._convert_weight_to_int4pack that the reference calls eagerly
// (moss_tts_lite/fast.py:97-99, 118; gptq.py:75-76, 582; fast_native.py:169), and
// mtl::gptq_gemm / mtl::strip_rows_gemm / mtl::strip_gemv, the int4 products of the GPTQ
// linear module's forward over its AutoGPTQ tensors and their strip copy (the layer the
// reference's kernel_linear serves, gptq.py:577-585), so an eager module call costs one
// dispatcher call per launch group.
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

constexpr int64_t kMaxRows = 16;   // rows per launch of both GPTQ-layout entries

// x[..., K] as a contiguous bf16 [M, K] on one device with the weights
at::Tensor rows_of(const at::Tensor& x, int64_t K) {
  TORCH_CHECK(x.dim() >= 1 && x.size(-1) == K, "x must be [..., ", K, "], got ", x.sizes());
  TORCH_CHECK(x.scalar_type() == at::kBFloat16, "expected x to be bfloat16, got ",
              x.scalar_type());
  return x.reshape({-1, K}).contiguous();
}

std::vector<int64_t> out_shape(const at::Tensor& x, int64_t N) {
  std::vector<int64_t> s(x.sizes().begin(), x.sizes().end());
  s.back() = N;
  return s;
}

int32_t out_code(at::ScalarType dt) {
  TORCH_CHECK(dt == at::kBFloat16 || dt == at::kFloat, "out_dtype must be bfloat16 or float32");
  return dt == at::kFloat ? MTL_OUT_F32 : MTL_OUT_BF16;
}

void check_gptq_meta(const at::Tensor& qzeros, const at::Tensor& scales, int64_t K, int64_t N,
                     int64_t g) {
  TORCH_CHECK(g == 32 || g == 64 || g == 128 || g == 256,
              "group_size must be 32, 64, 128 or 256, got ", g);
  TORCH_CHECK(K % g == 0, "K=", K, " is not a multiple of group_size ", g);
  TORCH_CHECK(scales.scalar_type() == at::kHalf && scales.dim() == 2 && scales.size(0) == K / g &&
                  scales.size(1) == N,
              "scales must be float16 [", K / g, ", ", N, "]");
  TORCH_CHECK(qzeros.scalar_type() == at::kInt && qzeros.dim() == 2 && qzeros.size(0) == K / g &&
                  qzeros.size(1) == N / 8,
              "qzeros must be int32 [", K / g, ", ", N / 8, "]");
}

const int32_t* perm_ptr(const c10::optional<at::Tensor>& perm, int64_t K, at::Tensor& keep) {
  if (!perm.has_value()) return nullptr;
  TORCH_CHECK(perm->scalar_type() == at::kInt && perm->numel() == K, "perm must be int32 [", K, "]");
  keep = perm->contiguous();
  return keep.data_ptr<int32_t>();
}

// The split-K GEMM over the AutoGPTQ layout (mtl_gptq_gemm), 16 rows per launch; its split
// partials go to a workspace from torch's caching allocator (the entry sums them in a second
// launch and reads no counter, so the workspace needs no clearing).
at::Tensor gptq_gemm(const at::Tensor& x, const at::Tensor& qweight, const at::Tensor& qzeros,
                     const at::Tensor& scales, int64_t group_size,
                     const c10::optional<at::Tensor>& perm, int64_t zero_offset,
                     at::ScalarType out_dtype) {
  TORCH_CHECK(qweight.scalar_type() == at::kInt && qweight.dim() == 2,
              "qweight must be int32 [K/8, N]");
  const int64_t K = qweight.size(0) * 8, N = qweight.size(1);
  check_gptq_meta(qzeros, scales, K, N, group_size);
  const at::Tensor x2 = rows_of(x, K);
  TORCH_CHECK(x2.is_cuda() && qweight.device() == x2.device() && qzeros.device() == x2.device() &&
                  scales.device() == x2.device(),
              "x and the GPTQ tensors must be on one HIP device");
  const c10::DeviceGuard guard(x2.device());
  at::Tensor pk;
  const int32_t* pp = perm_ptr(perm, K, pk);
  const at::Tensor w = qweight.contiguous(), z = qzeros.contiguous(), sc = scales.contiguous();
  const int64_t M = x2.size(0);
  at::Tensor y = at::empty({M, N}, x2.options().dtype(out_dtype));
  const int32_t odt = out_code(out_dtype);
  if (M > 0) {
    const int64_t ws = mtl_gemm_workspace_bytes(std::min(M, kMaxRows), K, N, (int32_t)group_size);
    at::Tensor wsb = at::empty({(ws + 3) / 4}, x2.options().dtype(at::kFloat));
    const hipStream_t stream = c10::hip::getCurrentHIPStream(x2.device().index()).stream();
    const int64_t esz = y.element_size();
    for (int64_t r0 = 0; r0 < M; r0 += kMaxRows) {
      const int64_t rows = std::min(kMaxRows, M - r0);
      check_status(mtl_gptq_gemm(static_cast<const uint16_t*>(x2.data_ptr()) + r0 * K, rows, K,
                                 w.data_ptr<int32_t>(), z.data_ptr<int32_t>(), sc.data_ptr(), pp,
                                 N, (int32_t)group_size, (int32_t)zero_offset,
                                 static_cast<char*>(y.data_ptr()) + r0 * N * esz, odt,
                                 wsb.data_ptr(), wsb.numel() * 4, stream),
                   "mtl_gptq_gemm");
    }
  }
  return y.view(out_shape(x, N));
}

at::Tensor gptq_gemm_meta(const at::Tensor& x, const at::Tensor& qweight, const at::Tensor& qzeros,
                          const at::Tensor& scales, int64_t group_size,
                          const c10::optional<at::Tensor>& perm, int64_t zero_offset,
                          at::ScalarType out_dtype) {
  const int64_t K = qweight.size(0) * 8, N = qweight.size(1);
  check_gptq_meta(qzeros, scales, K, N, group_size);
  TORCH_CHECK(x.size(-1) == K, "x must be [..., ", K, "]");
  return at::empty(out_shape(x, N), x.options().dtype(out_dtype));
}

// The skinny strip GEMM (mtl_w4_gemm_strip_rows_ex) on the strip copy of an AutoGPTQ
// linear, 16 rows per launch, x gathered through perm for an act-order linear.
at::Tensor strip_rows_gemm(const at::Tensor& x, const at::Tensor& strip_weight,
                           const at::Tensor& qzeros, const at::Tensor& scales, int64_t n,
                           int64_t group_size, int64_t zero_offset,
                           const c10::optional<at::Tensor>& perm, at::ScalarType out_dtype) {
  const int64_t K = x.size(-1);
  check_gptq_meta(qzeros, scales, K, n, group_size);
  TORCH_CHECK(strip_weight.scalar_type() == at::kInt && strip_weight.numel() * 8 == n * K,
              "strip_weight must be the int32 strip copy of a [", K, ", ", n, "] weight");
  const at::Tensor x2 = rows_of(x, K);
  TORCH_CHECK(x2.is_cuda() && strip_weight.device() == x2.device() &&
                  qzeros.device() == x2.device() && scales.device() == x2.device(),
              "x and the GPTQ tensors must be on one HIP device");
  const c10::DeviceGuard guard(x2.device());
  at::Tensor pk;
  const int32_t* pp = perm_ptr(perm, K, pk);
  const at::Tensor w = strip_weight.contiguous(), z = qzeros.contiguous(), sc = scales.contiguous();
  const int64_t M = x2.size(0);
  at::Tensor y = at::empty({M, n}, x2.options().dtype(out_dtype));
  const int32_t odt = out_code(out_dtype);
  const hipStream_t stream = c10::hip::getCurrentHIPStream(x2.device().index()).stream();
  const int64_t esz = y.element_size();
  for (int64_t r0 = 0; r0 < M; r0 += kMaxRows) {
    const int64_t rows = std::min(kMaxRows, M - r0);
    check_status(mtl_w4_gemm_strip_rows_ex(static_cast<const uint16_t*>(x2.data_ptr()) + r0 * K,
                                           rows, K, K, pp, w.data_ptr<int32_t>(), sc.data_ptr(),
                                           z.data_ptr<int32_t>(), n, (int32_t)group_size,
                                           (int32_t)zero_offset, MTL_META_GPTQ,
                                           static_cast<char*>(y.data_ptr()) + r0 * n * esz, n, odt,
                                           stream),
                 "mtl_w4_gemm_strip_rows_ex");
  }
  return y.view(out_shape(x, n));
}

// One row on the full-K strip GEMV (mtl_w4_gemv_strip) over the strip copy of an AutoGPTQ
// linear and its strip-ordered metadata, x gathered through perm (int16, the act-order index
// narrowed) for an act-order linear.
at::Tensor strip_gemv(const at::Tensor& x, const at::Tensor& strip_weight,
                      const at::Tensor& strip_scales, const at::Tensor& strip_zeros, int64_t n,
                      int64_t group_size, int64_t zero_offset,
                      const c10::optional<at::Tensor>& perm, at::ScalarType out_dtype) {
  const int64_t K = x.size(-1);
  TORCH_CHECK(x.numel() == K, "strip_gemv takes one row of x, got ", x.sizes());
  TORCH_CHECK(strip_weight.scalar_type() == at::kInt && strip_weight.numel() * 8 == n * K,
              "strip_weight must be the int32 strip copy of a [", K, ", ", n, "] weight");
  TORCH_CHECK(strip_scales.scalar_type() == at::kHalf && strip_scales.numel() == n * K / group_size,
              "strip_scales must be the fp16 strip-ordered scales (mtl_w4_strip_meta)");
  TORCH_CHECK(strip_zeros.scalar_type() == at::kInt, "strip_zeros must be int32");
  const at::Tensor x2 = rows_of(x, K);
  TORCH_CHECK(x2.is_cuda() && strip_weight.device() == x2.device() &&
                  strip_scales.device() == x2.device() && strip_zeros.device() == x2.device(),
              "x and the strip tensors must be on one HIP device");
  const c10::DeviceGuard guard(x2.device());
  at::Tensor pk;
  const uint16_t* pp = nullptr;
  if (perm.has_value()) {
    TORCH_CHECK(perm->scalar_type() == at::kShort && perm->numel() == K,
                "perm must be int16 [", K, "] (the act-order index, narrowed)");
    pk = perm->contiguous();
    pp = reinterpret_cast<const uint16_t*>(pk.data_ptr());
  }
  const at::Tensor w = strip_weight.contiguous(), sc = strip_scales.contiguous(),
                   z = strip_zeros.contiguous();
  at::Tensor y = at::empty({1, n}, x2.options().dtype(out_dtype));
  const hipStream_t stream = c10::hip::getCurrentHIPStream(x2.device().index()).stream();
  check_status(mtl_w4_gemv_strip(x2.data_ptr(), K, pp, w.data_ptr<int32_t>(), sc.data_ptr(),
                                 z.data_ptr<int32_t>(), n, (int32_t)group_size,
                                 (int32_t)zero_offset, out_code(out_dtype), y.data_ptr(), stream),
               "mtl_w4_gemv_strip");
  return y.view(out_shape(x, n));
}

at::Tensor strip_gemv_meta(const at::Tensor& x, const at::Tensor& strip_weight,
                           const at::Tensor& strip_scales, const at::Tensor& strip_zeros,
                           int64_t n, int64_t group_size, int64_t zero_offset,
                           const c10::optional<at::Tensor>& perm, at::ScalarType out_dtype) {
  return at::empty(out_shape(x, n), x.options().dtype(out_dtype));
}

at::Tensor strip_rows_gemm_meta(const at::Tensor& x, const at::Tensor& strip_weight,
                                const at::Tensor& qzeros, const at::Tensor& scales, int64_t n,
                                int64_t group_size, int64_t zero_offset,
                                const c10::optional<at::Tensor>& perm, at::ScalarType out_dtype) {
  check_gptq_meta(qzeros, scales, x.size(-1), n, group_size);
  return at::empty(out_shape(x, n), x.options().dtype(out_dtype));
}

}  // namespace

TORCH_LIBRARY(mtl, m) {
  m.def("weight_int4pack_mm(Tensor x, Tensor packed, int q_group_size, "
        "Tensor q_scale_and_zeros) -> Tensor");
  m.def("convert_weight_to_int4pack(Tensor prepacked, int inner_k_tiles) -> Tensor");
  m.def("gptq_gemm(Tensor x, Tensor qweight, Tensor qzeros, Tensor scales, int group_size, "
        "Tensor? perm=None, int zero_offset=0, ScalarType out_dtype=bfloat16) -> Tensor");
  m.def("strip_rows_gemm(Tensor x, Tensor strip_weight, Tensor qzeros, Tensor scales, int n, "
        "int group_size, int zero_offset=0, Tensor? perm=None, "
        "ScalarType out_dtype=bfloat16) -> Tensor");
  m.def("strip_gemv(Tensor x, Tensor strip_weight, Tensor strip_scales, Tensor strip_zeros, "
        "int n, int group_size, int zero_offset=0, Tensor? perm=None, "
        "ScalarType out_dtype=bfloat16) -> Tensor");
}

TORCH_LIBRARY_IMPL(mtl, CUDA, m) {
  m.impl("weight_int4pack_mm", &weight_int4pack_mm);
  m.impl("convert_weight_to_int4pack", &convert_weight_to_int4pack);
  m.impl("gptq_gemm", &gptq_gemm);
  m.impl("strip_rows_gemm", &strip_rows_gemm);
  m.impl("strip_gemv", &strip_gemv);
}

TORCH_LIBRARY_IMPL(mtl, Meta, m) {
  m.impl("weight_int4pack_mm", &weight_int4pack_mm_meta);
  m.impl("convert_weight_to_int4pack", &convert_weight_to_int4pack_meta);
  m.impl("gptq_gemm", &gptq_gemm_meta);
  m.impl("strip_rows_gemm", &strip_rows_gemm_meta);
  m.impl("strip_gemv", &strip_gemv_meta);
}
