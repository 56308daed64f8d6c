// torch.ops.consumer_int8.* registration over the C ABI (libci8_amd.so).
//
// Same schemas, dispatch key and error wording as the reference's stable-ABI bindings
// (csrc/bindings.cpp:593-634): tensors are checked for device, dtype, contiguity and
// shape here; geometry, alignment and overlap rules are checked by the C ABI, whose
// messages become the RuntimeError text. Calls run on the current stream of the
// input's device under a device guard, allocate nothing and never synchronize.
#include <Python.h>
#include <torch/csrc/inductor/aoti_torch/c/shim.h>
#include <torch/csrc/stable/accelerator.h>
#include <torch/csrc/stable/library.h>
#include <torch/csrc/stable/tensor.h>
#include <torch/headeronly/util/Exception.h>

#include <climits>
#include <string>

#include "consumer_int8_amd.h"

using torch::headeronly::ScalarType;
using torch::stable::Tensor;

namespace {

// csrc/bindings.cpp:17-22
void check(const Tensor& t, ScalarType dtype, int device) {
  STD_TORCH_CHECK(t.is_cuda() && t.get_device_index() == device,
                  "All tensors must be on the same CUDA device");
  STD_TORCH_CHECK(t.is_contiguous() && t.scalar_type() == dtype,
                  "Unexpected dtype or noncontiguous tensor");
}

void* stream_for(int device) {
  void* stream = nullptr;
  TORCH_ERROR_CODE_CHECK(aoti_torch_get_current_cuda_stream(device, &stream));
  return stream;
}

void raise_on_error(int status) {
  STD_TORCH_CHECK(status == CI8_OK, std::string(ci8_last_error()));
}

bool same_sizes(const Tensor& a, const Tensor& b) {
  if (a.dim() != b.dim()) return false;
  for (int64_t i = 0; i < a.dim(); ++i)
    if (a.size(i) != b.size(i)) return false;
  return true;
}

// csrc/bindings.cpp:191-209
void quantize_rows(Tensor x, Tensor codes, Tensor scales) {
  const int device = x.get_device_index();
  check(x, ScalarType::BFloat16, device);
  check(codes, ScalarType::Char, device);
  check(scales, ScalarType::Float, device);
  STD_TORCH_CHECK(x.dim() == 2 && x.size(0) > 0 && x.size(1) > 0,
                  "Expected a nonempty BF16 matrix");
  STD_TORCH_CHECK(same_sizes(codes, x) && scales.dim() == 1 && scales.size(0) == x.size(0),
                  "Wrong output shapes");
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_quantize_rows(x.data_ptr(), static_cast<int8_t*>(codes.data_ptr()),
                                   static_cast<float*>(scales.data_ptr()), x.size(0),
                                   x.size(1), stream_for(device)));
}

// csrc/bindings.cpp:210-237
void quantize_grouped4096(Tensor x, Tensor codes, Tensor scales) {
  const int device = x.get_device_index();
  check(x, ScalarType::BFloat16, device);
  check(codes, ScalarType::Char, device);
  check(scales, ScalarType::Float, device);
  STD_TORCH_CHECK(
      x.dim() == 3 && x.size(1) > 0 && x.size(2) == 4096 && codes.dim() == 3 &&
          codes.size(0) == x.size(1) && codes.size(1) == x.size(0) && codes.size(2) == 4096 &&
          scales.dim() == 2 && scales.size(0) == x.size(1) && scales.size(1) == x.size(0),
      "Expected BF16 input[M,G,4096], INT8 codes[G,M,4096], FP32 scales[G,M]");
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_quantize_grouped4096(x.data_ptr(), static_cast<int8_t*>(codes.data_ptr()),
                                          static_cast<float*>(scales.data_ptr()), x.size(0),
                                          x.size(1), stream_for(device)));
}

// csrc/bindings.cpp:386-424 (shared by fused_channel_mm and cutlass_channel_mm)
void check_gemm_tensors(const Tensor& a, const Tensor& w, const Tensor& sa, const Tensor& sw,
                        const Tensor& out, ScalarType w_dtype, const char* geometry) {
  const int device = a.get_device_index();
  check(a, ScalarType::Char, device);
  check(w, w_dtype, device);
  check(sa, ScalarType::Float, device);
  check(sw, ScalarType::BFloat16, device);
  check(out, ScalarType::BFloat16, device);
  STD_TORCH_CHECK(a.dim() == 2 && w.dim() == 2 && out.dim() == 2, "Expected matrices");
  const int64_t m = a.size(0), n = w.size(0), k = a.size(1);
  STD_TORCH_CHECK(w.size(1) == k && out.size(0) == m && out.size(1) == n && sa.dim() == 1 &&
                      sw.dim() == 1 && sa.size(0) == m && sw.size(0) == n,
                  geometry);
}

void fused_channel_mm(Tensor a, Tensor w, Tensor sa, Tensor sw, Tensor out, int64_t schedule) {
  check_gemm_tensors(a, w, sa, sw, out, ScalarType::Char, "Invalid CUTLASS geometry");
  const int device = a.get_device_index();
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_fused_channel_mm(
      static_cast<int8_t*>(a.data_ptr()), static_cast<int8_t*>(w.data_ptr()),
      static_cast<float*>(sa.data_ptr()), sw.data_ptr(), out.data_ptr(), a.size(0), w.size(0),
      a.size(1), schedule, stream_for(device)));
}

void cutlass_channel_mm(Tensor a, Tensor w, Tensor sa, Tensor sw, Tensor workspace,
                        Tensor out) {
  check_gemm_tensors(a, w, sa, sw, out, ScalarType::Char, "Invalid CUTLASS geometry");
  const int device = a.get_device_index();
  check(workspace, ScalarType::Int, device);
  STD_TORCH_CHECK(same_sizes(workspace, out), "Expected matching workspace");
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_cutlass_channel_mm(
      static_cast<int8_t*>(a.data_ptr()), static_cast<int8_t*>(w.data_ptr()),
      static_cast<float*>(sa.data_ptr()), sw.data_ptr(),
      static_cast<int32_t*>(workspace.data_ptr()), out.data_ptr(), a.size(0), w.size(0),
      a.size(1), stream_for(device)));
}

// csrc/bindings.cpp:238-265
void channel_mm(Tensor a, Tensor w, Tensor sa, Tensor sw, Tensor out) {
  const int device = a.get_device_index();
  check(a, ScalarType::Char, device);
  check(w, ScalarType::Byte, device);
  check(sa, ScalarType::Float, device);
  check(sw, ScalarType::BFloat16, device);
  check(out, ScalarType::BFloat16, device);
  STD_TORCH_CHECK(a.dim() == 2 && w.dim() == 2 && out.dim() == 2, "Expected matrices");
  const int64_t m = a.size(0), n = w.size(0), k = a.size(1);
  STD_TORCH_CHECK(m > 0 && n > 0 && k > 0 && k % 32 == 0 && k <= 65536 && w.size(1) == k,
                  "Invalid matrix geometry");
  STD_TORCH_CHECK(sa.dim() == 1 && sa.size(0) == m && sw.dim() == 1 && sw.size(0) == n &&
                      out.size(0) == m && out.size(1) == n,
                  "Wrong scale or output shapes");
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_channel_mm(static_cast<int8_t*>(a.data_ptr()),
                                static_cast<uint8_t*>(w.data_ptr()),
                                static_cast<float*>(sa.data_ptr()), sw.data_ptr(),
                                out.data_ptr(), m, n, k, stream_for(device)));
}

// No reference op: configs[4]'s grouped W8A8 with the group partials scaled and summed.
void grouped_summed_mm(Tensor a, Tensor w, Tensor sa, Tensor sw, Tensor out) {
  const int device = a.get_device_index();
  check(a, ScalarType::Char, device);
  check(w, ScalarType::Char, device);
  check(sa, ScalarType::Float, device);
  check(sw, ScalarType::BFloat16, device);
  check(out, ScalarType::BFloat16, device);
  STD_TORCH_CHECK(a.dim() == 3 && w.dim() == 3 && sa.dim() == 2 && sw.dim() == 1 &&
                      out.dim() == 2,
                  "Expected INT8 a[G,M,K], INT8 w[G,N,K], FP32 a_scale[G,M], BF16 "
                  "w_scale[N], BF16 out[M,N]");
  const int64_t g = a.size(0), m = a.size(1), k = a.size(2), n = w.size(1);
  STD_TORCH_CHECK(w.size(0) == g && w.size(2) == k && sa.size(0) == g && sa.size(1) == m &&
                      sw.size(0) == n && out.size(0) == m && out.size(1) == n,
                  "Expected INT8 a[G,M,K], INT8 w[G,N,K], FP32 a_scale[G,M], BF16 "
                  "w_scale[N], BF16 out[M,N]");
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_grouped_summed_mm(static_cast<int8_t*>(a.data_ptr()),
                                       static_cast<int8_t*>(w.data_ptr()),
                                       static_cast<float*>(sa.data_ptr()), sw.data_ptr(),
                                       out.data_ptr(), g, m, n, k, stream_for(device)));
}

// csrc/bindings.cpp:289-310
void channel_gemv(Tensor x, Tensor w, Tensor scale, Tensor out) {
  const int device = x.get_device_index();
  check(x, ScalarType::BFloat16, device);
  check(w, ScalarType::Char, device);
  check(scale, ScalarType::BFloat16, device);
  check(out, ScalarType::BFloat16, device);
  STD_TORCH_CHECK(x.dim() == 2 && w.dim() == 2 && out.dim() == 2 && scale.dim() == 1,
                  "Expected input/weight/output matrices and channel scales");
  const int64_t m = x.size(0), n = w.size(0), k = x.size(1);
  STD_TORCH_CHECK(w.size(1) == k && scale.size(0) == n && out.size(0) == m && out.size(1) == n,
                  "Unsupported W8A16 GEMV geometry");
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_channel_gemv(x.data_ptr(), static_cast<int8_t*>(w.data_ptr()),
                                  scale.data_ptr(), out.data_ptr(), m, n, k,
                                  stream_for(device)));
}

// csrc/bindings.cpp:32-44
void silu_mul(Tensor x, Tensor out) {
  const int device = x.get_device_index();
  check(x, ScalarType::BFloat16, device);
  check(out, ScalarType::BFloat16, device);
  STD_TORCH_CHECK(x.dim() == 2 && out.dim() == 2 &&
                      (out.size(1) == 8704 || out.size(1) == 17408) &&
                      x.size(1) == 2 * out.size(1) && x.size(0) == out.size(0) &&
                      x.numel() <= INT_MAX,
                  "Unsupported SwiGLU shape");
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_silu_mul(x.data_ptr(), out.data_ptr(), x.size(0), out.size(1),
                              stream_for(device)));
}

// csrc/bindings.cpp:46-64
void silu_mul_quantize(Tensor x, Tensor codes, Tensor scales) {
  const int device = x.get_device_index();
  check(x, ScalarType::BFloat16, device);
  check(codes, ScalarType::Char, device);
  check(scales, ScalarType::Float, device);
  STD_TORCH_CHECK(x.dim() == 2 && codes.dim() == 2 && scales.dim() == 1 &&
                      (codes.size(1) == 8704 || codes.size(1) == 17408) &&
                      x.size(1) == 2 * codes.size(1) && x.size(0) == codes.size(0) &&
                      scales.size(0) == x.size(0) && x.numel() <= INT_MAX,
                  "Unsupported SwiGLU quantization shape");
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_silu_mul_quantize(x.data_ptr(), static_cast<int8_t*>(codes.data_ptr()),
                                       static_cast<float*>(scales.data_ptr()), x.size(0),
                                       codes.size(1), stream_for(device)));
}

// csrc/bindings.cpp:266-288
void unpack_allspark(Tensor packed, Tensor packed_scales, Tensor weight, Tensor scales) {
  const int device = packed.get_device_index();
  check(packed, ScalarType::Byte, device);
  check(packed_scales, ScalarType::BFloat16, device);
  check(weight, ScalarType::Char, device);
  check(scales, ScalarType::BFloat16, device);
  STD_TORCH_CHECK(packed.dim() == 2 && weight.dim() == 2 && packed_scales.dim() == 1 &&
                      scales.dim() == 1,
                  "Wrong tensor ranks");
  const int64_t n = weight.size(0), k = weight.size(1), padded_n = (n + 31) / 32 * 32;
  STD_TORCH_CHECK(n > 0 && n % 16 == 0 && k > 0 && k <= 65536 && k % 16 == 0 &&
                      packed.size(0) == padded_n && packed.size(1) == k &&
                      packed_scales.size(0) == padded_n && scales.size(0) == n,
                  "Expected AllSpark N32K16 weights and channel scales");
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_unpack_allspark(static_cast<uint8_t*>(packed.data_ptr()),
                                     packed_scales.data_ptr(),
                                     static_cast<int8_t*>(weight.data_ptr()), scales.data_ptr(),
                                     n, k, stream_for(device)));
}

// csrc/gguf_bindings.cpp:135-171: x may be strided over rows and groups (K contiguous);
// the C ABI checks strides, sizes, alignment and aliasing.
void gguf_q8_packed_mm(Tensor x, Tensor codes, Tensor scales, Tensor out) {
  const int device = x.get_device_index();
  STD_TORCH_CHECK(x.is_cuda() && codes.is_cuda() && scales.is_cuda() && out.is_cuda() &&
                      codes.get_device_index() == device &&
                      scales.get_device_index() == device && out.get_device_index() == device,
                  "Packed Q8 tensors must share a CUDA device");
  STD_TORCH_CHECK(x.scalar_type() == ScalarType::BFloat16 &&
                      codes.scalar_type() == ScalarType::Char &&
                      scales.scalar_type() == ScalarType::Half &&
                      out.scalar_type() == ScalarType::BFloat16,
                  "Packed Q8 requires BF16 input/output, INT8 codes and original FP16 scales");
  STD_TORCH_CHECK(x.dim() == 3 && codes.dim() == 3 && scales.dim() == 3 && out.dim() == 3,
                  "Expected x[M,G,K], q[G,N,K], scales[G,N,K/32], out[M,G,N]");
  const int64_t m = x.size(0), groups = x.size(1), k = x.size(2), n = codes.size(1);
  STD_TORCH_CHECK(codes.is_contiguous() && scales.is_contiguous() && out.is_contiguous() &&
                      x.stride(2) == 1 && x.stride(0) > 0 && x.stride(1) > 0 && k > 0 &&
                      k % 64 == 0 && codes.size(0) == groups && codes.size(2) == k &&
                      scales.size(0) == groups && scales.size(1) == n &&
                      scales.size(2) == k / 32 && out.size(0) == m && out.size(1) == groups &&
                      out.size(2) == n,
                  "Invalid packed Q8 shape/strides; K must be a multiple of 64");
  torch::stable::accelerator::DeviceGuard guard(device);
  raise_on_error(ci8_gguf_q8_packed_mm(x.data_ptr(), static_cast<int8_t*>(codes.data_ptr()),
                                       scales.data_ptr(), out.data_ptr(), m, n, k, groups,
                                       x.stride(0), x.stride(1), stream_for(device)));
}

}  // namespace

// Schemas: csrc/bindings.cpp:594-595, 598, 603-607, 610 and csrc/gguf_bindings.cpp:496;
// grouped_summed_mm has no reference op.
STABLE_TORCH_LIBRARY(consumer_int8, m) {
  m.def("fused_channel_mm(Tensor a, Tensor w, Tensor a_scale, Tensor w_scale, Tensor(a!) out, int schedule=0) -> ()");
  m.def("quantize_rows(Tensor input, Tensor(a!) codes, Tensor(b!) scales) -> ()");
  m.def("quantize_grouped4096(Tensor input, Tensor(a!) codes, Tensor(b!) scales) -> ()");
  m.def("channel_mm(Tensor a, Tensor w, Tensor a_scale, Tensor w_scale, Tensor(a!) out) -> ()");
  m.def("channel_gemv(Tensor x, Tensor w, Tensor scale, Tensor(a!) out) -> ()");
  m.def("cutlass_channel_mm(Tensor a, Tensor w, Tensor a_scale, Tensor w_scale, Tensor(a!) workspace, Tensor(b!) out) -> ()");
  m.def("grouped_summed_mm(Tensor a, Tensor w, Tensor a_scale, Tensor w_scale, Tensor(a!) out) -> ()");
  m.def("silu_mul(Tensor input, Tensor(a!) out) -> ()");
  m.def("silu_mul_quantize(Tensor input, Tensor(a!) codes, Tensor(b!) scales) -> ()");
  m.def("unpack_allspark(Tensor packed, Tensor packed_scales, Tensor(a!) weight, Tensor(b!) scales) -> ()");
  m.def("gguf_q8_packed_mm(Tensor x, Tensor codes, Tensor scales, Tensor(a!) out) -> ()");
}

// HIP tensors carry the CUDA dispatch key in PyTorch-ROCm.
STABLE_TORCH_LIBRARY_IMPL(consumer_int8, CUDA, m) {
  m.impl("fused_channel_mm", TORCH_BOX(&fused_channel_mm));
  m.impl("quantize_rows", TORCH_BOX(&quantize_rows));
  m.impl("quantize_grouped4096", TORCH_BOX(&quantize_grouped4096));
  m.impl("channel_mm", TORCH_BOX(&channel_mm));
  m.impl("channel_gemv", TORCH_BOX(&channel_gemv));
  m.impl("cutlass_channel_mm", TORCH_BOX(&cutlass_channel_mm));
  m.impl("grouped_summed_mm", TORCH_BOX(&grouped_summed_mm));
  m.impl("silu_mul", TORCH_BOX(&silu_mul));
  m.impl("silu_mul_quantize", TORCH_BOX(&silu_mul_quantize));
  m.impl("unpack_allspark", TORCH_BOX(&unpack_allspark));
  m.impl("gguf_q8_packed_mm", TORCH_BOX(&gguf_q8_packed_mm));
}

extern "C" PyObject* PyInit__C() {
  static PyModuleDef module = {PyModuleDef_HEAD_INIT, "_C", nullptr, -1, nullptr};
  return PyModule_Create(&module);
}
