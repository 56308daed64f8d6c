// The C ABI (include/consumer_int8_amd.h): argument validation, then the launch.
//
// Validation is pure host code and runs before any HIP call, so every rejection can be
// exercised on a machine without a GPU. Messages reuse the reference's wording
// (csrc/bindings.cpp) so callers matching on it keep working.
#include "consumer_int8_amd.h"

#include <climits>
#include <cstdint>
#include <cstdio>
#include <string>

#include "launch.h"

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* message) {
  g_last_error = message;
  return status;
}

int launched(hipError_t error) {
  if (error != hipSuccess) {
    g_last_error = std::string("HIP launch failed: ") + hipGetErrorString(error);
    return CI8_ERR_LAUNCH;
  }
  g_last_error.clear();
  return CI8_OK;
}

bool aligned(const void* p, uintptr_t bytes) {
  return reinterpret_cast<uintptr_t>(p) % bytes == 0;
}

bool overlap(const void* a, int64_t bytes_a, const void* b, int64_t bytes_b) {
  const auto first = reinterpret_cast<uintptr_t>(a);
  const auto second = reinterpret_cast<uintptr_t>(b);
  return bytes_a > 0 && bytes_b > 0 && first < second + uint64_t(bytes_b) &&
         second < first + uint64_t(bytes_a);
}

hipStream_t as_stream(void* stream) { return static_cast<hipStream_t>(stream); }

// Shared GEMM geometry (csrc/bindings.cpp:402-408 for the signed ops,
// csrc/bindings.cpp:252-258 for channel_mm).
int check_gemm(int64_t m, int64_t n, int64_t k, bool need_n4, const char* what) {
  if (!(m > 0 && n > 0 && k > 0 && k % 32 == 0 && k <= 65536 && (!need_n4 || n % 4 == 0)))
    return fail(CI8_ERR_GEOMETRY, what);
  if (m * k > INT_MAX || n * k > INT_MAX || m * n > INT_MAX)
    return fail(CI8_ERR_TOO_LARGE, "Matrix too large");
  return CI8_OK;
}

// benchmarks/cuda/q8_block_int8.cu:142-174: m, n, k > 0 and k % 32 == 0.
int check_q8(int64_t m, int64_t n, int64_t k) {
  if (!(m > 0 && n > 0 && k > 0 && k % 32 == 0))
    return fail(CI8_ERR_GEOMETRY, "Invalid block-32 geometry");
  if (m * k > INT_MAX || n * k > INT_MAX || m * n > INT_MAX)
    return fail(CI8_ERR_TOO_LARGE, "Matrix too large");
  return CI8_OK;
}

}  // namespace

extern "C" {

const char* ci8_last_error(void) { return g_last_error.c_str(); }

const char* ci8_version(void) { return "0.1.0"; }

int ci8_quantize_rows(const void* x, int8_t* codes, float* scales, int64_t m, int64_t k,
                      void* stream) {
  if (!(m > 0 && k > 0)) return fail(CI8_ERR_GEOMETRY, "Expected a nonempty BF16 matrix");
  if (m * k > INT_MAX) return fail(CI8_ERR_TOO_LARGE, "Matrix too large");
  if (!aligned(x, 2) || !aligned(scales, 4))
    return fail(CI8_ERR_ALIGNMENT, "quantize_rows requires aligned buffers");
  return launched(ci8::launch_quantize_rows(x, codes, scales, int(m), int(k), as_stream(stream)));
}

int ci8_quantize_grouped4096(const void* x, int8_t* codes, float* scales, int64_t m,
                             int64_t groups, void* stream) {
  constexpr int64_t kWidth = 4096;
  if (!(m >= 0 && groups > 0))
    return fail(CI8_ERR_GEOMETRY,
                "Expected BF16 input[M,G,4096], INT8 codes[G,M,4096], FP32 scales[G,M]");
  if (m * groups * kWidth > INT_MAX)
    return fail(CI8_ERR_GEOMETRY,
                "Expected BF16 input[M,G,4096], INT8 codes[G,M,4096], FP32 scales[G,M]");
  if (!aligned(x, 16) || !aligned(codes, 8) || !aligned(scales, 4))
    return fail(CI8_ERR_ALIGNMENT, "Grouped quantization requires aligned buffers");
  const int64_t elems = m * groups * kWidth;
  if (overlap(x, elems * 2, codes, elems) || overlap(x, elems * 2, scales, m * groups * 4) ||
      overlap(codes, elems, scales, m * groups * 4))
    return fail(CI8_ERR_OVERLAP, "Grouped quantization buffers must not overlap");
  return launched(ci8::launch_quantize_grouped(x, codes, scales, int(m), int(groups),
                                               int(kWidth), as_stream(stream)));
}

int ci8_fused_channel_mm(const int8_t* a, const int8_t* w, const float* a_scale,
                         const void* w_scale, void* out, int64_t m, int64_t n, int64_t k,
                         int64_t schedule, void* stream) {
  if (int s = check_gemm(m, n, k, true, "Invalid CUTLASS geometry")) return s;
  if (!(schedule >= 0 && schedule <= 6))
    return fail(CI8_ERR_SCHEDULE, "Invalid fused GEMM schedule");
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(a_scale, 4) || !aligned(w_scale, 2) ||
      !aligned(out, 2))
    return fail(CI8_ERR_ALIGNMENT, "fused_channel_mm requires aligned buffers");
  return launched(ci8::launch_channel_gemm(a, w, ci8::WeightCode::kSigned, a_scale, w_scale,
                                           out, nullptr, int(m), int(n), int(k), int(schedule),
                                           as_stream(stream)));
}

int ci8_cutlass_channel_mm(const int8_t* a, const int8_t* w, const float* a_scale,
                           const void* w_scale, int32_t* workspace, void* out, int64_t m,
                           int64_t n, int64_t k, void* stream) {
  if (int s = check_gemm(m, n, k, true, "Invalid CUTLASS geometry")) return s;
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(a_scale, 4) || !aligned(w_scale, 2) ||
      !aligned(out, 2) || !aligned(workspace, 4))
    return fail(CI8_ERR_ALIGNMENT, "cutlass_channel_mm requires aligned buffers");
  return launched(ci8::launch_channel_gemm(a, w, ci8::WeightCode::kSigned, a_scale, w_scale,
                                           out, workspace, int(m), int(n), int(k), 0,
                                           as_stream(stream)));
}

int ci8_cutlass_channel_mm_noalloc(const int8_t* a, const int8_t* w, const float* a_scale,
                                   const void* w_scale, void* out, int64_t m, int64_t n,
                                   int64_t k, void* stream) {
  if (int s = check_gemm(m, n, k, true, "Invalid CUTLASS geometry")) return s;
  if (m * n > ci8::noalloc_scratch_ints())
    return fail(CI8_ERR_TOO_LARGE,
                "cutlass_channel_mm_noalloc: m * n exceeds the library's scratch of "
                "8388608 INT32 accumulators; use cutlass_channel_mm with a workspace");
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(a_scale, 4) || !aligned(w_scale, 2) ||
      !aligned(out, 2))
    return fail(CI8_ERR_ALIGNMENT, "cutlass_channel_mm requires aligned buffers");
  const hipError_t e = ci8::launch_cutlass_channel_mm_noalloc(a, w, a_scale, w_scale, out,
                                                              int(m), int(n), int(k),
                                                              as_stream(stream));
  if (e == hipErrorStreamCaptureUnsupported)
    return fail(CI8_ERR_LAUNCH,
                "cutlass_channel_mm_noalloc: the first call on a device must run outside "
                "graph capture (it looks up the device's scratch address)");
  return launched(e);
}

int ci8_channel_mm(const int8_t* a, const uint8_t* w_u8, const float* a_scale,
                   const void* w_scale, void* out, int64_t m, int64_t n, int64_t k,
                   void* stream) {
  if (!(m > 0 && n > 0 && k > 0 && k % 32 == 0 && k <= 65536))
    return fail(CI8_ERR_GEOMETRY, "Invalid matrix geometry");
  if (m * k > INT_MAX || n * k > INT_MAX || m * n > INT_MAX)
    return fail(CI8_ERR_TOO_LARGE, "Matrix too large");
  if (!aligned(a_scale, 4) || !aligned(w_scale, 2) || !aligned(out, 2))
    return fail(CI8_ERR_ALIGNMENT, "channel_mm requires aligned buffers");
  // The reference accepts operands at any offset (csrc/bindings.cpp:238-265); the MFMA
  // kernels copy 16-byte chunks, so other alignments take the byte-load kernel.
  if (!aligned(a, 16) || !aligned(w_u8, 16))
    return launched(ci8::launch_channel_gemm_bytes(a, w_u8, ci8::WeightCode::kBiasedU8,
                                                   a_scale, w_scale, out, int(m), int(n),
                                                   int(k), as_stream(stream)));
  return launched(ci8::launch_channel_gemm(a, w_u8, ci8::WeightCode::kBiasedU8, a_scale,
                                           w_scale, out, nullptr, int(m), int(n), int(k), 0,
                                           as_stream(stream)));
}

int ci8_grouped_summed_mm(const int8_t* a, const int8_t* w, const float* a_scale,
                          const void* w_scale, void* out, int64_t groups, int64_t m,
                          int64_t n, int64_t k, void* stream) {
  if (groups <= 0) return fail(CI8_ERR_GEOMETRY, "Invalid grouped GEMM geometry");
  const int status = check_gemm(m, n, k, true, "Invalid grouped GEMM geometry");
  if (status != CI8_OK) return status;
  if (groups * m > INT_MAX || groups > 65536)
    return fail(CI8_ERR_TOO_LARGE, "Matrix too large");
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(a_scale, 4) || !aligned(w_scale, 2) ||
      !aligned(out, 2))
    return fail(CI8_ERR_ALIGNMENT, "grouped_summed_mm requires aligned buffers");
  return launched(ci8::launch_grouped_summed_gemm(a, w, a_scale, w_scale, out, int(groups),
                                                  int(m), int(n), int(k), as_stream(stream)));
}

int ci8_channel_gemv(const void* x, const int8_t* w, const void* scale, void* out, int64_t m,
                     int64_t n, int64_t k, void* stream) {
  if (!(m > 0 && m <= 16 && n > 0 && k > 0 && k <= 65536 && k % 16 == 0))
    return fail(CI8_ERR_GEOMETRY, "Unsupported W8A16 GEMV geometry");
  if (n * k > INT_MAX) return fail(CI8_ERR_TOO_LARGE, "Weight matrix too large");
  if (!aligned(w, 16) || !aligned(x, 4) || !aligned(scale, 2) || !aligned(out, 2))
    return fail(CI8_ERR_ALIGNMENT, "Unaligned vector inputs");
  return launched(
      ci8::launch_channel_gemv(x, w, scale, out, int(m), int(n), int(k), as_stream(stream)));
}

// csrc/bindings.cpp:36-40: the two SwiGLU widths of the reference's models.
int ci8_silu_mul(const void* x, void* out, int64_t m, int64_t k, void* stream) {
  if (!(m >= 0 && (k == 8704 || k == 17408) && m * 2 * k <= INT_MAX))
    return fail(CI8_ERR_GEOMETRY, "Unsupported SwiGLU shape");
  if (!aligned(x, 2) || !aligned(out, 2))
    return fail(CI8_ERR_ALIGNMENT, "SwiGLU requires aligned buffers");
  if (overlap(x, m * 2 * k * 2, out, m * k * 2))
    return fail(CI8_ERR_OVERLAP, "SwiGLU buffers must not overlap");
  return launched(ci8::launch_silu_mul(x, out, int(m), int(k), as_stream(stream)));
}

// csrc/bindings.cpp:51-59
int ci8_silu_mul_quantize(const void* x, int8_t* codes, float* scales, int64_t m, int64_t k,
                          void* stream) {
  if (!(m >= 0 && (k == 8704 || k == 17408) && m * 2 * k <= INT_MAX))
    return fail(CI8_ERR_GEOMETRY, "Unsupported SwiGLU quantization shape");
  if (!aligned(x, 16) || !aligned(codes, 8) || !aligned(scales, 4))
    return fail(CI8_ERR_ALIGNMENT, "SwiGLU quantization requires aligned buffers");
  if (overlap(x, m * 2 * k * 2, codes, m * k) || overlap(x, m * 2 * k * 2, scales, m * 4) ||
      overlap(codes, m * k, scales, m * 4))
    return fail(CI8_ERR_OVERLAP, "SwiGLU quantization buffers must not overlap");
  return launched(
      ci8::launch_silu_mul_quantize(x, codes, scales, int(m), int(k), as_stream(stream)));
}

// csrc/bindings.cpp:276-284
int ci8_unpack_allspark(const uint8_t* packed, const void* packed_scales, int8_t* weight,
                        void* scales, int64_t n, int64_t k, void* stream) {
  if (!(n > 0 && n % 16 == 0 && k > 0 && k <= 65536 && k % 16 == 0))
    return fail(CI8_ERR_GEOMETRY, "Expected AllSpark N32K16 weights and channel scales");
  const int64_t padded_n = (n + 31) / 32 * 32;
  if (padded_n * k > INT_MAX) return fail(CI8_ERR_TOO_LARGE, "Weight too large");
  if (!aligned(packed, 4) || !aligned(weight, 16) || !aligned(packed_scales, 2) ||
      !aligned(scales, 2))
    return fail(CI8_ERR_ALIGNMENT, "Unaligned weights");
  if (overlap(packed, padded_n * k, weight, n * k) ||
      overlap(packed, padded_n * k, scales, n * 2) ||
      overlap(packed_scales, padded_n * 2, weight, n * k) ||
      overlap(packed_scales, padded_n * 2, scales, n * 2) || overlap(weight, n * k, scales, n * 2))
    return fail(CI8_ERR_OVERLAP, "AllSpark buffers must not overlap");
  return launched(ci8::launch_unpack_allspark(packed, packed_scales, weight, scales, int(n),
                                              int(k), as_stream(stream)));
}

int ci8_quantize_block32(const void* x, int8_t* a, float* sa, int64_t m, int64_t k,
                         void* stream) {
  if (int status = check_q8(m, 1, k)) return status;
  if (!aligned(x, 2) || !aligned(sa, 4))
    return fail(CI8_ERR_ALIGNMENT, "Block-32 quantization requires aligned buffers");
  if (overlap(x, m * k * 2, a, m * k) || overlap(x, m * k * 2, sa, m * k / 8) ||
      overlap(a, m * k, sa, m * k / 8))
    return fail(CI8_ERR_OVERLAP, "Block-32 buffers must not overlap");
  return launched(ci8::launch_quantize_block32(x, a, sa, int(m), int(k), as_stream(stream)));
}

int ci8_q8_block_mm(const int8_t* a, const float* sa, const int8_t* w, const void* sw, void* y,
                    int64_t m, int64_t n, int64_t k, void* stream) {
  if (int status = check_q8(m, n, k)) return status;
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(sa, 4) || !aligned(sw, 2) ||
      !aligned(y, 2))
    return fail(CI8_ERR_ALIGNMENT, "Block-32 GEMM requires aligned buffers");
  if (overlap(y, m * n * 2, a, m * k) || overlap(y, m * n * 2, w, n * k) ||
      overlap(y, m * n * 2, sa, m * k / 8) || overlap(y, m * n * 2, sw, n * k / 16))
    return fail(CI8_ERR_OVERLAP, "Block-32 buffers must not overlap");
  return launched(
      ci8::launch_q8_block_mm(a, sa, w, sw, y, int(m), int(n), int(k), as_stream(stream)));
}

int ci8_q8_block_int8(const void* x, int8_t* a, float* sa, const int8_t* w, const void* sw,
                      void* y, int64_t m, int64_t n, int64_t k, void* stream) {
  if (int status = check_q8(m, n, k)) return status;
  if (!aligned(x, 2) || !aligned(a, 16) || !aligned(w, 16) || !aligned(sa, 4) ||
      !aligned(sw, 2) || !aligned(y, 2))
    return fail(CI8_ERR_ALIGNMENT, "Block-32 GEMM requires aligned buffers");
  if (overlap(x, m * k * 2, a, m * k) || overlap(x, m * k * 2, sa, m * k / 8) ||
      overlap(a, m * k, sa, m * k / 8) || overlap(y, m * n * 2, x, m * k * 2) ||
      overlap(y, m * n * 2, a, m * k) || overlap(y, m * n * 2, w, n * k) ||
      overlap(y, m * n * 2, sa, m * k / 8) || overlap(y, m * n * 2, sw, n * k / 16))
    return fail(CI8_ERR_OVERLAP, "Block-32 buffers must not overlap");
  const hipStream_t s = as_stream(stream);
  const hipError_t q = ci8::launch_quantize_block32(x, a, sa, int(m), int(k), s);
  if (q != hipSuccess) return launched(q);
  return launched(ci8::launch_q8_block_mm(a, sa, w, sw, y, int(m), int(n), int(k), s));
}

// csrc/gguf_bindings.cpp:135-171, the same checks in the same order.
int ci8_gguf_q8_packed_mm(const void* x, const int8_t* codes, const void* scales, void* out,
                          int64_t m, int64_t n, int64_t k, int64_t groups,
                          int64_t x_row_stride, int64_t x_group_stride, void* stream) {
  if (!(m >= 0 && n >= 0 && groups >= 0 && k > 0 && k % 64 == 0 && x_row_stride > 0 &&
        x_group_stride > 0))
    return fail(CI8_ERR_GEOMETRY, "Invalid packed Q8 shape/strides; K must be a multiple of 64");
  if (!(m <= 65535LL * 32 && groups <= 65535 && k <= 2147483584LL && n <= 2147483584LL))
    return fail(CI8_ERR_TOO_LARGE, "Packed Q8 grid too large");
  if (x_row_stride % 8 || x_group_stride % 8 || !aligned(x, 16) || !aligned(codes, 16) ||
      !aligned(scales, 4))
    return fail(CI8_ERR_ALIGNMENT, "Packed Q8 copy alignment violation");
  if (m == 0 || n == 0 || groups == 0) {
    g_last_error.clear();
    return CI8_OK;
  }
  // Byte extents in 128-bit arithmetic: no device buffer reaches 2^62 bytes, so larger
  // extents (which would also overflow the kernels' 64-bit offsets) are rejected.
  using u128 = unsigned __int128;
  const u128 out_extent = u128(m) * u128(groups) * u128(n) * 2;
  const u128 x_extent =
      (u128(m - 1) * u128(x_row_stride) + u128(groups - 1) * u128(x_group_stride) + u128(k)) * 2;
  const u128 codes_extent = u128(groups) * u128(n) * u128(k);
  constexpr u128 kMaxExtent = u128(1) << 62;
  if (out_extent > kMaxExtent || x_extent > kMaxExtent || codes_extent > kMaxExtent)
    return fail(CI8_ERR_TOO_LARGE, "Packed Q8 grid too large");
  const auto out_bytes = int64_t(out_extent), x_bytes = int64_t(x_extent);
  if (overlap(out, out_bytes, x, x_bytes) || overlap(out, out_bytes, codes, groups * n * k) ||
      overlap(out, out_bytes, scales, groups * n * (k / 32) * 2))
    return fail(CI8_ERR_OVERLAP, "Packed Q8 output must not alias inputs");
  return launched(ci8::launch_gguf_q8_packed_mm(x, codes, scales, out, int(m), int(n), int(k),
                                                int(groups), x_row_stride, x_group_stride,
                                                as_stream(stream)));
}

}  // extern "C"
