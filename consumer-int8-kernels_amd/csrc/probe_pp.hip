// Measurement build of the persistent GEMM (gemm_pp_kernel.h) with clock stamps, for
// bench.py's --phase-profile only: part of libci8_probe.so, not of the drop-in library.
// It compiles the library's kernel source with the same flags, adding only the stamps.
#include "gemm_pp_kernel.h"

extern "C" {

// The stamp record: int64 values per workgroup, and phase kinds (pp_gemm_kernel's layout).
int ci8probe_pp_stamp_words() { return ci8::kStampWords; }
int ci8probe_pp_stamp_kinds() { return ci8::kStampKinds; }

// Workgroups of the persistent kernel's launch at m x n (one per CU, at most one per tile).
int ci8probe_pp_grid(int m, int n) {
  using C = ci8::PPConfig;
  const int tiles = ((n + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
  const int cus = ci8::device_cu_count();
  return cus > 0 && cus < tiles ? cus : tiles;
}

// fused_channel_mm with signed weights through the persistent kernel, recording
// ci8probe_pp_stamp_words() values per workgroup into `stamps`: mode 1 the shader-clock
// and wall-clock start and end times, mode 2 also the per-phase cycle sums. `stamps` holds
// at least ci8probe_pp_grid(m, n) * ci8probe_pp_stamp_words() values, zeroed by the
// caller. Same requirements as fused_channel_mm's persistent path: a, w 16-byte aligned,
// sw 8-byte aligned, n % 4 == 0.
int ci8probe_pp_gemm_stamped(const int8_t* a, const int8_t* w, const float* sa, const void* sw,
                             void* out, int m, int n, int k, int mode, int64_t* stamps,
                             void* stream) {
  using C = ci8::PPConfig;
  using ci8::WeightCode;
  if (a == nullptr || w == nullptr || sa == nullptr || sw == nullptr || out == nullptr ||
      stamps == nullptr || m <= 0 || n <= 0 || n % 4 != 0 || k <= 0 || k % 32 != 0 ||
      (mode != 1 && mode != 2) || reinterpret_cast<uintptr_t>(a) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(w) % 16 != 0 || reinterpret_cast<uintptr_t>(sw) % 8 != 0 ||
      reinterpret_cast<uintptr_t>(stamps) % 8 != 0)
    return int(hipErrorInvalidValue);
  const int grid = ci8probe_pp_grid(m, n);
  const bool out16 = (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  auto launch = [&](auto kernel_constant) {
    constexpr auto kernel = decltype(kernel_constant)::value;
    if (const hipError_t e = ci8::prepare_lds<kernel>(C::kLdsBytes); e != hipSuccess) return e;
    kernel<<<grid, C::kThreads, C::kLdsBytes, static_cast<hipStream_t>(stream)>>>(
        a, w, sa, static_cast<const uint16_t*>(sw), static_cast<uint16_t*>(out), m, n, k, n,
        out16, stamps);
    return hipGetLastError();
  };
  const bool exact = k % C::BK == 0;
  hipError_t e;
  if (mode == 1)
    e = exact ? launch(ci8::kernel_constant<ci8::pp_gemm_kernel<true, WeightCode::kSigned, 1>>{})
              : launch(ci8::kernel_constant<ci8::pp_gemm_kernel<false, WeightCode::kSigned, 1>>{});
  else
    e = exact ? launch(ci8::kernel_constant<ci8::pp_gemm_kernel<true, WeightCode::kSigned, 2>>{})
              : launch(ci8::kernel_constant<ci8::pp_gemm_kernel<false, WeightCode::kSigned, 2>>{});
  return int(e);
}

}  // extern "C"
