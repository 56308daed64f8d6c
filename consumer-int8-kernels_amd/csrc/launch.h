// Internal host launchers (C++), called by the validated C ABI in abi.cpp. Arguments
// are assumed valid; each returns the launch status.
#pragma once
#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "tile_plan.h"

namespace ci8 {

hipError_t launch_quantize_rows(const void* x, int8_t* codes, float* scales, int m, int k,
                                hipStream_t stream);
// x [m, groups, k] -> codes [groups, m, k], scales [groups, m].
hipError_t launch_quantize_grouped(const void* x, int8_t* codes, float* scales, int m,
                                   int groups, int k, hipStream_t stream);

// Weight encodings accepted by the GEMM.
enum class WeightCode { kSigned, kBiasedU8 };

// out = bf16((float(A W^T) * sa) * sw); optional INT32 copy of the accumulators.
hipError_t launch_channel_gemm(const int8_t* a, const void* w, WeightCode code,
                               const float* sa, const void* sw, void* out,
                               int32_t* workspace, int m, int n, int k, int schedule,
                               hipStream_t stream);

// launch_channel_gemm for signed weights with the INT32 accumulators written to the
// library's own device array instead of a caller workspace (noalloc.hip). Requires
// m * n <= noalloc_scratch_ints(); allocates nothing.
int64_t noalloc_scratch_ints();
hipError_t launch_cutlass_channel_mm_noalloc(const int8_t* a, const int8_t* w, const float* sa,
                                             const void* sw, void* out, int m, int n, int k,
                                             hipStream_t stream);

// launch_channel_gemm (schedule 0, no INT32 copy) for a and w at any byte alignment
// (gemm_bytes.hip): byte loads and the VALU's 4-way dot product; identical bits, slow.
hipError_t launch_channel_gemm_bytes(const int8_t* a, const void* w, WeightCode code,
                                     const float* sa, const void* sw, void* out, int m, int n,
                                     int k, hipStream_t stream);

// Small-M variant of launch_channel_gemm (gemm_small.hip): small output tiles, K split
// over the workgroup's waves; identical bits. `cus` is the device's CU count.
hipError_t launch_small_m_gemm(const int8_t* a, const void* w, WeightCode code, const float* sa,
                               const void* sw, void* out, int32_t* workspace, int m, int n,
                               int k, int cus, hipStream_t stream);

// Large-M GEMM with two waves per SIMD (gemm_pp.hip), signed or biased UINT8 weights;
// identical bits. Requires a and w 16-byte aligned, sw 8-byte aligned, n % 4 == 0.
hipError_t launch_pp_gemm(const int8_t* a, const void* w, WeightCode code, const float* sa,
                          const void* sw, void* out, int m, int n, int k, hipStream_t stream);

// The current device's CU count, queried once per device and cached (0 if unknown).
int device_cu_count();

// out = bf16(sum_g (float(A_g W_g^T) * sa[g]) * sw), A [groups, m, k], W [groups, n, k],
// sa [groups, m]; FP32 sum over ascending g.
hipError_t launch_grouped_summed_gemm(const int8_t* a, const int8_t* w, const float* sa,
                                      const void* sw, void* out, int groups, int m, int n,
                                      int k, hipStream_t stream);

// The same on the two-waves-per-SIMD scheme (gemm_grouped.hip); identical bits. Requires a
// and w 16-byte aligned, sw 8-byte aligned, n % 4 == 0, groups <= grouped_pp_max_groups().
int grouped_pp_max_groups();
hipError_t launch_grouped_pp_gemm(const int8_t* a, const int8_t* w, const float* sa,
                                  const void* sw, void* out, int groups, int m, int n, int k,
                                  hipStream_t stream);

// x BF16 [m, 2k] = [gate | up] -> out BF16 [m, k] = bf16(silu(gate) * up).
hipError_t launch_silu_mul(const void* x, void* out, int m, int k, hipStream_t stream);
// The same activations quantized per row like launch_quantize_rows, never written out.
hipError_t launch_silu_mul_quantize(const void* x, int8_t* codes, float* scales, int m, int k,
                                    hipStream_t stream);

// AllSpark N32K16 packed [ceil(n/32)*32, k] UINT8 + permuted BF16 scales -> row-major
// signed INT8 [n, k] + BF16 [n]. Requires n % 16 == 0, k % 16 == 0, packed 4-byte and
// weight 16-byte aligned.
hipError_t launch_unpack_allspark(const uint8_t* packed, const void* packed_scales,
                                  int8_t* weight, void* scales, int n, int k,
                                  hipStream_t stream);

// x BF16 [m, k] -> a INT8 [m, k], sa FP32 [m, k/32] (per 32 values as quantize_rows).
hipError_t launch_quantize_block32(const void* x, int8_t* a, float* sa, int m, int k,
                                   hipStream_t stream);
// y BF16 [m, n] from block-32 W8A8: a INT8 [m, k], sa FP32 [m, k/32], w INT8 [n, k],
// sw FP16 [n, k/32]. Requires k % 32 == 0, a and w 16-byte aligned.
hipError_t launch_q8_block_mm(const int8_t* a, const float* sa, const int8_t* w,
                              const void* sw, void* y, int m, int n, int k,
                              hipStream_t stream);

// Grouped W8A16 on GGUF Q8_0 codes: x BF16 [m, groups, k] (row stride xs, group stride
// xg elements), codes INT8 [groups, n, k], scales FP16 [groups, n, k/32] -> out BF16
// [m, groups, n]. Requires k % 64 == 0, x and codes 16-byte aligned, xs, xg % 8 == 0.
hipError_t launch_gguf_q8_packed_mm(const void* x, const int8_t* codes, const void* scales,
                                    void* out, int m, int n, int k, int groups, int64_t xs,
                                    int64_t xg, hipStream_t stream);

hipError_t launch_channel_gemv(const void* x, const int8_t* w, const void* scale, void* out,
                               int m, int n, int k, hipStream_t stream);

}  // namespace ci8
