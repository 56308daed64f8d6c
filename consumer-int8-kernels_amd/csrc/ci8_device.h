// Device-side helpers shared by the gfx950 kernels: vector types, BF16 conversion,
// raw buffer resources and wait-count encodings.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ci8 {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

typedef __attribute__((address_space(3))) void lds_void;

// BF16 bit pattern -> FP32 (exact).
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
// FP32 -> BF16 bit pattern, IEEE round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f32_to_bf16(float value) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(value));
}
// Two FP32 -> packed BF16 pair (low half = first).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16(lo) | (f32_to_bf16(hi) << 16);
}

// Raw buffer resource over `bytes` bytes starting at `base`. Loads at byte offsets
// >= bytes return zero, which covers row and column tails without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
// An offset past every valid buffer (buffers are limited to INT_MAX bytes).
constexpr uint32_t kOutOfRange = 0x80000000u;

// s_waitcnt immediate that waits until at most `n` vector-memory operations are
// outstanding and leaves the other counters unconstrained (gfx9 encoding).
constexpr int vmcnt_imm(int n) {
  return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}
// s_waitcnt immediate that waits for all LDS/scalar operations (lgkmcnt = 0).
constexpr int lgkmcnt0_imm() { return 0xF | (0x3 << 14) | (0x7 << 4); }

}  // namespace ci8
