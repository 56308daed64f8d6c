// Device-side helpers shared by the gfx950 kernels: vector types, BF16 conversion,
// raw buffer resources and wait-count encodings.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "lds_budget.h"

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
// Two FP32 -> packed BF16 pair (low half = first), one v_cvt_pk_bf16_f32 (RNE).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// Low and high BF16 halves of a packed pair, widened to FP32 (exact).
__device__ __forceinline__ float bf16_lo(uint32_t word) { return __uint_as_float(word << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t word) {
  return __uint_as_float(word & 0xFFFF0000u);
}

// rne(q) for |q| <= 127.5 as the low byte of fl(q + 1.5 * 2^23), the two's-complement
// INT8 code; a NaN q gives 0.
__device__ __forceinline__ uint32_t code_byte(float q) {
  return __float_as_uint(q + 12582912.0f) & 0xFFu;
}

// INT8 codes of eight BF16 values (four packed pairs) for a scale of the row or block they
// belong to: code = rne(fl(v / scale)), the IEEE quotient, as two words of four bytes.
// The quotient comes from q0 = fl(v * inv), inv = fl(1 / scale). For every finite v of
// the row, |v / scale| < 128 (scale >= amax / 127 rounded, or the 1e-20 floor), so
// |q0 - v/scale| <= 2^-17 + 2^-17 and |fl(v/scale) - v/scale| <= 2^-17: when q0 is more
// than 2^-15 from every half-integer, fl(v / scale) lies on the same side of each and
// rounds to the same integer. Lanes holding a value inside that band (about 1 in 16000)
// take the division. NaN and infinite products give NaN, whose code is 0 as with the
// division.
__device__ __forceinline__ u32x2 codes8(const u32x4& packed, float scale, float inv) {
#pragma clang fp contract(off)
  float q[8];
  bool near = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    q[2 * j] = bf16_lo(packed[j]) * inv;
    q[2 * j + 1] = bf16_hi(packed[j]) * inv;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) near |= fabsf(q[j] - __builtin_floorf(q[j]) - 0.5f) <= 0x1p-15f;
  if (near) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      q[2 * j] = bf16_lo(packed[j]) / scale;
      q[2 * j + 1] = bf16_hi(packed[j]) / scale;
    }
  }
  u32x2 out;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t bytes = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) bytes |= code_byte(q[4 * h + j]) << (8 * j);
    out[h] = bytes;
  }
  return out;
}

// Inputs larger than MI355X's 256 MB Infinity Cache (MALL) cannot stay cached between
// the kernels that write and read them; the streaming kernels read those with
// nontemporal loads (measured: quantize_rows [16384, 17408] 155 -> 138 us, silu_mul
// [16384, 2 x 17408] 285 -> 261 us; at [4096, 5120], where the input fits, nontemporal
// loads were 6% slower).
constexpr int64_t kMallBytes = int64_t(256) << 20;

// One 16-byte load, nontemporal when kNt.
template <bool kNt>
__device__ __forceinline__ u32x4 load16(const void* p) {
  if constexpr (kNt)
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else
    return *reinterpret_cast<const u32x4*>(p);
}

// Cache-policy operand of a buffer load that marks it nontemporal (the nt bit of gfx950's
// cache-policy field): for streams read once, such as a GEMV's weights.
constexpr int kBufferLoadNontemporal = 2;

// Raw buffer resource over `bytes` bytes starting at `base`. Loads at byte offsets
// >= bytes return zero, which covers row and column tails without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
// An offset past every valid buffer (buffers are limited to INT_MAX bytes).
constexpr uint32_t kOutOfRange = 0x80000000u;

// A kernel as a type, for launch helpers that take several kernels of one signature.
template <auto Kernel>
struct kernel_constant {
  static constexpr auto value = Kernel;
};

// Every launch that requests dynamic LDS calls prepare_lds<kernel>(bytes) first, with the
// bytes it requests. It returns hipErrorInvalidConfiguration (and the caller launches
// nothing) when the kernel's static LDS plus those bytes exceed the 160 KiB a workgroup
// can hold; otherwise, on the first launch of that kernel that needs more than the default
// 64 KiB, it raises the kernel's dynamic-LDS attribute to the rest of the budget. The
// kernel's static LDS is looked up once. State is kept per kernel (per template
// argument); concurrent first calls may both query or set the idempotent attributes.
template <auto Kernel>
inline hipError_t prepare_lds(int64_t dynamic_bytes) {
  static std::atomic<int64_t> static_bytes_cache{-1};
  static std::atomic<bool> raised{false};
  int64_t static_bytes = static_bytes_cache.load(std::memory_order_acquire);
  if (static_bytes < 0) {
    hipFuncAttributes attributes{};
    if (const hipError_t e =
            hipFuncGetAttributes(&attributes, reinterpret_cast<const void*>(Kernel));
        e != hipSuccess)
      return e;
    static_bytes = int64_t(attributes.sharedSizeBytes);
    static_bytes_cache.store(static_bytes, std::memory_order_release);
  }
  if (!lds_fits(static_bytes, dynamic_bytes)) return hipErrorInvalidConfiguration;
  if (dynamic_bytes > kDefaultDynamicLds && !raised.load(std::memory_order_acquire)) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(Kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             int(dynamic_lds_limit(static_bytes)));
    if (e != hipSuccess) return e;
    raised.store(true, std::memory_order_release);
  }
  return hipSuccess;
}

// s_waitcnt immediate that waits until at most `n` vector-memory operations are
// outstanding and leaves the other counters unconstrained (gfx9 encoding).
constexpr int vmcnt_imm(int n) {
  return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}
// s_waitcnt immediate that waits for all LDS/scalar operations (lgkmcnt = 0).
constexpr int lgkmcnt0_imm() { return 0xF | (0x3 << 14) | (0x7 << 4); }
// s_waitcnt immediate for at most `vm` vector-memory and `lgkm` LDS/scalar operations
// outstanding (lgkm <= 15).
constexpr int vm_lgkm_imm(int vm, int lgkm) {
  return (vm & 0xF) | ((vm >> 4) << 14) | (0x7 << 4) | ((lgkm & 0xF) << 8);
}

}  // namespace ci8
