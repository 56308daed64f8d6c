// SwiGLU producers for configs[3]'s down projection (csrc/silu_quant.cu:10-88 of the
// reference):
//
//   silu_mul:          out[m, j] = bf16_rn( silu(g) * u ),  g = x[m, j], u = x[m, K + j]
//   silu_mul_quantize: the same BF16 values, quantized per row exactly as quantize_rows
//                      (the activations never leave registers)
//
// with silu(g) = g / (1 + e^-g), evaluated in FP32. The input is BF16 [M, 2K] holding
// the gate in columns [0, K) and the up projection in [K, 2K).
//
// Arithmetic. e^x is the hardware base-2 exponential (v_exp_f32) of x * log2(e), with
// the product carried as t_hi + t_lo (t_lo the FMA residual of the rounded product plus
// the low part of log2(e)) and 2^t = 2^t_hi * (1 + t_lo ln 2); the quotient is
// g * rcp(1 + e) with the hardware reciprocal, then the product with u and one BF16
// rounding. Each step is within a few ULP, so the value before the BF16 rounding stays
// within 2^-20 of silu(g) * u (relative), and the BF16 result is the correctly rounded
// one except where the exact value lies that close to a rounding midpoint. Gates with
// |g| >= 87 (where 1 + e^-g leaves the range of a normal reciprocal), infinite or NaN
// take an IEEE division instead, and e^-g overflows to +inf for g <= -89, giving
// silu = -0 as in FP32 arithmetic. The quantizer's codes are bit-exact with
// quantize_rows applied to the activations this file produces.
#include "ci8_device.h"
#include "launch.h"

// Every rounding below is the one written: no multiply-add contraction.
#pragma clang fp contract(off)

namespace ci8 {
namespace {

constexpr int kWave = 64;

// e^x = 2^t_hi * 2^t_lo with t_hi + t_lo = x * log2(e) to about 2^-40 relative:
// returns 2^t_hi (v_exp_f32) and t_lo * ln 2, with 2^t_lo = 1 + t_lo ln 2 + O(2^-35)
// since |t_lo| <= 2^-17 for |x| < 128.
struct ExpParts {
  float pow2;
  float tail;
};
__device__ __forceinline__ ExpParts exp_parts(float x) {
  constexpr float kLog2e = 1.44269502162933349609375f;     // log2(e) rounded to FP32
  constexpr float kLog2eLo = 1.925963033500011e-08f;       // log2(e) - kLog2e
  constexpr float kLn2 = 0.693147180559945309f;
  const float t_hi = x * kLog2e;
  float t_lo = fmaf(x, kLog2e, -t_hi);                     // exact residual of the product
  t_lo = fmaf(x, kLog2eLo, t_lo);
  return {__builtin_amdgcn_exp2f(t_hi), t_lo * kLn2};
}

// e^x for |x| < 87 (the fast path).
__device__ __forceinline__ float exp_core(float x) {
  const ExpParts p = exp_parts(x);
  return fmaf(p.pow2, p.tail, p.pow2);
}

// e^x for every x: clamped to [-104, 89] first, so it is 0 below (e^-104 is under half
// the smallest subnormal) and +inf above ln(FLT_MAX) (the product form keeps an
// infinite 2^t_hi infinite). A NaN argument gives a finite value; callers carry NaN
// through their other operand.
__device__ __forceinline__ float exp_clamped(float x) {
  const ExpParts p = exp_parts(__builtin_fminf(__builtin_fmaxf(x, -104.0f), 89.0f));
  return p.pow2 * (1.f + p.tail);
}

// silu(g) * u for any g: IEEE division.
__device__ __forceinline__ float swiglu_exact(float g, float u) {
  const float silu = g / (1.f + exp_clamped(-g));
  return silu * u;
}

// silu(g) * u for |g| < 87, where 1 <= 1 + e^-g < 2^126: hardware reciprocal (1 ULP).
__device__ __forceinline__ float swiglu_fast(float g, float u) {
  const float silu = g * __builtin_amdgcn_rcpf(1.f + exp_core(-g));
  return silu * u;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset >= 1; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, kWave));
  return v;
}

// Eight BF16 activations (four packed words) from eight gate and eight up values.
__device__ __forceinline__ u32x4 swiglu8(const u32x4& gate, const u32x4& up) {
  u32x4 out;
  bool outside = false;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float g0 = bf16_lo(gate[j]), g1 = bf16_hi(gate[j]);
    outside |= !(fabsf(g0) < 87.f) | !(fabsf(g1) < 87.f);
    out[j] = pack_bf16x2(swiglu_fast(g0, bf16_lo(up[j])), swiglu_fast(g1, bf16_hi(up[j])));
  }
  if (outside) {  // |g| >= 87, infinite or NaN gates (essentially never in practice)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      out[j] = pack_bf16x2(swiglu_exact(bf16_lo(gate[j]), bf16_lo(up[j])),
                           swiglu_exact(bf16_hi(gate[j]), bf16_hi(up[j])));
  }
  return out;
}

// One row per workgroup of kWaves waves; each lane keeps kPacks packs of 8 activations
// in registers between the row maximum and the codes. Requires k % 8 == 0,
// k <= kPacks * kWaves * 512, x 16-byte and codes 8-byte aligned.
template <int kPacks, int kWaves>
__global__ void __launch_bounds__(64 * kWaves) silu_mul_quantize_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ codes, float* __restrict__ scales,
    int k) {
  __shared__ float partial[kWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row = blockIdx.x;
  const uint16_t* gate = x + row * 2 * k;
  const uint16_t* up = gate + k;

  u32x4 act[kPacks];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < kPacks; ++i) {
    const int col = ((i * kWaves + wave) * kWave + lane) * 8;
    act[i] = u32x4{0, 0, 0, 0};
    if (col < k)
      act[i] = swiglu8(*reinterpret_cast<const u32x4*>(gate + col),
                       *reinterpret_cast<const u32x4*>(up + col));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(act[i][j])), fabsf(bf16_hi(act[i][j]))));
  }
  amax = wave_max(amax);
  if (lane == 0) partial[wave] = amax;
  __syncthreads();
  amax = partial[0];
#pragma unroll
  for (int v = 1; v < kWaves; ++v) amax = fmaxf(amax, partial[v]);
  const float scale = fmaxf(amax / 127.f, 1e-20f);
  const float inv = 1.f / scale;
  if (threadIdx.x == 0) scales[row] = scale;
  int8_t* dst = codes + row * k;
#pragma unroll
  for (int i = 0; i < kPacks; ++i) {
    const int col = ((i * kWaves + wave) * kWave + lane) * 8;
    if (col < k)
      __builtin_nontemporal_store(codes8(act[i], scale, inv), reinterpret_cast<u32x2*>(dst + col));
  }
}

// Elementwise SwiGLU, eight outputs per lane; blockIdx.y is the row. Requires
// k % 8 == 0 and 16-byte aligned x and out.
template <bool kNt>
__global__ void __launch_bounds__(256) silu_mul_kernel(const uint16_t* __restrict__ x,
                                                       uint16_t* __restrict__ out, int k) {
  const int col = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (col >= k) return;
  const int64_t row = blockIdx.y;
  const uint16_t* gate = x + row * 2 * k + col;
  const u32x4 v = swiglu8(load16<kNt>(gate), load16<kNt>(gate + k));
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(out + row * k + col));
}

// Scalar fallback for rows not 16-byte aligned (silu_mul accepts any BF16 tensor).
__global__ void __launch_bounds__(256) silu_mul_scalar_kernel(const uint16_t* __restrict__ x,
                                                              uint16_t* __restrict__ out,
                                                              int64_t m, int k) {
  const int64_t index = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (index >= m * k) return;
  const int64_t row = index / k;
  const int col = int(index % k);
  const float g = bf16_to_f32(x[row * 2 * k + col]);
  const float u = bf16_to_f32(x[row * 2 * k + k + col]);
  out[index] = uint16_t(f32_to_bf16(swiglu_exact(g, u)));
}

}  // namespace

hipError_t launch_silu_mul_quantize(const void* x, int8_t* codes, float* scales, int m, int k,
                                    hipStream_t stream) {
  if (m == 0) return hipSuccess;
  const auto* src = static_cast<const uint16_t*>(x);
  // k = 8704 is 17 wave-wide packs of 512 values: 4 waves x 5 packs; k = 17408 is 34:
  // 8 waves x 5 packs (launch-shape sweep at M = 16384).
  if (k <= 4 * 5 * 512)
    silu_mul_quantize_kernel<5, 4><<<m, 256, 0, stream>>>(src, codes, scales, k);
  else
    silu_mul_quantize_kernel<5, 8><<<m, 512, 0, stream>>>(src, codes, scales, k);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const void* x, void* out, int m, int k, hipStream_t stream) {
  const int64_t count = int64_t(m) * k;
  if (count == 0) return hipSuccess;
  const auto* src = static_cast<const uint16_t*>(x);
  auto* dst = static_cast<uint16_t*>(out);
  const bool vec = reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0 && k % 8 == 0;
  if (vec) {
    // Inputs past the MALL's size are read with nontemporal loads (kMallBytes).
    const dim3 grid((k / 8 + 255) / 256, m);
    if (count * 4 > kMallBytes)
      silu_mul_kernel<true><<<grid, 256, 0, stream>>>(src, dst, k);
    else
      silu_mul_kernel<false><<<grid, 256, 0, stream>>>(src, dst, k);
  } else {
    silu_mul_scalar_kernel<<<int((count + 255) / 256), 256, 0, stream>>>(src, dst, m, k);
  }
  return hipGetLastError();
}

}  // namespace ci8
