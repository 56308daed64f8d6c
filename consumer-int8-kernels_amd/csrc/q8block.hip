// Block-32 Q8_0 W8A8 (the reference's benchmarks/cuda/q8_block_int8.cu:11-174):
//
//   quantize_block32: x BF16 [m, k] -> a INT8 [m, k], sa FP32 [m, k/32]; each run of 32
//                     consecutive values is quantized as quantize_rows quantizes a row
//                     (scale = max(amax/127, 1e-20), code = rne(x/scale), IEEE division)
//   q8_block_mm:      y[r, c] = bf16_rn( sum over blocks b = 0, 1, ... of
//                               fma(float(acc_b[r, c]), fl(sa[r, b] * float(sw[c, b])), sum) )
//                     with acc_b the exact INT32 dot product of block b, w INT8 [n, k] and
//                     sw FP16 [n, k/32] (GGUF Q8_0 codes and scales, stored apart), and
//                     the FP32 sum starting at +0. One rounding per multiply and per
//                     multiply-add, in ascending b.
//
// The integer accumulation restarts every 32 values of K, so each block is one
// v_mfma_i32_16x16x32_i8 into a zeroed accumulator followed by the FP32 rescale of its
// 4 outputs per lane: a convert, the scale product and a multiply-add, 3 VALU
// instructions per output per block. That rescale, not the matrix cores, bounds the
// kernel: one 16x16x32 MFMA (8 K of MAC per lane-cycle) against 12 VALU instructions.
//
// Layout: a workgroup computes a 64 x 64 output tile on 8 waves (16 rows x 32 columns
// each: 1 x 2 MFMA tiles), or 32 x 32 on 4 waves for small problems. K advances 256
// values (8 blocks) a step: the A and W slabs (16-byte loads, rows padded in LDS against
// bank conflicts) and their scales (W's converted to FP32) are staged in LDS, with the
// next step's global loads issued into registers before the current step's arithmetic.
// Measured at M=2048, N=1024, K=4096: 55 us, 37% of the VALU bound of the rescale; the
// LDS reads (operands and scales, about 5 bytes per output per block) run close to their
// own limit beside it.
#include "ci8_device.h"
#include "launch.h"

#pragma clang fp contract(off)

namespace ci8 {
namespace {

constexpr int kWave = 64;
typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ quantizer

// Four lanes per block, eight values per lane. Requires x 16-byte, a 8-byte aligned.
__global__ void __launch_bounds__(256) quantize_block32_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ a, float* __restrict__ sa,
    int64_t blocks) {
  const int64_t lane_id = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int64_t block = lane_id >> 2;
  const bool live = block < blocks;
  u32x4 v = u32x4{0, 0, 0, 0};
  if (live) v = reinterpret_cast<const u32x4*>(x)[lane_id];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(v[j] << 16)),
                             fabsf(__uint_as_float(v[j] & 0xFFFF0000u))));
  amax = fmaxf(amax, __shfl_xor(amax, 1, kWave));
  amax = fmaxf(amax, __shfl_xor(amax, 2, kWave));
  if (!live) return;
  const float scale = fmaxf(amax / 127.f, 1e-20f);
  if ((threadIdx.x & 3) == 0) sa[block] = scale;
  reinterpret_cast<u32x2*>(a)[lane_id] = codes8(v, scale, 1.f / scale);
}

// One thread per block of 32, any alignment of x and a.
__global__ void __launch_bounds__(256) quantize_block32_scalar_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ a, float* __restrict__ sa,
    int64_t blocks) {
  const int64_t block = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (block >= blocks) return;
  const uint16_t* src = x + block * 32;
  float amax = 0.f;
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(bf16_to_f32(src[j])));
  const float scale = fmaxf(amax / 127.f, 1e-20f);
  sa[block] = scale;
  for (int j = 0; j < 32; ++j)
    a[block * 32 + j] = int8_t(code_byte(bf16_to_f32(src[j]) / scale));
}

// ------------------------------------------------------------------ GEMM

// Tile shape: kWR x kWC waves, each owning kWM x kWN MFMA tiles of 16 x 16; K advances
// kBK values (kBK / 32 blocks) a step.
template <int kWR, int kWC, int kWM, int kWN, int kBKv>
struct Q8Tile {
  static constexpr int kThreads = 64 * kWR * kWC;
  static constexpr int kBM = kWR * kWM * 16, kBN = kWC * kWN * 16;
  static constexpr int kBK = kBKv, kSteps = kBK / 32;
  static constexpr int kPitch = kBK + 16;  // LDS row pitch in bytes
  static constexpr int kRowChunks = kBK / 16;
  static constexpr int kAChunks = kBM * kRowChunks / kThreads;  // 16-byte chunks per thread
  static constexpr int kWChunks = kBN * kRowChunks / kThreads;
  static_assert(kBM * kRowChunks % kThreads == 0 && kBN * kRowChunks % kThreads == 0,
                "tile / threads");
  static_assert(kBM <= kThreads && kBN <= kThreads, "one scale row per thread");
  static_assert(kSteps % 2 == 0, "FP16 scales travel in pairs");
};

template <class T>
struct Staged {
  u32x4 a[T::kAChunks];
  u32x4 w[T::kWChunks];
  float sa[T::kSteps];         // thread t < kBM: the step's block scales of row t
  uint32_t sw[T::kSteps / 2];  // thread t < kBN: the step's FP16 block scales of column t
};

template <class T>
struct Lds {
  alignas(16) int8_t a[T::kBM * T::kPitch];
  alignas(16) int8_t w[T::kBN * T::kPitch];
  alignas(16) float sa[T::kSteps][T::kBM];
  alignas(16) float sw[T::kSteps][T::kBN];
};

template <class T>
__device__ __forceinline__ void load_step(Staged<T>& st, const int8_t* a, const float* sa,
                                          const int8_t* w, const uint16_t* sw, int m, int n,
                                          int k, int row0, int col0, int kb) {
  const int t = threadIdx.x;
  const int kblocks = k / 32;
#pragma unroll
  for (int i = 0; i < T::kAChunks; ++i) {
    const int chunk = t + T::kThreads * i;
    const int row = row0 + chunk / T::kRowChunks, col = kb + (chunk % T::kRowChunks) * 16;
    st.a[i] = u32x4{0, 0, 0, 0};
    if (row < m && col < k) st.a[i] = *reinterpret_cast<const u32x4*>(a + int64_t(row) * k + col);
  }
#pragma unroll
  for (int i = 0; i < T::kWChunks; ++i) {
    const int chunk = t + T::kThreads * i;
    const int row = col0 + chunk / T::kRowChunks, col = kb + (chunk % T::kRowChunks) * 16;
    st.w[i] = u32x4{0, 0, 0, 0};
    if (row < n && col < k) st.w[i] = *reinterpret_cast<const u32x4*>(w + int64_t(row) * k + col);
  }
#pragma unroll
  for (int j = 0; j < T::kSteps; ++j) st.sa[j] = 0.f;
  if (t < T::kBM && row0 + t < m) {
    const float* src = sa + int64_t(row0 + t) * kblocks + kb / 32;
#pragma unroll
    for (int j = 0; j < T::kSteps; ++j)
      if (kb / 32 + j < kblocks) st.sa[j] = src[j];
  }
#pragma unroll
  for (int j = 0; j < T::kSteps / 2; ++j) st.sw[j] = 0u;
  if (t < T::kBN && col0 + t < n) {
    const uint16_t* src = sw + int64_t(col0 + t) * kblocks + kb / 32;
#pragma unroll
    for (int j = 0; j < T::kSteps / 2; ++j) {
      const uint32_t lo = kb / 32 + 2 * j < kblocks ? src[2 * j] : 0u;
      const uint32_t hi = kb / 32 + 2 * j + 1 < kblocks ? src[2 * j + 1] : 0u;
      st.sw[j] = lo | (hi << 16);
    }
  }
}

__device__ __forceinline__ float half_to_float(uint32_t bits) {
  return float(__builtin_bit_cast(_Float16, uint16_t(bits)));
}

template <class T>
__device__ __forceinline__ void store_step(Lds<T>& lds, const Staged<T>& st) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < T::kAChunks; ++i) {
    const int chunk = t + T::kThreads * i;
    *reinterpret_cast<u32x4*>(lds.a + (chunk / T::kRowChunks) * T::kPitch +
                              (chunk % T::kRowChunks) * 16) = st.a[i];
  }
#pragma unroll
  for (int i = 0; i < T::kWChunks; ++i) {
    const int chunk = t + T::kThreads * i;
    *reinterpret_cast<u32x4*>(lds.w + (chunk / T::kRowChunks) * T::kPitch +
                              (chunk % T::kRowChunks) * 16) = st.w[i];
  }
  if (t < T::kBM)
#pragma unroll
    for (int j = 0; j < T::kSteps; ++j) lds.sa[j][t] = st.sa[j];
  if (t < T::kBN)
#pragma unroll
    for (int j = 0; j < T::kSteps / 2; ++j) {
      lds.sw[2 * j][t] = half_to_float(st.sw[j] & 0xFFFFu);
      lds.sw[2 * j + 1][t] = half_to_float(st.sw[j] >> 16);
    }
}

// One block of 32 K for this wave's kWM x kWN tiles: MFMA into zeroed accumulators,
// then sum = fma(float(acc), fl(sa * sw), sum) per output.
template <class T, int kWM, int kWN>
__device__ __forceinline__ void q8_block(const Lds<T>& lds, int b, int wrow, int wcol, int lane,
                                         float (&sum)[kWM][kWN][4]) {
  const int lr = lane & 15, lk = (lane >> 4) * 8;
  int64_t af[kWM], wf[kWN];
  float swc[kWN];
  f32x4 sar[kWM];
#pragma unroll
  for (int ti = 0; ti < kWM; ++ti) {
    af[ti] = *reinterpret_cast<const int64_t*>(lds.a + (wrow + ti * 16 + lr) * T::kPitch + b * 32 + lk);
    sar[ti] = *reinterpret_cast<const f32x4*>(&lds.sa[b][wrow + ti * 16 + (lane >> 4) * 4]);
  }
#pragma unroll
  for (int tj = 0; tj < kWN; ++tj) {
    wf[tj] = *reinterpret_cast<const int64_t*>(lds.w + (wcol + tj * 16 + lr) * T::kPitch + b * 32 + lk);
    swc[tj] = lds.sw[b][wcol + tj * 16 + lr];
  }
#pragma unroll
  for (int ti = 0; ti < kWM; ++ti)
#pragma unroll
    for (int tj = 0; tj < kWN; ++tj) {
      const i32x4_t acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[ti], wf[tj],
                                                               i32x4_t{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sum[ti][tj][i] = __builtin_fmaf(float(acc[i]), sar[ti][i] * swc[tj], sum[ti][tj][i]);
    }
}

// Requires k % 32 == 0, a and w 16-byte aligned. kOcc: waves per SIMD the register
// allocation must allow (the unrolled blocks otherwise keep every block's operands live).
template <int kWR, int kWC, int kWM, int kWN, int kBK, int kOcc, int kUnroll>
__global__ void __launch_bounds__(64 * kWR * kWC, kOcc) q8_block_mm_kernel(
    const int8_t* __restrict__ a, const float* __restrict__ sa, const int8_t* __restrict__ w,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ y, int m, int n, int k) {
  using T = Q8Tile<kWR, kWC, kWM, kWN, kBK>;
  __shared__ Lds<T> lds;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = blockIdx.y * T::kBM, col0 = blockIdx.x * T::kBN;
  const int wrow = (wave / kWC) * kWM * 16, wcol = (wave % kWC) * kWN * 16;

  float sum[kWM][kWN][4];
#pragma unroll
  for (int ti = 0; ti < kWM; ++ti)
#pragma unroll
    for (int tj = 0; tj < kWN; ++tj)
#pragma unroll
      for (int i = 0; i < 4; ++i) sum[ti][tj][i] = 0.f;

  Staged<T> st;
  load_step<T>(st, a, sa, w, sw, m, n, k, row0, col0, 0);
  for (int kb = 0; kb < k; kb += T::kBK) {
    __syncthreads();  // the previous step's reads of lds are done
    store_step<T>(lds, st);
    __syncthreads();
    if (kb + T::kBK < k) load_step<T>(st, a, sa, w, sw, m, n, k, row0, col0, kb + T::kBK);
    if (kb + T::kBK <= k) {
#pragma unroll kUnroll
      for (int b = 0; b < T::kSteps; ++b) q8_block<T, kWM, kWN>(lds, b, wrow, wcol, lane, sum);
    } else {
      for (int b = 0; b < (k - kb) / 32; ++b) q8_block<T, kWM, kWN>(lds, b, wrow, wcol, lane, sum);
    }
  }
  const int lr = lane & 15;
#pragma unroll
  for (int ti = 0; ti < kWM; ++ti)
#pragma unroll
    for (int tj = 0; tj < kWN; ++tj) {
      const int col = col0 + wcol + tj * 16 + lr;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = row0 + wrow + ti * 16 + (lane >> 4) * 4 + i;
        if (row < m && col < n) y[int64_t(row) * n + col] = uint16_t(f32_to_bf16(sum[ti][tj][i]));
      }
    }
}

template <int kWR, int kWC, int kWM, int kWN, int kBK, int kOcc, int kUnroll>
void launch_q8_tile(const int8_t* a, const float* sa, const int8_t* w, const uint16_t* sw,
                    uint16_t* y, int m, int n, int k, hipStream_t stream) {
  using T = Q8Tile<kWR, kWC, kWM, kWN, kBK>;
  const dim3 grid((n + T::kBN - 1) / T::kBN, (m + T::kBM - 1) / T::kBM);
  q8_block_mm_kernel<kWR, kWC, kWM, kWN, kBK, kOcc, kUnroll>
      <<<grid, T::kThreads, 0, stream>>>(a, sa, w, sw, y, m, n, k);
}

}  // namespace

hipError_t launch_quantize_block32(const void* x, int8_t* a, float* sa, int m, int k,
                                   hipStream_t stream) {
  const int64_t blocks = int64_t(m) * (k / 32);
  const auto* src = static_cast<const uint16_t*>(x);
  if (reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(a) % 8 == 0) {
    const int64_t lanes = blocks * 4;
    quantize_block32_kernel<<<int((lanes + 255) / 256), 256, 0, stream>>>(src, a, sa, blocks);
  } else {
    quantize_block32_scalar_kernel<<<int((blocks + 255) / 256), 256, 0, stream>>>(src, a, sa,
                                                                               blocks);
  }
  return hipGetLastError();
}

hipError_t launch_q8_block_mm(const int8_t* a, const float* sa, const int8_t* w,
                              const void* sw, void* y, int m, int n, int k,
                              hipStream_t stream) {
  // 64 x 64 tiles on 8 waves (each 16 rows x 32 columns), K steps of 256; 32 x 32 tiles on
  // 4 waves when the larger tiles would leave CUs idle (tile-shape sweep at N = 1024,
  // K = 4096, M = 512 and 2048).
  const auto* s16 = static_cast<const uint16_t*>(sw);
  auto* out = static_cast<uint16_t*>(y);
  const int64_t big_tiles = int64_t((m + 63) / 64) * ((n + 63) / 64);
  if (big_tiles >= 256)
    launch_q8_tile<4, 2, 1, 2, 256, 4, 2>(a, sa, w, s16, out, m, n, k, stream);
  else
    launch_q8_tile<2, 2, 1, 1, 256, 4, 2>(a, sa, w, s16, out, m, n, k, stream);
  return hipGetLastError();
}

}  // namespace ci8
