// Measurement helpers for bench.py; not part of the drop-in library (they have no
// counterpart in the reference and no declaration in include/).
//
// A full-chip INT8 MFMA loop: one workgroup of 4 waves per CU, each wave running 8
// independent v_mfma_i32_16x16x64_i8 accumulator chains over 4 operand sets, so the
// operand registers change every instruction as they do in a GEMM. Thread 0 of each
// workgroup records the shader-clock cycles (s_memtime) and constant-rate wall-clock
// ticks (s_memrealtime) its loop took. From these the host gets the INT8 MFMA rate the
// chip sustains under a pure MFMA load and the shader clock it ran at, which gives the
// dense INT8 peak at the measured clock (CUs x 8192 op/clk x f).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t mix(uint32_t x) {
  x ^= x << 13;
  x ^= x >> 17;
  x ^= x << 5;
  return x;
}

__global__ void __launch_bounds__(256) mfma_loop_kernel(int rounds, int64_t* record) {
  uint32_t h = (blockIdx.x * 256u + threadIdx.x) * 2654435761u + 0x9E3779B9u;
  i32x4 a[4], b[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h = mix(h);
      a[s][e] = int32_t(h);
      h = mix(h);
      b[s][e] = int32_t(h);
    }
  i32x4 acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = i32x4{0, 0, 0, 0};

  const int64_t cycles0 = clock64(), ticks0 = wall_clock64();
  for (int r = 0; r < rounds; ++r) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int c = 0; c < 8; ++c)
        acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[(c + s) & 3], b[(c + 2 * s + 1) & 3],
                                                       acc[c], 0, 0, 0);
  }
  const int64_t cycles1 = clock64(), ticks1 = wall_clock64();

  int32_t fold = 0;
#pragma unroll
  for (int c = 0; c < 8; ++c) fold ^= acc[c][0] ^ acc[c][1] ^ acc[c][2] ^ acc[c][3];
  if (threadIdx.x == 0) {
    record[3 * blockIdx.x] = cycles1 - cycles0;
    record[3 * blockIdx.x + 1] = ticks1 - ticks0;
    record[3 * blockIdx.x + 2] = fold;  // keeps every MFMA live
  }
}

// HBM streaming references for the HBM-bound kernels: a plain read of `units` 16-byte
// units (a weight stream), and a read of 16 bytes with a write of 8 per unit (the bytes
// of a BF16 -> INT8 quantizer, without its per-row dependency). Each thread keeps 8 loads
// in flight over a grid-stride loop; the loaded words are folded into a value that is
// stored only if it matches a sentinel, so no load is dead.
// kIn loads in flight per thread; kNt marks them nontemporal.
template <int kIn, bool kNt>
__global__ void __launch_bounds__(256) stream_read_kernel(const i32x4* __restrict__ src,
                                                          int64_t units, int32_t* sink) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  int32_t fold = 0;
  for (; i + (kIn - 1) * stride < units; i += kIn * stride) {
    i32x4 v[kIn];
#pragma unroll
    for (int j = 0; j < kIn; ++j)
      v[j] = kNt ? __builtin_nontemporal_load(src + i + j * stride) : src[i + j * stride];
#pragma unroll
    for (int j = 0; j < kIn; ++j) fold ^= v[j][0] ^ v[j][1] ^ v[j][2] ^ v[j][3];
  }
  for (; i < units; i += stride) {
    const i32x4 v = src[i];
    fold ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (fold == 0x13579BDF) sink[0] = fold;
}

__global__ void __launch_bounds__(256) stream_read2_write1_kernel(const i32x4* __restrict__ src,
                                                                  int64_t units,
                                                                  int64_t* __restrict__ dst) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  for (; i + 7 * stride < units; i += 8 * stride) {
    i32x4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = src[i + j * stride];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      __builtin_nontemporal_store(int64_t(uint32_t(v[j][0] ^ v[j][1])) |
                                      int64_t(uint32_t(v[j][2] ^ v[j][3])) << 32,
                                  dst + i + j * stride);
  }
  for (; i < units; i += stride) {
    const i32x4 v = src[i];
    __builtin_nontemporal_store(int64_t(uint32_t(v[0] ^ v[1])) | int64_t(uint32_t(v[2] ^ v[3])) << 32,
                                dst + i);
  }
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) from `src` with `blocks` workgroups of 256 threads;
// variant 0: 8 plain loads in flight per thread, 1: 16 nontemporal loads (measured on
// MI355X over 89 MB of random bytes: 14.7 us at 2,048 workgroups against 15.0 us for
// variant 0 at its best grid).
int ci8probe_stream_read(const void* src, int64_t bytes, int32_t* sink, int blocks, int variant,
                         void* stream) {
  if (src == nullptr || sink == nullptr || bytes <= 0 || bytes % 16 || blocks <= 0 ||
      variant < 0 || variant > 1)
    return int(hipErrorInvalidValue);
  if (variant == 0)
    stream_read_kernel<8, false><<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const i32x4*>(src), bytes / 16, sink);
  else
    stream_read_kernel<16, true><<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const i32x4*>(src), bytes / 16, sink);
  return int(hipGetLastError());
}

// Reads `bytes` (a multiple of 16) from `src` and writes bytes / 2 to `dst`.
int ci8probe_stream_read2_write1(const void* src, int64_t bytes, void* dst, int blocks,
                                 void* stream) {
  if (src == nullptr || dst == nullptr || bytes <= 0 || bytes % 16 || blocks <= 0)
    return int(hipErrorInvalidValue);
  stream_read2_write1_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const i32x4*>(src), bytes / 16, static_cast<int64_t*>(dst));
  return int(hipGetLastError());
}


// MFMAs per wave per round, and INT8 ops per MFMA (16 x 16 x 64 x 2).
int ci8probe_mfma_per_round(void) { return 32; }
int64_t ci8probe_ops_per_mfma(void) { return 16 * 16 * 64 * 2; }

// Launches `blocks` workgroups of 256 threads, each running `rounds` rounds; `record`
// is a device buffer of 3 * blocks int64 (cycles, wall ticks, fold per workgroup).
int ci8probe_mfma_loop(int rounds, int blocks, int64_t* record, void* stream) {
  if (rounds <= 0 || blocks <= 0 || record == nullptr) return int(hipErrorInvalidValue);
  mfma_loop_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(rounds, record);
  return int(hipGetLastError());
}

// hipDeviceAttributeClockRate and hipDeviceAttributeWallClockRate of the current device,
// in kHz.
int ci8probe_clock_rates(int* shader_khz, int* wall_khz) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e == hipSuccess) e = hipDeviceGetAttribute(shader_khz, hipDeviceAttributeClockRate, device);
  if (e == hipSuccess) e = hipDeviceGetAttribute(wall_khz, hipDeviceAttributeWallClockRate, device);
  return int(e);
}

}  // extern "C"
