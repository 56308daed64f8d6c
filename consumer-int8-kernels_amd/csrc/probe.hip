// Measurement helper for bench.py; not part of the drop-in library (it has no
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

}  // namespace

extern "C" {

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
