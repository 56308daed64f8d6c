// Row quantizers for gfx950: BF16 [rows, k] -> INT8 codes + FP32 per-row scales.
//
// Numerics follow csrc/kernels.cu:13-35 and :41-86 of the reference exactly:
//   amax  = NaN-ignoring max |x| over the row, starting from 0
//   scale = max(fl(amax / 127), 1e-20f)                       (IEEE division)
//   code  = clamp(rne(fl(x / scale)), -127, 127)              (IEEE division, RNE)
// fl(x/scale) never exceeds 127 in magnitude for finite x, so the clamp only matters
// for non-finite input; rounding uses the 1.5*2^23 add, whose low byte is the
// two's-complement code and which maps NaN to 0 like the reference's
// float->int conversion. The vector path takes the quotient from the row reciprocal and
// divides only near half-integers (codes8 in ci8_device.h), with the same codes.
//
// Layout: one, two or four waves own a row (four past 1024 values, so a lane holds
// at most a few 16-byte packs; eight when a few rows of 2,561..4,096 values leave most
// CUs idle) and keep it in registers between the max reduction and the
// store, so HBM sees a single read of x and a single write of the codes, with 16-byte
// loads and 8-byte stores (nontemporal outside 256..1,024 rows) fully coalesced across the wave.
#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int offset = 32; offset >= 1; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, kWave));
  return v;
}

// Vector path. Requires k % 8 == 0, x 16-byte aligned, codes 8-byte aligned.
// kWaves waves cooperate on one row when kWaves > 1 (very wide rows).
// Grouped: output row o reads input row (o % m) * groups + o / m ([m,g,k] -> [g,m,k]).
// Workgroups hold four waves (1, 2 or 4 rows), or kWaves waves and one row for kWaves > 4.
template <int kPacks, int kWaves, bool kGrouped, int kPolicy>
__global__ void __launch_bounds__(kWaves > 4 ? 64 * kWaves : 256) quantize_rows_vec_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ codes, float* __restrict__ scales,
    int rows, int k, int m, int groups) {
  constexpr int kRowsPerBlock = kWaves > 4 ? 1 : 4 / kWaves;
  __shared__ float partial[kWaves > 4 ? kWaves : 4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int out_row = blockIdx.x * kRowsPerBlock + wave / kWaves;
  const int part = wave % kWaves;
  const bool active = out_row < rows;
  const int64_t in_row = kGrouped ? int64_t(out_row % m) * groups + out_row / m : out_row;
  const uint16_t* src = x + in_row * k;

  u32x4 packed[kPacks];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < kPacks; ++i) {
    const int col = ((i * kWaves + part) * kWave + lane) * 8;
    packed[i] = u32x4{0, 0, 0, 0};
    if (active && col < k) packed[i] = load16<(kPolicy == 2)>(src + col);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t word = packed[i][j];
      amax = fmaxf(amax, fabsf(__uint_as_float(word << 16)));
      amax = fmaxf(amax, fabsf(__uint_as_float(word & 0xFFFF0000u)));
    }
  }
  amax = wave_max(amax);
  if constexpr (kWaves > 1) {
    // Waves (wave / kWaves) * kWaves .. + kWaves - 1 share this row.
    if (lane == 0) partial[wave] = amax;
    __syncthreads();
    const int first = wave - part;
    amax = partial[first];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) amax = fmaxf(amax, partial[first + w]);
  }
  if (!active) return;
  const float scale = fmaxf(amax / 127.f, 1e-20f);
  const float inv = 1.f / scale;
  if (part == 0 && lane == 0) scales[out_row] = scale;
  int8_t* dst = codes + int64_t(out_row) * k;
#pragma unroll
  for (int i = 0; i < kPacks; ++i) {
    const int col = ((i * kWaves + part) * kWave + lane) * 8;
    if (col < k) {
      const u32x2 code = codes8(packed[i], scale, inv);
      if constexpr (kPolicy >= 1)
        __builtin_nontemporal_store(code, reinterpret_cast<u32x2*>(dst + col));
      else
        *reinterpret_cast<u32x2*>(dst + col) = code;
    }
  }
}

// Fallback for any k and any 2-byte alignment: one wave per row, two passes.
template <bool kGrouped>
__global__ void __launch_bounds__(256) quantize_rows_scalar_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ codes, float* __restrict__ scales,
    int rows, int k, int m, int groups) {
  const int lane = threadIdx.x & 63;
  const int out_row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (out_row >= rows) return;
  const int64_t in_row = kGrouped ? int64_t(out_row % m) * groups + out_row / m : out_row;
  const uint16_t* src = x + in_row * k;
  float amax = 0.f;
  for (int col = lane; col < k; col += kWave) amax = fmaxf(amax, fabsf(bf16_to_f32(src[col])));
  amax = wave_max(amax);
  const float scale = fmaxf(amax / 127.f, 1e-20f);
  if (lane == 0) scales[out_row] = scale;
  int8_t* dst = codes + int64_t(out_row) * k;
  for (int col = lane; col < k; col += kWave)
    dst[col] = static_cast<int8_t>(code_byte(bf16_to_f32(src[col]) / scale));
}

template <bool kGrouped>
hipError_t dispatch(const void* x, int8_t* codes, float* scales, int rows, int k, int m,
                    int groups, hipStream_t stream) {
  const auto* src = static_cast<const uint16_t*>(x);
  const bool vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                   (reinterpret_cast<uintptr_t>(codes) % 8 == 0) && (k % 8 == 0);
  const int packs = (k + 511) / 512;  // 16-byte packs per lane with one wave per row
  // Inputs past the MALL's size are read with nontemporal loads (kMallBytes).
  const bool nt = int64_t(rows) * k * 2 > kMallBytes;
  // Codes are stored nontemporally (past the caches) except for 256 to 1,024 rows. There the
  // GEMM that reads them next runs faster when they stay cached (measured on MI355X, graph
  // replays of quantize_rows + fused_channel_mm, identical outputs). At M = 1024, N = 5120
  // and K = 5120 / 8704 / 17408 the pair took 52.8 / 75.6 / 136.0 us against 59.0 / 86.3 /
  // 153.9 us, and M = 256, N = 5120, K = 17408 took 66.7 against 70.0 us. The quantizer alone
  // is faster with nontemporal stores ([1024, 17408]: 11.3 against 13.7 us). At 4,096 rows
  // ([4096, 5120], N = 5120) the pair gained only 1.4 us against a 0.6 us slower quantizer,
  // so larger inputs keep them, and so do fewer rows, whose GEMM is latency-bound.
  // Policy (a template argument, so the store loop has no branch): 0 plain loads and
  // stores, 1 nontemporal stores, 2 nontemporal loads and stores.
  const int policy = nt ? 2 : (rows >= 256 && rows <= 1024 ? 0 : 1);
#define CI8_QW(W, P)                                                                       \
  if (packs <= (W) * (P)) {                                                                \
    constexpr int kPerBlock = (W) > 4 ? 1 : 4 / (W);                                       \
    constexpr int kThreads = (W) > 4 ? 64 * (W) : 256;                                     \
    const int blocks = (rows + kPerBlock - 1) / kPerBlock;                                 \
    if (policy == 2)                                                                       \
      quantize_rows_vec_kernel<P, W, kGrouped, 2><<<blocks, kThreads, 0, stream>>>(         \
          src, codes, scales, rows, k, m, groups);                                         \
    else if (policy == 1)                                                                  \
      quantize_rows_vec_kernel<P, W, kGrouped, 1><<<blocks, kThreads, 0, stream>>>(         \
          src, codes, scales, rows, k, m, groups);                                         \
    else                                                                                   \
      quantize_rows_vec_kernel<P, W, kGrouped, 0><<<blocks, kThreads, 0, stream>>>(         \
          src, codes, scales, rows, k, m, groups);                                         \
    return hipGetLastError();                                                              \
  }
  // Waves per row: four once a row has four packs, so each lane holds at most a few
  // 16-byte packs and a workgroup is one row. Measured on MI355X (us, 4 / 2 / 1 waves per
  // row): [128, 4096] 3.04 / 4.05 / 7.33, [16, 5120] 3.76 / 5.20 / 8.12, [256, 5120]
  // 3.37 / 4.31 / 7.11, [4096, 5120] 13.87 / 14.42 / 15.84: more waves keep more loads
  // in flight and let a row's stores start sooner.
  // When the rows do not fill the chip (configs[0]'s 128 rows on 256 CUs) the op is one
  // memory latency long, and eight waves of one pack per lane shorten it a little
  // (measured on MI355X in configs[0]'s quantize + fused_channel_mm step, 128 x 4096,
  // against four waves of two packs, same box and process: 11.80-11.86 against
  // 12.04-12.18 us on one box, 12.27-12.48 against 12.41-12.57 us on another; identical
  // codes).
  const bool few_rows = rows <= 256;
  if (vec && few_rows && packs > 4 && packs <= 8) {
    CI8_QW(8, 1)
  }
  if (vec) {
    CI8_QW(1, 1) CI8_QW(2, 1) CI8_QW(4, 1) CI8_QW(4, 2) CI8_QW(4, 3) CI8_QW(4, 4)
    CI8_QW(4, 5) CI8_QW(4, 6) CI8_QW(4, 7) CI8_QW(4, 8) CI8_QW(4, 9) CI8_QW(4, 10)
    CI8_QW(4, 12) CI8_QW(4, 14) CI8_QW(4, 16) CI8_QW(4, 20) CI8_QW(4, 24) CI8_QW(4, 32)
  }
#undef CI8_QW
  quantize_rows_scalar_kernel<kGrouped><<<(rows + 3) / 4, 256, 0, stream>>>(
      src, codes, scales, rows, k, m, groups);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_quantize_rows(const void* x, int8_t* codes, float* scales, int m, int k,
                                hipStream_t stream) {
  return dispatch<false>(x, codes, scales, m, k, m, 1, stream);
}

hipError_t launch_quantize_grouped(const void* x, int8_t* codes, float* scales, int m,
                                   int groups, int k, hipStream_t stream) {
  if (m == 0) return hipSuccess;
  return dispatch<true>(x, codes, scales, m * groups, k, m, groups, stream);
}

}  // namespace ci8
