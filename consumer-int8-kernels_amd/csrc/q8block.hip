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
// 4 outputs per lane.
//
// Main kernel (K a multiple of 128, sw 4-byte aligned): A, W and both scale arrays go
// through a four-stage LDS ring filled by buffer_load ... lds (three stages in flight
// per workgroup), 128 K values (4 blocks) a stage. The scale products fl(sa * sw) of a
// stage's 4 blocks come from one v_mfma_f32_16x16x1f32 per 16 x 16 tile: its four
// 16 x 16 outer products (A column = sa of block lane / 16, B row = sw of that block)
// are exact products rounded once each, as the FP32 multiply rounds (checked on MI355X
// over 4.2 M operand pairs: identical bits, except that a zero product is +0 where the
// multiply gives -0, which cannot reach the output because the running sum, starting
// at +0, is never -0), and they land in the layout of the INT32 MFMA output. That
// leaves 2 VALU instructions per output per block (a convert and the multiply-add).
// Tiles: 64 x 64 on 8 waves (2 x 4 waves of 32 x 16), or 128 x 128 on 16 waves once
// those fill the chip twice over. Measured on MI355X: M=2048, N=1024, K=4096 56 -> 38
// us, M=N=K=4096 366 -> 257 us against the kernel below.
//
// Fallback (any K % 32 == 0): a workgroup computes a 64 x 64 output tile on 8 waves
// (16 rows x 32 columns each), or 32 x 32 on 4 waves for small problems. K advances 256
// values (8 blocks) a step: the A and W slabs (16-byte loads, rows padded in LDS against
// bank conflicts) and their scales (W's converted to FP32) are staged in LDS, with the
// next step's global loads issued into registers before the current step's arithmetic,
// and the scale product is a VALU multiply (3 VALU instructions per output per block).
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
  const int tiles_n = (n + T::kBN - 1) / T::kBN;
  const int row0 = int(blockIdx.x) / tiles_n * T::kBM, col0 = int(blockIdx.x) % tiles_n * T::kBN;
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
  // One-dimensional grid: m * n <= INT_MAX keeps the tile count far below 2^31 - 1.
  const unsigned grid = unsigned((n + T::kBN - 1) / T::kBN) * unsigned((m + T::kBM - 1) / T::kBM);
  q8_block_mm_kernel<kWR, kWC, kWM, kWN, kBK, kOcc, kUnroll>
      <<<grid, T::kThreads, 0, stream>>>(a, sa, w, sw, y, m, n, k);
}

// ------------------------------------------------------------------ ring kernel

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x32_t __attribute__((ext_vector_type(32)));
typedef int32_t i32x16_t __attribute__((ext_vector_type(16)));

// LDS DMA copies (non-template helpers: the host pass of a kernel template rejects the
// 16-byte form of the builtin, which only gfx950 has).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, lds_void* dst,
                                      uint32_t offset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, offset, 0, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t rsrc, lds_void* dst,
                                     uint32_t offset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 4, offset, 0, 0, 0);
}

// kWM x kWN waves, each owning kTM x kTN MFMA tiles of 16 x 16 (or, with kMfma32, one
// 32 x 32 tile: kTM = kTN = 2); kNS ring stages of 128 K values; kOcc waves per SIMD
// the register allocation must allow.
template <int kWM_, int kWN_, int kTM_, int kTN_, int kNS_, int kOcc_, bool kMfma32_ = false>
struct RingTile {
  static constexpr int kWM = kWM_, kWN = kWN_, kTM = kTM_, kTN = kTN_, kNS = kNS_;
  static constexpr int kOcc = kOcc_;
  static constexpr bool kMfma32 = kMfma32_;
  static_assert(!kMfma32 || (kTM == 2 && kTN == 2), "a 32 x 32 tile per wave");
  static constexpr int kWaves = kWM * kWN, kThreads = 64 * kWaves;
  static constexpr int kBM = kWM * kTM * 16, kBN = kWN * kTN * 16, kBK = 128;
  // One stage: A rows of 128 bytes, W rows, sa [row][4 blocks] FP32, and sw as two
  // planes (blocks 0-1, 2-3) of [column][2 blocks] FP16.
  static constexpr int kA = kBM * kBK, kW = kBN * kBK, kSa = kBM * 16, kSw = kBN * 8;
  static constexpr int kStage = kA + kW + kSa + kSw;
  // Copies per stage: 1 KiB of A or W rows (8 rows x 128 bytes), 1 KiB of sa (64 rows),
  // 256 bytes of one sw plane (64 columns x 4 bytes).
  static constexpr int nA = kBM / 8, nW = kBN / 8, nSa = kBM / 64, nSw = kBN / 32;
  static constexpr int nCopies = nA + nW + nSa + nSw;
  static constexpr int kPerWave = (nCopies + kWaves - 1) / kWaves;  // the rest: junk copies
  static constexpr int kJunk = kNS * kStage;
  static constexpr int kLds = kJunk + 1024;
  static_assert(kBM % 64 == 0 && kBN % 64 == 0, "scale copies cover 64 rows or columns");
  static_assert(kLds <= 160 * 1024, "LDS");
  static_assert(kPerWave * (kNS - 2) <= 63, "vmcnt holds 6 bits");
};

// Requires k % 128 == 0, a and w 16-byte aligned, sa 4-byte and sw 4-byte aligned.
// 16 x 16 tiles: v_mfma_i32_16x16x32_i8, one per block, reads 8 bytes a lane; A and W
// rows sit in LDS with their 16-byte chunks XOR-swizzled by (row / 2) % 8. Those 8-byte
// reads of 16 rows still meet 2-way bank conflicts (the copies move 16-byte chunks, so
// no swizzle can separate the two 8-byte halves of a chunk): measured on MI355X, 17.8%
// of the kernel's cycles against 21.8% with row % 8.
// 32 x 32 tiles: two v_mfma_i32_32x32x16_i8 per block. Lane (row r = lane % 32, half
// h = lane / 32) feeds K values 16 h + 8 s .. + 7 of the block in step s (A and W alike,
// so the exact INT32 sums are the block's), i.e. one 16-byte chunk 2 q + h per block:
// 16-byte reads, chunks swizzled by row % 8, as in the other GEMMs. The scale products
// of two blocks come from one v_mfma_f32_32x32x1f32 (two 32 x 32 outer products,
// rounded as the FP32 multiply: checked on MI355X over 4.2 M operand pairs, like the
// 16 x 16 form), in the layout of the INT32 output: register 16 b + i holds block b's
// row 8 (i / 4) + 4 h + i % 4, column lane % 32 (checked on MI355X).
template <class T>
__global__ void __launch_bounds__(T::kThreads, T::kOcc) q8_ring_kernel(
    const int8_t* __restrict__ a, const float* __restrict__ sa, const int8_t* __restrict__ w,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ y, int m, int n, int k) {
  extern __shared__ __attribute__((aligned(1024))) char lds_raw[];
  auto* lds = (char __attribute__((address_space(3)))*)(lds_raw);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tiles_n = (n + T::kBN - 1) / T::kBN;
  // Workgroup -> tile: the hardware deals workgroups to the 8 XCDs round-robin, so each
  // XCD's workgroups take a contiguous range of a raster grouped by 8 m tiles, and the
  // tiles one XCD runs share A and W panels in its L2 (measured on MI355X, identical
  // outputs: M = 2048, N = 1024, K = 4096 43.6 against 44.5-45.2 us; M = 1000, N = 3000,
  // K = 2048 30.1 against 31.3-31.6 us, for the row-major order).
  int row0, col0;
  {
    const int tiles_m = (m + T::kBM - 1) / T::kBM;
    const int tiles = tiles_m * tiles_n;
    const int per = tiles / 8, extra = tiles % 8;
    const int xcd = int(blockIdx.x) % 8, idx = int(blockIdx.x) / 8;
    const int logical =
        (xcd < extra ? xcd * (per + 1) : extra * (per + 1) + (xcd - extra) * per) + idx;
    constexpr int kGroupM = 8;
    const int group_span = kGroupM * tiles_n;
    const int first_m = (logical / group_span) * kGroupM;
    const int group_rows = min(tiles_m - first_m, kGroupM);
    row0 = (first_m + (logical % group_span) % group_rows) * T::kBM;
    col0 = ((logical % group_span) / group_rows) * T::kBN;
  }
  const int kb32 = k / 32;
  const int stages = k / T::kBK;
  const auto a_rsrc = make_rsrc(a, uint32_t(m) * uint32_t(k));
  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto sa_rsrc = make_rsrc(sa, uint32_t(m) * uint32_t(kb32) * 4u);
  const auto sw_rsrc = make_rsrc(sw, uint32_t(n) * uint32_t(kb32) * 2u);

  // Stage st's copies into ring slot st % kNS: copy j = wave + kWaves * i of the list
  // A, W, sa, sw, junk (every wave issues kPerWave, so one vmcnt fits all). Stages past
  // the end copy nothing but zeros from out of range, which keeps the counts uniform.
  // Each of this wave's copies is fixed up front as (buffer, LDS offset in the slot,
  // this lane's offset at stage 0 or out of range, bytes per stage, 16 or 4 bytes per
  // lane), so a stage issues them without walking the list.
  __amdgpu_buffer_rsrc_t c_rsrc[T::kPerWave];
  int c_lds[T::kPerWave];
  uint32_t c_off[T::kPerWave], c_step[T::kPerWave];
  bool c_wide[T::kPerWave];
#pragma unroll
  for (int i = 0; i < T::kPerWave; ++i) {
    const int j = wave + T::kWaves * i;  // uniform over the wave
    if (j < T::nA + T::nW) {
      const bool is_a = j < T::nA;
      const int jj = is_a ? j : j - T::nA;
      const int r = jj * 8 + (lane >> 3);
      const int chunk = (lane & 7) ^ (T::kMfma32 ? (r & 7) : ((r >> 1) & 7));
      const int first = is_a ? row0 : col0;
      c_rsrc[i] = is_a ? a_rsrc : w_rsrc;
      c_lds[i] = (is_a ? 0 : T::kA) + jj * 1024;
      c_off[i] = first + r < (is_a ? m : n) ? uint32_t(first + r) * uint32_t(k) + uint32_t(chunk * 16)
                                            : kOutOfRange;
      c_step[i] = T::kBK;
      c_wide[i] = true;
    } else if (j < T::nA + T::nW + T::nSa) {
      const int jj = j - T::nA - T::nW;
      const int r = jj * 64 + lane;
      c_rsrc[i] = sa_rsrc;
      c_lds[i] = T::kA + T::kW + jj * 1024;
      c_off[i] = row0 + r < m ? uint32_t(row0 + r) * uint32_t(kb32) * 4u : kOutOfRange;
      c_step[i] = 16;  // 4 blocks x FP32
      c_wide[i] = true;
    } else if (j < T::nCopies) {
      const int jj = j - T::nA - T::nW - T::nSa;  // plane jj % 2, columns 64 (jj / 2) ..
      const int plane = jj & 1, c = (jj >> 1) * 64 + lane;
      c_rsrc[i] = sw_rsrc;
      c_lds[i] = T::kA + T::kW + T::kSa + plane * (T::kBN * 4) + (jj >> 1) * 256;
      c_off[i] = col0 + c < n ? uint32_t(col0 + c) * uint32_t(kb32) * 2u + 4u * plane : kOutOfRange;
      c_step[i] = 8;  // 4 blocks x FP16
      c_wide[i] = false;
    } else {
      c_rsrc[i] = sw_rsrc;
      c_lds[i] = -1;  // the junk KiB, outside the ring
      c_off[i] = kOutOfRange;
      c_step[i] = 0;
      c_wide[i] = false;
    }
  }
  auto issue = [&](int st) __attribute__((always_inline)) {
    const int slot = (st % T::kNS) * T::kStage;
    const bool live = st < stages;
#pragma unroll
    for (int i = 0; i < T::kPerWave; ++i) {
      const uint32_t off =
          live && c_off[i] != kOutOfRange ? c_off[i] + uint32_t(st) * c_step[i] : kOutOfRange;
      auto* dst = (lds_void*)(lds + (c_lds[i] < 0 ? T::kJunk : slot + c_lds[i]));
      // A copy slot that holds A, W or sa rows for every wave needs no branch.
      if ((i + 1) * T::kWaves <= T::nA + T::nW + T::nSa || c_wide[i])
        dma16(c_rsrc[i], dst, off);
      else
        dma4(c_rsrc[i], dst, off);
    }
  };

  const int wm = wave % T::kWM, wn = wave / T::kWM;
  float sum[T::kTM * T::kTN * 4];
#pragma unroll
  for (int i = 0; i < T::kTM * T::kTN * 4; ++i) sum[i] = 0.f;

#pragma unroll
  for (int st = 0; st < T::kNS - 1; ++st) issue(st);
  for (int t = 0; t < stages; ++t) {
    // This wave's copies of stage t have landed (those of the kNS - 2 later stages may
    // be in flight); after the barrier every wave's have, and slot (t - 1) % kNS, read
    // in stage t - 1, is free for stage t + kNS - 1.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(T::kPerWave * (T::kNS - 2)));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(t + T::kNS - 1);
    __builtin_amdgcn_sched_barrier(0);
    const auto* base = lds + (t % T::kNS) * T::kStage;
    if constexpr (T::kMfma32) {
      const int lr = lane & 31, lh = lane >> 5;
      const int arow = wm * 32 + lr, wrow = wn * 32 + lr;
#pragma unroll
      for (int p = 0; p < 2; ++p) {  // blocks 2p and 2p + 1
        const float sa_op = *reinterpret_cast<const __attribute__((address_space(3))) float*>(
            base + T::kA + T::kW + arow * 16 + (2 * p + lh) * 4);
        const float sw_op = half_to_float(*reinterpret_cast<const __attribute__((address_space(3))) uint16_t*>(
            base + T::kA + T::kW + T::kSa + p * (T::kBN * 4) + wrow * 4 + lh * 2));
        const f32x32_t scl = __builtin_amdgcn_mfma_f32_32x32x1f32(sa_op, sw_op, f32x32_t{}, 0, 0, 0);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int chunk = 2 * (2 * p + b) + lh;
          const u32x4 af = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
              base + arow * 128 + ((chunk ^ (arow & 7)) * 16));
          const u32x4 wf = *reinterpret_cast<const __attribute__((address_space(3))) u32x4*>(
              base + T::kA + wrow * 128 + ((chunk ^ (wrow & 7)) * 16));
          i32x16_t acc = {};
#pragma unroll
          for (int st2 = 0; st2 < 2; ++st2)
            acc = __builtin_amdgcn_mfma_i32_32x32x16_i8(
                int64_t(af[2 * st2]) | (int64_t(af[2 * st2 + 1]) << 32),
                int64_t(wf[2 * st2]) | (int64_t(wf[2 * st2 + 1]) << 32), acc, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 16; ++i) sum[i] = __builtin_fmaf(float(acc[i]), scl[16 * b + i], sum[i]);
        }
      }
    } else {
      const int lr = lane & 15, lq = lane >> 4;
      f32x16_t scl[T::kTM][T::kTN];
      {
        float sa_op[T::kTM], sw_op[T::kTN];
#pragma unroll
        for (int ti = 0; ti < T::kTM; ++ti) {
          const int row = (wm * T::kTM + ti) * 16 + lr;
          sa_op[ti] = *reinterpret_cast<const __attribute__((address_space(3))) float*>(
              base + T::kA + T::kW + row * 16 + lq * 4);
        }
#pragma unroll
        for (int tj = 0; tj < T::kTN; ++tj) {
          const int col = (wn * T::kTN + tj) * 16 + lr;
          sw_op[tj] = half_to_float(*reinterpret_cast<const __attribute__((address_space(3))) uint16_t*>(
              base + T::kA + T::kW + T::kSa + (lq >> 1) * (T::kBN * 4) + col * 4 + (lq & 1) * 2));
        }
#pragma unroll
        for (int ti = 0; ti < T::kTM; ++ti)
#pragma unroll
          for (int tj = 0; tj < T::kTN; ++tj)
            scl[ti][tj] = __builtin_amdgcn_mfma_f32_16x16x1f32(sa_op[ti], sw_op[tj], f32x16_t{}, 0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // Lane group lq takes bytes 8 lq .. 8 lq + 7 of block q: chunk 2q + lq / 2.
        const int chunk = 2 * q + (lq >> 1);
        int64_t af[T::kTM], wf[T::kTN];
#pragma unroll
        for (int ti = 0; ti < T::kTM; ++ti) {
          const int row = (wm * T::kTM + ti) * 16 + lr;
          af[ti] = *reinterpret_cast<const __attribute__((address_space(3))) int64_t*>(
              base + row * 128 + ((chunk ^ ((row >> 1) & 7)) * 16) + (lq & 1) * 8);
        }
#pragma unroll
        for (int tj = 0; tj < T::kTN; ++tj) {
          const int row = (wn * T::kTN + tj) * 16 + lr;
          wf[tj] = *reinterpret_cast<const __attribute__((address_space(3))) int64_t*>(
              base + T::kA + row * 128 + ((chunk ^ ((row >> 1) & 7)) * 16) + (lq & 1) * 8);
        }
#pragma unroll
        for (int ti = 0; ti < T::kTM; ++ti)
#pragma unroll
          for (int tj = 0; tj < T::kTN; ++tj) {
            const i32x4_t acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(af[ti], wf[tj],
                                                                     i32x4_t{0, 0, 0, 0}, 0, 0, 0);
            float* o = sum + (ti * T::kTN + tj) * 4;
#pragma unroll
            for (int i = 0; i < 4; ++i)
              o[i] = __builtin_fmaf(float(acc[i]), scl[ti][tj][4 * q + i], o[i]);
          }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // drain the trailing (out-of-range) copies
  if constexpr (T::kMfma32) {
    const int lr = lane & 31, lh = lane >> 5;
    const int col = col0 + wn * 32 + lr;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = row0 + wm * 32 + 8 * (i / 4) + 4 * lh + (i % 4);
      if (row < m && col < n) y[int64_t(row) * n + col] = uint16_t(f32_to_bf16(sum[i]));
    }
  } else {
    const int lr = lane & 15, lq = lane >> 4;
#pragma unroll
    for (int ti = 0; ti < T::kTM; ++ti)
#pragma unroll
      for (int tj = 0; tj < T::kTN; ++tj) {
        const int col = col0 + (wn * T::kTN + tj) * 16 + lr;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = row0 + (wm * T::kTM + ti) * 16 + lq * 4 + i;
          if (row < m && col < n)
            y[int64_t(row) * n + col] = uint16_t(f32_to_bf16(sum[(ti * T::kTN + tj) * 4 + i]));
        }
      }
  }
}

template <class T>
hipError_t launch_ring(const int8_t* a, const float* sa, const int8_t* w, const uint16_t* sw,
                       uint16_t* y, int m, int n, int k, hipStream_t stream) {
  auto kernel = q8_ring_kernel<T>;
  if (const hipError_t e = prepare_lds<q8_ring_kernel<T>>(T::kLds); e != hipSuccess)
    return e;
  // One-dimensional grid: m * n <= INT_MAX keeps the tile count far below 2^31 - 1.
  const unsigned grid = unsigned((m + T::kBM - 1) / T::kBM) * unsigned((n + T::kBN - 1) / T::kBN);
  kernel<<<grid, T::kThreads, T::kLds, stream>>>(a, sa, w, sw, y, m, n, k);
  return hipGetLastError();
}

using Ring64 = RingTile<2, 4, 2, 1, 4, 2>;         // 64 x 64, waves of 32 x 16, two per CU
using Ring128 = RingTile<4, 4, 2, 2, 4, 4, true>;  // 128 x 128, 16 waves of 32 x 32, one per CU

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
  const auto* s16 = static_cast<const uint16_t*>(sw);
  auto* out = static_cast<uint16_t*>(y);
  if (k % 128 == 0 && reinterpret_cast<uintptr_t>(sw) % 4 == 0) {
    // The ring kernel; 128 x 128 tiles on 32 x 32 MFMAs once there are two per CU
    // (M = N = K = 4096: 228 us, against 246 us for 16 x 16 MFMAs and 272 us for 64 x 64
    // tiles), else 64 x 64 on 16 x 16 MFMAs (at M = 2048, N = 1024, K = 4096 the 32 x 32
    // form of any of three tile shapes is no faster).
    const int cus = device_cu_count();
    const int64_t tiles128 = int64_t((m + 127) / 128) * ((n + 127) / 128);
    if (cus > 0 && tiles128 >= 2 * int64_t(cus))
      return launch_ring<Ring128>(a, sa, w, s16, out, m, n, k, stream);
    return launch_ring<Ring64>(a, sa, w, s16, out, m, n, k, stream);
  }
  // Other K or 2-byte-aligned sw: the step kernel, 64 x 64 tiles on 8 waves (each 16 rows
  // x 32 columns), K steps of 256; 32 x 32 tiles on 4 waves when the larger tiles would
  // leave CUs idle (tile-shape sweep at N = 1024, K = 4096, M = 512 and 2048).
  const int64_t big_tiles = int64_t((m + 63) / 64) * ((n + 63) / 64);
  if (big_tiles >= 256)
    launch_q8_tile<4, 2, 1, 2, 256, 4, 2>(a, sa, w, s16, out, m, n, k, stream);
  else
    launch_q8_tile<2, 2, 1, 1, 256, 4, 2>(a, sa, w, s16, out, m, n, k, stream);
  return hipGetLastError();
}

}  // namespace ci8
