// Grouped W8A16 with GGUF Q8_0 weights (gguf_q8_packed_mm) for gfx950.
//
//   wq[g, n, k]  = bf16_rn( float(code[g, n, k]) * float(scale[g, n, k / 32]) )
//   out[m, g, n] = bf16_rn( sum_k float(x[m, g, k]) * float(wq[g, n, k]) )   (FP32 sums)
//
// The arithmetic of csrc/gguf_q8_packed.cu:176-183 and :230-244 of the reference: the
// original signed codes and FP16 block scales of each 32-value block are multiplied
// (exactly, in FP32: 8-bit by 11-bit significands), rounded once to BF16, and fed with
// the BF16 activations to a BF16 matrix product with FP32 accumulation. The summation
// order is the hardware's, so parity is by tolerance, as in the reference's test
// (tests/test_gguf_q8.py:20-62).
//
// Layout: x BF16 [M, G, K] with independent row and group strides (K contiguous), codes
// INT8 [G, N, K], scales FP16 [G, N, K / 32], out BF16 [M, G, N] contiguous; K % 64 == 0.
//
// Design: a workgroup computes a BM x 64 (rows x channels) tile of one group; its four
// waves each own a 16-channel block and BM / 16 row blocks of
// v_mfma_f32_16x16x32_bf16 accumulators (the MFMA computes D[n][m] = Wq . x^T, so a lane
// holds 4 consecutive channels of one row and stores 8 bytes). K advances 64 at a time
// through two LDS buffers: while a stage is multiplied, the next stage's x and codes
// are already in registers; the codes are dequantized to BF16 on their way into LDS,
// once per workgroup. Rows past M or N read as zero and are not stored.
#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

constexpr int kBK = 64;  // K per stage
constexpr int kBN = 64;  // channels per workgroup

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// FP16 bit pattern -> FP32 (exact).
__device__ __forceinline__ float f16_to_f32(uint32_t bits) {
  return float(__builtin_bit_cast(_Float16, uint16_t(bits)));
}

// LDS tiles are [rows][64 BF16] = 128 bytes per row, 16-byte chunks XOR-swizzled by
// row % 8 so the 16 rows of a fragment read at one chunk fall in distinct banks.
__device__ __forceinline__ int tile_offset(int row, int chunk) {
  return row * 128 + ((chunk ^ (row & 7)) * 16);
}

template <int BM>
__global__ void __launch_bounds__(256) gguf_q8_packed_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, uint16_t* __restrict__ out, int m, int n, int k,
    int groups, int64_t xs, int64_t xg) {
  constexpr int TM = BM / 16;                  // row blocks per wave
  constexpr int kXChunks = BM * kBK / 8;       // 16-byte x chunks per stage
  constexpr int kXPerThread = (kXChunks + 255) / 256;
  __shared__ __attribute__((aligned(16))) char xs_lds[2][BM * 128];
  __shared__ __attribute__((aligned(16))) char ws_lds[2][kBN * 128];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.z;
  const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * BM;
  const int8_t* gcodes = codes + int64_t(g) * n * k;
  const uint16_t* gscales = scales + int64_t(g) * n * (k / 32);

  // Global -> register staging. x: chunk c of the stage is row c / 8, 16-byte chunk c % 8.
  // Codes: thread t takes row t / 4, 16 codes at k offset (t % 4) * 16, and their scale.
  u32x4 xr[kXPerThread];
  u32x4 cr;
  uint32_t sr;
  const int c_row = tid >> 2, c_col = (tid & 3) * 16;
  const bool c_live = n0 + c_row < n;
  auto load = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kXPerThread; ++i) {
      const int c = i * 256 + tid;
      const int row = c >> 3, chunk = c & 7;
      xr[i] = u32x4{0, 0, 0, 0};
      if (c < kXChunks && m0 + row < m)
        xr[i] = *reinterpret_cast<const u32x4*>(x + int64_t(m0 + row) * xs + int64_t(g) * xg +
                                                 k0 + chunk * 8);
    }
    cr = u32x4{0, 0, 0, 0};
    sr = 0;
    if (c_live) {
      cr = *reinterpret_cast<const u32x4*>(gcodes + int64_t(n0 + c_row) * k + k0 + c_col);
      sr = gscales[int64_t(n0 + c_row) * (k / 32) + (k0 + c_col) / 32];
    }
  };
  // Registers -> LDS buffer b, dequantizing the codes: 16 codes -> 16 BF16 (2 chunks).
  auto store = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kXPerThread; ++i) {
      const int c = i * 256 + tid;
      if (c < kXChunks)
        *reinterpret_cast<u32x4*>(xs_lds[b] + tile_offset(c >> 3, c & 7)) = xr[i];
    }
    const float s = f16_to_f32(sr);
    uint32_t packed[8];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t word = cr[w];
      packed[2 * w] = pack_bf16x2(float(int8_t(word)) * s, float(int8_t(word >> 8)) * s);
      packed[2 * w + 1] = pack_bf16x2(float(int8_t(word >> 16)) * s, float(int8_t(word >> 24)) * s);
    }
    const int chunk = c_col / 8;
    *reinterpret_cast<u32x4*>(ws_lds[b] + tile_offset(c_row, chunk)) =
        u32x4{packed[0], packed[1], packed[2], packed[3]};
    *reinterpret_cast<u32x4*>(ws_lds[b] + tile_offset(c_row, chunk + 1)) =
        u32x4{packed[4], packed[5], packed[6], packed[7]};
  };

  // Wave w owns channel block w (16 channels) and all TM row blocks. Fragment lane
  // layout (16x16x32 BF16 MFMA): row lane % 16, K elements 8 * (lane / 16) .. + 7 of
  // the 32-wide K-step, i.e. 16-byte chunk 4h + lane / 16 of the 64-wide stage.
  const int f_row = lane & 15, f_chunk = lane >> 4;
  f32x4 acc[TM];
#pragma unroll
  for (int j = 0; j < TM; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};

  load(0);
  store(0);
  __syncthreads();
  const int stages = k / kBK;
  for (int t = 0; t < stages; ++t) {
    const int b = t & 1;
    if (t + 1 < stages) load((t + 1) * kBK);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4 wfrag = *reinterpret_cast<const u32x4*>(
          ws_lds[b] + tile_offset(wave * 16 + f_row, 4 * h + f_chunk));
#pragma unroll
      for (int j = 0; j < TM; ++j) {
        const u32x4 xfrag = *reinterpret_cast<const u32x4*>(
            xs_lds[b] + tile_offset(j * 16 + f_row, 4 * h + f_chunk));
        acc[j] = mfma_bf16(wfrag, xfrag, acc[j]);
      }
    }
    if (t + 1 < stages) store(b ^ 1);  // buffer b ^ 1 was last read in stage t - 1
    __syncthreads();
  }

  // Lane holds D[n][m] for n = 4 * (lane / 16) + e of the wave's channel block and
  // m = lane % 16 of each row block.
  const int col = n0 + wave * 16 + 4 * f_chunk;
  const bool vec = (n & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0;
#pragma unroll
  for (int j = 0; j < TM; ++j) {
    const int row = m0 + j * 16 + f_row;
    if (row >= m) continue;
    uint16_t* dst = out + (int64_t(row) * groups + g) * n + col;
    if (vec && col + 3 < n) {
      *reinterpret_cast<u32x2*>(dst) =
          u32x2{pack_bf16x2(acc[j][0], acc[j][1]), pack_bf16x2(acc[j][2], acc[j][3])};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (col + e < n) dst[e] = uint16_t(f32_to_bf16(acc[j][e]));
    }
  }
}

}  // namespace

hipError_t launch_gguf_q8_packed_mm(const void* x, const int8_t* codes, const void* scales,
                                    void* out, int m, int n, int k, int groups, int64_t xs,
                                    int64_t xg, hipStream_t stream) {
  if (m == 0 || n == 0 || groups == 0) return hipSuccess;
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* sp = static_cast<const uint16_t*>(scales);
  auto* op = static_cast<uint16_t*>(out);
  const unsigned tiles_n = unsigned((n + kBN - 1) / kBN);
  if (m <= 16) {
    gguf_q8_packed_kernel<16><<<dim3(tiles_n, unsigned(m + 15) / 16, unsigned(groups)), 256, 0,
                                stream>>>(xp, codes, sp, op, m, n, k, groups, xs, xg);
  } else {
    gguf_q8_packed_kernel<64><<<dim3(tiles_n, unsigned(m + 63) / 64, unsigned(groups)), 256, 0,
                                stream>>>(xp, codes, sp, op, m, n, k, groups, xs, xg);
  }
  return hipGetLastError();
}

}  // namespace ci8
