// Small-batch W8A16 (channel_gemv) for gfx950.
//
//   wq[n, k]  = bf16_rn( float(w[n, k]) * float(scale[n]) )       (csrc/gemv.cu:25)
//   out[m, n] = bf16_rn( sum_k float(x[m, k]) * float(wq[n, k]) )  (FP32 accumulation)
//
// The dequantized multiplicand is bit-identical to the reference's. Only the FP32
// summation order differs (the reference uses a per-lane FMA chain and a 32-lane
// butterfly, csrc/gemv.cu:16-45; here the products are summed by the MFMA and the
// partial sums of four waves are added in a fixed order), so parity is by tolerance
// as in tests/test_gemv.py:24-33.
//
// Design: the op is HBM-bound on the INT8 weights (N*K bytes), so the VALU work per
// weight must stay well below the load rate. The multiply-accumulate goes to
// v_mfma_f32_16x16x32_bf16 (rows = 16 channels, columns = up to 16 batch rows, so
// m <= 16 costs the same as m = 1), leaving the VALU only the dequantization:
// XOR 0x80 (one op per four weights), v_cvt_f32_ubyteN, one FMA u*s - 128*s (exact,
// since code*scale fits in FP32), and v_cvt_pk_bf16_f32 (one op per two weights).
// A workgroup owns 16*kBlocks channels and its four waves split K; weight rows past
// N and K chunks past K read as zero through the buffer range check.
#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kGemvWaves = 4;

__device__ __forceinline__ uint32_t dequant_pair(uint32_t word, int shift, float s,
                                                 float bias) {
  // word holds (code + 128) bytes; bytes `shift/8` and `shift/8 + 1` are converted.
  const float lo = fmaf(float((word >> shift) & 0xFFu), s, bias);
  const float hi = fmaf(float((word >> (shift + 8)) & 0xFFu), s, bias);
  return pack_bf16x2(lo, hi);
}

template <int kBlocks, int kUnroll>
__global__ void __launch_bounds__(64 * kGemvWaves) channel_gemv_kernel(
    const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
    const uint16_t* __restrict__ scale, uint16_t* __restrict__ out, int m, int n, int k) {
  __shared__ f32x4 partial[kGemvWaves][kBlocks][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row = lane & 15;   // MFMA row (channel) / column (batch row)
  const int group = lane >> 4; // 16-element K group within a 64-wide K block
  const int n0 = blockIdx.x * (16 * kBlocks);

  const auto w_rsrc = make_rsrc(w, uint32_t(n) * uint32_t(k));
  const auto x_rsrc = make_rsrc(x, uint32_t(m) * uint32_t(k) * 2u);

  float s[kBlocks], bias[kBlocks];
  uint32_t w_off[kBlocks];
#pragma unroll
  for (int b = 0; b < kBlocks; ++b) {
    const int channel = n0 + b * 16 + row;
    s[b] = channel < n ? bf16_to_f32(scale[channel]) : 0.f;
    bias[b] = -128.f * s[b];
    w_off[b] = channel < n ? uint32_t(channel) * uint32_t(k) : kOutOfRange;
  }
  const uint32_t x_off = row < m ? uint32_t(row) * uint32_t(k) * 2u : kOutOfRange;

  f32x4 acc[kBlocks];
#pragma unroll
  for (int b = 0; b < kBlocks; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int kblocks = (k + 63) / 64;
  for (int kb0 = wave; kb0 < kblocks; kb0 += kGemvWaves * kUnroll) {
    u32x4 wv[kUnroll][kBlocks];
    u32x4 xv[kUnroll][2];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int kb = kb0 + u * kGemvWaves;
      const int kcol = kb * 64 + group * 16;
      const bool valid = kb < kblocks && kcol < k;
#pragma unroll
      for (int b = 0; b < kBlocks; ++b) {
        const uint32_t off = valid && w_off[b] != kOutOfRange ? w_off[b] + uint32_t(kcol)
                                                              : kOutOfRange;
        wv[u][b] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 w_rsrc, off, 0, 0));
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t off = valid && x_off != kOutOfRange
                                 ? x_off + uint32_t(kcol + h * 8) * 2u
                                 : kOutOfRange;
        xv[u][h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 x_rsrc, off, 0, 0));
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int b = 0; b < kBlocks; ++b) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t w0 = wv[u][b][2 * h] ^ 0x80808080u;
          const uint32_t w1 = wv[u][b][2 * h + 1] ^ 0x80808080u;
          const u32x4 wq{dequant_pair(w0, 0, s[b], bias[b]), dequant_pair(w0, 16, s[b], bias[b]),
                         dequant_pair(w1, 0, s[b], bias[b]), dequant_pair(w1, 16, s[b], bias[b])};
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, wq), __builtin_bit_cast(bf16x8, xv[u][h]), acc[b], 0,
              0, 0);
        }
      }
    }
  }

  // Sum the four waves' partials in a fixed order, then round once to BF16.
#pragma unroll
  for (int b = 0; b < kBlocks; ++b) partial[wave][b][lane] = acc[b];
  __syncthreads();
  for (int slot = threadIdx.x; slot < kBlocks * 64 * 4; slot += 64 * kGemvWaves) {
    const int e = slot & 3, l = (slot >> 2) & 63, b = slot >> 8;
    const int out_row = l & 15;                            // batch row m
    const int channel = n0 + b * 16 + (l >> 4) * 4 + e;    // output column n
    if (out_row >= m || channel >= n) continue;
    float sum = partial[0][b][l][e];
#pragma unroll
    for (int v = 1; v < kGemvWaves; ++v) sum += partial[v][b][l][e];
    out[int64_t(out_row) * n + channel] = uint16_t(f32_to_bf16(sum));
  }
}

}  // namespace

hipError_t launch_channel_gemv(const void* x, const int8_t* w, const void* scale, void* out,
                               int m, int n, int k, hipStream_t stream) {
  constexpr int kBlocks = 2, kUnroll = 4;
  const int grid = (n + 16 * kBlocks - 1) / (16 * kBlocks);
  channel_gemv_kernel<kBlocks, kUnroll><<<grid, 64 * kGemvWaves, 0, stream>>>(
      static_cast<const uint16_t*>(x), w, static_cast<const uint16_t*>(scale),
      static_cast<uint16_t*>(out), m, n, k);
  return hipGetLastError();
}

}  // namespace ci8
