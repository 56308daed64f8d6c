// channel_mm for operands at any byte alignment.
//
// The reference's channel_mm binding (csrc/bindings.cpp:238-265) accepts any INT8 and
// UINT8 views, and its kernel reads the operands as 4-byte words (csrc/kernels.cu:99-110).
// The MFMA kernels here copy 16-byte chunks (buffer_load ... lds) and so need 16-byte
// aligned rows; an operand that starts elsewhere (a sliced view) takes this kernel
// instead. It is a plain, correct fallback, not a fast path: byte loads into LDS and
// v_dot4_i32_i8 on the VALU. The products are exact INT32 sums and the epilogue is the
// same two FP32 multiplies and one BF16 rounding as every other GEMM kernel here, so
// its output is bit-identical to theirs.
#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

constexpr int kTile = 64;  // output rows and columns per workgroup
constexpr int kKStep = 32;  // K bytes per LDS stage

// 8 bytes at an arbitrary address, little-endian into two words.
__device__ __forceinline__ void load8(const uint8_t* p, uint32_t& lo, uint32_t& hi) {
  lo = uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24;
  hi = uint32_t(p[4]) | uint32_t(p[5]) << 8 | uint32_t(p[6]) << 16 | uint32_t(p[7]) << 24;
}

template <WeightCode kCode>
__global__ void __launch_bounds__(256) gemm_bytes_kernel(
    const uint8_t* __restrict__ a, const uint8_t* __restrict__ w, const float* __restrict__ sa,
    const uint16_t* __restrict__ sw, uint16_t* __restrict__ out, int m, int n, int k) {
  // [row][word] with one word of padding so the 16 rows a thread group reads at one word
  // fall in different banks.
  __shared__ uint32_t as[kTile][kKStep / 4 + 1];
  __shared__ uint32_t ws[kTile][kKStep / 4 + 1];
  const int tid = threadIdx.x;
  const int tiles_n = (n + kTile - 1) / kTile;
  const int m0 = int(blockIdx.x) / tiles_n * kTile, n0 = int(blockIdx.x) % tiles_n * kTile;
  const int ty = tid / 16, tx = tid % 16;  // outputs rows ty*4 .. +3, columns tx*4 .. +3
  const int l_row = tid / 4, l_byte = (tid % 4) * 8;
  const bool a_live = m0 + l_row < m, w_live = n0 + l_row < n;
  const uint8_t* a_src = a + int64_t(m0 + l_row) * k + l_byte;
  const uint8_t* w_src = w + int64_t(n0 + l_row) * k + l_byte;

  int acc[4][4] = {};
  for (int k0 = 0; k0 < k; k0 += kKStep) {
    uint32_t a_lo = 0, a_hi = 0, w_lo = 0, w_hi = 0;
    if (a_live) load8(a_src + k0, a_lo, a_hi);
    if (w_live) load8(w_src + k0, w_lo, w_hi);
    if constexpr (kCode == WeightCode::kBiasedU8) {
      // code + 128 -> signed code: flip each byte's top bit (rows past N stay zero).
      if (w_live) {
        w_lo ^= 0x80808080u;
        w_hi ^= 0x80808080u;
      }
    }
    as[l_row][l_byte / 4] = a_lo;
    as[l_row][l_byte / 4 + 1] = a_hi;
    ws[l_row][l_byte / 4] = w_lo;
    ws[l_row][l_byte / 4 + 1] = w_hi;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kKStep / 4; ++q) {
      int av[4], wv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = int(as[ty * 4 + i][q]);
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[j] = int(ws[tx * 4 + j][q]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_sdot4(av[i], wv[j], acc[i][j], false);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = m0 + ty * 4 + i;
    if (row >= m) continue;
    const float rs = sa[row];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + tx * 4 + j;
      if (col < n)
        out[int64_t(row) * n + col] =
            uint16_t(f32_to_bf16((float(acc[i][j]) * rs) * bf16_to_f32(sw[col])));
    }
  }
}

}  // namespace

hipError_t launch_channel_gemm_bytes(const int8_t* a, const void* w, WeightCode code,
                                     const float* sa, const void* sw, void* out, int m, int n,
                                     int k, hipStream_t stream) {
  // One-dimensional grid: m * n <= INT_MAX (checked by the caller) keeps the tile count
  // far below the 2^31 - 1 workgroup limit.
  const unsigned grid = unsigned((n + kTile - 1) / kTile) * unsigned((m + kTile - 1) / kTile);
  const auto* ap = reinterpret_cast<const uint8_t*>(a);
  const auto* wp = static_cast<const uint8_t*>(w);
  const auto* swp = static_cast<const uint16_t*>(sw);
  auto* op = static_cast<uint16_t*>(out);
  if (code == WeightCode::kBiasedU8)
    gemm_bytes_kernel<WeightCode::kBiasedU8><<<grid, 256, 0, stream>>>(ap, wp, sa, swp, op, m, n, k);
  else
    gemm_bytes_kernel<WeightCode::kSigned><<<grid, 256, 0, stream>>>(ap, wp, sa, swp, op, m, n, k);
  return hipGetLastError();
}

}  // namespace ci8
