// unpack_allspark: AllSpark N32K16 packed UINT8 weights and permuted BF16 scales ->
// row-major signed INT8 weights [n, k] and channel scales [n] (the reference's
// csrc/allspark_layout.cu:8-35, whose index map defines the format).
//
// The format, read off that map: output rows come in groups of 32; rows
// 32G + r8 + 8q (r8 = 0..7, q = 0..3) share packed row 8G + r8 of 4k bytes, which is
// k/16 tiles of 64 bytes. Tile t holds k = 16t .. 16t + 15 of those four rows as four
// 16-byte chunks j = 0..3; chunk j is four 4-byte pieces, one per q, holding the biased
// codes (code + 128) of k = 16t + 2j, 16t + 2j + 1, 16t + 8 + 2j, 16t + 9 + 2j. Scale
// 32G + r8 + 8q sits at packed position 32G + 4 r8 + q.
//
// One lane per (packed row, tile): it loads the whole 64-byte tile (four 16-byte loads;
// the lanes of a wave take consecutive tiles, so together they read 4 KiB of one packed
// row), rebuilds the four output rows' 16-byte pieces with byte selects and a XOR of
// 0x80 per byte, and stores them; consecutive lanes write consecutive 16-byte pieces of
// each output row (nontemporal stores: the restored layer is not read back by this
// kernel). Rows at or beyond n (the last group when n % 32 == 16) are neither stored nor
// their bytes used. Pure data movement: HBM-bound at 2 bytes per weight.
#include "ci8_device.h"
#include "launch.h"

namespace ci8 {
namespace {

// Output piece (16 bytes, k = 16t .. 16t + 15) of row q from the four chunk words of q.
__device__ __forceinline__ u32x4 restore_piece(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  constexpr uint32_t kDebias = 0x80808080u;
  return u32x4{((a & 0xFFFFu) | (b << 16)) ^ kDebias, ((c & 0xFFFFu) | (d << 16)) ^ kDebias,
               ((a >> 16) | (b & 0xFFFF0000u)) ^ kDebias,
               ((c >> 16) | (d & 0xFFFF0000u)) ^ kDebias};
}

// blockIdx.y = packed row p, lanes over tiles. kVec: packed is 16-byte aligned (else
// 4-byte words).
template <bool kVec>
__global__ void __launch_bounds__(256) unpack_allspark_kernel(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ packed_scales,
    int8_t* __restrict__ weight, uint16_t* __restrict__ scales, int n, int k) {
  const int tile = blockIdx.x * 256 + threadIdx.x;
  if (tile >= k / 16) return;
  const int p = blockIdx.y;
  const int first = (p / 8) * 32 + p % 8;  // output row of q = 0; rows first + 8q
  const uint8_t* src = packed + int64_t(p) * 4 * k + int64_t(tile) * 64;
  u32x4 chunk[4];
  if constexpr (kVec) {
    // Plain loads: the four chunks of neighbouring lanes share cache lines, which a
    // nontemporal hint would evict between the loads (40 us instead of 27 us at
    // [5120, 17408]).
#pragma unroll
    for (int j = 0; j < 4; ++j) chunk[j] = reinterpret_cast<const u32x4*>(src)[j];
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) chunk[j][q] = reinterpret_cast<const uint32_t*>(src)[4 * j + q];
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = first + 8 * q;
    if (row < n)
      __builtin_nontemporal_store(
          restore_piece(chunk[0][q], chunk[1][q], chunk[2][q], chunk[3][q]),
          reinterpret_cast<u32x4*>(weight + int64_t(row) * k + int64_t(tile) * 16));
  }
  if (tile == 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = first + 8 * q;
      if (row < n) scales[row] = packed_scales[(p / 8) * 32 + (p % 8) * 4 + q];
    }
  }
}

}  // namespace

hipError_t launch_unpack_allspark(const uint8_t* packed, const void* packed_scales,
                                  int8_t* weight, void* scales, int n, int k,
                                  hipStream_t stream) {
  const int packed_rows = (n + 31) / 32 * 8;
  const dim3 grid((k / 16 + 255) / 256, packed_rows);
  const auto* ps = static_cast<const uint16_t*>(packed_scales);
  auto* s = static_cast<uint16_t*>(scales);
  if (reinterpret_cast<uintptr_t>(packed) % 16 == 0)
    unpack_allspark_kernel<true><<<grid, 256, 0, stream>>>(packed, ps, weight, s, n, k);
  else
    unpack_allspark_kernel<false><<<grid, 256, 0, stream>>>(packed, ps, weight, s, n, k);
  return hipGetLastError();
}

}  // namespace ci8
