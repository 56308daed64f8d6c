// Large-M INT8 GEMM for gfx950 with two waves per SIMD in alternating roles.
//
//   out[m, n] = bf16_rn( fl( fl( float_rn(acc[m, n]) * sa[m] ) * float(sw[n]) ) )
//   acc[m, n] = sum_k a[m, k] * w[n, k]            (exact INT32)
//
// the arithmetic of csrc/fused_mm.cu:24-38 (and of gemm.hip, bit for bit). Biased UINT8
// weights (channel_mm, code + 128) are turned into the signed codes in registers, one XOR
// per four bytes after each W fragment read.
//
// Persistent: one workgroup of eight waves per CU walks the 256 (m) x 224 (n) output
// tiles b, b + grid, ... (grid = CU count). Where the 224-wide tiles would leave the last
// round partly empty and 160-wide tiles fill it, the columns are split between two
// launches (pp_plan below): whole rounds of 224-wide tiles, then 160-wide tiles over the
// rest (configs[3], M = 16384, N = 5120: 5 rounds over 4480 columns, then one round of
// 256 x 160 tiles over 640, in place of 5.75 rounds of 224-wide tiles). The 160-wide
// kernel is the same source with 5 n blocks per wave, 5 W copies per W wave and a copy
// after every second fragment read (gemm_pp_kernel.h); the numbers below are the 224-wide
// kernel's.
//
// The copy stream runs on across tiles: the K
// stages g = r * ns + t of the whole launch (tile r, stage t) use ring slots g % 2 (A)
// and g % 3 (W), and a tile's last stages copy the next tile's first stages just as they
// copy their own, so the tile switch issues no copies and the address unit is free for
// the epilogue's stores (measured on MI355X at configs[2]: 105 K against 108 K cycles
// per tile, 255.6-257.4 against 259.6-261.0 us, identical outputs). The epilogue runs
// through the A slot of the tile's last stage, which the next tile's first copies do not
// use. The tile's row and channel scales are copied into LDS at the tile start and read
// back by the epilogue, so they hold no registers through the K loop. With one K stage
// (K <= 128) the next tile's first copies go out at the tile switch instead.
//
// Within a tile, wave w owns rows 64 * (w % 4)
// and columns 112 * (w / 4) of the tile, as 4 x 7 blocks of v_mfma_i32_16x16x64_i8
// accumulators (112 registers). Waves w and w + 4 share SIMD w % 4. The waves of group
// g = w / 4 alternate between a memory phase (read the stage's 22 MFMA fragments from
// LDS and issue this wave's copies of a later stage) and a compute phase (56 MFMAs from
// registers), and the two groups are offset by one phase, so each SIMD always has one
// wave issuing MFMAs while the other waits on memory. Phases end at workgroup barriers:
//
//   phase:     0        1        2        3        4      ...
//   group 0:   M0       C0       M1       C1       M2
//   group 1:   -        M0       C0       M1       C1
//
// Measured on MI355X (per-wave clock stamps), one wave of each SIMD issuing 56 MFMAs
// while the other reads its fragments keeps the MFMA pipes about 96% busy when the
// operands are already in LDS; where a single wave per SIMD does both, the lock-step
// barriers of its K loop idle the pipes about a quarter of the time.
//
// Operands go through LDS rings of 128-byte K stages filled by buffer_load ... lds
// (8 rows x 128 bytes per copy; rows past M or N and bytes past K come back as zeros
// from the buffer range check). Copies are issued between the fragment reads of the
// memory phases: the vector-memory unit takes about 16 cycles per 1 KiB copy per CU and
// a wave stalls when it issues into a full queue, which in a compute phase would stall
// the MFMAs (measured: about 40 cycles per copy there). Group 0 copies A, group 1 W:
//   A: two 32 KB slots. A(t + 1) is copied in phase 2t into the slot of A(t - 1), which
//      both groups read in phases 2t - 2 and 2t - 1; group 0 waits for it at the end of
//      phase 2t + 1.
//   W: three 28 KB slots. W(t + 2) is copied in phase 2t + 1 into the slot of W(t - 1),
//      read in phases 2t - 2 and 2t - 1; group 1 waits for W(t + 1) at the end of phase
//      2t + 1.
// In a tile's last stage group 0 copies the next tile's A(0), and in its last two group
// 1 copies the next tile's W(0) and W(1); those are waited for at the tile switch.
// Stage t of a tile is K stage (t + t0) % ns with a per-tile start t0, so the tiles of an
// XCD that share a panel do not fetch its K slices all at once (gemm_pp_kernel.h).
// A W wave has 7 copies per stage against an A wave's 8; its eighth reads nothing into a
// junk KiB, which keeps the copy sequence identical and branch-free.
//
// MFMA lane layouts: the MFMA computes D[n][m] = W . A^T; within a 128-byte stage, lane
// group g (lane / 16) reads logical chunk 4h + g in K-step h (A and W alike, so the
// exact INT32 sums are those of any other K order), and LDS rows hold their 16-byte
// chunks XOR-swizzled by row % 8. With this order the 16 lanes of a group read one
// chunk column of 16 rows and a fragment read has no bank conflicts (measured on
// MI355X: the order 2g + h, where the four groups read every other chunk, stalls each
// 1 KiB read about 4 cycles on bank conflicts, a quarter of the kernel's LDS time).
#include "gemm_pp_kernel.h"

namespace ci8 {

// The host plan (tile_plan.h) prices these tiles.
static_assert(PPConfig::BM == kPlanBM && PPConfig::BN == kPlanBN &&
                  PPConfigNarrow::BM == kPlanBM && PPConfigNarrow::BN == kPlanNarrowBN,
              "tile_plan.h prices the kernel's tiles");

// Requires a and w 16-byte aligned, sw 8-byte aligned and n % 4 == 0 (the fused op's
// contract); out needs 2-byte alignment (16-byte aligned rows take 16-byte stores).
hipError_t launch_pp_gemm(const int8_t* a, const void* w, WeightCode code, const float* sa,
                          const void* sw, void* out, int m, int n, int k, hipStream_t stream) {
  const int cus = device_cu_count();
  const bool out16 = (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  const bool exact = k % PPConfig::BK == 0;
  // Columns [c0, c0 + nc) of the output with tiles of width kBN.
  auto launch = [&](auto width, int c0, int nc) {
    constexpr int kBN = decltype(width)::value;
    using C = PPConfigT<kBN>;
    const int tiles = ((nc + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
    const int grid = cus > 0 && cus < tiles ? cus : tiles;  // one workgroup per CU
    const int8_t* wc = static_cast<const int8_t*>(w) + int64_t(c0) * k;
    const uint16_t* swc = static_cast<const uint16_t*>(sw) + c0;
    uint16_t* outc = static_cast<uint16_t*>(out) + c0;
    auto go = [&](auto kernel_constant) {
      constexpr auto kernel = decltype(kernel_constant)::value;
      if (const hipError_t e = prepare_lds<kernel>(C::kLdsBytes); e != hipSuccess) return e;
      kernel<<<grid, C::kThreads, C::kLdsBytes, stream>>>(a, wc, sa, swc, outc, m, nc, k, n,
                                                           out16, nullptr);
      return hipGetLastError();
    };
    constexpr auto kS = WeightCode::kSigned, kU = WeightCode::kBiasedU8;
    if (code == kS)
      return exact ? go(kernel_constant<pp_gemm_kernel<true, kS, 0, kBN>>{})
                   : go(kernel_constant<pp_gemm_kernel<false, kS, 0, kBN>>{});
    return exact ? go(kernel_constant<pp_gemm_kernel<true, kU, 0, kBN>>{})
                 : go(kernel_constant<pp_gemm_kernel<false, kU, 0, kBN>>{});
  };
  const PPPlan plan = pp_plan(m, n, cus);
  if (plan.n_head == 0) return launch(std::integral_constant<int, PPConfig::BN>{}, 0, n);
  if (const hipError_t e = launch(std::integral_constant<int, PPConfig::BN>{}, 0, plan.n_head);
      e != hipSuccess)
    return e;
  return launch(std::integral_constant<int, PPConfigNarrow::BN>{}, plan.n_head, n - plan.n_head);
}

}  // namespace ci8
