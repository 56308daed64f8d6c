// Host-side tile plans of the large-M GEMMs: how many rounds of one tile per CU a launch
// takes, and the column split of the persistent kernel. Plain C++ (no HIP), so a CPU test
// compiles it with g++ and checks the plans the dispatcher picks.
#pragma once
#include <stdint.h>

namespace ci8 {

// Tile sizes these rules price (the persistent kernel's 256 x 224 and 256 x 160 tiles,
// gemm_pp_kernel.h, and the one-wave-per-SIMD kernel's 256 x 256 tiles, gemm.hip).
constexpr int kPlanBM = 256, kPlanBN = 224, kPlanNarrowBN = 160, kPlanWideBN = 256;

// Time of a round of 160-wide tiles, in units where a round of 224-wide tiles takes 224
// (measured on MI355X at configs[3], M = 16384, K = 17408: 5 rounds of 224-wide tiles
// over N = 4480 took 966-978 us, and the split launch over N = 5120 1114-1129 us, so the
// 160-wide round and the second launch took ~0.8 of a 224-wide round).
//
// The split gains less than its rounds suggest: the chip runs at its power limit, so a
// partly filled last round runs faster per tile than a full one. At configs[3] the single
// launch's sixth round (192 of 256 CUs busy, 672 columns for 640) took ~161 us against
// ~195 us for a full round, and the split launch measured 1114-1129 against 1131-1145 us
// (same process, alternating, identical outputs; at K = 5120, 326.5-327.7 against
// 328.4-329.8 us): about 1%, mostly the 32 padded columns that the 160-wide tiles do not
// compute.
constexpr int64_t kNarrowRoundCost = 180;

// Column plan of the two-waves-per-SIMD GEMM (gemm_pp.hip) at m x n on `cus` CUs: 224-wide
// tiles over the first n_head columns and 160-wide tiles over the rest (n_head = 0: one
// launch of 224-wide tiles over all n). `cost` is the planned rounds' time in units where a
// round of 224-wide tiles takes 224.
struct PPPlan {
  int n_head;
  int64_t cost;
};

inline PPPlan pp_plan(int m, int n, int cus) {
  const int64_t tiles_m = (m + kPlanBM - 1) / kPlanBM;
  const int64_t tiles = tiles_m * ((n + kPlanBN - 1) / kPlanBN);
  PPPlan plan{0, 0};
  if (cus <= 0) return plan;
  plan.cost = (tiles + cus - 1) / cus * kPlanBN;
  // A last round that keeps under half the CUs busy runs faster per tile than the split's
  // round of 160-wide tiles (same process, identical outputs: M = 2048, N = 17408, whose
  // third round holds 112 tiles, 155.4-155.7 us in one launch against 156.7-157.4 us
  // split; M = 1100, N = 15516, 94 tiles, 106.4-106.9 us either way).
  const int64_t last = tiles % cus;
  if (last == 0 || 2 * last < cus) return plan;
  // Split: 224-wide tiles over the columns that the launch's whole rounds cover, then
  // 160-wide tiles over the rest.
  const int64_t head_tiles_n = tiles / cus * cus / tiles_m;
  const int64_t n_head = head_tiles_n * kPlanBN;
  if (head_tiles_n == 0 || n_head >= n) return plan;
  const int64_t head_rounds = (head_tiles_n * tiles_m + cus - 1) / cus;
  const int64_t tail_tiles = tiles_m * ((n - n_head + kPlanNarrowBN - 1) / kPlanNarrowBN);
  const int64_t cost = head_rounds * kPlanBN + (tail_tiles + cus - 1) / cus * kNarrowRoundCost;
  if (cost < plan.cost) plan = PPPlan{int(n_head), cost};
  return plan;
}

// Whether 256-wide large tiles finish an m x n GEMM sooner than 224-wide ones. A launch
// runs its tiles in rounds of one per CU, and a round takes time in proportion to the
// tile width, so the cost of a width is rounds x width. 224 suits N = 17408 at M = 4096
// (1,248 tiles, 4.9 rounds on 256 CUs, where 256-wide tiles need 4.25 rounds, i.e. 5);
// 256 suits N = 5120 at M = 16384 (5 full rounds against 5.75).
inline bool wide_tiles_pay(int m, int n, int cus) {
  if (cus <= 0) return false;
  const int64_t tiles_m = (m + kPlanBM - 1) / kPlanBM;
  const int64_t rounds224 = (tiles_m * ((n + kPlanBN - 1) / kPlanBN) + cus - 1) / cus;
  const int64_t rounds256 = (tiles_m * ((n + kPlanWideBN - 1) / kPlanWideBN) + cus - 1) / cus;
  return rounds256 * kPlanWideBN < rounds224 * kPlanBN;
}

// Whether the persistent kernel (one tile per CU per round, about 1.2x the MFMA rate of
// the 256-wide kernel) finishes sooner than 256-wide tiles: the cost of its column plan
// (rounds x width) against rounds x 256, weighted by that rate.
inline bool pp_beats_wide_tiles(int m, int n, int cus) {
  if (cus <= 0) return false;
  const int64_t tiles_m = (m + kPlanBM - 1) / kPlanBM;
  const int64_t rounds256 = (tiles_m * ((n + kPlanWideBN - 1) / kPlanWideBN) + cus - 1) / cus;
  return pp_plan(m, n, cus).cost * 6 <= rounds256 * kPlanWideBN * 7;
}

}  // namespace ci8
