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

// Tile shapes of the small-M kernel (gemm_small.hip), as (BM, BN). A launch runs its tiles
// in rounds of one per CU, and a round lasts about as long as one tile takes to stream its
// (BM + BN) x K operand bytes, so the cost of a shape is rounds x (BM + BN); ties go to the
// larger tile (the earlier entry).
struct SmallShape {
  int bm, bn;
};
constexpr SmallShape kSmallShapes[] = {{64, 32}, {32, 64}, {16, 64}, {32, 32},
                                       {32, 16}, {16, 32}, {16, 16}};

inline int64_t small_shape_cost(SmallShape s, int m, int n, int cus) {
  const int64_t tiles = int64_t((m + s.bm - 1) / s.bm) * ((n + s.bn - 1) / s.bn);
  return (tiles + cus - 1) / cus * (s.bm + s.bn);
}

inline SmallShape small_best_shape(int m, int n, int cus) {
  SmallShape best = kSmallShapes[0];
  for (const SmallShape s : kSmallShapes)
    if (small_shape_cost(s, m, n, cus) < small_shape_cost(best, m, n, cus)) best = s;
  return best;
}

// Largest M the small-M kernel takes under schedule 0, and the M above which it competes
// with the 128 x 128 and 256 x 224 kernels (mid_m_schedule).
constexpr int kSmallMaxM = 256, kSmallOnlyMaxM = 128;

// Schedule 0 for kSmallOnlyMaxM < M <= kSmallMaxM: 0 (the small-M kernel), 1 (128 x 128
// tiles) or 4 (256 x 224 tiles), whichever a time model of the three finishes first. The
// model's figures are per-launch times measured on MI355X at K = 5120 (each kernel's time
// is proportional to K, so the comparison holds at any K), conditioned graph replays,
// identical outputs:
//   small-M:  (its shape cost) / 13.3 us (M = 256, 64 x 32 tiles: 4 / 8 / 17 rounds took
//             29.7 / 57.3 / 119.2 us at N = 8192 / 16384 / 34816);
//   128x128:  35.5 us while its tiles fit one round (34.6-36.4 us from 80 to 256 tiles);
//             past that, whole rounds plus the rest's share of a round but at least 0.37
//             of one, as two workgroups fit a CU (M = 256: 272 / 384 / 544 tiles took
//             48.5 / 53.2 / 86.8 us);
//   256x224:  60 us a round (57.1-61.0 us from 23 to 156 tiles).
// At M = 256 this takes N = 11264-24576 from 43.4-85.0 us to 34.9-53.2 us and N = 34816
// from 119.2 to 60.3 us, and keeps the small-M kernel up to N = 8192, where it is fastest
// (160 <= M <= 256, N from 5120 to 34816, K = 2048-17408). M <= kSmallOnlyMaxM keeps the
// small-M kernel: its rows fill every tile of the other two, and streaming the weights
// bounds all three alike.
inline int mid_m_schedule(int m, int n, int cus) {
  if (cus <= 0 || m <= kSmallOnlyMaxM || m > kSmallMaxM) return 0;
  const double small = double(small_shape_cost(small_best_shape(m, n, cus), m, n, cus)) / 13.3;
  const int64_t tiles128 = int64_t((m + 127) / 128) * ((n + 127) / 128);
  double rounds128 = 1.0;
  if (tiles128 > cus) {
    const int64_t rest = tiles128 % cus;
    rounds128 = double(tiles128 / cus);
    if (rest > 0) rounds128 += rest * 100 > cus * 37 ? double(rest) / cus : 0.37;
  }
  const double medium = 35.5 * rounds128;
  const int64_t tiles224 = int64_t((m + kPlanBM - 1) / kPlanBM) * ((n + kPlanBN - 1) / kPlanBN);
  const double wide = 60.0 * double((tiles224 + cus - 1) / cus);
  if (small <= medium && small <= wide) return 0;
  return medium <= wide ? 1 : 4;
}

// Whether 128 x 128 tiles beat the persistent kernel at M >= 1024: when its 256 x 224 tiles
// would keep under half the CUs busy and 128 x 128 tiles fit in one round (measured on
// MI355X, conditioned graph replays, identical outputs: M = 1024, N = 2560 / 3072 / 2048,
// K = 10240 / 5120 / 8192: 63.5 / 35.0 / 51.6 against 76.7 / 43.8 / 62.0 us; with more than
// one round of 128 x 128 tiles it is not faster: M = 1024, N = 5120, K = 10240: 81.0
// against 77.3 us, M = 2048, N = 2560: 44.4 against 44.7 us).
inline bool medium_tiles_pay(int m, int n, int cus) {
  if (cus <= 0 || m < 1024) return false;
  const int64_t tiles224 = int64_t((m + kPlanBM - 1) / kPlanBM) * ((n + kPlanBN - 1) / kPlanBN);
  const int64_t tiles128 = int64_t((m + 127) / 128) * ((n + 127) / 128);
  return 2 * tiles224 < cus && tiles128 <= cus;
}

}  // namespace ci8
