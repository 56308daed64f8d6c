"""The large-M GEMM tile plans (csrc/tile_plan.h), compiled on the CPU with g++.

The dispatcher runs the persistent 256 x 224 kernel, split into whole rounds of 224-wide
tiles plus a round of 160-wide tiles where that costs less, or the 256-wide kernel where
its rounds are fewer. The expected plans below are worked out by hand from the tile
counts on 256 CUs (an MI355X), not from the header's formulas.
"""

import shutil
import subprocess

import pytest

from tests.conftest import PKG

PROGRAM = r"""
#include <cstdio>
#include "tile_plan.h"
using namespace ci8;
int main() {
  const int cases[][3] = {{4096, 17408, 256}, {16384, 5120, 256}, {4096, 4096, 256},
                          {1024, 15520, 256}, {1100, 15516, 256}, {2048, 17408, 256},
                          {16384, 5120, 0}, {1024, 128, 256}, {1024, 23040, 256},
                          {1100, 18500, 256}, {8192, 17408, 256}};
  for (const auto& c : cases) {
    const PPPlan p = pp_plan(c[0], c[1], c[2]);
    std::printf("%d %d %d %d %lld %d %d\n", c[0], c[1], c[2], p.n_head, (long long)p.cost,
                int(wide_tiles_pay(c[0], c[1], c[2])), int(pp_beats_wide_tiles(c[0], c[1], c[2])));
  }
  return 0;
}
"""


def test_tile_plans(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src = tmp_path / "tile_plan_check.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "tile_plan_check"
    subprocess.run([gxx, "-std=c++17", "-O1", f"-I{PKG / 'csrc'}", str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.split("\n"):
        if line:
            m, n, cus, n_head, cost, wide, pp = map(int, line.split())
            got[(m, n, cus)] = (n_head, cost, wide, pp)
    # 16 x 78 = 1,248 tiles, 4.875 rounds -> 5 x 224; the last round holds 224
    # tiles, but whole rounds would cover 64 column tiles (14,336 columns) and leave 3,072
    # for 20 x 16 = 320 narrow tiles, two rounds: 4 x 224 + 2 x 180 = 1,256 > 1,120, so
    # one launch. 256-wide: 16 x 68 = 1,088 tiles, 5 rounds (1,280): the persistent kernel
    # wins (1,120 x 6 <= 1,280 x 7).
    assert got[(4096, 17408, 256)] == (0, 1120, 0, 1)
    # 64 x 23 = 1,472 tiles, 5.75 rounds -> 6 x 224 = 1,344, last round 192
    # tiles; split after 5 rounds = 1,280 tiles = 20 column tiles (4,480 columns), tail 640
    # = 4 x 160, 256 tiles, one round: 5 x 224 + 180 = 1,300.
    assert got[(16384, 5120, 256)] == (4480, 1300, 1, 1)
    # M = N = 4096: 304 tiles, 2 rounds (448), the second 48 tiles: no split; one round of
    # 256-wide tiles (16 x 16) wins (448 x 6 > 256 x 7).
    assert got[(4096, 4096, 256)] == (0, 448, 1, 0)
    # 4 x 70 = 280 tiles, the second round 24: no split; 4 x 61 = 244 tiles of 256-wide
    # fill one round, so the 256-wide kernel takes it.
    assert got[(1024, 15520, 256)] == (0, 448, 1, 0)
    # 5 x 70 = 350 tiles, the second round 94 (under half): one launch of 224-wide tiles
    # (256-wide: 5 x 61 = 305 tiles, also 2 rounds, 512).
    assert got[(1100, 15516, 256)] == (0, 448, 0, 1)
    # 8 x 78 = 624 tiles, the third round 112 tiles (under half): one launch, 3 x 224.
    assert got[(2048, 17408, 256)] == (0, 672, 0, 1)
    # No CU count: no plan, no preference.
    assert got[(16384, 5120, 0)] == (0, 0, 0, 0)
    # Fewer tiles than CUs: one round, nothing to split.
    assert got[(1024, 128, 256)] == (0, 224, 0, 1)
    # The GPU tests' split shapes. 4 x 103 = 412 tiles, the second round 156: one round of
    # 224-wide tiles over 64 column tiles (14,336 columns), then 8,704 columns as 55 x 4 =
    # 220 narrow tiles: 224 + 180 = 404 < 448 (256-wide: 4 x 90 = 360 tiles, 2 rounds).
    assert got[(1024, 23040, 256)] == (14336, 404, 0, 1)
    # 5 x 83 = 415 tiles, the second round 159; 256 // 5 = 51 column tiles (11,424
    # columns), then 7,076 columns as 45 x 5 = 225 narrow tiles.
    assert got[(1100, 18500, 256)] == (11424, 404, 0, 1)
    # 32 x 78 = 2,496 tiles, 9.75 rounds (2,240), last round 192: 9 rounds = 2,304 tiles =
    # 72 column tiles (16,128 columns), 1,280 columns = 8 x 32 = 256 narrow tiles:
    # 9 x 224 + 180 = 2,196.
    assert got[(8192, 17408, 256)] == (16128, 2196, 0, 1)


MID_PROGRAM = r"""
#include <cstdio>
#include "tile_plan.h"
using namespace ci8;
int main() {
  const int cases[][3] = {{256, 8192, 256}, {256, 11264, 256}, {256, 16384, 256},
                          {256, 17408, 256}, {256, 24576, 256}, {256, 34816, 256},
                          {160, 11264, 256}, {160, 16384, 256}, {256, 5120, 256},
                          {128, 34816, 256}, {257, 34816, 256}, {256, 34816, 0},
                          {1024, 2560, 256}, {1024, 2048, 256}, {1024, 5120, 256},
                          {2048, 2560, 256}, {1024, 7168, 256}, {1024, 2560, 0}};
  for (const auto& c : cases)
    std::printf("%d %d %d %d %d\n", c[0], c[1], c[2], mid_m_schedule(c[0], c[1], c[2]),
                int(medium_tiles_pay(c[0], c[1], c[2])));
  return 0;
}
"""


def test_mid_m_schedule_choices(tmp_path):
    """Schedule 0's kernel for 128 < M <= 256 and the 128 x 128 tiles at M >= 1024, worked
    out by hand from the tile counts on 256 CUs and the per-kernel times the header states
    (small-M: shape cost / 13.3 us; 128 x 128: 35.5 us a round; 256 x 224: 60 us a round)."""
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src = tmp_path / "mid_m_check.cpp"
    src.write_text(MID_PROGRAM)
    exe = tmp_path / "mid_m_check"
    subprocess.run([gxx, "-std=c++17", "-O1", f"-I{PKG / 'csrc'}", str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.split("\n"):
        if line:
            m, n, cus, mid, medium = map(int, line.split())
            got[(m, n, cus)] = (mid, medium)
    # M = 256, N = 8192: 64 x 32 tiles 4 x 256 = 1,024, 4 rounds x 96 = 384 -> 28.9 us;
    # 128 x 128: 2 x 64 = 128 tiles, one round, 35.5 us: the small-M kernel.
    assert got[(256, 8192, 256)] == (0, 0)
    # N = 11264: 4 x 352 = 1,408 tiles, 6 rounds x 96 = 576 -> 43.3 us against 176 tiles of
    # 128 x 128 (35.5 us).
    assert got[(256, 11264, 256)] == (1, 0)
    # N = 16384: 8 rounds, 57.7 us against 256 tiles of 128 x 128, one round.
    assert got[(256, 16384, 256)] == (1, 0)
    # N = 17408: 9 rounds, 65.0 us; 272 tiles of 128 x 128 = 1 round + 16 tiles (0.37 of a
    # round) = 48.6 us; 78 tiles of 256 x 224, 60 us.
    assert got[(256, 17408, 256)] == (1, 0)
    # N = 24576: 384 tiles of 128 x 128 = 1.5 rounds = 53.3 us against 110 of 256 x 224.
    assert got[(256, 24576, 256)] == (1, 0)
    # N = 34816: 544 tiles of 128 x 128 = 2 rounds + 32 tiles = 2.37 x 35.5 = 84.1 us;
    # 156 tiles of 256 x 224, one round, 60 us; small-M 17 rounds, 122.7 us.
    assert got[(256, 34816, 256)] == (4, 0)
    # M = 160, N = 11264: 32 x 64 tiles 5 x 176 = 880, 4 rounds x 96 = 384 -> 28.9 us.
    assert got[(160, 11264, 256)] == (0, 0)
    # M = 160, N = 16384: 32 x 64 tiles 5 x 256 = 1,280, 5 rounds x 96 = 480 -> 36.1 us
    # against 256 tiles of 128 x 128 (35.5 us).
    assert got[(160, 16384, 256)] == (1, 0)
    # N = 5120: 640 tiles of 64 x 32, 3 rounds, 21.7 us.
    assert got[(256, 5120, 256)] == (0, 0)
    # M <= 128 and M > 256 are outside the rule; no CU count, no rule.
    assert got[(128, 34816, 256)] == (0, 0)
    assert got[(257, 34816, 256)] == (0, 0)
    assert got[(256, 34816, 0)] == (0, 0)
    # M = 1024: N = 2560 has 4 x 12 = 48 persistent tiles (under half of 256) and 8 x 20 =
    # 160 tiles of 128 x 128; N = 2048 40 and 128.
    assert got[(1024, 2560, 256)] == (0, 1)
    assert got[(1024, 2048, 256)] == (0, 1)
    # N = 5120: 92 persistent tiles but 320 of 128 x 128 (two rounds); M = 2048, N = 2560:
    # 96 and 320; N = 7168: 128 persistent tiles, half the CUs.
    assert got[(1024, 5120, 256)] == (0, 0)
    assert got[(2048, 2560, 256)] == (0, 0)
    assert got[(1024, 7168, 256)] == (0, 0)
    assert got[(1024, 2560, 0)] == (0, 0)
