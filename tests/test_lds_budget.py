"""The LDS budget every dynamic-LDS launcher checks before launching (csrc/lds_budget.h).

A gfx950 workgroup holds at most 160 KiB (163,840 bytes) of LDS, static plus dynamic. A
launch asking for more is accepted by the launch call and then aborts the device queue
(HSA_STATUS_ERROR_INVALID_ALLOCATION); such a launch of 163,840 bytes of dynamic LDS in a
kernel with 1 KiB of static LDS did abort on an MI355X during development. The launchers
call prepare_lds<kernel>(bytes), which applies lds_fits() to the kernel's static LDS and
the request and returns an error instead. This CPU test compiles the header on its own
with g++ and checks the rule at and around the limit, including that failing case.
"""

import shutil
import subprocess

import pytest

from tests.conftest import PKG

PROGRAM = r"""
#include <cstdio>
#include "lds_budget.h"
using namespace ci8;
static_assert(kLdsPerWorkgroup == 163840, "160 KiB");
int main() {
  const long long cases[][2] = {
      {0, 163840}, {1024, 163840}, {1024, 162816}, {0, 163841}, {163840, 0},
      {163840, 1}, {0, 0}, {-1, 0}, {0, -1}, {64 * 1024, 96 * 1024}, {32768, 131073}};
  for (const auto& c : cases)
    std::printf("%lld %lld %d %lld\n", c[0], c[1], int(lds_fits(c[0], c[1])),
                dynamic_lds_limit(c[0] < 0 ? 0 : c[0]));
  return 0;
}
"""


def test_lds_budget_rule(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src = tmp_path / "lds_budget_check.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "lds_budget_check"
    subprocess.run([gxx, "-std=c++17", "-O1", f"-I{PKG / 'csrc'}", str(src), "-o", str(exe)],
                   check=True)
    lines = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {(int(a), int(b)): (int(ok), int(limit))
           for a, b, ok, limit in (line.split() for line in lines if line)}
    assert got[(0, 163840)] == (1, 163840)        # the whole budget, no static LDS
    assert got[(1024, 163840)][0] == 0            # the launch that aborted on the device
    assert got[(1024, 162816)] == (1, 162816)     # the same kernel at its true limit
    assert got[(0, 163841)][0] == 0
    assert got[(163840, 0)][0] == 1 and got[(163840, 1)][0] == 0
    assert got[(0, 0)][0] == 1
    assert got[(-1, 0)][0] == 0 and got[(0, -1)][0] == 0
    assert got[(64 * 1024, 96 * 1024)][0] == 1
    assert got[(32768, 131073)][0] == 0


def launch_configs(text):
    """(offset, [grid, block, lds, stream]) of every kernel launch in `text`, split on the
    top-level commas of its <<<...>>> (grid expressions may hold commas)."""
    pos = 0
    while (start := text.find("<<<", pos)) >= 0:
        end = text.index(">>>", start)
        args, depth, cur = [], 0, ""
        for ch in text[start + 3:end]:
            if ch == "," and depth == 0:
                args.append(cur.strip())
                cur = ""
                continue
            depth += ch in "([{"
            depth -= ch in ")]}"
            cur += ch
        args.append(cur.strip())
        yield start, args
        pos = end + 3


def test_every_dynamic_lds_launch_is_checked():
    """Every launch that passes a nonzero dynamic LDS size is preceded, in the same
    launcher, by prepare_lds (and no launcher still raises the attribute by itself)."""
    csrc = PKG / "csrc"
    launches = 0
    for path in sorted(csrc.glob("*.hip")):
        text = path.read_text()
        assert "raise_lds_limit_once" not in text, path.name
        for start, args in launch_configs(text):
            assert len(args) == 4, (path.name, args)
            launches += 1
            if args[2] == "0":
                continue
            before = text[max(0, start - 1500):start]
            assert "prepare_lds<" in before, f"{path.name}: launch with {args[2]} bytes of LDS"
    assert launches >= 30
