"""Grid-tail split planner (CPU).

Compiles a host-only program against the kernels' own header
(``avgen_amd/csrc/avattn_kernels.h``) and checks ``plan_tail_split``, which
decides how the dK/dV kernel's partial last round is shared out:

* no split when the grid fits one round, fills its last round exactly, or no
  part count shortens the last round;
* otherwise ``nsplit`` is the last round's block count (``total % cus``),
  ``nparts`` lies in 2..8, ``nsplit * nparts`` fits the partial-sum slots, and
  the last round it leaves (``ceil(nsplit * nparts / cus) / nparts`` of a full
  round) is shorter than one round and no longer than with any other
  admissible part count (the smaller count on ties);
* the configurations the benchmarks run: c3 (5,920 blocks) -> 32 x 8, a c4
  pass (4,760) -> 152 x 3, a window / varlen pass (4,728) -> 120 x 2, c2
  (5,120, whole rounds) -> none.
"""

import shutil
import subprocess
from fractions import Fraction
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "avgen_amd" / "csrc"

PROGRAM = r"""
#include "avattn_kernels.h"
#include <cstdio>
using namespace avattn;
int main() {
  const int cus_list[] = {32, 80, 256, 304};
  const int slots_list[] = {64, 256, 512};
  for (int cus : cus_list)
    for (int slots : slots_list)
      for (long total = 1; total <= 4 * cus + 7; ++total) {
        const TailSplit t = plan_tail_split(total, cus, slots);
        std::printf("%ld %d %d %d %d\n", total, cus, slots, t.nsplit, t.nparts);
      }
  const long extra[][2] = {{5920, 256}, {4760, 256}, {4728, 256}, {5120, 256}};
  for (const auto& e : extra) {
    const TailSplit t = plan_tail_split(e[0], (int)e[1], kSplitSlots);
    std::printf("%ld %ld %d %d %d\n", e[0], e[1], kSplitSlots, t.nsplit, t.nparts);
  }
  return 0;
}
"""


@pytest.fixture(scope="module")
def plans(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("tail_split")
    src, exe = d / "plan.cpp", d / "plan"
    src.write_text(PROGRAM)
    cmd = [hipcc, "-x", "hip", "--offload-host-only", "-std=c++17", "-O1", f"-I{CSRC}",
           f"-I{ROOT / 'include'}", str(src), "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    rows = {}
    for line in out.stdout.split("\n"):
        if line.strip():
            total, cus, slots, ns, np_ = map(int, line.split())
            rows[(total, cus, slots)] = (ns, np_)
    return rows


def _last_round(r, p, cus):
    return Fraction(-(-r * p // cus), p)


def test_planner_properties(plans):
    for (total, cus, slots), (ns, np_) in plans.items():
        r = total % cus
        options = [p for p in range(2, 9) if r * p <= slots and _last_round(r, p, cus) < 1]
        if total <= cus or r == 0 or not options:
            assert (ns, np_) == (0, 0), (total, cus, slots, ns, np_)
            continue
        assert ns == r and 2 <= np_ <= 8 and ns * np_ <= slots, (total, cus, slots, ns, np_)
        mine = _last_round(r, np_, cus)
        assert mine < 1
        for p in options:
            assert mine <= _last_round(r, p, cus), (total, cus, slots, np_, p)
            if _last_round(r, p, cus) == mine:
                assert np_ <= p  # ties go to the smaller part count


def test_planner_on_benchmark_grids(plans):
    assert plans[(5920, 256, 512)] == (32, 8)   # c3 chunk: 1 x 40 x 148 key blocks
    assert plans[(4760, 256, 512)] == (152, 3)  # c4 pass: 8 pairs x 595 blocks
    assert plans[(4728, 256, 512)] == (120, 2)  # window / varlen pass: 8 pairs x 591 blocks
    assert plans[(5120, 256, 512)] == (0, 0)    # c2: 2 x 20 x 128 blocks, 20 whole rounds
