"""LDS tile layout and direct-staging address maps (CPU).

Compiles a host-only program against the kernels' own header
(``avgen_amd/csrc/avattn_device.h``) and checks, for every tile shape the
kernels stage (K/Q/dO row tiles of head_dim channels, V^T/Q^T/dO^T/K^T tiles
of 32 or 64 sequence positions, head_dim 64 and 128, 8 waves):

* ``TileLayout<RL>::off`` is a bijection of the tile's 16-byte chunks;
* ``TileStager``: the chunk lane j loads in wave instruction i is the
  logical chunk that ``TileLayout`` places at the LDS slot the hardware
  writes (block base + 16*j), and the waves' instructions cover every block
  of the tile (repeats only where waves outnumber instructions);
* every 16-byte operand read pattern of the kernels (16 lanes reading the
  same logical chunk of 16 rows of an aligned group, rows in identity or
  perm23 order) touches 16 distinct 16-byte bank groups of a 64-bank x
  4-byte LDS, i.e. is bank-conflict free;
* perm23 is an involution that maps 8 consecutive C-layout rows of each
  16-row k-step to one aligned 8-row chunk;
* staged dS (``DsUnit``): the dK/dV kernel's stores cover every element of
  a unit once and stay in it, and the dQ kernel's stage loads plus
  transposed reads hand every lane the (row, key) pairs of its B operand,
  for 64- and 32-key stages;
* ``tr_read_off``: the dK/dV kernel's transposed reads of the row-major Q
  and dO tiles hand every lane channel ``32*dt + lane%32`` of the eight
  consecutive rows of its A operand, for head_dim 128 and 64.
"""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "avgen_amd" / "csrc"

PROGRAM = r"""
#include "avattn_device.h"
#include <cstdio>
#include <vector>
using namespace avattn;

static int failures = 0;
#define CHECK(c, ...) do { if (!(c)) { if (failures++ < 20) std::printf(__VA_ARGS__); } } while (0)

template <int ROWS, int RL, int NW>
void check_tile() {
  using L = TileLayout<RL>;
  using S = TileStager<ROWS, RL, NW>;
  constexpr int cpr = RL / 8, chunks = ROWS * cpr;
  // 1. layout bijection (element offsets of chunk starts).
  std::vector<int> seen(chunks, 0);
  for (int r = 0; r < ROWS; ++r)
    for (int c = 0; c < cpr; ++c) {
      const int o = L::off(r, 8 * c);
      CHECK(o % 8 == 0 && o / 8 >= 0 && o / 8 < chunks, "off out of range %d %d %d\n", RL, r, c);
      CHECK(o / RL == r, "off leaves row %d (RL %d)\n", r, RL);
      if (o % 8 == 0 && o / 8 >= 0 && o / 8 < chunks) seen[o / 8]++;
      for (int e = 0; e < 8; e += 4) CHECK(L::off(r, 8 * c + e) == o + e, "chunk not contiguous\n");
    }
  for (int i = 0; i < chunks; ++i) CHECK(seen[i] == 1, "slot %d hit %d times (RL %d)\n", i, seen[i], RL);
  // 2. stager: lane j of instruction i writes LDS bytes i*kRpi*RL*2 + 16*j.
  const long stride = RL + 24;  // any source row stride (elements)
  std::vector<int> block(S::kNi, 0);
  for (int w = 0; w < NW; ++w)
    for (int k = 0; k < S::kPer; ++k) {
      const int instr = S::first_instr(w) + k;
      CHECK(instr < S::kNi, "instruction %d out of tile\n", instr);
      block[instr]++;
      for (int j = 0; j < 64; ++j) {
        const int lds_elem = instr * S::kRpi * RL + 8 * j;  // physical element offset
        const int row = S::row_of(instr, j);
        const uint32_t src = S::src_offset(instr, j, stride);
        const long src_elem = src / 2;
        CHECK(src % 16 == 0, "source not 16-byte aligned\n");
        CHECK(src_elem / stride == row, "source row %ld != %d\n", src_elem / stride, row);
        const int col = (int)(src_elem % stride);
        CHECK(col % 8 == 0 && col < RL, "source column %d\n", col);
        CHECK(L::off(row, col) == lds_elem, "stager/layout mismatch RL %d row %d col %d: %d vs %d\n", RL, row,
              col, L::off(row, col), lds_elem);
      }
    }
  for (int i = 0; i < S::kNi; ++i)
    CHECK(block[i] == (S::kNi >= NW ? 1 : NW / S::kNi), "block %d staged %d times\n", i, block[i]);
  // 3. operand reads: 16 lanes, same logical chunk, 16 rows of an aligned group.
  for (int g = 0; g < ROWS; g += 16)
    for (int c = 0; c < cpr; ++c)
      for (int perm = 0; perm < 2; ++perm) {
        int hit[16] = {0};
        for (int l = 0; l < 16; ++l) {
          const int r = g + (perm ? perm23(l) : l);
          const int byte = 2 * L::off(r, 8 * c);
          hit[(byte / 16) % 16]++;
        }
        for (int b = 0; b < 16; ++b) CHECK(hit[b] == 1, "bank group %d hit %d (RL %d rows %d chunk %d)\n", b, hit[b], RL, g, c);
      }
}

// Staged dS: the dK/dV kernel's 16-byte stores and the dQ kernel's 1 KB
// stage loads plus transposed reads (ds_read_b64_tr_b16: in each 16-lane
// group, lane j receives element j % 4 of the 4 elements lane 4*r + j/4
// points at, r = 0..3, as checked on the GPU) deliver every lane the
// (row, key) pairs of its MFMA B operand.
template <int BK>
void check_ds(int nkt) {
  // One query group's units for nkt key blocks, written as the dK/dV waves
  // of sub 0 write them (the sub-1 half goes to the next group's units).
  const int unit_elems = 4096;
  std::vector<int> row_of(nkt * unit_elems, -1), key_of(nkt * unit_elems, -1);
  for (int kt = 0; kt < nkt; ++kt)
    for (int kw = 0; kw < 4; ++kw)
      for (int lane = 0; lane < 64; ++lane)
        for (int sub = 0; sub < 2; ++sub)
          for (int k2 = 0; k2 < 2; ++k2) {
            const int j = 32 * kw + (lane & 31);
            const uint32_t off = DsUnit::store_offset(j, lane, sub, k2, nkt);
            CHECK(off % 16 == 0 && off + 16 <= (uint32_t)(nkt + 1) * 8192, "store offset %u out of range\n", off);
            CHECK((int)(off / (nkt * 8192)) == sub && off % (nkt * 8192) < 8192, "store leaves its unit\n");
            if (sub) continue;
            for (int e = 0; e < 8; ++e) {
              const int el = kt * unit_elems + (int)(off / 2) + e;
              CHECK(row_of[el] < 0, "element %d stored twice\n", el);
              row_of[el] = 16 * k2 + 8 * (lane >> 5) + e;
              key_of[el] = 128 * kt + j;
            }
          }
  for (int el = 0; el < nkt * unit_elems; ++el) CHECK(row_of[el] >= 0, "element %d never stored\n", el);
  constexpr int per_stage = 2 * BK * 16;  // bf16 elements of one wave's stage
  for (int s = 0; s < nkt * 128 / BK; ++s) {
    std::vector<int> lrow(per_stage, -1), lkey(per_stage, -1);
    for (int i = 0; i < BK / 16; ++i)
      for (int lane = 0; lane < 64; ++lane) {
        const uint32_t src = DsUnit::stage_src<BK>(s, i, lane);
        CHECK(src == DsUnit::stage_src<BK>(s, 0, 0) + DsUnit::stage_src<BK>(0, i, lane), "stage offset not separable\n");
        CHECK(src % 16 == 0 && src + 16 <= (uint32_t)nkt * 8192, "stage source %u out of range\n", src);
        for (int e = 0; e < 8; ++e) {
          const int d = (1024 * i + 16 * lane) / 2 + e;
          CHECK(d < per_stage && lrow[d] < 0, "stage element %d written twice\n", d);
          lrow[d] = row_of[src / 2 + e];
          lkey[d] = key_of[src / 2 + e];
        }
      }
    for (int ks = 0; ks < BK / 16; ++ks)
      for (int half = 0; half < 2; ++half)
        for (int lane = 0; lane < 64; ++lane) {
          const int g = lane >> 4, j = lane & 15;
          for (int r = 0; r < 4; ++r) {
            const int src_lane = 16 * g + 4 * r + j / 4;
            const int el = DsUnit::tr_elem<BK>(src_lane, ks, half) + j % 4;
            CHECK(el >= 0 && el < per_stage, "tr read out of the stage\n");
            const int want_key = BK * s + 16 * ks + 8 * (lane >> 5) + 4 * half + r;
            CHECK(lrow[el] == (lane & 31) && lkey[el] == want_key,
                  "BK %d stage %d ks %d half %d lane %d r %d: row %d key %d, want %d %d\n", BK, s, ks, half, lane,
                  r, lrow[el], lkey[el], lane & 31, want_key);
          }
        }
  }
}

// Transposed reads of row-major tiles (dK/dV kernel: Q^T and dO^T operands
// from the Q and dO row tiles): lane l must receive channel 32*dt + l%32 of
// rows 16*s + 8*(l/32) + 4*h + r, r = 0..3, for every 16-row step s.
template <int RL, int ROWS>
void check_tr_reads() {
  using L = TileLayout<RL>;
  // physical element -> (row, column)
  std::vector<int> prow(ROWS * RL, -1), pcol(ROWS * RL, -1);
  for (int r = 0; r < ROWS; ++r)
    for (int c = 0; c < RL; ++c) {
      const int o = L::off(r, c & ~3) + (c & 3);
      prow[o] = r;
      pcol[o] = c;
    }
  for (int s = 0; s < ROWS / 16; ++s)
    for (int dt = 0; dt < RL / 32; ++dt)
      for (int h = 0; h < 2; ++h)
        for (int lane = 0; lane < 64; ++lane) {
          const int g = lane >> 4, j = lane & 15;
          const int own = tr_read_off<RL>(lane, dt, h) + 16 * s * RL;
          CHECK(own % 4 == 0 && own >= 0 && own + 4 <= ROWS * RL, "tr offset out of the tile\n");
          for (int r = 0; r < 4; ++r) {
            const int src_lane = 16 * g + 4 * r + j / 4;
            const int el = tr_read_off<RL>(src_lane, dt, h) + 16 * s * RL + j % 4;
            CHECK(prow[el] == 16 * s + 8 * (lane >> 5) + 4 * h + r && pcol[el] == 32 * dt + (lane & 31),
                  "RL %d s %d dt %d h %d lane %d r %d: row %d col %d\n", RL, s, dt, h, lane, r, prow[el], pcol[el]);
          }
        }
}

int main() {
  check_tr_reads<128, 64>();
  check_tr_reads<64, 64>();
  check_ds<64>(3);
  check_ds<32>(2);
  check_tile<64, 128, 8>();  // forward K tile; dK/dV Q, dO row tiles (d128)
  check_tile<128, 64, 8>();  // forward V^T tile; dK/dV Q^T, dO^T tiles (d128)
  check_tile<32, 128, 8>();  // dQ K, V row tiles (d128)
  check_tile<128, 32, 8>();  // dQ K^T tile (d128)
  check_tile<64, 64, 8>();   // d64 row and column tiles of 64
  check_tile<32, 64, 8>();   // dQ K, V row tiles (d64)
  check_tile<64, 32, 8>();   // dQ K^T tile (d64)
  // perm23: involution; C-layout rows 16*k2 + 8*h + e (e = 0..7) come from
  // lanes whose perm23 row index is consecutive.
  for (int x = 0; x < 32; ++x) CHECK(perm23(perm23(x)) == x, "perm23 not an involution at %d\n", x);
  for (int k2 = 0; k2 < 2; ++k2)
    for (int h = 0; h < 2; ++h)
      for (int e = 0; e < 8; ++e) {
        // C layout of 32x32 MFMA: register r of lane l holds row 8*(r/4) + 4*(l/32) + r%4.
        const int reg = 8 * k2 + e, row_c = 8 * (reg / 4) + 4 * h + reg % 4;
        CHECK(perm23(row_c) == 16 * k2 + 8 * h + e, "perm23 C-layout order k2 %d h %d e %d\n", k2, h, e);
      }
  if (failures) { std::printf("FAILURES %d\n", failures); return 1; }
  std::printf("OK\n");
  return 0;
}
"""


@pytest.fixture(scope="module")
def layout_binary(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("layout")
    src = d / "layout_check.hip"
    src.write_text(PROGRAM)
    exe = d / "layout_check"
    cmd = [hipcc, "-x", "hip", "--offload-host-only", "-std=c++17", "-O1", f"-I{CSRC}", str(src), "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    return exe


def test_tile_layout_and_staging(layout_binary):
    res = subprocess.run([str(layout_binary)], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0 and res.stdout.strip().endswith("OK"), res.stdout[-3000:]
