"""The GEMM block -> work mapping (csrc/tile_map.hpp), checked exhaustively on the CPU.

The same header is compiled into the gfx950 kernels; here it is compiled for
the host.  For every (row tiles, column tiles) pair in a broad range, every
block of the padded grid either is rejected as padding or names a tile in
range, and every tile is named exactly once.  For the work units (whole
tiles, plus the K-split parts of a short last round) every live tile is
covered exactly once, or by exactly `parts` distinct parts that share one
workspace slot; split units come after every whole tile in time order and
fill at most one round.  With the run-time tail (the last units handed out
by ticket), every unit still runs exactly once and there are enough blocks.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "hy-nomas-rs_amd", "csrc", "tile_map.hpp")

PROG = r"""
#include "tile_map.hpp"
#include <cstdio>
#include <vector>
int main() {
  long pairs = 0;
  for (int max_tiles = 1; max_tiles <= 260; ++max_tiles)
    for (int ntn = 1; ntn <= 66; ++ntn) {
      const long long G = (long long)max_tiles * ntn, Gp = nomas::tile_grid(max_tiles, ntn);
      if (Gp < G || Gp % (nomas::kXcds * nomas::kCusPerXcd) != 0) { printf("bad grid\n"); return 1; }
      std::vector<int> hit(G, 0);
      for (long long pid = 0; pid < Gp; ++pid) {
        int mt = -1, nt = -1;
        if (!nomas::tile_coords((int)pid, ntn, max_tiles, &mt, &nt)) continue;
        if (mt < 0 || mt >= max_tiles || nt < 0 || nt >= ntn) {
          printf("out of range: pid %lld -> (%d, %d) for (%d, %d)\n", pid, mt, nt, max_tiles, ntn);
          return 1;
        }
        hit[(long long)mt * ntn + nt]++;
      }
      for (long long i = 0; i < G; ++i)
        if (hit[i] != 1) { printf("tile %lld named %d times (%d, %d)\n", i, hit[i], max_tiles, ntn); return 1; }
      ++pairs;
    }
  // work units
  const int turns_set[] = {1, 2, 3, 6, 12, 24, 64};
  long units_checked = 0;
  for (int max_tiles = 1; max_tiles <= 150; ++max_tiles)
    for (int tiles = 0; tiles <= max_tiles; tiles += (max_tiles > 40 ? 7 : 1))
      for (int ntn = 1; ntn <= 66; ntn += (tiles > 60 ? 5 : 1))
        for (int turns : turns_set) {
          const long long T = (long long)tiles * ntn;
          const long long grid = nomas::tile_grid(max_tiles, ntn) + nomas::kRound;
          std::vector<int> whole(T, 0), parts_seen(T, 0), slot_of(T, -1), pmask(T, 0), npart(T, 0);
          std::vector<int> slot_used(nomas::kRound, 0);
          long long last_whole = -1, first_split = 1LL << 60;
          for (long long pid = 0; pid < grid; ++pid) {
            nomas::WorkUnit u;
            if (!nomas::unit_coords((int)pid, ntn, tiles, turns, &u)) continue;
            if (u.mt < 0 || u.mt >= tiles || u.nt < 0 || u.nt >= ntn) { printf("unit out of range\n"); return 1; }
            const long long t = (long long)u.mt * ntn + u.nt, L = nomas::time_order((int)pid);
            if (u.parts == 1) { whole[t]++; if (L > last_whole) last_whole = L; continue; }
            if (u.parts < 2 || u.parts > nomas::kMaxSplit || turns % u.parts || u.part < 0 || u.part >= u.parts ||
                u.slot < 0 || u.slot * u.parts >= nomas::kRound) { printf("bad split unit\n"); return 1; }
            if (slot_of[t] != -1 && slot_of[t] != u.slot) { printf("slot mismatch\n"); return 1; }
            slot_of[t] = u.slot; npart[t] = u.parts;
            if (pmask[t] & (1 << u.part)) { printf("part twice\n"); return 1; }
            pmask[t] |= 1 << u.part; parts_seen[t]++;
            if (L < first_split) first_split = L;
          }
          for (long long t = 0; t < T; ++t) {
            const bool ok = (whole[t] == 1 && parts_seen[t] == 0) ||
                            (whole[t] == 0 && parts_seen[t] == npart[t] && pmask[t] == (1 << npart[t]) - 1);
            if (!ok) { printf("tile %lld covered wrongly (%d, %d, %d)\n", t, tiles, ntn, turns); return 1; }
            if (slot_of[t] >= 0) { if (slot_used[slot_of[t]]++) { printf("slot shared\n"); return 1; } }
          }
          if (first_split < (1LL << 60) && first_split < last_whole) { printf("split before whole\n"); return 1; }
          // the run-time tail: blocks before tail_start run their own unit,
          // every other block takes a ticket (tickets 0, 1, ... in any order);
          // each unit must run exactly once
          const long long W = nomas::unit_count(tiles, ntn, turns), Ws = nomas::tail_start(W);
          if (Ws > W || Ws % nomas::kRound || W - Ws >= nomas::kTailUnits + nomas::kRound ||
              (W > nomas::kTailUnits && W - Ws < nomas::kTailUnits)) { printf("bad tail\n"); return 1; }
          std::vector<int> runs(W, 0);
          long long tail_blocks = 0;
          for (long long pid = 0; pid < grid; ++pid) {
            const long long L = nomas::time_order((int)pid);
            if (L < Ws) {
              nomas::WorkUnit a, b;
              if (!nomas::unit_coords((int)pid, ntn, tiles, turns, &a)) { printf("static block idle\n"); return 1; }
              nomas::unit_at(L, ntn, tiles, turns, &b);
              if (a.mt != b.mt || a.nt != b.nt || a.part != b.part || a.parts != b.parts || a.slot != b.slot) {
                printf("unit_at differs from unit_coords\n"); return 1;
              }
              runs[L]++;
            } else {
              ++tail_blocks;
            }
          }
          if (tail_blocks < W - Ws) { printf("fewer tail blocks than tail units\n"); return 1; }
          for (long long t = 0; t < tail_blocks && Ws + t < W; ++t) runs[Ws + t]++;
          for (long long i = 0; i < W; ++i)
            if (runs[i] != 1) { printf("unit %lld runs %d times (%d, %d, %d)\n", i, runs[i], tiles, ntn, turns); return 1; }
          ++units_checked;
        }
  printf("ok %ld %ld\n", pairs, units_checked);
  return 0;
}
"""


def test_tile_and_work_unit_mappings(tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    src = tmp_path / "tile_map_check.cpp"
    src.write_text(PROG)
    exe = tmp_path / "tile_map_check"
    subprocess.run([hipcc, "-O2", "-std=c++17", "-I", os.path.dirname(HDR), str(src), "-o",
                    str(exe)], check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("ok")
