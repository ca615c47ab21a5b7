"""The GEMM block -> tile mapping (csrc/tile_map.hpp), checked exhaustively on the CPU.

The same header is compiled into the gfx950 kernels; here it is compiled for
the host.  For every (row tiles, column tiles) pair in a broad range, every
block of the padded grid either is rejected as padding or names a tile in
range, and every tile is named exactly once.
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
  printf("ok %ld\n", pairs);
  return 0;
}
"""


def test_tile_mapping_is_a_bijection_onto_valid_tiles(tmp_path):
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
