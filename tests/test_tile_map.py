"""The GEMM's workgroup -> tile map (csrc/tile_map.hpp) on the host: for every
grid shape up to 130 x 130 tiles (and the 720p MLP's 99 x 54 and 99 x 20) each
workgroup id in [0, tiles_m * tiles_n) gets a distinct in-range tile, so
every output tile is computed exactly once; and each XCD's workgroups cover
one contiguous run of logical tiles."""

import shutil
import subprocess

import pytest

from conftest import ROOT

HARNESS = r"""
#include <cstdio>
#include <vector>
#include "tile_map.hpp"

int check(int tm_n, int tn_n) {
  const int total = tm_n * tn_n;
  std::vector<int> seen(total, 0);
  for (int pid = 0; pid < total; ++pid) {
    int tm, tn;
    xmh3::tile_coords(pid, tm_n, tn_n, tm, tn);
    if (tm < 0 || tm >= tm_n || tn < 0 || tn >= tn_n) {
      std::printf("out of range: grid %dx%d pid %d -> (%d,%d)\n", tm_n, tn_n, pid, tm, tn);
      return 1;
    }
    if (seen[tm * tn_n + tn]++) {
      std::printf("tile twice: grid %dx%d pid %d -> (%d,%d)\n", tm_n, tn_n, pid, tm, tn);
      return 1;
    }
  }
  return 0;
}

int main() {
  long shapes = 0;
  for (int a = 1; a <= 130; ++a)
    for (int b = 1; b <= 130; ++b, ++shapes)
      if (check(a, b)) return 1;
  if (check(99, 54) || check(99, 20) || check(1024, 3) || check(7, 997)) return 1;
  std::printf("ok %ld shapes\n", shapes + 4);
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_tile_coords_is_a_bijection(tmp_path):
    src = tmp_path / "tile_map_check.cpp"
    src.write_text(HARNESS)
    exe = tmp_path / "tile_map_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", str(ROOT / "x-minimaxh3_amd" / "csrc"), str(src), "-o",
                    str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout
    assert r.stdout.startswith("ok 16904 shapes")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_each_xcd_walks_a_contiguous_logical_run(tmp_path):
    src = tmp_path / "xcd_runs.cpp"
    src.write_text(r"""
#include <cstdio>
#include "tile_map.hpp"
int main() {
  // fc1 at 720p: 99 x 54 tiles. Workgroup pid runs on XCD pid % 8; logical
  // index = band-major order of the returned tile; per XCD it must rise by 1.
  const int tm_n = 99, tn_n = 54, total = tm_n * tn_n;
  for (int x = 0; x < xmh3::NUM_XCD; ++x) {
    int prev = -1;
    for (int pid = x; pid < total; pid += xmh3::NUM_XCD) {
      int tm, tn;
      xmh3::tile_coords(pid, tm_n, tn_n, tm, tn);
      const int band = tm / xmh3::GROUP_M, first = band * xmh3::GROUP_M;
      const int gsize = tm_n - first < xmh3::GROUP_M ? tm_n - first : xmh3::GROUP_M;
      const int logical = first * tn_n + tn * gsize + (tm - first);
      if (prev >= 0 && logical != prev + 1) { std::printf("xcd %d breaks at pid %d\n", x, pid); return 1; }
      prev = logical;
    }
  }
  std::printf("ok\n");
  return 0;
}
""")
    exe = tmp_path / "xcd_runs"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", str(ROOT / "x-minimaxh3_amd" / "csrc"), str(src), "-o",
                    str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout
