"""The XCD tile mapping of the implicit-GEMM kernels (csrc/tile_map.h), compiled for the host with g++: for every grid
the kernels may launch, workgroup ids [0, gx*gy*gz) must map one-to-one onto the tiles and stay inside the grid (a tile
outside it would be written out of bounds, a tile never visited left unwritten). Also checks the locality the mapping
is for: the 8 XCDs each receive one contiguous run of tile ids."""

import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
CSRC = ROOT / "omarchy-mac-torch_amd" / "csrc"

CHECK = r"""
#include <cstdio>
#include <vector>
#include "tile_map.h"
using omt::TileId;

static long check(int gx, int gy, int gz, int gm) {
  const int n = gx * gy * gz;
  std::vector<char> seen(n, 0);
  long bad = 0;
  for (int pid = 0; pid < n; ++pid) {
    const TileId t = omt::xcd_tile(pid, gx, gy, gz, gm);
    if (t.x < 0 || t.x >= gx || t.y < 0 || t.y >= gy || t.z < 0 || t.z >= gz) { ++bad; continue; }
    char& s = seen[t.x + gx * (t.y + gy * t.z)];
    bad += s;
    s = 1;
  }
  // locality: with n a multiple of 8, XCD j (workgroups j, j+8, ...) visits the ids [j*n/8, (j+1)*n/8) in order
  if (n % omt::kXCDs == 0) {
    const int per = n / omt::kXCDs;
    for (int pid = 0; pid < n; ++pid) {
      const int want = (pid % omt::kXCDs) * per + pid / omt::kXCDs;
      const TileId a = omt::xcd_tile(pid, gx, gy, gz, gm);
      // the id `want` sits in z-plane want / (gx*gy)
      if (a.z != want / (gx * gy)) ++bad;
    }
  }
  return bad;
}

int main() {
  long bad = 0, cases = 0;
  for (int gx = 1; gx <= 70; ++gx)
    for (int gy = 1; gy <= 40; gy += (gy < 10 ? 1 : 7))
      for (int gz = 1; gz <= 23; gz += (gz < 5 ? 1 : 6))
        for (int gm : {1, 3, 8}) bad += check(gx, gy, gz, gm), ++cases;
  // grids of the ResNet-50 body at batch 256 (gather 196x8, 98x32, 12544x1; wgrad 9x1x203) and a split gather
  const int big[][3] = {{196, 8, 1}, {98, 32, 1}, {9, 1, 203}, {12544, 1, 1}, {1568, 4, 3}, {25, 16, 16}};
  for (const auto& g : big) bad += check(g[0], g[1], g[2], 8), ++cases;
  printf("cases %ld bad %ld\n", cases, bad);
  return bad != 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_xcd_tile_mapping_is_a_bijection(tmp_path):
    src = tmp_path / "check.cpp"
    src.write_text(CHECK)
    exe = tmp_path / "check"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("bad 0")
