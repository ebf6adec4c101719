// Workgroup -> tile mapping of the implicit-GEMM kernels (host- and device-compilable: the CPU tests check that it
// is a bijection onto the tile grid).
#pragma once

#ifndef __HIPCC__
#define __host__
#define __device__
#endif

namespace omt {

// Workgroups go to the 8 XCDs round robin in dispatch order (x fastest), so workgroup `pid` of a launch runs on XCD
// (pid + c) % 8 for a launch-wide c, and each XCD has an L2 of its own. The tile mapping hands each XCD a contiguous
// run of tile ids, walked in groups of `gm` tile rows (y) with the rows fastest: the workgroups resident on one XCD at
// a time then cover a compact block of output tiles, whose operand rows they share in that L2, rather than every
// eighth tile of a row. A bijection of [0, gx*gy*gz) onto the tiles (the ids past the last full round of 8 keep their
// place).
constexpr int kXCDs = 8;
struct TileId {
  int x, y, z;
};
__host__ __device__ inline TileId xcd_tile(int pid, int gx, int gy, int gz, int gm) {
  const int per = gx * gy * gz / kXCDs;
  const int t = pid < per * kXCDs ? (pid % kXCDs) * per + pid / kXCDs : pid;
  const int plane = gx * gy;
  const int z = t / plane;
  int r = t - z * plane;
  const int g = r / (gm * gx);
  const int y0 = g * gm;
  const int rows = gy - y0 < gm ? gy - y0 : gm;
  r -= g * gm * gx;
  return {r / rows, y0 + r % rows, z};
}

}  // namespace omt
