// Host check of smx::tile_of (csrc/common.hpp): every tile order maps the
// workgroups of a launch one-to-one onto its tile grid, for every grid up to
// 72 x 72 tiles and every group size SMX_GROUP_M accepts (1-64), and for the
// Qwen3-32B sites' grids (128 x 128 and 128 x 256 product tiles).
// Built and run by tests/test_tile_order.py.
#include <cstdio>
#include <vector>

#include "../strassen_tpu_amd/csrc/common.hpp"

static bool bijective(int tiles_m, int tiles_n, int group_m, int raster) {
  const int total = tiles_m * tiles_n;
  std::vector<int> seen(total, 0);
  for (int bid = 0; bid < total; ++bid) {
    int tm, tn;
    smx::tile_of(bid, tiles_m, tiles_n, group_m, raster, tm, tn);
    if (tm < 0 || tm >= tiles_m || tn < 0 || tn >= tiles_n || seen[tm * tiles_n + tn]++) {
      printf("order %d, group %d, grid %d x %d: workgroup %d -> tile (%d, %d)\n", raster, group_m, tiles_m,
             tiles_n, bid, tm, tn);
      return false;
    }
  }
  return true;
}

int main() {
  const int orders[] = {smx::kRasterSpread, smx::kRasterChunks, smx::kRasterBlocks};
  const int sites[][2] = {{32, 32}, {32, 4}, {32, 20}, {32, 200}, {64, 40}, {1, 20}, {1, 200}, {256, 4},
                          {32, 100}, {32, 10}, {32, 16}, {32, 2}};
  long grids = 0;
  for (int raster : orders) {
    for (int group_m = 1; group_m <= 64; ++group_m)
      for (int tiles_m = 1; tiles_m <= 72; ++tiles_m)
        for (int tiles_n = 1; tiles_n <= 72; ++tiles_n, ++grids)
          if (!bijective(tiles_m, tiles_n, group_m, raster)) return 1;
    for (const auto& s : sites) {
      if (!bijective(s[0], s[1], 8, raster)) return 1;
      ++grids;
    }
  }
  printf("ok %ld grids\n", grids);
  return 0;
}
