// Tile scheduling and operand windows of the large-tile fp8 GEMM, as __host__
// __device__ functions so the host-side test build can check them exhaustively.
#pragma once

#include <stdint.h>

namespace ayk {

// Workgroup b runs on XCD b % 8. Give each XCD a contiguous range of logical tile
// ids, then walk tiles in an M-grouped order (kGroupM M tiles per group, N varying
// within the group), so the tiles one XCD runs together share operand panels in its
// L2. The mapping b -> (tm, tn) is a bijection onto [0, tiles_m) x [0, tiles_n).
__host__ __device__ inline void big_tile_coords(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int xcd = b & 7, local = b >> 3, per = total >> 3, rem = total & 7;
  const int t = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + local;
  constexpr int kGroupM = 8;
  const int group = t / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int gsize = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
  const int in_group = t - group * kGroupM * tiles_n;
  tm = first_m + in_group % gsize;
  tn = in_group / gsize;
}

// Buffer window of one wavefront's operand rows [row0, row0 + 128): byte offset of
// the window base from the operand base, and the number of readable bytes from it
// (rows row0 .. total_rows-1). A window entirely past the last row is empty: zero
// records (every load returns zero) and a base inside the allocation.
struct OperandWindow {
  int64_t base_offset;
  int32_t records;
};
__host__ __device__ inline OperandWindow operand_window(int64_t row0, int64_t total_rows, int64_t ld) {
  const int64_t rows_left = total_rows - row0;
  if (rows_left <= 0) return {0, 0};
  const int64_t bytes = rows_left * ld;
  return {row0 * ld, (int32_t)(bytes < 0x7FFFFFFF ? bytes : 0x7FFFFFFF)};
}

}  // namespace ayk
