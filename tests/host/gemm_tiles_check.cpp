// Host check of the large-tile GEMM scheduling arithmetic (csrc/gemm_tiles.h):
// tile order bijectivity and buffer-window bounds for every wavefront of every tile.
// Built with g++ by tests/test_gemm_tiles_host.py; prints "ok" or the first violation.
#include <cstdio>
#include <cstdint>
#include <vector>
#define __host__
#define __device__
#include "gemm_tiles.h"

using namespace ayk;

static int check_shape(int64_t M, int64_t N, int64_t K, int64_t lda, int64_t ldw) {
  const int tile = 256, half = 128;
  const int tm_n = (int)((M + tile - 1) / tile), tn_n = (int)((N + tile - 1) / tile);
  std::vector<int> seen((size_t)tm_n * tn_n, 0);
  for (int b = 0; b < tm_n * tn_n; ++b) {
    int tm, tn;
    big_tile_coords(b, tm_n, tn_n, tm, tn);
    if (tm < 0 || tm >= tm_n || tn < 0 || tn >= tn_n) { printf("coords out of range b=%d M=%lld N=%lld\n", b, (long long)M, (long long)N); return 1; }
    if (seen[(size_t)tm * tn_n + tn]++) { printf("coords not a bijection b=%d\n", b); return 1; }
    for (int wave = 0; wave < 4; ++wave) {
      const bool w = wave < 2;
      const int64_t rows = w ? N : M, ld = w ? ldw : lda;
      const int64_t row0 = (int64_t)(w ? tn : tm) * tile + (wave & 1) * half;
      const OperandWindow win = operand_window(row0, rows, ld);
      const int64_t alloc = rows * ld;
      if (win.records < 0) { printf("negative records\n"); return 1; }
      if (win.records > 0 && (win.base_offset < 0 || win.base_offset >= alloc)) { printf("base outside allocation\n"); return 1; }
      if (win.base_offset + win.records > alloc) { printf("window past allocation\n"); return 1; }
      for (int r = 0; r < half; ++r) {
        const int64_t row = row0 + r;
        // last byte this row's loads touch: the row's K bytes
        const int64_t first = (int64_t)r * ld, last = first + K - 1;
        if (row < rows) {
          if (last >= win.records) { printf("valid row %lld not readable\n", (long long)row); return 1; }
        } else if (first < win.records) {
          printf("row %lld past the end is readable (M=%lld N=%lld)\n", (long long)row, (long long)M, (long long)N);
          return 1;
        }
      }
    }
  }
  return 0;
}

int main() {
  const int64_t Ms[] = {256, 300, 384, 513, 777, 1024, 4096, 8192};
  const int64_t Ns[] = {256, 260, 520, 772, 1028, 3584, 18432, 37888, 57344};
  const int64_t Ks[] = {128, 1024, 3584};
  for (int64_t M : Ms)
    for (int64_t N : Ns)
      for (int64_t K : Ks)
        for (int64_t pad : {0, 128})
          if (check_shape(M, N, K, K + pad, K)) return 1;
  printf("ok\n");
  return 0;
}
