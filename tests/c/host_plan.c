/* A plain C host building one phase of a paired bridge_k plan with the host table builder
 * (include/hilberta_hip.h, the hb_*_host entry points) and printing it:
 *   host_plan GRID TILES K PHASE KEY_BLOCK
 * prints "shared S", "rows R width W", then R lines "count: id/flag id/flag ...".
 * No GPU is needed.  tests/test_capi.py compiles it with gcc and checks the output against the
 * oracle's bridge_k_plan + pair_metadata. */
#include <stdio.h>
#include <stdlib.h>

#include "hilberta_hip.h"

#define CHECK(call)                                                   \
  do {                                                                \
    if ((call) != 0) {                                                \
      fprintf(stderr, "%s: %s\n", #call, hb_last_error());            \
      return 1;                                                       \
    }                                                                 \
  } while (0)

int main(int argc, char** argv) {
  if (argc != 6) {
    fprintf(stderr, "usage: %s GRID TILES K PHASE KEY_BLOCK\n", argv[0]);
    return 2;
  }
  const int grid = atoi(argv[1]), tiles = atoi(argv[2]), k = atoi(argv[3]);
  const int phase = atoi(argv[4]), key_block = atoi(argv[5]);
  const int bs = 64, text = 512;
  const long n = (long)grid * grid;
  const int nb = (int)(n / bs), T = text / bs + nb, words = (T + 31) / 32;
  int64_t* orders = malloc(sizeof(int64_t) * (4 * n + 2 * nb));
  int32_t status[3];
  if (!orders) return 1;
  int64_t *orig = orders, *inv = orders + n, *img = orders + 2 * n, *inv_img = orders + 3 * n;
  int64_t *packed = orders + 4 * n, *to_phys = packed + nb;
  CHECK(hb_plan_layout_host(grid, bs, text, 0, orig, inv, img, inv_img, packed, to_phys, status));
  const int rows = T - text / bs - status[0];
  int32_t* scores = malloc(sizeof(int32_t) * (size_t)nb * nb);
  int64_t* chosen = malloc(sizeof(int64_t) * (size_t)nb * k);
  uint32_t* bits = malloc(sizeof(uint32_t) * (size_t)rows * words);
  int32_t* counts = malloc(sizeof(int32_t) * (size_t)(rows / 2));
  if (!scores || !chosen || !bits || !counts) return 1;
  CHECK(hb_plan_phase_bits_host(inv, packed, to_phys, grid, tiles, text, bs, status[0], phase, 2, k,
                                scores, chosen, bits));
  int32_t widest[2];
  CHECK(hb_bits_counts_host(bits, rows, T, key_block, NULL, counts, widest));
  const int width = widest[1] > 0 ? widest[1] : 1;
  int32_t* ids = malloc(sizeof(int32_t) * (size_t)(rows / 2) * width);
  int32_t* flags = malloc(sizeof(int32_t) * (size_t)(rows / 2) * width);
  if (!ids || !flags) return 1;
  CHECK(hb_bits_emit_host(bits, rows, T, key_block, NULL, 0, ids, flags, width));
  printf("shared %d\nrows %d width %d\n", status[0], rows / 2, width);
  for (int r = 0; r < rows / 2; ++r) {
    printf("%d:", counts[r]);
    for (int e = 0; e < counts[r]; ++e) printf(" %d/%d", ids[r * width + e], flags[r * width + e]);
    printf("\n");
  }
  free(ids);
  free(flags);
  free(counts);
  free(bits);
  free(chosen);
  free(scores);
  free(orders);
  return 0;
}
