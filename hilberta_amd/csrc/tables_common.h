// Integer helpers of the block-table builder, shared by the device kernels (tables.hip) and the
// host builder (tables_host.hip) so that both compute every table from the same arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hb {

// Token at position d of the Hilbert curve over a g x g grid (g a power of two), as a raster id
// (g-1-y)*g + x: d2xy with the quadrant rotation (geometry.py:6-25).
__host__ __device__ __forceinline__ int64_t hilbert_raster(int64_t d, int g) {
  int64_t x = 0, y = 0, t = d;
  for (int s = 1; s < g; s *= 2) {
    const int64_t rx = (t / 2) & 1;
    const int64_t ry = (t ^ (t / 2)) & 1;
    if (ry == 0) {
      if (rx) {
        x = s - 1 - x;
        y = s - 1 - y;
      }
      const int64_t tmp = x;
      x = y;
      y = tmp;
    }
    x += s * rx;
    y += s * ry;
    t /= 4;
  }
  return (int64_t)(g - 1 - y) * g + x;
}

// Tile of composite-order position `pos` in a phase shifted by `off` tokens: tiles are runs of
// `width` positions of the cyclic order over n image tokens (plan.py:159-183).
__host__ __device__ __forceinline__ int tile_label(int64_t pos, int64_t off, int64_t n, int64_t width) {
  return (int)((((pos - off) % n) + n) % n / width);
}

// Flag of key block kb in the paired row built from bitmap rows ra (query half 0) and rb (query
// half 1) at key granularity `ratio` 64-token blocks: bit (half + 2*key_half) is set where that
// half holds that 64-token key half (paired_metadata.py:38-51).  0 when neither row holds it.
__host__ __device__ __forceinline__ int pair_flag(const uint32_t* ra, const uint32_t* rb, int kb, int ratio) {
  int flag = 0;
  for (int kh = 0; kh < ratio; ++kh) {
    const int p = kb * ratio + kh;
    const uint32_t a = (ra[p / 32] >> (p % 32)) & 1u;
    const uint32_t b = (rb[p / 32] >> (p % 32)) & 1u;
    flag |= (int)(a << (2 * kh)) | (int)(b << (1 + 2 * kh));
  }
  return flag;
}

}  // namespace hb
