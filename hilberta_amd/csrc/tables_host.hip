// Host (CPU) builder of the HilbertA block tables: the same tables as the device kernels of
// tables.hip, bit for bit, for callers that set a plan up on a host without a GPU (the reference
// builds every table on the CPU: geometry.py:6-25, plan.py:114-197, bridge_k.py:10-51,
// paired_metadata.py:26-51).  Each entry point takes the arguments of its device counterpart
// except the stream, with host pointers, runs synchronously on the calling thread and touches no
// HIP API.  The attention kernels have no host counterpart.
//
// The integer helpers (Hilbert curve, tile labels, pair flags) are the device builder's own
// (tables_common.h); the steps that the device spreads over lanes and atomics run here as plain
// loops whose results do not depend on order: sums, ORs, a stable partition and a top-K over
// distinct keys.
#include <string.h>

#include <algorithm>
#include <new>
#include <vector>

#include "common.h"
#include "tables_common.h"
#include "../../include/hilberta_hip.h"

namespace hb {
namespace {

// key blocks per row the device pairing kernel covers; the host accepts the same tables
constexpr int PAIR_MAX_BLOCKS = 16384;

// Runs f, turning a failed host allocation into an error code: nothing throws across the C ABI.
template <class F>
int guarded(F&& f) {
  try {
    return f();
  } catch (const std::bad_alloc&) {
    set_error("host allocation failed");
    return HB_EINVAL;
  }
}

void composite_order(int g, int64_t* original, int64_t* inverse) {
  const int64_t n = (int64_t)g * g, half = n / 2;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t h = hilbert_raster(n / 4 + (i < half ? i : i - half), g);
    const int64_t tok = i < half ? h : n - 1 - h;
    original[i] = tok;
    inverse[tok] = i;
  }
}

// Emits row `row` of a bitmap (mode 0) or paired row `row` (mode 1, rows 2*row and 2*row + 1 at
// key granularity `ratio`) as ascending key blocks, zero padded to `width`; returns the number of
// entries the row holds (entries past `width` are dropped).
int emit_row(const uint32_t* bits, int words, int T, int mode, int ratio, int row, int32_t* ids,
             int32_t* flags, int width) {
  const uint32_t* ra = bits + (int64_t)(mode ? 2 * row : row) * words;
  const uint32_t* rb = ra + words;
  const int kblocks = mode ? (T + ratio - 1) / ratio : T;
  int base = 0;
  for (int kb = 0; kb < kblocks; ++kb) {
    const int flag = mode ? pair_flag(ra, rb, kb, ratio) : (int)((ra[kb / 32] >> (kb % 32)) & 1u);
    if (!flag) continue;
    if (base < width) {
      ids[base] = kb;
      if (flags) flags[base] = flag;
    }
    ++base;
  }
  for (int e = base; e < width; ++e) {
    ids[e] = 0;
    if (flags) flags[e] = 0;
  }
  return base;
}

int count_row(const uint32_t* bits, int words, int T, int mode, int ratio, int row) {
  int c = 0;
  if (mode == 0) {
    const uint32_t* r = bits + (int64_t)row * words;
    for (int w = 0; w < words; ++w) c += __builtin_popcount(r[w]);
  } else {
    const uint32_t* ra = bits + (int64_t)(2 * row) * words;
    const uint32_t* rb = ra + words;
    const int kblocks = (T + ratio - 1) / ratio;
    for (int kb = 0; kb < kblocks; ++kb) c += pair_flag(ra, rb, kb, ratio) != 0;
  }
  return c;
}

}  // namespace
}  // namespace hb

using namespace hb;

extern "C" int hb_hilbert_order_host(int32_t grid_size, int64_t* out) {
  HB_REQUIRE(grid_size >= 2 && (grid_size & (grid_size - 1)) == 0,
             "Hilbert grid side must be a power of two >= 2");
  HB_REQUIRE(out, "null output");
  const int64_t n = (int64_t)grid_size * grid_size;
  for (int64_t d = 0; d < n; ++d) out[d] = hilbert_raster(d, grid_size);
  return HB_OK;
}

extern "C" int hb_plan_layout_host(int32_t grid_size, int32_t block_size, int32_t text_tokens,
                                   int32_t shared, int64_t* original_order,
                                   int64_t* inverse_original, int64_t* image_order,
                                   int64_t* inverse_image_order, int64_t* physical_original_blocks,
                                   int64_t* original_to_physical, int32_t* status) {
  HB_REQUIRE(grid_size >= 8 && (grid_size & (grid_size - 1)) == 0,
             "grid_size must be a power of two >= 8");
  HB_REQUIRE(block_size > 0 && text_tokens > 0 && text_tokens % block_size == 0,
             "text prefix must be block aligned");
  const int64_t n = (int64_t)grid_size * grid_size;
  HB_REQUIRE(n % block_size == 0 && n / block_size <= (1 << 20), "image tokens must be whole blocks");
  HB_REQUIRE(original_order && inverse_original && image_order && inverse_image_order &&
                 physical_original_blocks && original_to_physical && status,
             "null output");
  const int g = grid_size, bs = block_size, nb = (int)(n / bs), text_blocks = text_tokens / bs;
  return guarded([&] {
    composite_order(g, original_order, inverse_original);
    // shared blocks: every token inside the centre square [3g/8, 5g/8)^2 (plan.py:138-150)
    const int start = 3 * g / 8, end = 5 * g / 8;
    std::vector<char> is_shared(nb, 0);
    int n_shared = 0, partial = 0;
    for (int b = 0; b < nb; ++b) {
      int cnt = 0;
      if (shared) {
        for (int j = 0; j < bs; ++j) {
          const int64_t tok = original_order[(int64_t)b * bs + j];
          const int y = (int)(tok / g), x = (int)(tok % g);
          cnt += (y >= start && y < end && x >= start && x < end);
        }
      }
      if (cnt != 0 && cnt != bs) partial = 1;
      is_shared[b] = cnt == bs;
      n_shared += cnt == bs;
    }
    // stable partition, shared blocks first
    int sh = 0, ord = n_shared;
    for (int b = 0; b < nb; ++b) {
      const int slot = is_shared[b] ? sh++ : ord++;
      physical_original_blocks[slot] = b;
      original_to_physical[b] = slot + text_blocks;
    }
    for (int64_t i = 0; i < n; ++i) inverse_image_order[i] = -1;
    for (int64_t i = 0; i < n; ++i) {
      const int64_t tok = original_order[physical_original_blocks[i / bs] * bs + i % bs];
      image_order[i] = tok;
      if (tok >= 0 && tok < n) inverse_image_order[tok] = i;
    }
    int bad = 0;
    for (int64_t i = 0; i < n; ++i) {
      const int64_t tok = image_order[i];
      bad |= tok < 0 || tok >= n || inverse_image_order[tok] != i;
    }
    status[0] = n_shared;
    status[1] = partial;
    status[2] = bad;
    return HB_OK;
  });
}

extern "C" int hb_plan_phase_bits_host(const int64_t* inverse_original,
                                       const int64_t* physical_original_blocks,
                                       const int64_t* original_to_physical, int32_t grid_size,
                                       int32_t tile_count, int32_t text_tokens, int32_t block_size,
                                       int32_t shared_blocks, int32_t phase, int32_t bridge_mode,
                                       int32_t k, int32_t* scores, int64_t* bridge_original_blocks,
                                       uint32_t* bits) {
  const int64_t n = (int64_t)grid_size * grid_size;
  HB_REQUIRE(grid_size >= 8 && tile_count > 0 && block_size > 0, "invalid plan geometry");
  HB_REQUIRE(n % tile_count == 0 && (n / tile_count) % (4 * block_size) == 0 &&
                 text_tokens % block_size == 0,
             "Tile quarter offsets and text prefix must be block aligned");
  HB_REQUIRE(phase >= 0 && phase < 4, "phase must be 0..3");
  HB_REQUIRE(bridge_mode >= 0 && bridge_mode <= 2, "bridge_mode must be 0 (none), 1 (directed), 2 (reciprocal)");
  HB_REQUIRE(bridge_mode == 0 || (k >= 1 && k <= 4), "bridge K must be 1..4");
  HB_REQUIRE(inverse_original && physical_original_blocks && original_to_physical && bits, "null pointer");
  HB_REQUIRE(bridge_mode == 0 || (scores && bridge_original_blocks), "bridges need scores and chosen buffers");
  const int g = grid_size, bs = block_size;
  const int nb = (int)(n / bs);
  const int text_blocks = text_tokens / bs;
  const int T = text_blocks + nb;
  const int gb = text_blocks + shared_blocks;
  HB_REQUIRE(shared_blocks >= 0 && shared_blocks < nb, "shared_blocks out of range");
  const int nq = T - gb;
  const int words = (T + 31) / 32;
  const int64_t width = n / tile_count;
  const int64_t off = phase * (width / 4);
  // base rows (plan.py:173-183): the global prefix, then every ordinary block with the row's tile
  // label; the rows of one label are equal, so each label's row is built once and copied
  const int labels = tile_count;
  return guarded([&] {
    std::vector<uint32_t> label_rows((size_t)labels * words, 0u);
    for (int p = 0; p < gb; ++p)
      for (int l = 0; l < labels; ++l) label_rows[(size_t)l * words + p / 32] |= 1u << (p % 32);
    std::vector<int> block_label(T, -1);
    for (int p = gb; p < T; ++p) {
      const int l = tile_label(physical_original_blocks[p - text_blocks] * bs, off, n, width);
      block_label[p] = l;
      label_rows[(size_t)l * words + p / 32] |= 1u << (p % 32);
    }
    for (int r = 0; r < nq; ++r)
      memcpy(bits + (int64_t)r * words, &label_rows[(size_t)block_label[gb + r] * words],
             sizeof(uint32_t) * words);
    if (!bridge_mode) return HB_OK;
    // bridge scores: cross-tile 4-neighbour token pairs between two original blocks, counted in
    // both directions (bridge_k.py:22-28)
    memset(scores, 0, sizeof(int32_t) * (size_t)nb * nb);
    for (int64_t y = 0; y < g; ++y)
      for (int64_t x = 0; x < g; ++x) {
        const int64_t a = y * g + x;
        for (int dir = 0; dir < 2; ++dir) {
          if (dir == 0 ? x + 1 >= g : y + 1 >= g) continue;
          const int64_t c = dir == 0 ? a + 1 : a + g;
          const int64_t pa = inverse_original[a], pc = inverse_original[c];
          if (tile_label(pa, off, n, width) == tile_label(pc, off, n, width)) continue;
          const int ba = (int)(pa / bs), bc = (int)(pc / bs);
          ++scores[(int64_t)ba * nb + bc];
          ++scores[(int64_t)bc * nb + ba];
        }
      }
    // top-K key blocks of each query block by (-score, (key - offset/bs) mod nb) (bridge_k.py:36-40):
    // code (score << 32 | nb-1-rolled) is distinct per key, so the K largest codes are the picks
    const int offset_blocks = (int)(off / bs);
    for (int q = 0; q < nb; ++q) {
      uint64_t top[4] = {0, 0, 0, 0};  // descending
      const int32_t* row = scores + (int64_t)q * nb;
      for (int key = 0; key < nb; ++key) {
        const int s = row[key];
        if (s <= 0) continue;
        const int rolled = ((key - offset_blocks) % nb + nb) % nb;
        uint64_t code = ((uint64_t)(uint32_t)s << 32) | (uint32_t)(nb - 1 - rolled);
        for (int j = 0; j < k; ++j)
          if (code > top[j]) {
            const uint64_t t = top[j];
            top[j] = code;
            code = t;
          }
      }
      for (int j = 0; j < k; ++j) {
        int64_t chosen = -1;
        if (top[j]) chosen = ((nb - 1 - (int)(top[j] & 0xffffffffu)) + offset_blocks) % nb;
        bridge_original_blocks[(int64_t)q * k + j] = chosen;
      }
    }
    // bridge bits: directed (query -> key) or reciprocal (both directions, bridge_k.py:44)
    for (int64_t idx = 0; idx < (int64_t)nb * k; ++idx) {
      const int64_t key = bridge_original_blocks[idx];
      if (key < 0) continue;
      const int pq = (int)original_to_physical[idx / k];
      const int pk = (int)original_to_physical[key];
      if (pq >= gb) bits[(int64_t)(pq - gb) * words + pk / 32] |= 1u << (pk % 32);
      if (bridge_mode == 2 && pk >= gb) bits[(int64_t)(pk - gb) * words + pq / 32] |= 1u << (pq % 32);
    }
    return HB_OK;
  });
}

extern "C" int hb_table_bits_host(const int32_t* kv_indices, const int32_t* kv_counts, int32_t rows,
                                  int32_t width, int32_t total_blocks, uint32_t* bits) {
  HB_REQUIRE(kv_indices && kv_counts && bits && rows > 0 && width > 0 && total_blocks > 0,
             "invalid table arguments");
  const int words = (total_blocks + 31) / 32;
  memset(bits, 0, sizeof(uint32_t) * (size_t)rows * words);
  for (int r = 0; r < rows; ++r) {
    const int c = kv_counts[r] < width ? kv_counts[r] : width;
    for (int e = 0; e < c; ++e) {
      const int p = kv_indices[(int64_t)r * width + e];
      if (p < 0 || p >= total_blocks) continue;
      bits[(int64_t)r * words + p / 32] |= 1u << (p % 32);
    }
  }
  return HB_OK;
}

extern "C" int hb_bits_counts_host(const uint32_t* bits, int32_t rows, int32_t total_blocks,
                                   int32_t key_block_size, int32_t* counts, int32_t* paired_counts,
                                   int32_t* max_counts) {
  HB_REQUIRE(bits && max_counts && rows > 0 && total_blocks > 0, "invalid bitmap arguments");
  HB_REQUIRE(key_block_size == 64 || key_block_size == 128, "key_block_size must be 64 or 128");
  HB_REQUIRE(!paired_counts || rows % 2 == 0, "paired rows need an even row count");
  const int words = (total_blocks + 31) / 32;
  max_counts[0] = max_counts[1] = 0;
  if (counts)
    for (int r = 0; r < rows; ++r) {
      counts[r] = count_row(bits, words, total_blocks, 0, 1, r);
      if (counts[r] > max_counts[0]) max_counts[0] = counts[r];
    }
  if (paired_counts)
    for (int r = 0; r < rows / 2; ++r) {
      paired_counts[r] = count_row(bits, words, total_blocks, 1, key_block_size / 64, r);
      if (paired_counts[r] > max_counts[1]) max_counts[1] = paired_counts[r];
    }
  return HB_OK;
}

extern "C" int hb_bits_emit_host(const uint32_t* bits, int32_t rows, int32_t total_blocks,
                                 int32_t key_block_size, int32_t* ids, int32_t width,
                                 int32_t* paired_ids, int32_t* paired_flags, int32_t paired_width) {
  HB_REQUIRE(bits && rows > 0 && total_blocks > 0, "invalid bitmap arguments");
  HB_REQUIRE(key_block_size == 64 || key_block_size == 128, "key_block_size must be 64 or 128");
  const int words = (total_blocks + 31) / 32;
  if (ids) {
    HB_REQUIRE(width > 0, "width must be positive");
    for (int r = 0; r < rows; ++r)
      emit_row(bits, words, total_blocks, 0, 1, r, ids + (int64_t)r * width, nullptr, width);
  }
  if (paired_ids) {
    HB_REQUIRE(paired_flags && paired_width > 0 && rows % 2 == 0, "paired output needs flags and width");
    for (int r = 0; r < rows / 2; ++r)
      emit_row(bits, words, total_blocks, 1, key_block_size / 64, r,
               paired_ids + (int64_t)r * paired_width, paired_flags + (int64_t)r * paired_width,
               paired_width);
  }
  return HB_OK;
}

extern "C" int hb_pair_rows_host(const int32_t* kv_indices, const int32_t* kv_counts, int32_t rows,
                                 int32_t width, int32_t total_blocks, int32_t key_block_size,
                                 int32_t* paired_ids, int32_t* paired_flags, int32_t* paired_counts,
                                 int32_t paired_width, int32_t* overflow) {
  HB_REQUIRE(kv_indices && kv_counts && paired_ids && paired_flags && paired_counts,
             "null pointer argument");
  HB_REQUIRE(rows > 0, "rows must be positive (got %d)", rows);
  HB_REQUIRE(width > 0 && paired_width > 0, "table widths must be positive");
  HB_REQUIRE(total_blocks > 0 && total_blocks <= PAIR_MAX_BLOCKS,
             "total_blocks must be in [1, %d] (got %d)", PAIR_MAX_BLOCKS, total_blocks);
  HB_REQUIRE(key_block_size == 64 || key_block_size == 128, "key_block_size must be 64 or 128");
  // an odd row count is paired from the end: paired row 0 holds an empty half 0 and row 0
  const int lead = rows & 1, prows = (rows + 1) / 2, ratio = key_block_size / 64;
  // two bitmap rows, one word beyond the last key block (pair_flag reads up to bit T)
  const int words = total_blocks / 32 + 2;
  return guarded([&] {
    std::vector<uint32_t> bm(2 * (size_t)words);
    for (int pr = 0; pr < prows; ++pr) {
      std::fill(bm.begin(), bm.end(), 0u);
      for (int h = 0; h < 2; ++h) {
        const int row = 2 * pr + h - lead;
        if (row < 0) continue;
        int c = kv_counts[row] < width ? kv_counts[row] : width;
        if (c < 0) c = 0;
        for (int e = 0; e < c; ++e) {
          const int p = kv_indices[(int64_t)row * width + e];
          if (p >= 0 && p < total_blocks) bm[(size_t)h * words + p / 32] |= 1u << (p % 32);
        }
      }
      const int n = emit_row(bm.data(), words, total_blocks, 1, ratio, 0,
                             paired_ids + (int64_t)pr * paired_width,
                             paired_flags + (int64_t)pr * paired_width, paired_width);
      paired_counts[pr] = n < paired_width ? n : paired_width;
      if (n > paired_width && overflow) *overflow |= 1;
    }
    return HB_OK;
  });
}
