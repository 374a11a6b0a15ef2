// Device construction of HilbertA block tables (integer-only, deterministic, bit-exact).
//
// Replaces the CPU setup of the reference (hilberta/geometry.py, plan.py:114-212,
// bridge_k.py:10-51, paired_metadata.py:26-51) with gfx950 kernels.  The intermediate form is a
// per-phase adjacency bitmap over physical 64-token blocks, one row of ceil(T/32) words for each
// ordinary query block:
//
//   layout   composite Hilbert order cat(h[n/4:3n/4], n-1-h[n/4:3n/4]), its inverse, the optional
//            shared centre square moved to the global prefix (plan.py:133-150, :186-197)
//   bits     row of ordinary block o = global prefix | ordinary blocks with o's tile label
//            (plan.py:173-183) | bridges: top-K key blocks of each query block ranked by
//            (-score, (key - offset/bs) mod nb), where score counts cross-tile 4-neighbour token
//            pairs between the two blocks in both directions (plan.py:159-172, bridge_k.py:22-43);
//            directed (build_plan) or reciprocal (bridge_k: adj | adj^T, bridge_k.py:44)
//   emit     rows of set bits in ascending order, zero padded to the widest row; paired rows merge
//            query blocks 2r and 2r+1 with flag bit (half + 2*key_half) (paired_metadata.py:38-51)
//
// Integer atomics only (order-independent sums and ORs), so results do not depend on scheduling.
#include "common.h"
#include "tables_common.h"
#include "../../include/hilberta_hip.h"

namespace hb {
namespace {

constexpr int TPB = 256;

__global__ void hilbert_kernel(int g, int64_t* out) {
  const int64_t n = (int64_t)g * g;
  for (int64_t d = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; d < n; d += (int64_t)gridDim.x * blockDim.x)
    out[d] = hilbert_raster(d, g);
}

// original[i] = h[n/4 + i] (i < n/2), n-1-h[n/4 + i - n/2] (i >= n/2); inverse[original[i]] = i.
__global__ void composite_kernel(int g, int64_t* original, int64_t* inverse) {
  const int64_t n = (int64_t)g * g;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t half = n / 2;
    const int64_t src = n / 4 + (i < half ? i : i - half);
    const int64_t h = hilbert_raster(src, g);
    const int64_t tok = i < half ? h : n - 1 - h;
    original[i] = tok;
    inverse[tok] = i;
  }
}

// One workgroup: classify original blocks as shared (inside the centre square) or ordinary, then
// pack them stably: shared blocks first (plan.py:138-150).  status[0] = #shared, [1] = partial,
// [2] cleared for order_check_kernel.
__global__ void __launch_bounds__(1024) pack_blocks_kernel(int g, int bs, int shared,
                                                           const int64_t* original, int text_blocks,
                                                           int64_t* packed, int64_t* to_physical,
                                                           int32_t* status) {
  const int64_t n = (int64_t)g * g;
  const int nb = (int)(n / bs);
  __shared__ int s_total[2];
  __shared__ int s_scan[1024];
  const int t = threadIdx.x;
  const int per = (nb + 1023) / 1024;  // contiguous run of blocks per thread keeps the order stable
  const int lo = min(t * per, nb), hi = min(lo + per, nb);
  const int start = 3 * g / 8, end = 5 * g / 8;
  int my_shared = 0, partial = 0;
  for (int b = lo; b < hi; ++b) {
    int cnt = 0;
    if (shared) {
      for (int j = 0; j < bs; ++j) {
        const int64_t tok = original[(int64_t)b * bs + j];
        const int y = (int)(tok / g), x = (int)(tok % g);
        cnt += (y >= start && y < end && x >= start && x < end);
      }
    }
    if (cnt != 0 && cnt != bs) partial = 1;
    my_shared += (cnt == bs);
  }
  s_scan[t] = my_shared;
  if (t == 0) s_total[1] = 0;
  __syncthreads();
  if (partial) atomicOr(&s_total[1], 1);
  // inclusive scan of shared counts (Hillis-Steele)
  for (int off = 1; off < 1024; off *= 2) {
    const int v = t >= off ? s_scan[t - off] : 0;
    __syncthreads();
    s_scan[t] += v;
    __syncthreads();
  }
  const int n_shared = s_scan[1023];
  int sh_before = s_scan[t] - my_shared;
  int ord_before = lo - sh_before;  // ordinary blocks before this thread's run
  for (int b = lo; b < hi; ++b) {
    int cnt = 0;
    if (shared) {
      for (int j = 0; j < bs; ++j) {
        const int64_t tok = original[(int64_t)b * bs + j];
        const int y = (int)(tok / g), x = (int)(tok % g);
        cnt += (y >= start && y < end && x >= start && x < end);
      }
    }
    int slot;
    if (cnt == bs) slot = sh_before++;
    else slot = n_shared + ord_before++;
    packed[slot] = b;
    to_physical[b] = slot + text_blocks;
  }
  if (t == 0) {
    status[0] = n_shared;
    status[1] = s_total[1];
    status[2] = 0;  // set by order_check_kernel if the image order is no permutation
  }
}

// image_order[j*bs + u] = original[packed[j]*bs + u]; inverse_image_order[image_order[i]] = i
__global__ void image_order_kernel(int64_t n, int bs, const int64_t* original, const int64_t* packed,
                                   int64_t* order, int64_t* inverse_order) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tok = original[packed[i / bs] * bs + i % bs];
    order[i] = tok;
    if (tok >= 0 && tok < n) inverse_order[tok] = i;
  }
}

// status[2] = 1 unless order is a permutation of [0, n) (then inverse_order[order[i]] = i for
// every i; two positions holding one token leave one of them unmatched).
__global__ void order_check_kernel(int64_t n, const int64_t* order, const int64_t* inverse_order,
                                   int32_t* status) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t tok = order[i];
    if (tok < 0 || tok >= n || inverse_order[tok] != i) atomicOr(&status[2], 1);
  }
}

__global__ void zero_kernel(uint32_t* p, int64_t words) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < words; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

// scores[qa*nb + qc] += 1 and [qc*nb + qa] += 1 for every 4-neighbour raster pair (a, c) whose
// tokens carry different tile labels; qa, qc are original block ids (bridge_k.py:22-28).
__global__ void scores_kernel(int g, int bs, int64_t off, int64_t width, const int64_t* inverse,
                              int32_t* scores) {
  const int64_t n = (int64_t)g * g;
  const int nb = (int)(n / bs);
  const int64_t pairs = 2 * (int64_t)g * (g - 1);
  for (int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; p < pairs; p += (int64_t)gridDim.x * blockDim.x) {
    int64_t a, c;
    if (p < (int64_t)g * (g - 1)) {  // horizontal: (y, x) - (y, x+1)
      const int64_t y = p / (g - 1), x = p % (g - 1);
      a = y * g + x;
      c = a + 1;
    } else {  // vertical: (y, x) - (y+1, x)
      const int64_t q = p - (int64_t)g * (g - 1);
      a = q;
      c = q + g;
    }
    const int64_t pa = inverse[a], pc = inverse[c];
    if (tile_label(pa, off, n, width) != tile_label(pc, off, n, width)) {
      const int ba = (int)(pa / bs), bc = (int)(pc / bs);
      atomicAdd(&scores[(int64_t)ba * nb + bc], 1);
      atomicAdd(&scores[(int64_t)bc * nb + ba], 1);
    }
  }
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = __shfl_xor((unsigned)(v & 0xffffffffu), off);
    const uint32_t hi = __shfl_xor((unsigned)(v >> 32), off);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

// One wave per query block q: K rounds of "largest (score, nb-1-rolled) strictly below the last
// pick" give the top-K by (-score, (key - offset_blocks) mod nb) (bridge_k.py:36-40).
__global__ void topk_kernel(int nb, int k, int offset_blocks, const int32_t* scores, int64_t* chosen) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wave >= nb) return;
  const int q = wave;
  uint64_t bound = ~0ull;
  for (int j = 0; j < k; ++j) {
    uint64_t best = 0;
    for (int key = lane; key < nb; key += 64) {
      const int s = scores[(int64_t)q * nb + key];
      if (s <= 0) continue;
      const int rolled = ((key - offset_blocks) % nb + nb) % nb;
      const uint64_t code = ((uint64_t)(uint32_t)s << 32) | (uint32_t)(nb - 1 - rolled);
      if (code < bound && code > best) best = code;
    }
    best = wave_max_u64(best);
    if (lane == 0) {
      if (best) {
        const int rolled = nb - 1 - (int)(best & 0xffffffffu);
        chosen[(int64_t)q * k + j] = (rolled + offset_blocks) % nb;
      } else {
        chosen[(int64_t)q * k + j] = -1;
      }
    }
    bound = best ? best : 0;  // once exhausted every later round finds nothing
  }
}

// Base rows: word w of ordinary row r = globals (physical id < gb) | ordinary blocks whose tile
// label equals that of the row's block (plan.py:173-183).  One lane per (row, key block): a wave
// covers 64 key blocks of one row, ballots its bits and writes the two words (rows are laid out
// in 64-lane spans, the tail lanes of a row's last span idle), so every label is computed once
// per lane instead of 32 times in a serial loop per word.
__global__ void base_bits_kernel(int nq, int words, int T, int gb, int text_blocks, int bs,
                                 int64_t off, int64_t n, int64_t width, const int64_t* packed,
                                 uint32_t* bits) {
  const int spans = (T + 63) / 64;  // 64-lane spans per row
  const int64_t total = (int64_t)nq * spans * 64;
  const int lane = threadIdx.x & 63;
  // every lane of a wave runs the same number of iterations (total is a multiple of 64)
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t span = idx >> 6;
    const int r = (int)(span / spans), sp = (int)(span % spans);
    const int p = sp * 64 + lane;
    bool on = false;
    if (p < gb) {
      on = true;
    } else if (p < T) {
      const int lab = tile_label(packed[gb - text_blocks + r] * bs, off, n, width);
      on = tile_label(packed[p - text_blocks] * bs, off, n, width) == lab;
    }
    const uint64_t m = __ballot(on);
    const int w = sp * 2 + (lane >> 5);
    if ((lane & 31) == 0 && w < words) bits[(int64_t)r * words + w] = (uint32_t)(m >> (lane & 32));
  }
}

// Bridge bits: directed adds (phys q -> phys key) to ordinary rows; reciprocal adds both directions.
__global__ void bridge_bits_kernel(int nb, int k, int words, int gb, int reciprocal,
                                   const int64_t* chosen, const int64_t* to_physical, uint32_t* bits) {
  const int64_t total = (int64_t)nb * k;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t key = chosen[idx];
    if (key < 0) continue;
    const int pq = (int)to_physical[idx / k];
    const int pk = (int)to_physical[key];
    if (pq >= gb) atomicOr(&bits[(int64_t)(pq - gb) * words + pk / 32], 1u << (pk % 32));
    if (reciprocal && pk >= gb) atomicOr(&bits[(int64_t)(pk - gb) * words + pq / 32], 1u << (pq % 32));
  }
}

// Existing unpaired tables -> bits (used to pair arbitrary validated tables).
__global__ void table_bits_kernel(const int32_t* ids, const int32_t* counts, int rows, int width,
                                  int words, int T, uint32_t* bits) {
  const int64_t total = (int64_t)rows * width;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * blockDim.x) {
    const int r = (int)(idx / width), e = (int)(idx % width);
    if (e >= counts[r]) continue;
    const int p = ids[idx];
    if (p < 0 || p >= T) continue;  // tables are validated on the host; never write out of range
    atomicOr(&bits[(int64_t)r * words + p / 32], 1u << (p % 32));
  }
}

// Counts: one wave per row.  mode 0: unpaired rows (popcount); mode 1: paired rows at ratio.
// max_counts[mode] receives the widest row (atomicMax).
__global__ void count_kernel(const uint32_t* bits, int rows_out, int words, int T, int mode, int ratio,
                             int32_t* counts, int32_t* max_counts) {
  const int row = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (row >= rows_out) return;
  int c = 0;
  if (mode == 0) {
    const uint32_t* r = bits + (int64_t)row * words;
    for (int w = lane; w < words; w += 64) c += __popc(r[w]);
  } else {
    const uint32_t* ra = bits + (int64_t)(2 * row) * words;
    const uint32_t* rb = ra + words;
    const int kblocks = (T + ratio - 1) / ratio;
    for (int kb = lane; kb < kblocks; kb += 64) c += pair_flag(ra, rb, kb, ratio) != 0;
  }
  for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off);
  if (lane == 0) {
    counts[row] = c;
    atomicMax(&max_counts[mode], c);
  }
}

// Emit ascending ids (and flags) of each row, zero padded to `width`; one wave per row walking
// 64 key blocks per step with a ballot-based prefix.
__global__ void emit_kernel(const uint32_t* bits, int rows_out, int words, int T, int mode, int ratio,
                            int32_t* ids, int32_t* flags, int width) {
  const int row = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (row >= rows_out) return;
  const uint32_t* ra = bits + (int64_t)(mode ? 2 * row : row) * words;
  const uint32_t* rb = ra + words;
  const int kblocks = mode ? (T + ratio - 1) / ratio : T;
  int base = 0;
  for (int k0 = 0; k0 < kblocks; k0 += 64) {
    const int kb = k0 + lane;
    int flag = 0;
    if (kb < kblocks) {
      if (mode) flag = pair_flag(ra, rb, kb, ratio);
      else flag = (int)((ra[kb / 32] >> (kb % 32)) & 1u);
    }
    const uint64_t ballot = __ballot(flag != 0);
    const int before = __popcll(ballot & ((1ull << lane) - 1ull));
    if (flag && base + before < width) {
      ids[(int64_t)row * width + base + before] = kb;
      if (flags) flags[(int64_t)row * width + base + before] = flag;
    }
    base += __popcll(ballot);
  }
  for (int e = base + lane; e < width; e += 64) {
    ids[(int64_t)row * width + e] = 0;
    if (flags) flags[(int64_t)row * width + e] = 0;
  }
}

int grid_for(int64_t work) {
  int64_t g = (work + TPB - 1) / TPB;
  if (g > 65536) g = 65536;
  return g < 1 ? 1 : (int)g;
}

}  // namespace
}  // namespace hb

using namespace hb;

extern "C" int hb_hilbert_order(int32_t grid_size, int64_t* out, hb_stream_t stream) {
  HB_REQUIRE(grid_size >= 2 && (grid_size & (grid_size - 1)) == 0,
             "Hilbert grid side must be a power of two >= 2");
  HB_REQUIRE(out, "null output");
  const int64_t n = (int64_t)grid_size * grid_size;
  hipLaunchKernelGGL(hilbert_kernel, dim3(grid_for(n)), dim3(TPB), 0, stream, grid_size, out);
  HB_HIP(hipGetLastError());
  return HB_OK;
}

extern "C" int hb_plan_layout(int32_t grid_size, int32_t block_size, int32_t text_tokens,
                              int32_t shared, int64_t* original_order, int64_t* inverse_original,
                              int64_t* image_order, int64_t* inverse_image_order,
                              int64_t* physical_original_blocks, int64_t* original_to_physical,
                              int32_t* status, hb_stream_t stream) {
  HB_REQUIRE(grid_size >= 8 && (grid_size & (grid_size - 1)) == 0,
             "grid_size must be a power of two >= 8");
  HB_REQUIRE(block_size > 0 && text_tokens > 0 && text_tokens % block_size == 0,
             "text prefix must be block aligned");
  const int64_t n = (int64_t)grid_size * grid_size;
  HB_REQUIRE(n % block_size == 0 && n / block_size <= (1 << 20), "image tokens must be whole blocks");
  HB_REQUIRE(original_order && inverse_original && image_order && inverse_image_order &&
                 physical_original_blocks && original_to_physical && status,
             "null output");
  hipLaunchKernelGGL(composite_kernel, dim3(grid_for(n)), dim3(TPB), 0, stream, grid_size,
                     original_order, inverse_original);
  hipLaunchKernelGGL(pack_blocks_kernel, dim3(1), dim3(1024), 0, stream, grid_size, block_size,
                     shared, (const int64_t*)original_order, text_tokens / block_size,
                     physical_original_blocks, original_to_physical, status);
  hipLaunchKernelGGL(image_order_kernel, dim3(grid_for(n)), dim3(TPB), 0, stream, n, block_size,
                     (const int64_t*)original_order, (const int64_t*)physical_original_blocks,
                     image_order, inverse_image_order);
  hipLaunchKernelGGL(order_check_kernel, dim3(grid_for(n)), dim3(TPB), 0, stream, n,
                     (const int64_t*)image_order, (const int64_t*)inverse_image_order, status);
  HB_HIP(hipGetLastError());
  return HB_OK;
}

extern "C" int64_t hb_plan_scratch_bytes(int32_t grid_size, int32_t block_size) {
  if (grid_size <= 0 || block_size <= 0) return -1;
  const int64_t nb = (int64_t)grid_size * grid_size / block_size;
  return nb * nb * 4;
}

extern "C" int hb_plan_phase_bits(const int64_t* inverse_original,
                                  const int64_t* physical_original_blocks,
                                  const int64_t* original_to_physical, int32_t grid_size,
                                  int32_t tile_count, int32_t text_tokens, int32_t block_size,
                                  int32_t shared_blocks, int32_t phase, int32_t bridge_mode,
                                  int32_t k, int32_t* scores, int64_t* bridge_original_blocks,
                                  uint32_t* bits, hb_stream_t stream) {
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
  const int nb = (int)(n / block_size);
  const int text_blocks = text_tokens / block_size;
  const int T = text_blocks + nb;
  const int gb = text_blocks + shared_blocks;
  const int nq = T - gb;
  const int words = (T + 31) / 32;
  const int64_t width = n / tile_count;
  const int64_t off = phase * (width / 4);
  hipLaunchKernelGGL(base_bits_kernel, dim3(grid_for((int64_t)nq * ((T + 63) / 64) * 64)), dim3(TPB), 0, stream, nq,
                     words, T, gb, text_blocks, block_size, off, n, width, physical_original_blocks,
                     bits);
  if (bridge_mode) {
    hipLaunchKernelGGL(zero_kernel, dim3(grid_for((int64_t)nb * nb)), dim3(TPB), 0, stream,
                       (uint32_t*)scores, (int64_t)nb * nb);
    hipLaunchKernelGGL(scores_kernel, dim3(grid_for(2 * n)), dim3(TPB), 0, stream, grid_size,
                       block_size, off, width, inverse_original, scores);
    hipLaunchKernelGGL(topk_kernel, dim3((nb * 64 + TPB - 1) / TPB), dim3(TPB), 0, stream, nb, k,
                       (int)(off / block_size), (const int32_t*)scores, bridge_original_blocks);
    hipLaunchKernelGGL(bridge_bits_kernel, dim3(grid_for((int64_t)nb * k)), dim3(TPB), 0, stream, nb,
                       k, words, gb, bridge_mode == 2, (const int64_t*)bridge_original_blocks,
                       original_to_physical, bits);
  }
  HB_HIP(hipGetLastError());
  return HB_OK;
}

extern "C" int hb_table_bits(const int32_t* kv_indices, const int32_t* kv_counts, int32_t rows,
                             int32_t width, int32_t total_blocks, uint32_t* bits,
                             hb_stream_t stream) {
  HB_REQUIRE(kv_indices && kv_counts && bits && rows > 0 && width > 0 && total_blocks > 0,
             "invalid table arguments");
  const int words = (total_blocks + 31) / 32;
  hipLaunchKernelGGL(zero_kernel, dim3(grid_for((int64_t)rows * words)), dim3(TPB), 0, stream, bits,
                     (int64_t)rows * words);
  hipLaunchKernelGGL(table_bits_kernel, dim3(grid_for((int64_t)rows * width)), dim3(TPB), 0, stream,
                     kv_indices, kv_counts, rows, width, words, total_blocks, bits);
  HB_HIP(hipGetLastError());
  return HB_OK;
}

extern "C" int hb_bits_counts(const uint32_t* bits, int32_t rows, int32_t total_blocks,
                              int32_t key_block_size, int32_t* counts, int32_t* paired_counts,
                              int32_t* max_counts, hb_stream_t stream) {
  HB_REQUIRE(bits && max_counts && rows > 0 && total_blocks > 0, "invalid bitmap arguments");
  HB_REQUIRE(key_block_size == 64 || key_block_size == 128, "key_block_size must be 64 or 128");
  HB_REQUIRE(!paired_counts || rows % 2 == 0, "paired rows need an even row count");
  const int words = (total_blocks + 31) / 32;
  hipLaunchKernelGGL(zero_kernel, dim3(1), dim3(64), 0, stream, (uint32_t*)max_counts, (int64_t)2);
  if (counts)
    hipLaunchKernelGGL(count_kernel, dim3((rows * 64 + TPB - 1) / TPB), dim3(TPB), 0, stream, bits, rows,
                       words, total_blocks, 0, 1, counts, max_counts);
  if (paired_counts)
    hipLaunchKernelGGL(count_kernel, dim3((rows / 2 * 64 + TPB - 1) / TPB), dim3(TPB), 0, stream, bits,
                       rows / 2, words, total_blocks, 1, key_block_size / 64, paired_counts, max_counts);
  HB_HIP(hipGetLastError());
  return HB_OK;
}

extern "C" int hb_bits_emit(const uint32_t* bits, int32_t rows, int32_t total_blocks,
                            int32_t key_block_size, int32_t* ids, int32_t width, int32_t* paired_ids,
                            int32_t* paired_flags, int32_t paired_width, hb_stream_t stream) {
  HB_REQUIRE(bits && rows > 0 && total_blocks > 0, "invalid bitmap arguments");
  HB_REQUIRE(key_block_size == 64 || key_block_size == 128, "key_block_size must be 64 or 128");
  const int words = (total_blocks + 31) / 32;
  if (ids) {
    HB_REQUIRE(width > 0, "width must be positive");
    hipLaunchKernelGGL(emit_kernel, dim3((rows * 64 + TPB - 1) / TPB), dim3(TPB), 0, stream, bits, rows,
                       words, total_blocks, 0, 1, ids, (int32_t*)nullptr, width);
  }
  if (paired_ids) {
    HB_REQUIRE(paired_flags && paired_width > 0 && rows % 2 == 0, "paired output needs flags and width");
    hipLaunchKernelGGL(emit_kernel, dim3((rows / 2 * 64 + TPB - 1) / TPB), dim3(TPB), 0, stream, bits,
                       rows / 2, words, total_blocks, 1, key_block_size / 64, paired_ids, paired_flags,
                       paired_width);
  }
  HB_HIP(hipGetLastError());
  return HB_OK;
}

// Pairs an unpaired table in one launch (pair_metadata, paired_metadata.py:26-51): one wave per
// paired row r builds the key-block bitmaps of rows 2r - lead and 2r + 1 - lead in LDS, then writes
// their union in ascending key-block order with flag bit (half + 2*key_half) set where row `half`
// holds key half `key_half`, zero-pads the row to out_width and stores its count.  lead is 1 for
// an odd row count: paired rows are aligned to the end of the table (as the attention kernel
// aligns them to the end of the sequence), so paired row 0 holds an empty half 0 and row 0 as
// half 1.  Ids outside [0, T) and entries past a row's count (clamped to width) are ignored.  A
// union longer than out_width is cut to out_width entries and sets *overflow (when given) to 1.
// key blocks per row the LDS bitmaps cover (N up to 2^20 tokens; 16 KiB of LDS per workgroup)
constexpr int PAIR_MAX_BLOCKS = 16384;
constexpr int PAIR_WORDS = PAIR_MAX_BLOCKS / 32 + 2;
__global__ __launch_bounds__(TPB) void pair_rows_kernel(const int32_t* ids, const int32_t* counts,
                                                        int prows, int lead, int width, int T,
                                                        int ratio, int out_width, int32_t* out_ids,
                                                        int32_t* out_flags, int32_t* out_counts,
                                                        int32_t* overflow) {
  __shared__ uint32_t bm[TPB / 64][2][PAIR_WORDS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int pr = blockIdx.x * (TPB / 64) + w;
  // only the words this table's key blocks reach (pair_flag reads bit kb * ratio + kh <= T)
  const int nwords = T / 32 + 2;
  for (int i = lane; i < 2 * nwords; i += 64) bm[w][i / nwords][i % nwords] = 0u;
  __syncthreads();
  if (pr < prows) {
    for (int h = 0; h < 2; ++h) {
      const int row = 2 * pr + h - lead;
      if (row < 0) continue;  // the empty half of an odd table's first paired row
      const int c = min(max(counts[row], 0), width);
      const int32_t* rid = ids + (int64_t)row * width;
      for (int e = lane; e < c; e += 64) {
        const int p = rid[e];
        if (p >= 0 && p < T) atomicOr(&bm[w][h][p >> 5], 1u << (p & 31));
      }
    }
  }
  __syncthreads();
  if (pr >= prows) return;
  // pair_flag reads bit kb * ratio + kh <= T, inside the PAIR_WORDS words
  const int nkb = (T + ratio - 1) / ratio;
  int32_t* oid = out_ids + (int64_t)pr * out_width;
  int32_t* ofl = out_flags + (int64_t)pr * out_width;
  int base = 0;
  for (int kb0 = 0; kb0 < nkb; kb0 += 64) {
    const int kb = kb0 + lane;
    const int flag = kb < nkb ? pair_flag(bm[w][0], bm[w][1], kb, ratio) : 0;
    const uint64_t live = __ballot(flag != 0);
    const int pos = base + __popcll(live & ((1ull << lane) - 1));
    if (flag && pos < out_width) {
      oid[pos] = kb;
      ofl[pos] = flag;
    }
    base += __popcll(live);
  }
  const int cnt = min(base, out_width);
  for (int e = cnt + lane; e < out_width; e += 64) {
    oid[e] = 0;
    ofl[e] = 0;
  }
  if (lane == 0) out_counts[pr] = cnt;
  if (lane == 0 && base > out_width && overflow) atomicOr(overflow, 1);
}

extern "C" int hb_pair_rows(const int32_t* kv_indices, const int32_t* kv_counts, int32_t rows,
                            int32_t width, int32_t total_blocks, int32_t key_block_size,
                            int32_t* paired_ids, int32_t* paired_flags, int32_t* paired_counts,
                            int32_t paired_width, int32_t* overflow, hb_stream_t stream) {
  HB_REQUIRE(kv_indices && kv_counts && paired_ids && paired_flags && paired_counts,
             "null pointer argument");
  HB_REQUIRE(rows > 0, "rows must be positive (got %d)", rows);
  HB_REQUIRE(width > 0 && paired_width > 0, "table widths must be positive");
  HB_REQUIRE(total_blocks > 0 && total_blocks <= PAIR_MAX_BLOCKS,
             "total_blocks must be in [1, %d] (got %d)", PAIR_MAX_BLOCKS, total_blocks);
  HB_REQUIRE(key_block_size == 64 || key_block_size == 128, "key_block_size must be 64 or 128");
  const int lead = rows & 1, prows = (rows + 1) / 2, per_block = TPB / 64;
  hipLaunchKernelGGL(pair_rows_kernel, dim3((prows + per_block - 1) / per_block), dim3(TPB), 0,
                     stream, kv_indices, kv_counts, prows, lead, width, total_blocks,
                     key_block_size / 64, paired_width, paired_ids, paired_flags, paired_counts,
                     overflow);
  HB_HIP(hipGetLastError());
  return HB_OK;
}

// Quad rows for the 256-query attention items: one wave per quad row r merges the rows of r's
// group (group 2: paired rows 2r, 2r + 1 with 64-key flags bit half; group 4: unpaired rows
// 4r .. 4r + 3) into a per-key-block flag byte in LDS, bit b set where 64-query block b of the
// quad row (b = 2 * paired row + half, or the unpaired row) sees the key block, then writes the
// union in ascending key-block order, zero padded to out_width, with its count.  The same union
// as pair_metadata (paired_metadata.py:38-51) taken over four query blocks instead of two.  Ids
// outside [0, T) and entries past a row's count (clamped to width) are ignored; a union longer
// than out_width is cut to out_width entries and sets *overflow (when given) to 1.
constexpr int QUAD_MAX_BLOCKS = 2048;            // key blocks per row of a quad table
constexpr int QUAD_WORDS = QUAD_MAX_BLOCKS / 4;  // four flag bytes per word
__global__ __launch_bounds__(TPB) void quad_rows_kernel(const int32_t* ids, const int32_t* flags,
                                                        const int32_t* counts, int qrows, int width,
                                                        int T, int group, int out_width,
                                                        int32_t* out_ids, int32_t* out_flags,
                                                        int32_t* out_counts, int32_t* overflow) {
  __shared__ uint32_t fm[TPB / 64][QUAD_WORDS];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int qr = blockIdx.x * (TPB / 64) + w;
  for (int i = lane; i < QUAD_WORDS; i += 64) fm[w][i] = 0u;
  __syncthreads();
  if (qr < qrows) {
    const int bits = 4 / group;  // flag bits each input row contributes
    for (int j = 0; j < group; ++j) {
      const int row = group * qr + j;
      const int c = min(max(counts[row], 0), width);
      const int32_t* rid = ids + (int64_t)row * width;
      const int32_t* rfl = flags ? flags + (int64_t)row * width : nullptr;
      for (int e = lane; e < c; e += 64) {
        const int p = rid[e];
        if (p < 0 || p >= T) continue;
        const uint32_t f = rfl ? (uint32_t)(rfl[e] & 3) : 1u;
        atomicOr(&fm[w][p >> 2], (f << (bits * j)) << (8 * (p & 3)));
      }
    }
  }
  __syncthreads();
  if (qr >= qrows) return;
  int32_t* oid = out_ids + (int64_t)qr * out_width;
  int32_t* ofl = out_flags + (int64_t)qr * out_width;
  int base = 0;
  for (int kb0 = 0; kb0 < T; kb0 += 64) {
    const int kb = kb0 + lane;
    const int flag = kb < T ? (int)((fm[w][kb >> 2] >> (8 * (kb & 3))) & 15u) : 0;
    const uint64_t live = __ballot(flag != 0);
    const int pos = base + __popcll(live & ((1ull << lane) - 1));
    if (flag && pos < out_width) {
      oid[pos] = kb;
      ofl[pos] = flag;
    }
    base += __popcll(live);
  }
  const int cnt = min(base, out_width);
  for (int e = cnt + lane; e < out_width; e += 64) {
    oid[e] = 0;
    ofl[e] = 0;
  }
  if (lane == 0) out_counts[qr] = cnt;
  if (lane == 0 && base > out_width && overflow) atomicOr(overflow, 1);
}

extern "C" int hb_quad_rows(const int32_t* kv_indices, const int32_t* kv_flags,
                            const int32_t* kv_counts, int32_t rows, int32_t width,
                            int32_t total_blocks, int32_t* quad_ids, int32_t* quad_flags,
                            int32_t* quad_counts, int32_t quad_width, int32_t* overflow,
                            hb_stream_t stream) {
  HB_REQUIRE(kv_indices && kv_counts && quad_ids && quad_flags && quad_counts,
             "null pointer argument");
  const int group = kv_flags ? 2 : 4;
  HB_REQUIRE(rows > 0 && rows % group == 0,
             "rows must be a positive multiple of %d (got %d)", group, rows);
  HB_REQUIRE(width > 0 && quad_width > 0, "table widths must be positive");
  HB_REQUIRE(total_blocks > 0 && total_blocks <= QUAD_MAX_BLOCKS,
             "total_blocks must be in [1, %d] (got %d)", QUAD_MAX_BLOCKS, total_blocks);
  const int qrows = rows / group, per_block = TPB / 64;
  hipLaunchKernelGGL(quad_rows_kernel, dim3((qrows + per_block - 1) / per_block), dim3(TPB), 0,
                     stream, kv_indices, kv_flags, kv_counts, qrows, width, total_blocks, group,
                     quad_width, quad_ids, quad_flags, quad_counts, overflow);
  HB_HIP(hipGetLastError());
  return HB_OK;
}

// ---------------------------------------------------------------------------------------------
// Fused device plan (bridge_k_plan + pair_metadata for all four phases, reciprocal top-K bridges,
// paired_plan_device): six launches and one host read instead of one launch sequence per phase.
// The global-prefix length (the shared blocks of the layout) stays on the device: the phase
// kernels read it from status[0], so nothing synchronises before the table widths are known.
//
//   P1 composite order (grid-wide) + clearing the four phases' score matrices
//   P2 one workgroup: block packing, image order and its inverse, the permutation check, status
//   P3 bridge scores of all four phases (atomic adds per raster 4-neighbour pair) + base rows
//   P4 top-K per (phase, query block), reciprocal bridge bits
//   P5 paired row counts per phase -> status[3 + phase] = widest row
//   -- host reads status (n_shared, partial, bad order, four widths), allocates exact tables --
//   P6 emit the four phases' paired ids / flags / counts at their exact widths
//
// Scratch: 4 nb^2 int32 scores, then 4 x nb x words uint32 bitmaps (rows = ordinary blocks, of
// which the first T - gb are used).  status: int32[7].
namespace {

constexpr int PLAN_PHASES = 4;

__global__ void plan_composite_kernel(int g, int64_t* original, int64_t* inverse, int32_t* scores,
                                      int64_t score_words) {
  const int64_t n = (int64_t)g * g;
  const int64_t total = n > score_words ? n : score_words;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    if (i < n) {
      const int64_t half = n / 2;
      const int64_t src = n / 4 + (i < half ? i : i - half);
      const int64_t h = hilbert_raster(src, g);
      const int64_t tok = i < half ? h : n - 1 - h;
      original[i] = tok;
      inverse[tok] = i;
    }
    if (i < score_words) scores[i] = 0;
  }
}

// The block packing of pack_blocks_kernel, then (same workgroup, after a barrier) the image order,
// its inverse and the permutation check of image_order_kernel / order_check_kernel.
__global__ void __launch_bounds__(1024) plan_pack_kernel(int g, int bs, int shared,
                                                         const int64_t* original, int text_blocks,
                                                         int64_t* packed, int64_t* to_physical,
                                                         int64_t* order, int64_t* inverse_order,
                                                         int32_t* status) {
  const int64_t n = (int64_t)g * g;
  const int nb = (int)(n / bs);
  __shared__ int s_total[3];
  __shared__ int s_scan[1024];
  const int t = threadIdx.x;
  const int per = (nb + 1023) / 1024;
  const int lo = min(t * per, nb), hi = min(lo + per, nb);
  const int start = 3 * g / 8, end = 5 * g / 8;
  auto shared_tokens = [&](int b) {
    int cnt = 0;
    if (shared) {
      for (int j = 0; j < bs; ++j) {
        const int64_t tok = original[(int64_t)b * bs + j];
        const int y = (int)(tok / g), x = (int)(tok % g);
        cnt += (y >= start && y < end && x >= start && x < end);
      }
    }
    return cnt;
  };
  int my_shared = 0, partial = 0;
  for (int b = lo; b < hi; ++b) {
    const int cnt = shared_tokens(b);
    if (cnt != 0 && cnt != bs) partial = 1;
    my_shared += (cnt == bs);
  }
  s_scan[t] = my_shared;
  if (t == 0) {
    s_total[1] = 0;
    s_total[2] = 0;
  }
  __syncthreads();
  if (partial) atomicOr(&s_total[1], 1);
  for (int off = 1; off < 1024; off *= 2) {
    const int v = t >= off ? s_scan[t - off] : 0;
    __syncthreads();
    s_scan[t] += v;
    __syncthreads();
  }
  const int n_shared = s_scan[1023];
  int sh_before = s_scan[t] - my_shared;
  int ord_before = lo - sh_before;
  for (int b = lo; b < hi; ++b) {
    const int slot = shared_tokens(b) == bs ? sh_before++ : n_shared + ord_before++;
    packed[slot] = b;
    to_physical[b] = slot + text_blocks;
  }
  __syncthreads();  // packed complete (global writes of this workgroup are visible after it)
  for (int64_t i = t; i < n; i += 1024) {
    const int64_t tok = original[packed[i / bs] * bs + i % bs];
    order[i] = tok;
    if (tok >= 0 && tok < n) inverse_order[tok] = i;
  }
  __syncthreads();
  int bad = 0;
  for (int64_t i = t; i < n; i += 1024) {
    const int64_t tok = order[i];
    bad |= tok < 0 || tok >= n || inverse_order[tok] != i;
  }
  if (bad) atomicOr(&s_total[2], 1);
  __syncthreads();
  if (t == 0) {
    status[0] = n_shared;
    status[1] = s_total[1];
    status[2] = s_total[2];
  }
  if (t < PLAN_PHASES) status[3 + t] = 0;
}

// Bridge scores of the four phases (blocks [0, score_blocks)) and their base rows (the rest).
__global__ void plan_scores_base_kernel(int g, int bs, int tiles, int text_blocks, int score_blocks,
                                        const int64_t* inverse, const int64_t* packed,
                                        const int32_t* status, int32_t* scores, uint32_t* bits) {
  const int64_t n = (int64_t)g * g;
  const int nb = (int)(n / bs);
  const int T = text_blocks + nb;
  const int words = (T + 31) / 32;
  const int64_t width = n / tiles;
  if ((int)blockIdx.x < score_blocks) {
    const int64_t pairs = 2 * (int64_t)g * (g - 1);
    for (int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; p < pairs; p += (int64_t)score_blocks * blockDim.x) {
      int64_t a, c;
      if (p < (int64_t)g * (g - 1)) {
        const int64_t y = p / (g - 1), x = p % (g - 1);
        a = y * g + x;
        c = a + 1;
      } else {
        const int64_t q = p - (int64_t)g * (g - 1);
        a = q;
        c = q + g;
      }
      const int64_t pa = inverse[a], pc = inverse[c];
      const int ba = (int)(pa / bs), bc = (int)(pc / bs);
      for (int ph = 0; ph < PLAN_PHASES; ++ph) {
        const int64_t off = ph * (width / 4);
        if (tile_label(pa, off, n, width) != tile_label(pc, off, n, width)) {
          int32_t* sc = scores + (int64_t)ph * nb * nb;
          atomicAdd(&sc[(int64_t)ba * nb + bc], 1);
          atomicAdd(&sc[(int64_t)bc * nb + ba], 1);
        }
      }
    }
    return;
  }
  // base rows (plan.py:173-183): one lane per (phase, row, key block), as base_bits_kernel
  const int gb = text_blocks + status[0];
  const int nq = T - gb;
  const int spans = (T + 63) / 64;
  const int64_t total = (int64_t)PLAN_PHASES * nb * spans * 64;
  const int lane = threadIdx.x & 63;
  const int64_t first = (blockIdx.x - score_blocks) * (int64_t)blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)(gridDim.x - score_blocks) * blockDim.x;
  for (int64_t idx = first; idx < total; idx += stride) {
    const int64_t span = idx >> 6;
    const int ph = (int)(span / ((int64_t)nb * spans));
    const int64_t rs = span - (int64_t)ph * nb * spans;
    const int r = (int)(rs / spans), sp = (int)(rs % spans);
    if (r >= nq) continue;  // whole wave: a span belongs to one row
    const int64_t off = ph * (width / 4);
    const int p = sp * 64 + lane;
    bool on = false;
    if (p < gb) {
      on = true;
    } else if (p < T) {
      const int lab = tile_label(packed[gb - text_blocks + r] * bs, off, n, width);
      on = tile_label(packed[p - text_blocks] * bs, off, n, width) == lab;
    }
    const uint64_t m = __ballot(on);
    const int w = sp * 2 + (lane >> 5);
    if ((lane & 31) == 0 && w < words)
      bits[((int64_t)ph * nb + r) * words + w] = (uint32_t)(m >> (lane & 32));
  }
}

// Top-K per (phase, original query block) as topk_kernel, then the reciprocal bridge bits of its
// picks as bridge_bits_kernel (adj | adj^T, bridge_k.py:36-44).
__global__ void plan_topk_bits_kernel(int g, int bs, int tiles, int k, int text_blocks,
                                      const int32_t* scores, const int64_t* to_physical,
                                      const int32_t* status, uint32_t* bits) {
  const int64_t n = (int64_t)g * g;
  const int nb = (int)(n / bs);
  const int T = text_blocks + nb;
  const int words = (T + 31) / 32;
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wave >= PLAN_PHASES * nb) return;
  const int ph = wave / nb, q = wave - ph * nb;
  const int offset_blocks = (int)(ph * (n / tiles / 4) / bs);
  const int32_t* sc = scores + (int64_t)ph * nb * nb + (int64_t)q * nb;
  const int gb = text_blocks + status[0];
  uint32_t* pb = bits + (int64_t)ph * nb * words;
  const int pq = (int)to_physical[q];
  uint64_t bound = ~0ull;
  for (int j = 0; j < k; ++j) {
    uint64_t best = 0;
    for (int key = lane; key < nb; key += 64) {
      const int s = sc[key];
      if (s <= 0) continue;
      const int rolled = ((key - offset_blocks) % nb + nb) % nb;
      const uint64_t code = ((uint64_t)(uint32_t)s << 32) | (uint32_t)(nb - 1 - rolled);
      if (code < bound && code > best) best = code;
    }
    best = wave_max_u64(best);
    if (!best) break;
    if (lane == 0) {
      const int rolled = nb - 1 - (int)(best & 0xffffffffu);
      const int key = (rolled + offset_blocks) % nb;
      const int pk = (int)to_physical[key];
      if (pq >= gb) atomicOr(&pb[(int64_t)(pq - gb) * words + pk / 32], 1u << (pk % 32));
      if (pk >= gb) atomicOr(&pb[(int64_t)(pk - gb) * words + pq / 32], 1u << (pq % 32));
    }
    bound = best;
  }
}

// Paired counts of the four phases: one wave per (phase, paired row); the widest row of each
// phase goes to status[3 + phase].
__global__ void plan_counts_kernel(int nb, int words, int T, int text_blocks, int ratio,
                                   const uint32_t* bits, int32_t* status) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  const int prows_max = nb / 2;
  if (wave >= PLAN_PHASES * prows_max) return;
  const int ph = wave / prows_max, pr = wave - ph * prows_max;
  const int nq = T - text_blocks - status[0];
  if (pr >= nq / 2) return;  // (an odd nq is rejected on the host)
  const uint32_t* ra = bits + ((int64_t)ph * nb + 2 * pr) * words;
  const uint32_t* rb = ra + words;
  const int kblocks = (T + ratio - 1) / ratio;
  int c = 0;
  for (int kb = lane; kb < kblocks; kb += 64) c += pair_flag(ra, rb, kb, ratio) != 0;
  for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off);
  if (lane == 0) atomicMax(&status[3 + ph], c);
}

struct PlanOut {
  int32_t* ids[PLAN_PHASES];
  int32_t* flags[PLAN_PHASES];
  int32_t* counts[PLAN_PHASES];
  int32_t width[PLAN_PHASES];
};

// Paired tables of the four phases at their exact widths (emit_kernel, mode 1).
__global__ void plan_emit_kernel(int nb, int words, int T, int prows, int ratio,
                                 const uint32_t* bits, PlanOut out) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  if (wave >= PLAN_PHASES * prows) return;
  const int ph = wave / prows, row = wave - ph * prows;
  const uint32_t* ra = bits + ((int64_t)ph * nb + 2 * row) * words;
  const uint32_t* rb = ra + words;
  const int kblocks = (T + ratio - 1) / ratio;
  const int width = out.width[ph];
  int32_t* ids = out.ids[ph] + (int64_t)row * width;
  int32_t* fl = out.flags[ph] + (int64_t)row * width;
  int base = 0;
  for (int k0 = 0; k0 < kblocks; k0 += 64) {
    const int kb = k0 + lane;
    const int flag = kb < kblocks ? pair_flag(ra, rb, kb, ratio) : 0;
    const uint64_t ballot = __ballot(flag != 0);
    const int pos = base + __popcll(ballot & ((1ull << lane) - 1ull));
    if (flag && pos < width) {
      ids[pos] = kb;
      fl[pos] = flag;
    }
    base += __popcll(ballot);
  }
  for (int e = base + lane; e < width; e += 64) {
    ids[e] = 0;
    fl[e] = 0;
  }
  if (lane == 0) out.counts[ph][row] = base < width ? base : width;
}

}  // namespace

extern "C" int64_t hb_paired_plan_scratch_bytes(int32_t grid_size, int32_t text_tokens) {
  if (grid_size < 8 || text_tokens < 0 || text_tokens % 64) return -1;
  const int64_t nb = (int64_t)grid_size * grid_size / 64;
  const int64_t words = (text_tokens / 64 + nb + 31) / 32;
  return PLAN_PHASES * (nb * nb * 4 + nb * words * 4);
}

extern "C" int hb_paired_plan_tables(int32_t grid_size, int32_t tile_count, int32_t k,
                                     int32_t text_tokens, int32_t shared, int32_t key_block_size,
                                     int64_t* original_order, int64_t* inverse_original,
                                     int64_t* image_order, int64_t* inverse_image_order,
                                     int64_t* physical_original_blocks,
                                     int64_t* original_to_physical, void* scratch,
                                     int32_t* status, hb_stream_t stream) {
  HB_REQUIRE(grid_size >= 8 && (grid_size & (grid_size - 1)) == 0,
             "grid_size must be a power of two >= 8");
  const int64_t n = (int64_t)grid_size * grid_size;
  HB_REQUIRE(tile_count > 0 && n % tile_count == 0 && (n / tile_count) % (4 * 64) == 0 &&
                 text_tokens > 0 && text_tokens % 64 == 0,
             "Tile quarter offsets and text prefix must be block aligned");
  HB_REQUIRE(k >= 1 && k <= 4, "bridge K must be 1..4");
  HB_REQUIRE(key_block_size == 64 || key_block_size == 128, "key_block_size must be 64 or 128");
  HB_REQUIRE(n / 64 <= (1 << 14), "at most 16384 image blocks");
  HB_REQUIRE(original_order && inverse_original && image_order && inverse_image_order &&
                 physical_original_blocks && original_to_physical && scratch && status,
             "null pointer argument");
  const int bs = 64;
  const int nb = (int)(n / bs), text_blocks = text_tokens / bs, T = text_blocks + nb;
  const int words = (T + 31) / 32;
  int32_t* scores = (int32_t*)scratch;
  uint32_t* bits = (uint32_t*)(scores + (int64_t)PLAN_PHASES * nb * nb);
  const int64_t score_words = (int64_t)PLAN_PHASES * nb * nb;
  hipLaunchKernelGGL(plan_composite_kernel, dim3(grid_for(n > score_words ? n : score_words)),
                     dim3(TPB), 0, stream, grid_size, original_order, inverse_original, scores,
                     score_words);
  hipLaunchKernelGGL(plan_pack_kernel, dim3(1), dim3(1024), 0, stream, grid_size, bs, shared,
                     (const int64_t*)original_order, text_blocks, physical_original_blocks,
                     original_to_physical, image_order, inverse_image_order, status);
  const int score_blocks = grid_for(2 * n);
  const int base_blocks = grid_for((int64_t)PLAN_PHASES * nb * ((T + 63) / 64) * 64);
  hipLaunchKernelGGL(plan_scores_base_kernel, dim3(score_blocks + base_blocks), dim3(TPB), 0,
                     stream, grid_size, bs, tile_count, text_blocks, score_blocks,
                     (const int64_t*)inverse_original, (const int64_t*)physical_original_blocks,
                     (const int32_t*)status, scores, bits);
  hipLaunchKernelGGL(plan_topk_bits_kernel, dim3(((int64_t)PLAN_PHASES * nb * 64 + TPB - 1) / TPB),
                     dim3(TPB), 0, stream, grid_size, bs, tile_count, k, text_blocks,
                     (const int32_t*)scores, (const int64_t*)original_to_physical,
                     (const int32_t*)status, bits);
  hipLaunchKernelGGL(plan_counts_kernel, dim3(((int64_t)PLAN_PHASES * (nb / 2) * 64 + TPB - 1) / TPB),
                     dim3(TPB), 0, stream, nb, words, T, text_blocks, key_block_size / 64,
                     (const uint32_t*)bits, status);
  HB_HIP(hipGetLastError());
  return HB_OK;
}

extern "C" int hb_paired_plan_emit(int32_t grid_size, int32_t text_tokens, int32_t shared_blocks,
                                   int32_t key_block_size, const void* scratch,
                                   int32_t* const* ids, int32_t* const* flags,
                                   int32_t* const* counts, const int32_t* widths,
                                   hb_stream_t stream) {
  HB_REQUIRE(grid_size >= 8 && text_tokens > 0 && text_tokens % 64 == 0, "invalid plan geometry");
  HB_REQUIRE(key_block_size == 64 || key_block_size == 128, "key_block_size must be 64 or 128");
  HB_REQUIRE(scratch && ids && flags && counts && widths, "null pointer argument");
  const int64_t n = (int64_t)grid_size * grid_size;
  const int nb = (int)(n / 64), text_blocks = text_tokens / 64, T = text_blocks + nb;
  HB_REQUIRE(shared_blocks >= 0 && shared_blocks < nb, "shared_blocks out of range");
  const int nq = nb - shared_blocks;
  HB_REQUIRE(nq % 2 == 0, "paired rows need an even number of ordinary blocks");
  PlanOut out;
  for (int p = 0; p < PLAN_PHASES; ++p) {
    HB_REQUIRE(ids[p] && flags[p] && counts[p] && widths[p] > 0, "phase %d: null table or width", p);
    out.ids[p] = ids[p];
    out.flags[p] = flags[p];
    out.counts[p] = counts[p];
    out.width[p] = widths[p];
  }
  const int words = (T + 31) / 32;
  const uint32_t* bits = (const uint32_t*)((const int32_t*)scratch + (int64_t)PLAN_PHASES * nb * nb);
  const int prows = nq / 2;
  hipLaunchKernelGGL(plan_emit_kernel, dim3(((int64_t)PLAN_PHASES * prows * 64 + TPB - 1) / TPB),
                     dim3(TPB), 0, stream, nb, words, T, prows, key_block_size / 64, bits, out);
  HB_HIP(hipGetLastError());
  return HB_OK;
}
