// Token-dimension gather for the persistent Hilbert layout (permute / unpermute).
//
// Replaces the torch index_select calls of the reference at transformer entry and exit
// (hilberta/flux_adapter.py:209-212, :243) and around sampling (sampling_layout.py:96-97, :110):
//   dst[o, i, :] = src[o, index[i], :]   for o < outer, i < rows
// Each row is `row_bytes` contiguous bytes.  The copy moves the widest vector (16/8/4/2/1 bytes)
// that every pointer, stride and the row size allow; consecutive threads walk consecutive vectors
// of one destination row, so both the gathered reads and the writes are coalesced.  This is an
// HBM-bound byte move: 2 * outer * rows * row_bytes plus the index reads per call.
#include "common.h"
#include "../../include/hilberta_hip.h"

namespace hb {
namespace {

template <int V>
struct Vec;
template <> struct Vec<16> { typedef u32x4 T; };
template <> struct Vec<8> { typedef u32x2 T; };
template <> struct Vec<4> { typedef uint32_t T; };
template <> struct Vec<2> { typedef uint16_t T; };
template <> struct Vec<1> { typedef uint8_t T; };

// I is the index type of the flat thread walk: 32-bit when the walk fits (cheap division).
template <int V, typename I>
__global__ __launch_bounds__(256) void gather_rows_kernel(const char* __restrict__ src, char* __restrict__ dst,
                                   const int64_t* __restrict__ index, I rows, I outer,
                                   int64_t src_outer, int64_t dst_outer, int64_t src_row,
                                   int64_t dst_row, I vec_per_row, int64_t src_rows,
                                   int32_t* error) {
  typedef typename Vec<V>::T T;
  const I total = outer * rows * vec_per_row;
  for (I t = blockIdx.x * (I)blockDim.x + threadIdx.x; t < total; t += (I)gridDim.x * blockDim.x) {
    const I row = t / vec_per_row;
    const I v = t - row * vec_per_row;
    const I o = row / rows;
    const I r = row - o * rows;
    const int64_t s = index[r];
    if (s < 0 || s >= src_rows) {  // never read out of bounds; report instead
      if (error) atomicOr(error, 1);
      continue;
    }
    const T val = *(const T*)(src + o * src_outer + s * src_row + v * V);
    *(T*)(dst + o * dst_outer + r * dst_row + v * V) = val;
  }
}

template <int V>
void launch_gather(const void* src, void* dst, const int64_t* index, int64_t rows, int64_t outer,
                   int64_t so, int64_t dso, int64_t sr, int64_t dr, int64_t row_bytes,
                   int64_t src_rows, int32_t* error, hipStream_t stream) {
  const int64_t vpr = row_bytes / V;
  const int64_t total = outer * rows * vpr;
  // One vector per thread and one pass for every size up to 2^28 vectors: a grid capped at a few
  // workgroups per CU with a grid-stride loop measured 9-11 % slower on 100-400 MB gathers (the
  // last pass leaves most CUs idle); beyond 2^20 workgroups the loop strides.
  int64_t blocks = (total + 255) / 256;
  const int64_t cap = (int64_t)1 << 20;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  if (total + (int64_t)blocks * 256 < (int64_t)0xffffffffu) {
    hipLaunchKernelGGL((gather_rows_kernel<V, uint32_t>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       (const char*)src, (char*)dst, index, (uint32_t)rows, (uint32_t)outer, so, dso,
                       sr, dr, (uint32_t)vpr, src_rows, error);
  } else {
    hipLaunchKernelGGL((gather_rows_kernel<V, uint64_t>), dim3((unsigned)blocks), dim3(256), 0, stream,
                       (const char*)src, (char*)dst, index, (uint64_t)rows, (uint64_t)outer, so, dso,
                       sr, dr, (uint64_t)vpr, src_rows, error);
  }
}

}  // namespace
}  // namespace hb

extern "C" int hb_gather_rows(const void* src, void* dst, const int64_t* index, int64_t rows, int64_t outer, int64_t src_outer_stride,
                              int64_t dst_outer_stride, int64_t src_row_stride,
                              int64_t dst_row_stride, int64_t row_bytes, int64_t src_rows,
                              int32_t* error, hb_stream_t stream) {
  HB_REQUIRE(src && dst && index, "null pointer argument");
  HB_REQUIRE(rows >= 0 && outer >= 0 && row_bytes > 0 && src_rows >= 0, "negative sizes");
  if (rows == 0 || outer == 0) return HB_OK;
  const int64_t vals[7] = {(int64_t)(uintptr_t)src, (int64_t)(uintptr_t)dst, src_outer_stride,
                           dst_outer_stride, src_row_stride, dst_row_stride, row_bytes};
  int width = 16;
  for (int i = 0; i < 7; ++i)
    while (width > 1 && vals[i] % width) width >>= 1;
  switch (width) {
    case 16: hb::launch_gather<16>(src, dst, index, rows, outer, src_outer_stride, dst_outer_stride, src_row_stride, dst_row_stride, row_bytes, src_rows, error, stream); break;
    case 8: hb::launch_gather<8>(src, dst, index, rows, outer, src_outer_stride, dst_outer_stride, src_row_stride, dst_row_stride, row_bytes, src_rows, error, stream); break;
    case 4: hb::launch_gather<4>(src, dst, index, rows, outer, src_outer_stride, dst_outer_stride, src_row_stride, dst_row_stride, row_bytes, src_rows, error, stream); break;
    case 2: hb::launch_gather<2>(src, dst, index, rows, outer, src_outer_stride, dst_outer_stride, src_row_stride, dst_row_stride, row_bytes, src_rows, error, stream); break;
    default: hb::launch_gather<1>(src, dst, index, rows, outer, src_outer_stride, dst_outer_stride, src_row_stride, dst_row_stride, row_bytes, src_rows, error, stream); break;
  }
  HB_HIP(hipGetLastError());
  return HB_OK;
}
