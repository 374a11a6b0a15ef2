// Gated residual update + AdaLN modulation of the FLUX transformer blocks, one pass per row.
//
// The FLUX blocks the reference runs (diffusers 0.36.0 FluxTransformerBlock /
// FluxSingleTransformerBlock / AdaLayerNormContinuous, called through the transformer that
// hilberta/flux_adapter.py wraps) repeat, per token row of `hidden` values:
//   r   = x + gate * y                      (gated residual; torch.addcmul, one rounding)
//   n   = LayerNorm(r)                      (no affine, eps; fp32 statistics, rounded)
//   out = shift + n * (1 + scale)           (1 + scale rounded first, as torch adds in 16 bit)
// as three to five separate passes over the row.  This kernel does it in one: it reads x (and
// y), writes the new residual (optional, may be in place) and the modulated row.  One wave per
// row: 64 lanes x NV 16-byte vectors cover hidden = 512 * NV values, the statistics are two
// wave reductions (mean, then the centred sum of squares) with no LDS.  HBM-bound: 2 bytes per
// value for each of x, y, the residual and the output.
#include "common.h"
#include "../../include/hilberta_hip.h"

namespace hb {
namespace {

struct AdaArgs {
  const uint16_t* x;
  int64_t x_b, x_n;
  const uint16_t* y;  // null: no residual update
  int64_t y_b, y_n;
  const uint16_t* gate;
  int64_t gate_b;
  uint16_t* x_out;    // null: residual not stored
  int64_t xo_b, xo_n;
  const uint16_t* shift;
  const uint16_t* scale;
  int64_t mod_b;
  uint16_t* out;
  int64_t out_b, out_n;
  uint32_t rows_total, rows;
  float inv_hidden, eps;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

template <bool F16, int NV>
__global__ __launch_bounds__(256) void adaln_kernel(AdaArgs a) {
#pragma clang fp contract(off)
  const uint32_t row = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (row >= a.rows_total) return;  // the whole wave leaves together
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t b = row / a.rows;
  const uint32_t i = row - b * a.rows;
  const uint16_t* xp = a.x + b * a.x_b + (int64_t)i * a.x_n + lane * 8;
  float r[NV][8];
  u32x4 raw[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) raw[v] = *(const u32x4*)(xp + v * 512);
  if (a.y) {
    const uint16_t* yp = a.y + b * a.y_b + (int64_t)i * a.y_n + lane * 8;
    const uint16_t* gp = a.gate + b * a.gate_b + lane * 8;
    u32x4 yr[NV], gr[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      yr[v] = *(const u32x4*)(yp + v * 512);
      gr[v] = *(const u32x4*)(gp + v * 512);
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      float xv[8], yv[8], gv[8];
      unpack8<F16>(raw[v], xv);
      unpack8<F16>(yr[v], yv);
      unpack8<F16>(gr[v], gv);
#pragma unroll
      for (int k = 0; k < 8; ++k) r[v][k] = round_f<F16>(xv[k] + gv[k] * yv[k]);
    }
    if (a.x_out) {
      uint16_t* op = a.x_out + b * a.xo_b + (int64_t)i * a.xo_n + lane * 8;
#pragma unroll
      for (int v = 0; v < NV; ++v) *(u32x4*)(op + v * 512) = pack8<F16>(r[v]);
    }
  } else {
#pragma unroll
    for (int v = 0; v < NV; ++v) unpack8<F16>(raw[v], r[v]);
  }
  float s = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int k = 0; k < 8; ++k) s += r[v][k];
  const float mean = wave_sum(s) * a.inv_hidden;
  float q = 0.f;
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float d = r[v][k] - mean;
      q += d * d;
    }
  const float rstd = __builtin_amdgcn_rsqf(wave_sum(q) * a.inv_hidden + a.eps);
  const uint16_t* sp = a.shift + b * a.mod_b + lane * 8;
  const uint16_t* cp = a.scale + b * a.mod_b + lane * 8;
  uint16_t* op = a.out + b * a.out_b + (int64_t)i * a.out_n + lane * 8;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float sh[8], sc[8], o[8];
    unpack8<F16>(*(const u32x4*)(sp + v * 512), sh);
    unpack8<F16>(*(const u32x4*)(cp + v * 512), sc);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float n = round_f<F16>((r[v][k] - mean) * rstd);
      o[k] = sh[k] + n * round_f<F16>(1.f + sc[k]);
    }
    *(u32x4*)(op + v * 512) = pack8<F16>(o);
  }
}

template <bool F16>
int launch(const AdaArgs& a, int nv, hipStream_t st) {
  const dim3 grid((a.rows_total + 3) / 4), block(256);
  switch (nv) {
    case 1: hipLaunchKernelGGL((adaln_kernel<F16, 1>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((adaln_kernel<F16, 2>), grid, block, 0, st, a); break;
    case 3: hipLaunchKernelGGL((adaln_kernel<F16, 3>), grid, block, 0, st, a); break;
    case 4: hipLaunchKernelGGL((adaln_kernel<F16, 4>), grid, block, 0, st, a); break;
    case 6: hipLaunchKernelGGL((adaln_kernel<F16, 6>), grid, block, 0, st, a); break;
    case 8: hipLaunchKernelGGL((adaln_kernel<F16, 8>), grid, block, 0, st, a); break;
    default: set_error("hidden must be 512, 1024, 1536, 2048, 3072 or 4096"); return HB_EINVAL;
  }
  HB_HIP(hipGetLastError());
  return HB_OK;
}

}  // namespace
}  // namespace hb

using namespace hb;

extern "C" int hb_adaln_modulate(int32_t batch, int32_t rows, int32_t hidden, int32_t dtype,
                                 float eps, const void* x, int64_t x_batch_stride,
                                 int64_t x_row_stride, const void* y, int64_t y_batch_stride,
                                 int64_t y_row_stride, const void* gate,
                                 int64_t gate_batch_stride, void* x_out,
                                 int64_t x_out_batch_stride, int64_t x_out_row_stride,
                                 const void* shift, const void* scale, int64_t mod_batch_stride,
                                 void* out, int64_t out_batch_stride, int64_t out_row_stride,
                                 hb_stream_t stream) {
  HB_REQUIRE(batch > 0 && rows > 0, "batch and rows must be positive");
  HB_REQUIRE((int64_t)batch * rows < (1ll << 31), "too many rows for one launch");
  HB_REQUIRE(hidden > 0 && hidden % 512 == 0, "hidden must be a multiple of 512 (got %d)", hidden);
  HB_REQUIRE(dtype == HB_DTYPE_BF16 || dtype == HB_DTYPE_F16, "dtype must be bf16 or fp16");
  HB_REQUIRE(eps > 0.f, "eps must be positive");
  HB_REQUIRE(x && shift && scale && out, "null pointer argument");
  HB_REQUIRE(!y || gate, "a residual update needs its gate");
  HB_REQUIRE(!x_out || y, "x_out is written only with a residual update");
  const void* ptrs[7] = {x, y, gate, x_out, shift, scale, out};
  for (int k = 0; k < 7; ++k)
    HB_REQUIRE(((uintptr_t)ptrs[k] & 15) == 0, "every pointer must be 16-byte aligned");
  const int64_t strides[10] = {x_batch_stride, x_row_stride, y_batch_stride, y_row_stride,
                               gate_batch_stride, x_out_batch_stride, x_out_row_stride,
                               mod_batch_stride, out_batch_stride, out_row_stride};
  for (int k = 0; k < 10; ++k)
    HB_REQUIRE(strides[k] >= 0 && strides[k] % 8 == 0, "strides must be non-negative multiples of 8");
  AdaArgs a;
  a.x = (const uint16_t*)x;
  a.x_b = x_batch_stride;
  a.x_n = x_row_stride;
  a.y = (const uint16_t*)y;
  a.y_b = y_batch_stride;
  a.y_n = y_row_stride;
  a.gate = (const uint16_t*)gate;
  a.gate_b = gate_batch_stride;
  a.x_out = (uint16_t*)x_out;
  a.xo_b = x_out_batch_stride;
  a.xo_n = x_out_row_stride;
  a.shift = (const uint16_t*)shift;
  a.scale = (const uint16_t*)scale;
  a.mod_b = mod_batch_stride;
  a.out = (uint16_t*)out;
  a.out_b = out_batch_stride;
  a.out_n = out_row_stride;
  a.rows_total = (uint32_t)(batch * rows);
  a.rows = (uint32_t)rows;
  a.inv_hidden = 1.f / (float)hidden;
  a.eps = eps;
  const int nv = hidden / 512;
  return dtype == HB_DTYPE_F16 ? launch<true>(a, nv, (hipStream_t)stream)
                               : launch<false>(a, nv, (hipStream_t)stream);
}
