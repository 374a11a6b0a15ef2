// Dense bf16 MFMA peak probe: back-to-back v_mfma_f32_32x32x16_bf16 on every SIMD, so that a
// benchmark can state its attention kernel's MFMA throughput against the rate this GPU sustains
// under the same clock conditions in the same process (the nominal 2.5 PFLOP/s assumes a clock
// the part does not hold under sustained MFMA load).
#include "common.h"
#include "../../include/hilberta_hip.h"

namespace hb {
namespace {

constexpr int PROBE_CHAINS = 4;  // independent accumulators per wave

__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, float* sink) {
  // operands that depend on the lane, so nothing folds; values stay small and finite
  const float x = (float)(threadIdx.x & 7) * 0.125f;
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(x + 0.01f * i);
    b[i] = (__bf16)(0.5f - 0.02f * i);
  }
  f32x16 c[PROBE_CHAINS];
#pragma unroll
  for (int j = 0; j < PROBE_CHAINS; ++j) c[j] = f32x16{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < PROBE_CHAINS; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[j], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < PROBE_CHAINS; ++j) s += c[j][0] + c[j][15];
  // the results reach memory only in a case that never occurs for these operands (keeps the
  // MFMAs live without a store per wave)
  if (s == -1.0f) sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace
}  // namespace hb

extern "C" int hb_mfma_peak_probe(int32_t iterations, int32_t groups, float* sink, int64_t* flops,
                                  hb_stream_t stream) {
  HB_REQUIRE(iterations > 0 && iterations <= (1 << 24), "iterations must be in [1, 2^24]");
  HB_REQUIRE(groups >= 0 && groups <= (1 << 16), "groups must be in [0, 65536]");
  HB_REQUIRE(sink && flops, "null pointer argument");
  const int g = groups > 0 ? groups : 2 * hb::device_cu_count();
  hipLaunchKernelGGL(hb::mfma_peak_kernel, dim3(g), dim3(256), 0, stream, iterations, sink);
  HB_HIP(hipGetLastError());
  // 32 x 32 x 16 multiply-adds per MFMA, 4 waves per workgroup
  *flops = (int64_t)g * 4 * (int64_t)iterations * hb::PROBE_CHAINS * 2 * 32 * 32 * 16;
  return HB_OK;
}
