// Per-head RMSNorm + rotary embedding + joint [text | image] BNHD write for FLUX attention inputs.
//
// Replaces, in one pass, what the FLUX attention processor does between the Q/K projections and
// the attention call (reference hilberta/flux_adapter.py:283-295, which runs diffusers'
// attn.norm_q / norm_k / norm_added_q / norm_added_k, torch.cat of text and image tokens and
// apply_rotary_emb):
//   y   = bf16(x * rsqrt(mean(x^2) + eps))     (fp32 statistics, per token and head; when asked)
//   y   = bf16(y * w)                          (per-dimension weight, when given)
//   out = bf16(y * cos + rot(y) * sin)         (fp32, rot(y)[2i] = -y[2i+1], rot(y)[2i+1] = y[2i];
//                                               when cos/sin are given)
// Text tokens [0, T) come from one source tensor and weight, image tokens [T, N) from another;
// with neither step asked for, the kernel is the [text; image] concatenation into BNHD (V).
// The rotary products and sum are not contracted into FMAs, so that step rounds exactly as the
// unfused fp32 formula does.
// Sixteen lanes own one (token, head) row of 128 elements, 8 per lane (one 16-byte load and
// store each), and reduce the sum of squares with cross-lane swaps.  HBM-bound: 2 bytes read and
// 2 written per element, the fp32 cos/sin rows are shared by all heads of a token.
#include "common.h"
#include "../../include/hilberta_hip.h"

namespace hb {
namespace {

struct PrepArgs {
  const uint16_t* src[2];   // text, image
  int64_t src_b[2], src_n[2];
  const uint16_t* w[2];     // per-dimension weights or null
  const float* cos;         // [tokens, head_dim] or null
  const float* sin;
  uint16_t* out;
  int64_t out_b, out_n;
  int32_t batch, text, tokens, heads, normalize;
  float eps;
};

template <bool F16>
__device__ __forceinline__ float to_f(uint16_t v) {
  if constexpr (F16) return (float)__builtin_bit_cast(_Float16, v);
  else return (float)__builtin_bit_cast(__bf16, v);
}
template <bool F16>
__device__ __forceinline__ uint16_t from_f(float v) {
  if constexpr (F16) return __builtin_bit_cast(uint16_t, (_Float16)v);
  else return __builtin_bit_cast(uint16_t, (__bf16)v);
}

// D = 128: 16 lanes x 8 elements per (token, head) row.
template <bool F16>
__global__ __launch_bounds__(256) void qk_prep_kernel(PrepArgs a) {
#pragma clang fp contract(off)
  constexpr int D = 128;
  const int64_t rows = (int64_t)a.batch * a.tokens * a.heads;
  const int sub = threadIdx.x & 15;
  for (int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4; row < rows;
       row += ((int64_t)gridDim.x * blockDim.x) >> 4) {
    const int h = (int)(row % a.heads);
    const int64_t bt = row / a.heads;
    const int t = (int)(bt % a.tokens);
    const int b = (int)(bt / a.tokens);
    const int part = t < a.text ? 0 : 1;
    const int tr = part ? t - a.text : t;
    const uint16_t* sp = a.src[part] + b * a.src_b[part] + tr * a.src_n[part] + h * D + sub * 8;
    const u32x4 raw = *(const u32x4*)sp;
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = to_f<F16>((uint16_t)(raw[i] & 0xffff));
      x[2 * i + 1] = to_f<F16>((uint16_t)(raw[i] >> 16));
    }
    if (a.normalize) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
      // sum over the 16 lanes of this row
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 16);
      const float r = __builtin_amdgcn_rsqf(ss * (1.f / D) + a.eps);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = to_f<F16>(from_f<F16>(x[i] * r));
      const uint16_t* w = a.w[part];
      if (w) {
        // the normalised value is rounded to the weight type before the weight multiply
        const u32x4 wr = *(const u32x4*)(w + sub * 8);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[2 * i] = to_f<F16>(from_f<F16>(x[2 * i] * to_f<F16>((uint16_t)(wr[i] & 0xffff))));
          x[2 * i + 1] = to_f<F16>(from_f<F16>(x[2 * i + 1] * to_f<F16>((uint16_t)(wr[i] >> 16))));
        }
      }
    }
    u32x4 res;
    if (a.cos) {
      const float* cp = a.cos + (int64_t)t * D + sub * 8;
      const float* sn = a.sin + (int64_t)t * D + sub * 8;
      const f32x4 c0 = *(const f32x4*)cp, c1 = *(const f32x4*)(cp + 4);
      const f32x4 s0 = *(const f32x4*)sn, s1 = *(const f32x4*)(sn + 4);
      const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
      const float s[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = x[2 * i] * c[2 * i] - x[2 * i + 1] * s[2 * i];
        const float o = x[2 * i + 1] * c[2 * i + 1] + x[2 * i] * s[2 * i + 1];
        res[i] = (uint32_t)from_f<F16>(e) | ((uint32_t)from_f<F16>(o) << 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        res[i] = (uint32_t)from_f<F16>(x[2 * i]) | ((uint32_t)from_f<F16>(x[2 * i + 1]) << 16);
    }
    *(u32x4*)(a.out + b * a.out_b + (int64_t)t * a.out_n + h * D + sub * 8) = res;
  }
}

}  // namespace
}  // namespace hb

using namespace hb;

extern "C" int hb_qk_prep(const void* src_text, const void* src_image, int64_t text_batch_stride,
                          int64_t text_row_stride, int64_t image_batch_stride,
                          int64_t image_row_stride, int32_t batch, int32_t text_tokens,
                          int32_t tokens, int32_t heads, int32_t head_dim, int32_t dtype,
                          int32_t normalize, const void* weight_text, const void* weight_image,
                          float eps,
                          const float* cos, const float* sin, void* out, int64_t out_batch_stride,
                          int64_t out_row_stride, hb_stream_t stream) {
  HB_REQUIRE(head_dim == 128, "head_dim must be 128 (got %d)", head_dim);
  HB_REQUIRE(batch > 0 && heads > 0 && tokens > 0 && text_tokens >= 0 && text_tokens <= tokens,
             "batch, heads and tokens must be positive with 0 <= text_tokens <= tokens");
  HB_REQUIRE(dtype == HB_DTYPE_BF16 || dtype == HB_DTYPE_F16, "dtype must be bf16 or fp16");
  HB_REQUIRE(out && (text_tokens == 0 || src_text) && (text_tokens == tokens || src_image),
             "null pointer argument");
  HB_REQUIRE((cos == nullptr) == (sin == nullptr), "cos and sin must be given together");
  HB_REQUIRE(normalize == 0 || normalize == 1, "normalize must be 0 or 1");
  HB_REQUIRE(!normalize || eps > 0.f, "eps must be positive");
  HB_REQUIRE(normalize || (!weight_text && !weight_image), "norm weights need normalize=1");
  const void* ptrs[7] = {src_text, src_image, out, weight_text, weight_image, cos, sin};
  for (int i = 0; i < 7; ++i)
    HB_REQUIRE(((uintptr_t)ptrs[i] & 15) == 0, "every pointer must be 16-byte aligned");
  const int64_t strides[6] = {text_batch_stride, text_row_stride, image_batch_stride,
                              image_row_stride, out_batch_stride, out_row_stride};
  for (int i = 0; i < 6; ++i)
    HB_REQUIRE(strides[i] >= 0 && strides[i] % 8 == 0, "strides must be non-negative multiples of 8");
  PrepArgs a;
  a.src[0] = (const uint16_t*)src_text;
  a.src[1] = (const uint16_t*)src_image;
  a.src_b[0] = text_batch_stride;
  a.src_n[0] = text_row_stride;
  a.src_b[1] = image_batch_stride;
  a.src_n[1] = image_row_stride;
  a.w[0] = (const uint16_t*)weight_text;
  a.w[1] = (const uint16_t*)weight_image;
  a.cos = cos;
  a.sin = sin;
  a.out = (uint16_t*)out;
  a.out_b = out_batch_stride;
  a.out_n = out_row_stride;
  a.batch = batch;
  a.text = text_tokens;
  a.tokens = tokens;
  a.heads = heads;
  a.normalize = normalize;
  a.eps = eps;
  const int64_t threads = (int64_t)batch * tokens * heads * 16;
  int64_t blocks = (threads + 255) / 256;
  const int64_t cap = (int64_t)device_cu_count() * 32;
  if (blocks > cap) blocks = cap;
  if (dtype == HB_DTYPE_F16)
    hipLaunchKernelGGL(qk_prep_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(qk_prep_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, a);
  HB_HIP(hipGetLastError());
  return HB_OK;
}
