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
// One launch may prepare two planes (Q and K, adjacent column ranges of a fused projection),
// which share the index arithmetic and the cos/sin loads.
// The rotary products and sum are not contracted into FMAs, so that step rounds exactly as the
// unfused fp32 formula does.
// Sixteen lanes own a (token, head) row of 128 elements, 8 per lane (one 16-byte load and store
// per plane and head), and reduce the sum of squares with cross-lane swaps; a group takes up to
// four heads of one token so the fp32 cos/sin row is loaded once for them.  HBM-bound: 2 bytes
// read and 2 written per element.
#include "common.h"
#include "../../include/hilberta_hip.h"

namespace hb {
namespace {

struct PrepArgs {
  const uint16_t* src[2];   // text, image
  int64_t src_b[2], src_n[2];
  int64_t src_p;            // element offset between the planes of a source row (Q -> K)
  const uint16_t* w[2][2];  // [plane][text, image] per-dimension weights or null
  const float* cos;         // [tokens, head_dim] or null
  const float* sin;
  uint16_t* out;
  int64_t out_p, out_b, out_n;
  uint32_t threads, text, tokens, heads;
  int32_t normalize;
  float eps;
};

// D = 128: 16 lanes x 8 elements per (token, head) row.  A 16-lane group handles HG heads of one
// token and PLANES tensors (Q, or Q and K): all HG * PLANES loads are issued first, and the fp32
// cos/sin values of the token are loaded once for the HG heads.  One group per (token, head
// group), no grid-stride loop (the launch covers every group).
template <bool F16, int PLANES, int HG>
__global__ __launch_bounds__(256) void qk_prep_kernel(PrepArgs a) {
#pragma clang fp contract(off)
  constexpr int D = 128;
  const uint32_t e = blockIdx.x * 256u + threadIdx.x;
  if (e >= a.threads) return;  // threads is a multiple of 16: whole groups leave together
  const uint32_t sub = e & 15;
  const uint32_t grp = e >> 4;
  const uint32_t groups_per_token = a.heads / HG;
  const uint32_t bt = grp / groups_per_token;
  const uint32_t col = (grp - bt * groups_per_token) * (HG * D) + sub * 8;
  const uint32_t b = bt / a.tokens;
  const uint32_t t = bt - b * a.tokens;
  const int part = t < a.text ? 0 : 1;
  const uint32_t tr = part ? t - a.text : t;
  const uint16_t* sp = a.src[part] + b * a.src_b[part] + (int64_t)tr * a.src_n[part] + col;
  u32x4 raw[HG][PLANES];
#pragma unroll
  for (int k = 0; k < HG; ++k)
#pragma unroll
    for (int p = 0; p < PLANES; ++p) raw[k][p] = *(const u32x4*)(sp + k * D + p * a.src_p);
  float c[8], s[8];
  if (a.cos) {
    const float* cp = a.cos + (int64_t)t * D + sub * 8;
    const float* sn = a.sin + (int64_t)t * D + sub * 8;
    const f32x4 c0 = *(const f32x4*)cp, c1 = *(const f32x4*)(cp + 4);
    const f32x4 s0 = *(const f32x4*)sn, s1 = *(const f32x4*)(sn + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      c[i] = c0[i];
      c[4 + i] = c1[i];
      s[i] = s0[i];
      s[4 + i] = s1[i];
    }
  }
  float wv[PLANES][8];
  if (a.normalize) {
#pragma unroll
    for (int p = 0; p < PLANES; ++p) {
      const uint16_t* w = a.w[p][part];
      if (w) unpack8<F16>(*(const u32x4*)(w + sub * 8), wv[p]);
    }
  }
  uint16_t* op = a.out + b * a.out_b + (int64_t)t * a.out_n + col;
#pragma unroll
  for (int k = 0; k < HG; ++k)
#pragma unroll
    for (int p = 0; p < PLANES; ++p) {
      float x[8];
      unpack8<F16>(raw[k][p], x);
      if (a.normalize) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
        // sum over the 16 lanes of this row
#pragma unroll
        for (int m = 8; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 16);
        const float r = __builtin_amdgcn_rsqf(ss * (1.f / D) + a.eps);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = round_f<F16>(x[i] * r);
        if (a.w[p][part]) {
          // the normalised value is rounded to the weight type before the weight multiply
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = round_f<F16>(x[i] * wv[p][i]);
        }
      }
      u32x4 res;
      if (a.cos) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ev = x[2 * i] * c[2 * i] - x[2 * i + 1] * s[2 * i];
          const float od = x[2 * i + 1] * c[2 * i + 1] + x[2 * i] * s[2 * i + 1];
          res[i] = (uint32_t)from_f<F16>(ev) | ((uint32_t)from_f<F16>(od) << 16);
        }
      } else {
        res = pack8<F16>(x);
      }
      *(u32x4*)(op + k * D + p * a.out_p) = res;
    }
}

template <bool F16, int PLANES>
void launch_planes(const PrepArgs& a0, int heads, hipStream_t st) {
  PrepArgs a = a0;
  const int hg = heads % 4 == 0 ? 4 : heads % 2 == 0 ? 2 : 1;
  a.threads = a0.threads / hg;
  const dim3 grid((a.threads + 255) / 256), block(256);
  if (hg == 4) hipLaunchKernelGGL((qk_prep_kernel<F16, PLANES, 4>), grid, block, 0, st, a);
  else if (hg == 2) hipLaunchKernelGGL((qk_prep_kernel<F16, PLANES, 2>), grid, block, 0, st, a);
  else hipLaunchKernelGGL((qk_prep_kernel<F16, PLANES, 1>), grid, block, 0, st, a);
}

}  // namespace
}  // namespace hb

using namespace hb;

extern "C" int hb_qk_prep(const void* src_text, const void* src_image, int64_t text_batch_stride,
                          int64_t text_row_stride, int64_t image_batch_stride,
                          int64_t image_row_stride, int32_t planes, int64_t src_plane_stride,
                          int32_t batch, int32_t text_tokens, int32_t tokens, int32_t heads,
                          int32_t head_dim, int32_t dtype, int32_t normalize,
                          const void* const* weights, float eps, const float* cos,
                          const float* sin, void* out, int64_t out_plane_stride,
                          int64_t out_batch_stride, int64_t out_row_stride, hb_stream_t stream) {
  HB_REQUIRE(head_dim == 128, "head_dim must be 128 (got %d)", head_dim);
  HB_REQUIRE(planes == 1 || planes == 2, "planes must be 1 or 2");
  HB_REQUIRE(batch > 0 && heads > 0 && tokens > 0 && text_tokens >= 0 && text_tokens <= tokens,
             "batch, heads and tokens must be positive with 0 <= text_tokens <= tokens");
  HB_REQUIRE((int64_t)batch * tokens * heads * 16 < (1ll << 32), "too many rows for one launch");
  HB_REQUIRE(dtype == HB_DTYPE_BF16 || dtype == HB_DTYPE_F16, "dtype must be bf16 or fp16");
  HB_REQUIRE(out && (text_tokens == 0 || src_text) && (text_tokens == tokens || src_image),
             "null pointer argument");
  HB_REQUIRE((cos == nullptr) == (sin == nullptr), "cos and sin must be given together");
  HB_REQUIRE(normalize == 0 || normalize == 1, "normalize must be 0 or 1");
  HB_REQUIRE(!normalize || eps > 0.f, "eps must be positive");
  const void* w[4] = {nullptr, nullptr, nullptr, nullptr};
  if (weights)
    for (int i = 0; i < 2 * planes; ++i) w[i] = weights[i];
  HB_REQUIRE(normalize || (!w[0] && !w[1] && !w[2] && !w[3]), "norm weights need normalize=1");
  const void* ptrs[9] = {src_text, src_image, out, w[0], w[1], w[2], w[3], cos, sin};
  for (int i = 0; i < 9; ++i)
    HB_REQUIRE(((uintptr_t)ptrs[i] & 15) == 0, "every pointer must be 16-byte aligned");
  const int64_t strides[8] = {text_batch_stride, text_row_stride, image_batch_stride,
                              image_row_stride, out_batch_stride, out_row_stride,
                              src_plane_stride, out_plane_stride};
  for (int i = 0; i < 8; ++i)
    HB_REQUIRE(strides[i] >= 0 && strides[i] % 8 == 0, "strides must be non-negative multiples of 8");
  PrepArgs a;
  a.src[0] = (const uint16_t*)src_text;
  a.src[1] = (const uint16_t*)src_image;
  a.src_b[0] = text_batch_stride;
  a.src_n[0] = text_row_stride;
  a.src_b[1] = image_batch_stride;
  a.src_n[1] = image_row_stride;
  a.src_p = src_plane_stride;
  for (int p = 0; p < 2; ++p)
    for (int part = 0; part < 2; ++part) a.w[p][part] = (const uint16_t*)w[2 * p + part];
  a.cos = cos;
  a.sin = sin;
  a.out = (uint16_t*)out;
  a.out_p = out_plane_stride;
  a.out_b = out_batch_stride;
  a.out_n = out_row_stride;
  a.threads = (uint32_t)((int64_t)batch * tokens * heads * 16);
  a.text = (uint32_t)text_tokens;
  a.tokens = (uint32_t)tokens;
  a.heads = (uint32_t)heads;
  a.normalize = normalize;
  a.eps = eps;
  const hipStream_t st = (hipStream_t)stream;
  if (dtype == HB_DTYPE_F16) {
    if (planes == 2) launch_planes<true, 2>(a, heads, st);
    else launch_planes<true, 1>(a, heads, st);
  } else {
    if (planes == 2) launch_planes<false, 2>(a, heads, st);
    else launch_planes<false, 1>(a, heads, st);
  }
  HB_HIP(hipGetLastError());
  return HB_OK;
}
