// Shared helpers for the HilbertA gfx950 kernels: error reporting for the C ABI,
// vector types and small device utilities.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define HB_OK 0
#define HB_EINVAL 1
#define HB_EHIP 2

namespace hb {

// Records a printf-style message retrievable through hb_last_error(); thread-local.
void set_error(const char* fmt, ...);

// Number of compute units on the current device (cached per device).
int device_cu_count();

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// 16-bit float (bf16 or fp16) <-> fp32, round to nearest even.
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
template <bool F16>
__device__ __forceinline__ float round_f(float v) { return to_f<F16>(from_f<F16>(v)); }

// Eight packed 16-bit values <-> fp32.
template <bool F16>
__device__ __forceinline__ void unpack8(const u32x4& raw, float (&x)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = to_f<F16>((uint16_t)(raw[i] & 0xffff));
    x[2 * i + 1] = to_f<F16>((uint16_t)(raw[i] >> 16));
  }
}
template <bool F16>
__device__ __forceinline__ u32x4 pack8(const float (&x)[8]) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r[i] = (uint32_t)from_f<F16>(x[2 * i]) | ((uint32_t)from_f<F16>(x[2 * i + 1]) << 16);
  return r;
}

}  // namespace hb

#define HB_REQUIRE(cond, ...)          \
  do {                                 \
    if (!(cond)) {                     \
      hb::set_error(__VA_ARGS__);      \
      return HB_EINVAL;                \
    }                                  \
  } while (0)

#define HB_HIP(call)                                                              \
  do {                                                                            \
    hipError_t hb_err_ = (call);                                                  \
    if (hb_err_ != hipSuccess) {                                                  \
      hb::set_error("%s failed: %s", #call, hipGetErrorString(hb_err_));          \
      return HB_EHIP;                                                             \
    }                                                                             \
  } while (0)
