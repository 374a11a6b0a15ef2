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
