// Error reporting and device queries shared by every C-ABI entry point.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "../../include/hilberta_hip.h"

namespace hb {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace hb

extern "C" const char* hb_last_error(void) { return hb::g_error; }

extern "C" int hb_version(void) { return HB_ABI_VERSION; }

extern "C" int hb_stream_capture_id(hb_stream_t stream, uint64_t* capture_id) {
  HB_REQUIRE(capture_id, "null pointer argument");
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  HB_HIP(hipStreamGetCaptureInfo(stream, &status, &id));
  *capture_id = status == hipStreamCaptureStatusActive ? (uint64_t)id : 0;
  return HB_OK;
}
