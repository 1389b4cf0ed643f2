// Library-level C ABI: version, device check, thread-local error message.
#include <string.h>

#include "common.hpp"

namespace grpo {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace grpo

extern "C" int grpo_version(void) { return 100; }

extern "C" const char* grpo_last_error(void) { return grpo::g_last_error; }

extern "C" int grpo_init(void) {
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) {
    grpo::set_error("no HIP device available (%s)", hipGetErrorString(e));
    return e != hipSuccess ? (int)e : 100;
  }
  int dev = 0;
  if (int rc = grpo::hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  hipDeviceProp_t prop;
  if (int rc = grpo::hip_check(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties"))
    return rc;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    grpo::set_error("device %d is %s; libgrpo_hip is built for gfx950 only", dev,
                    prop.gcnArchName);
    return GRPO_EUNSUPPORTED;
  }
  return GRPO_OK;
}
