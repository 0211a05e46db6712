// Library-level entry points of the crbq C ABI.
#include <string.h>

#include "common.h"

extern "C" int crbq_version(void) { return 100; }  // 0.1.0

extern "C" const char* crbq_status_string(int status) {
  switch (status) {
    case CRBQ_OK: return "ok";
    case CRBQ_ERR_ARG: return "invalid argument (size, stride, enum or alignment)";
    case CRBQ_ERR_HIP: return "HIP runtime call failed";
    case CRBQ_ERR_WORKSPACE: return "workspace missing or too small";
    case CRBQ_ERR_TOPK: return "selected index k out of range (block narrower than up_lim)";
    case CRBQ_ERR_TOO_LARGE:
      return "problem larger than the allocation-free entry point's static scratch";
    case CRBQ_ERR_CAPTURE:
      return "first call on this device made under stream capture (make one call outside "
             "capture first)";
    default: return "unknown status";
  }
}

extern "C" int crbq_device_ok(void) {
  int dev = 0;
  CRBQ_HIP(hipGetDevice(&dev));
  hipDeviceProp_t prop;
  CRBQ_HIP(hipGetDeviceProperties(&prop, dev));
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? CRBQ_OK : CRBQ_ERR_ARG;
}
