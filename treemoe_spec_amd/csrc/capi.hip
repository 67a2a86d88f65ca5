// Version and status text of the libtreemoe_amd.so C ABI.
#include <hip/hip_runtime.h>

#include "tm_common.h"

extern "C" int tm_version(void) { return 50000; }

extern "C" int tm_host_device_pointer(void* host, void** device) {
  if (host == nullptr || device == nullptr) return TM_ERR_ARG;
  const hipError_t e = hipHostGetDevicePointer(device, host, 0);
  return e == hipSuccess ? TM_OK : TM_ERR_HIP_BASE + (int)e;
}

extern "C" const char* tm_status_string(int code) {
  switch (code) {
    case TM_OK:
      return "ok";
    case TM_ERR_SHAPE:
      return "a size argument is outside the supported range";
    case TM_ERR_ALIGN:
      return "a pointer or stride is not 16-byte aligned";
    case TM_ERR_ARG:
      return "an enumerated argument has an unknown value";
    default:
      break;
  }
  if (code >= TM_ERR_HIP_BASE) return hipGetErrorString((hipError_t)(code - TM_ERR_HIP_BASE));
  return "unknown status";
}
