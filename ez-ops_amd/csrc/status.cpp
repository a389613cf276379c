#include "status.h"

#include <cstdarg>
#include <cstdio>

#include "../../include/ezops_hip.h"

namespace ez {

int num_cus() {
  static int cus = 0;  // the first device queried (one GPU per process)
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus = n;
  }
  return cus;
}

namespace {
thread_local char g_err[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(int(e), "%s: launch failed: %s", what, hipGetErrorString(e));
  return EZ_OK;
}
}  // namespace ez

extern "C" const char* ezops_hip_last_error(void) { return ez::g_err; }
extern "C" int ezops_hip_abi_version(void) { return EZOPS_HIP_ABI_VERSION; }
