// Status codes and last-error text shared by every C-ABI entry point.
#pragma once

#include <hip/hip_runtime.h>

#define EZ_OK 0
#define EZ_EINVAL (-22)

namespace ez {
int set_error(int code, const char* fmt, ...);
// Map the launch status of the kernels just enqueued to a return code.
int launch_status(const char* what);
// Compute units of the current device (256 on MI355X).
int num_cus();
}  // namespace ez

#define EZ_REQUIRE(cond, ...)                                      \
  do {                                                             \
    if (!(cond)) return ::ez::set_error(EZ_EINVAL, __VA_ARGS__);   \
  } while (0)
