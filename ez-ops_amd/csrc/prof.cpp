// Host side of the wave-level timelines: each instrumented translation unit
// registers a reader for its record buffer (profiling build only; the
// production build registers none and the entry points report that).
#include <hip/hip_runtime.h>

#include <utility>
#include <vector>

#include "prof.h"
#include "status.h"
#include "../../include/ezops_hip.h"

namespace ez {
namespace {
std::vector<std::pair<ProfRead, ProfReset>>& registry() {
  static std::vector<std::pair<ProfRead, ProfReset>> r;
  return r;
}
}  // namespace

bool prof_register(ProfRead read, ProfReset reset) {
  registry().emplace_back(read, reset);
  return true;
}
}  // namespace ez

extern "C" int64_t ezops_profile_read(void* records, int64_t capacity) {
  auto& reg = ez::registry();
  if (reg.empty())
    return ez::set_error(EZOPS_ENOSYS, "profiling is not compiled in (build the library with -DEZ_PROFILE=1)");
  EZ_REQUIRE(capacity >= 0 && (records || capacity == 0), "profile_read: bad buffer");
  if (hipDeviceSynchronize() != hipSuccess) return ez::launch_status("profile_read");
  auto* out = static_cast<ez::WaveRecord*>(records);
  size_t total = 0;
  for (auto& e : reg) {
    size_t n = 0;
    const int rc = e.first(out ? out + total : nullptr, size_t(capacity) - total, &n);
    if (rc < 0) return ez::set_error(EZ_EINVAL, "profile_read: copying a record buffer failed");
    total += n;
  }
  return int64_t(total);
}

extern "C" int ezops_profile_reset(void) {
  auto& reg = ez::registry();
  if (reg.empty())
    return ez::set_error(EZOPS_ENOSYS, "profiling is not compiled in (build the library with -DEZ_PROFILE=1)");
  if (hipDeviceSynchronize() != hipSuccess) return ez::launch_status("profile_reset");
  for (auto& e : reg)
    if (e.second() != 0) return ez::set_error(EZ_EINVAL, "profile_reset: clearing a record buffer failed");
  return 0;
}
