// Wave-level kernel timelines (the profiling build, -DEZ_PROFILE=1).
//
// Each instrumented kernel opens EZ_PROF_WAVE(kernel id) on entry; when the
// wave leaves the kernel, its lane 0 appends one WaveRecord (begin / end of
// the 100 MHz s_memrealtime clock and where the wave ran: XCC, shader
// engine, CU, SIMD) to a buffer of the translation unit.  Without
// EZ_PROFILE the macros expand to nothing, so the production library is
// unchanged.  The buffers are read and cleared through
// ezops_profile_read / ezops_profile_reset.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#ifndef EZ_PROFILE
#define EZ_PROFILE 0
#endif

namespace ez {

struct WaveRecord {
  unsigned long long t0, t1;  // s_memrealtime ticks (10 ns)
  uint32_t hw_id;             // HW_ID register: wave slot, SIMD, CU, SH, SE, ...
  uint32_t xcc_id;            // XCC_ID register (bits 3:0)
  uint16_t kernel, wave;      // ProfKernel id, wave index in the block
  uint32_t block;             // blockIdx.x
};
static_assert(sizeof(WaveRecord) == 32, "record layout is part of the profiling ABI");

enum ProfKernel : uint16_t {
  kProfGemvRows = 1, kProfGemvValu, kProfLinearScalar, kProfLinearMfma, kProfAttnSplit, kProfAttnCombine,
  kProfPrefillAttn, kProfSiluMul, kProfQkRope, kProfRmsnormF32, kProfRmsnormBf16, kProfSoftmax, kProfSum, kProfGemm,
};

// Records are appended per CU (region = XCC, SE, SH, CU from the hardware
// registers), each region with its own counter, so no counter is shared by
// more than the waves of one CU.
constexpr uint32_t kProfRegions = 8 * 8 * 2 * 16;
constexpr uint32_t kProfRegionCap = 512;
constexpr uint32_t kProfCap = kProfRegions * kProfRegionCap;  // records per translation unit (32 MiB)

// Host side: every translation unit with a buffer registers its reader.
using ProfRead = int (*)(WaveRecord* host, size_t cap, size_t* n);
using ProfReset = int (*)();
bool prof_register(ProfRead read, ProfReset reset);

#if EZ_PROFILE
struct ProfScope {
  unsigned long long t0;
  WaveRecord* buf;
  unsigned long long* count;
  uint16_t kid;
  __device__ ProfScope(uint16_t k, WaveRecord* b, unsigned long long* c) : buf(b), count(c), kid(k) {
    t0 = __builtin_amdgcn_s_memrealtime();
  }
  __device__ ~ProfScope() {
    const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
    if ((threadIdx.x & 63) == 0) {
      WaveRecord r;
      r.t0 = t0;
      r.t1 = t1;
      r.hw_id = __builtin_amdgcn_s_getreg((31 << 11) | 4);   // HW_ID, 32 bits
      r.xcc_id = __builtin_amdgcn_s_getreg((15 << 11) | 20); // XCC_ID, 16 bits
      r.kernel = kid;
      r.wave = uint16_t(threadIdx.x >> 6);
      r.block = blockIdx.x;
      const uint32_t region = ((((r.xcc_id & 7u) * 8u + ((r.hw_id >> 13) & 7u)) * 2u + ((r.hw_id >> 12) & 1u)) * 16u) +
                              ((r.hw_id >> 8) & 15u);
      const unsigned long long i = atomicAdd(count + region, 1ull);  // vector atomic from one lane
      if (i < kProfRegionCap) buf[region * kProfRegionCap + i] = r;
    }
  }
};

// One buffer per translation unit (kernels of different .hip files are
// separate code objects) plus its host reader, registered at load time.
#define EZ_PROF_DEFINE(tu)                                                                               \
  __device__ ::ez::WaveRecord ez_prof_buf_##tu[::ez::kProfCap];                                          \
  __device__ unsigned long long ez_prof_n_##tu[::ez::kProfRegions];                                      \
  namespace {                                                                                            \
  __device__ __forceinline__ ::ez::WaveRecord* ez_prof_buf() { return ez_prof_buf_##tu; }                \
  __device__ __forceinline__ unsigned long long* ez_prof_count() { return ez_prof_n_##tu; }              \
  int ez_prof_read_##tu(::ez::WaveRecord* host, size_t cap, size_t* n) {                                 \
    std::vector<unsigned long long> cnt(::ez::kProfRegions);                                             \
    std::vector<::ez::WaveRecord> all(::ez::kProfCap);                                                   \
    if (hipMemcpyFromSymbol(cnt.data(), HIP_SYMBOL(ez_prof_n_##tu), cnt.size() * sizeof(cnt[0]), 0,      \
                            hipMemcpyDeviceToHost) != hipSuccess ||                                      \
        hipMemcpyFromSymbol(all.data(), HIP_SYMBOL(ez_prof_buf_##tu), all.size() * sizeof(all[0]), 0,    \
                            hipMemcpyDeviceToHost) != hipSuccess)                                        \
      return -1;                                                                                         \
    size_t k = 0;                                                                                        \
    bool lost = false;                                                                                   \
    for (uint32_t g = 0; g < ::ez::kProfRegions; ++g) {                                                  \
      const size_t m = cnt[g] < ::ez::kProfRegionCap ? size_t(cnt[g]) : size_t(::ez::kProfRegionCap);    \
      lost |= cnt[g] > ::ez::kProfRegionCap;                                                             \
      for (size_t i = 0; i < m && k < cap; ++i) {                                                        \
        if (host) host[k] = all[size_t(g) * ::ez::kProfRegionCap + i];                                   \
        ++k;                                                                                             \
      }                                                                                                  \
    }                                                                                                    \
    *n = k;                                                                                              \
    return lost ? 1 : 0;                                                                                 \
  }                                                                                                      \
  int ez_prof_reset_##tu() {                                                                             \
    const std::vector<unsigned long long> z(::ez::kProfRegions, 0ull);                                   \
    return hipMemcpyToSymbol(HIP_SYMBOL(ez_prof_n_##tu), z.data(), z.size() * sizeof(z[0]), 0,           \
                             hipMemcpyHostToDevice) == hipSuccess                                        \
               ? 0                                                                                       \
               : -1;                                                                                     \
  }                                                                                                      \
  const bool ez_prof_registered_##tu = ::ez::prof_register(&ez_prof_read_##tu, &ez_prof_reset_##tu);     \
  }
#define EZ_PROF_WAVE(kid) ::ez::ProfScope ez_prof_scope_(kid, ez_prof_buf(), ez_prof_count())
#else
#define EZ_PROF_DEFINE(tu)
#define EZ_PROF_WAVE(kid) \
  do {                    \
  } while (0)
#endif

}  // namespace ez
