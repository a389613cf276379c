// Standalone split-KV GQA decode attention kernel and its launcher.  The
// per-block routine (and its design notes) is in attn_impl.h.
#include "attn_impl.h"
#include "status.h"
#include "../../include/ezops_hip.h"

namespace ez {
namespace {

using attn::AttnWs;
using attn::kMaxSplits;
using attn::kTile;

int num_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  return cus;
}

struct SplitPlan {
  int waves;
  int64_t nsplit;
};

// Splits per (b, kv head), planned on the cache capacity S: enough blocks to
// keep every CU busy, at least one tile per wave at full capacity, and at
// most kMaxSplits partials per merge.
SplitPlan plan_splits(int64_t B, int64_t Hkv, int64_t S, int64_t G) {
  const int64_t units = B * Hkv;
  const int64_t cus = num_cus();
  // 8-wave blocks for few units; group 8 keeps 4 waves (its accumulators need
  // the register budget of one wave per SIMD).
  const int waves = (units * 4 <= cus && G <= 4) ? 8 : 4;
  const int64_t target = waves == 8 ? 2 * cus : 8 * cus;  // blocks in flight
  int64_t ns = (target + units - 1) / units;
  const int64_t max_ns = (S + int64_t(waves) * kTile - 1) / (int64_t(waves) * kTile);
  if (ns > max_ns) ns = max_ns;
  if (ns > kMaxSplits) ns = kMaxSplits;
  if (ns < 1) ns = 1;
  return {waves, ns};
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

#ifndef EZ_ATTN_MERGE_LAST
#define EZ_ATTN_MERGE_LAST 0  // 1: the last block of a unit merges its splits (no combine launch)
#endif
constexpr bool kMergeLast = EZ_ATTN_MERGE_LAST;

template <int D, int G, int W, int QSRC>
__global__ __launch_bounds__(W * kWave) void attn_split_kernel(AttnArgs a, int64_t nsplit, AttnWs ws) {
  attn::attn_block<D, G, W, QSRC, attn::kOutBf16, kMergeLast>(a, blockIdx.x % nsplit, blockIdx.x / nsplit, nsplit,
                                                              ws);
}

// One wave per query head merges that head's split partials.
template <int D>
__global__ __launch_bounds__(kWave) void attn_combine_kernel(AttnArgs a, int64_t nsplit, AttnWs ws) {
  attn::attn_combine<D, attn::kOutBf16>(a, blockIdx.x, nsplit, ws);
}

template <int D, int W, int LAYER>
void launch_dw(const AttnArgs& a, const SplitPlan& pl, const AttnWs& ws, int64_t G, hipStream_t s) {
  const dim3 grid{unsigned(a.B * a.Hkv * pl.nsplit), 1, 1}, block{unsigned(W * kWave), 1, 1};
  switch (G) {
    case 1: hipLaunchKernelGGL((attn_split_kernel<D, 1, W, LAYER>), grid, block, 0, s, a, pl.nsplit, ws); break;
    case 2: hipLaunchKernelGGL((attn_split_kernel<D, 2, W, LAYER>), grid, block, 0, s, a, pl.nsplit, ws); break;
    case 4: hipLaunchKernelGGL((attn_split_kernel<D, 4, W, LAYER>), grid, block, 0, s, a, pl.nsplit, ws); break;
    default: break;  // group 8 launches from launch_d
  }
}

template <int D, int LAYER>
void launch_d(const AttnArgs& a, const SplitPlan& pl, const AttnWs& ws, int64_t G, hipStream_t s) {
  const dim3 block{unsigned(pl.waves * kWave), 1, 1};
  const dim3 grid{unsigned(a.B * a.Hkv * pl.nsplit), 1, 1};
  if (G == 8) {
    hipLaunchKernelGGL((attn_split_kernel<D, 8, 4, LAYER>), grid, block, 0, s, a, pl.nsplit, ws);
  } else if (pl.waves == 8) {
    launch_dw<D, 8, LAYER>(a, pl, ws, G, s);
  } else {
    launch_dw<D, 4, LAYER>(a, pl, ws, G, s);
  }
}

}  // namespace

size_t attn_workspace_size(int64_t B, int64_t H, int64_t Hkv, int64_t S, int64_t D) {
  if (B < 1 || H < 1 || Hkv < 1 || S < 1 || D < 1) return 0;
  const SplitPlan pl = plan_splits(B, Hkv, S, H / Hkv);
  return align256(size_t(B * H * pl.nsplit * D) * 4) + align256(size_t(B * H * pl.nsplit * 2) * 4) +
         align256(size_t(B * Hkv) * 4);
}

int launch_attn(const AttnArgs& a, void* ws, size_t ws_bytes, hipStream_t s) {
  const bool layer = a.Q == nullptr;
  EZ_REQUIRE(a.K && a.V && a.Out && (!layer || a.qkv), "attn_decode: null pointer");
  EZ_REQUIRE(a.B >= 1 && a.H >= 1 && a.Hkv >= 1 && a.S >= 1, "attn_decode: bad shape");
  EZ_REQUIRE(a.H % a.Hkv == 0, "attn_decode: num_heads must be divisible by num_kv_heads");
  const int64_t G = a.H / a.Hkv;
  EZ_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "attn_decode: group size %lld not in {1,2,4,8}", (long long)G);
  EZ_REQUIRE(a.D == 64 || a.D == 128, "attn_decode: head_dim must be 64 or 128");
  EZ_REQUIRE((a.cos == nullptr) == (a.sin == nullptr), "attn_decode: cos and sin go together");
  const SplitPlan pl = plan_splits(a.B, a.Hkv, a.S, G);
  AttnWs w{};
  if (pl.nsplit > 1) {
    EZ_REQUIRE(ws && ws_bytes >= attn_workspace_size(a.B, a.H, a.Hkv, a.S, a.D),
               "attn_decode: workspace too small (%zu < %zu)", ws_bytes,
               attn_workspace_size(a.B, a.H, a.Hkv, a.S, a.D));
    char* p = static_cast<char*>(ws);
    w.opart = reinterpret_cast<float*>(p);
    p += align256(size_t(a.B * a.H * pl.nsplit * a.D) * 4);
    w.ml = reinterpret_cast<float*>(p);
    p += align256(size_t(a.B * a.H * pl.nsplit * 2) * 4);
    w.counters = reinterpret_cast<int*>(p);
  }
  AttnArgs aa = a;
  if (aa.scale <= 0.f) aa.scale = 1.0f / sqrtf(float(a.D));
  if (layer) {
    if (a.D == 64) launch_d<64, attn::kQFromQkvBf16>(aa, pl, w, G, s);
    else launch_d<128, attn::kQFromQkvBf16>(aa, pl, w, G, s);
  } else {
    if (a.D == 64) launch_d<64, attn::kQFromQ>(aa, pl, w, G, s);
    else launch_d<128, attn::kQFromQ>(aa, pl, w, G, s);
  }
  if (pl.nsplit > 1 && !kMergeLast) {
    const dim3 grid{unsigned(a.B * a.H), 1, 1}, block{kWave, 1, 1};
    if (a.D == 64) hipLaunchKernelGGL(attn_combine_kernel<64>, grid, block, 0, s, aa, pl.nsplit, w);
    else hipLaunchKernelGGL(attn_combine_kernel<128>, grid, block, 0, s, aa, pl.nsplit, w);
  }
  return launch_status("attn_decode");
}

}  // namespace ez

extern "C" size_t ezops_attn_decode_workspace_size(int64_t B, int64_t H, int64_t Hkv, int64_t S, int64_t D) {
  return ez::attn_workspace_size(B, H, Hkv, S, D);
}

extern "C" int ezops_attn_decode_bf16(const void* Q, const void* K, const void* V, void* Out, int64_t B,
                                      int64_t H, int64_t Hkv, int64_t S, int64_t D, const int32_t* kv_lens,
                                      float scale, void* ws, size_t ws_bytes, hipStream_t stream) {
  EZ_REQUIRE(Q, "attn_decode: null pointer");
  ez::AttnArgs a{};
  a.Q = static_cast<const uint16_t*>(Q);
  a.K = static_cast<const uint16_t*>(K);
  a.V = static_cast<const uint16_t*>(V);
  a.Out = static_cast<uint16_t*>(Out);
  a.B = B; a.H = H; a.Hkv = Hkv; a.S = S; a.D = D;
  a.kv_lens = kv_lens;
  a.scale = scale;
  return ez::launch_attn(a, ws, ws_bytes, stream);
}
