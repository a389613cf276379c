// Qwen3 per-head QK RMSNorm + half-split RoPE + KV-cache slot write.
//
// One wave per head (B * (H + Hkv) waves).  Lane l owns the RoPE pairs
// (i, i + D/2) for i = l, l + 64, ..., so the rotation never leaves the lane.
// The fp32 pipeline and its operation order follow the reference
// (ezops/ops/fused_qk_norm_rope.py:138-147): x * rsqrt(mean(x^2) + eps) * w,
// then x * cos + rotate_half(x) * sin, one bf16 rounding.  Products and sums
// use explicit round-to-nearest intrinsics so no FMA contraction changes
// the rounding.
#include "common.h"
#include "internal.h"
#include "prof.h"
#include "status.h"
#include "../../include/ezops_hip.h"

namespace ez {

EZ_PROF_DEFINE(qkrope)
namespace {

constexpr int kMaxPairsPerLane = 4;  // D <= 512

__global__ __launch_bounds__(256) void qk_norm_rope_kernel(QkRopeArgs a) {
  EZ_PROF_WAVE(kProfQkRope);
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t heads = a.H + a.Hkv;
  const int64_t hid = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (hid >= a.B * heads) return;
  const int64_t b = hid / heads, h = hid % heads;
  const bool is_q = h < a.H;
  const int64_t kvh = h - a.H;
  const uint16_t* src = is_q ? a.q + b * a.q_bs + h * a.D : a.k + b * a.k_bs + kvh * a.D;
  const uint16_t* w = is_q ? a.qw : a.kw;
  int64_t seq = b, pos;
  if (a.cu) {  // prefill row: find its sequence (wave-uniform binary search)
    int64_t lo = 0, hi = a.nseq - 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) >> 1;
      if (a.cu[mid] <= b) lo = mid; else hi = mid - 1;
    }
    seq = lo;
    pos = (a.past ? int64_t(a.past[seq]) : 0) + b - a.cu[seq];
  } else {
    pos = (a.positions ? int64_t(a.positions[b]) : a.position) + a.pos_offset;
  }
  const int64_t half = a.D / 2;
  // Positions can come from device memory (per-sequence arrays), so they are
  // range-checked here: an out-of-range position writes nothing.
  if (pos < 0 || pos >= a.S) return;

  float x1[kMaxPairsPerLane], x2[kMaxPairsPerLane];
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < kMaxPairsPerLane; ++t) {
    const int64_t i = lane + int64_t(t) * kWave;
    x1[t] = i < half ? bf2f(src[i]) : 0.f;
    x2[t] = i < half ? bf2f(src[i + half]) : 0.f;
    ss += x1[t] * x1[t] + x2[t] * x2[t];
  }
  const float r = rsqrtf(wave_sum(ss) / float(a.D) + a.eps);

  const uint16_t* crow = a.cos ? a.cos + pos * a.D : nullptr;
  const uint16_t* srow = a.sin ? a.sin + pos * a.D : nullptr;
  // cache row offset (elements) of (seq, kvh, pos)
  int64_t crow_off = 0;
  if (!is_q) {
    if (a.block_table) {
      const int sh = __builtin_ctz(unsigned(a.page_size));
      const int64_t pg = pos >> sh;
      const uint32_t id = min(uint32_t(a.block_table[seq * a.bt_stride + pg]), uint32_t(a.num_pages - 1));
      crow_off = ((int64_t(id) * a.Hkv + kvh) * a.page_size + (pos - (pg << sh))) * a.D;
    } else {
      crow_off = ((seq * a.Hkv + kvh) * a.S + pos) * a.D;
    }
  }
  uint16_t* dst = is_q ? a.q_out + (b * a.H + h) * a.D : a.Kc + crow_off;
  uint16_t* kdst = (!is_q && a.k_out) ? a.k_out + (b * a.Hkv + kvh) * a.D : nullptr;
#pragma unroll
  for (int t = 0; t < kMaxPairsPerLane; ++t) {
    const int64_t i = lane + int64_t(t) * kWave;
    if (i >= half) break;
    float y1 = __fmul_rn(x1[t], r), y2 = __fmul_rn(x2[t], r);
    if (w) {
      y1 = __fmul_rn(y1, bf2f(w[i]));
      y2 = __fmul_rn(y2, bf2f(w[i + half]));
    }
    float o1 = y1, o2 = y2;
    if (crow) {
      o1 = __fadd_rn(__fmul_rn(y1, bf2f(crow[i])), __fmul_rn(-y2, bf2f(srow[i])));
      o2 = __fadd_rn(__fmul_rn(y2, bf2f(crow[i + half])), __fmul_rn(y1, bf2f(srow[i + half])));
    }
    const uint16_t b1 = f2bf(o1), b2 = f2bf(o2);
    dst[i] = b1;
    dst[i + half] = b2;
    if (kdst) {
      kdst[i] = b1;
      kdst[i + half] = b2;
    }
  }
  if (!is_q) {
    const uint16_t* vs = a.v + b * a.v_bs + kvh * a.D;
    uint16_t* vd = a.Vc + crow_off;
    for (int64_t i = lane; i < a.D; i += kWave) vd[i] = vs[i];
  }
}

}  // namespace

int launch_qk_norm_rope(const QkRopeArgs& a, hipStream_t s) {
  EZ_REQUIRE(a.q && a.k && a.v && a.Kc && a.Vc && a.q_out, "qk_norm_rope: null pointer");
  EZ_REQUIRE(a.B >= 1 && a.H >= 1 && a.Hkv >= 1 && a.S >= 1, "qk_norm_rope: bad shape");
  EZ_REQUIRE(a.D >= 2 && a.D <= 2 * kMaxPairsPerLane * kWave && a.D % 2 == 0,
             "qk_norm_rope: head_dim must be even and <= %d", 2 * kMaxPairsPerLane * kWave);
  EZ_REQUIRE((a.cos == nullptr) == (a.sin == nullptr), "qk_norm_rope: cos and sin go together");
  EZ_REQUIRE(!a.cu || a.nseq >= 1, "qk_norm_rope: prefill rows need nseq >= 1");
  EZ_REQUIRE(!a.block_table || (a.page_size >= 1 && (a.page_size & (a.page_size - 1)) == 0 && a.num_pages >= 1 &&
                                a.S == a.bt_stride * a.page_size),
             "qk_norm_rope: paged cache needs a power-of-two page_size and S = max_pages * page_size");
  const int64_t waves = a.B * (a.H + a.Hkv);
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(unsigned((waves + 3) / 4)), dim3(256), 0, s, a);
  return launch_status("qk_norm_rope");
}

}  // namespace ez

extern "C" int ezops_qk_norm_rope_bf16(const void* q, int64_t q_bs, const void* k, int64_t k_bs,
                                       const void* v, int64_t v_bs, const void* qw, const void* kw,
                                       const void* cos, const void* sin, void* Kc, void* Vc,
                                       void* q_out, void* k_out, int64_t B, int64_t H, int64_t Hkv,
                                       int64_t D, int64_t S, int64_t position,
                                       const int32_t* positions, int64_t pos_offset, float eps,
                                       hipStream_t stream) {
  ez::QkRopeArgs a{};
  a.q = static_cast<const uint16_t*>(q); a.q_bs = q_bs;
  a.k = static_cast<const uint16_t*>(k); a.k_bs = k_bs;
  a.v = static_cast<const uint16_t*>(v); a.v_bs = v_bs;
  a.qw = static_cast<const uint16_t*>(qw); a.kw = static_cast<const uint16_t*>(kw);
  a.cos = static_cast<const uint16_t*>(cos); a.sin = static_cast<const uint16_t*>(sin);
  a.Kc = static_cast<uint16_t*>(Kc); a.Vc = static_cast<uint16_t*>(Vc);
  a.q_out = static_cast<uint16_t*>(q_out); a.k_out = static_cast<uint16_t*>(k_out);
  a.B = B; a.H = H; a.Hkv = Hkv; a.D = D; a.S = S;
  a.position = position; a.positions = positions; a.pos_offset = pos_offset;
  a.eps = eps;
  EZ_REQUIRE(H % Hkv == 0, "qk_norm_rope: num_heads must be divisible by num_kv_heads");
  EZ_REQUIRE(positions || (position + pos_offset >= 0 && position + pos_offset < S),
             "qk_norm_rope: position out of range");
  return ez::launch_qk_norm_rope(a, stream);
}
