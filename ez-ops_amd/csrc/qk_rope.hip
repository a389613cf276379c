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

// Sequence and cache position of row b (a decode batch row or a prefill token).
__device__ __forceinline__ void row_position(const QkRopeArgs& a, int64_t b, int64_t& seq, int64_t& pos) {
  seq = b;
  if (a.cu) {  // prefill row: find its sequence (binary search over cu)
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
}

// Element offset of cache row (seq, kv head, pos): contiguous or paged.
__device__ __forceinline__ int64_t cache_offset(const QkRopeArgs& a, int64_t seq, int64_t kvh, int64_t pos) {
  if (a.block_table) {
    const int sh = __builtin_ctz(unsigned(a.page_size));
    const int64_t pg = pos >> sh;
    const uint32_t id = min(uint32_t(a.block_table[seq * a.bt_stride + pg]), uint32_t(a.num_pages - 1));
    return ((int64_t(id) * a.Hkv + kvh) * a.page_size + (pos - (pg << sh))) * a.D;
  }
  return ((seq * a.Hkv + kvh) * a.S + pos) * a.D;
}

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
  int64_t seq, pos;
  row_position(a, b, seq, pos);
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
  const int64_t crow_off = is_q ? 0 : cache_offset(a, seq, kvh, pos);
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

// D in {64, 128, 256}: D/8 lanes per head, each lane holding 8 consecutive
// elements (16-byte loads and stores), 64/(D/8) heads per wave.  RoPE pairs
// (i, i + D/2) sit in lanes l and l ^ (D/16) of the head's lane group, so the
// partner half arrives by one lane exchange.  Same fp32 operations and
// rounding as the kernel above.
template <int D>
__global__ __launch_bounds__(256) void qk_norm_rope_vec_kernel(QkRopeArgs a) {
  EZ_PROF_WAVE(kProfQkRope);
  constexpr int LPH = D / 8;
  constexpr int HPW = kWave / LPH;
  const int lane = threadIdx.x & (kWave - 1);
  const int l = lane % LPH;
  const int64_t h0 = a.q_out ? 0 : a.H;  // without q_out, the kv heads only
  const int64_t heads = a.H + a.Hkv - h0;
  const int64_t hid = (int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6)) * HPW + lane / LPH;
  const bool live = hid < a.B * heads;
  const int64_t hc = live ? hid : 0;  // dead lanes still join the exchanges, on a valid row
  const int64_t b = hc / heads, h = h0 + hc % heads;
  const bool is_q = h < a.H;
  const int64_t kvh = h - a.H;
  int64_t seq, pos;
  row_position(a, b, seq, pos);
  const bool ok = live && pos >= 0 && pos < a.S;
  const int64_t posc = ok ? pos : 0;
  const uint16_t* src = (is_q ? a.q + b * a.q_bs + h * D : a.k + b * a.k_bs + kvh * D) + 8 * l;
  const uint16_t* w = is_q ? a.qw : a.kw;

  float x[8];
  unpack8(*reinterpret_cast<const uint4*>(src), x);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
#pragma unroll
  for (int o = LPH / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
  const float r = rsqrtf(ss / float(D) + a.eps);
  float y[8], wf[8];
  if (w) unpack8(*reinterpret_cast<const uint4*>(w + 8 * l), wf);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    y[e] = __fmul_rn(x[e], r);
    if (w) y[e] = __fmul_rn(y[e], wf[e]);
  }
  float o[8];
  if (a.cos) {
    float c[8], sn[8], yp[8];
    unpack8(*reinterpret_cast<const uint4*>(a.cos + posc * D + 8 * l), c);
    unpack8(*reinterpret_cast<const uint4*>(a.sin + posc * D + 8 * l), sn);
    const bool first = l < LPH / 2;  // this lane holds y1 (i < D/2), its partner y2
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      yp[e] = __shfl_xor(y[e], LPH / 2, kWave);
      o[e] = __fadd_rn(__fmul_rn(y[e], c[e]), __fmul_rn(first ? -yp[e] : yp[e], sn[e]));
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = y[e];
  }
  if (!ok) return;
  const uint4 packed = make_uint4(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]), pack_bf2(o[4], o[5]), pack_bf2(o[6], o[7]));
  if (is_q) {
    *reinterpret_cast<uint4*>(a.q_out + (b * a.H + h) * D + 8 * l) = packed;
  } else {
    const int64_t off = cache_offset(a, seq, kvh, pos) + 8 * l;
    *reinterpret_cast<uint4*>(a.Kc + off) = packed;
    if (a.k_out) *reinterpret_cast<uint4*>(a.k_out + (b * a.Hkv + kvh) * D + 8 * l) = packed;
    *reinterpret_cast<uint4*>(a.Vc + off) = *reinterpret_cast<const uint4*>(a.v + b * a.v_bs + kvh * D + 8 * l);
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

namespace {
bool vec_form(const QkRopeArgs& a) {
  return (a.D == 64 || a.D == 128 || a.D == 256) && a.q_bs % 8 == 0 && a.k_bs % 8 == 0 && a.v_bs % 8 == 0 &&
         aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.Kc) && aligned16(a.Vc) &&
         (!a.q_out || aligned16(a.q_out)) && (!a.k_out || aligned16(a.k_out)) && (!a.qw || aligned16(a.qw)) &&
         (!a.kw || aligned16(a.kw)) && (!a.cos || aligned16(a.cos)) && (!a.sin || aligned16(a.sin));
}
}  // namespace

int check_qk_norm_rope(const QkRopeArgs& a) {
  EZ_REQUIRE(a.q && a.k && a.v && a.Kc && a.Vc, "qk_norm_rope: null pointer");
  EZ_REQUIRE(a.B >= 1 && a.H >= 1 && a.Hkv >= 1 && a.S >= 1, "qk_norm_rope: bad shape");
  EZ_REQUIRE(a.D >= 2 && a.D <= 2 * kMaxPairsPerLane * kWave && a.D % 2 == 0,
             "qk_norm_rope: head_dim must be even and <= %d", 2 * kMaxPairsPerLane * kWave);
  EZ_REQUIRE((a.cos == nullptr) == (a.sin == nullptr), "qk_norm_rope: cos and sin go together");
  EZ_REQUIRE(!a.cu || a.nseq >= 1, "qk_norm_rope: prefill rows need nseq >= 1");
  EZ_REQUIRE(!a.block_table || (a.page_size >= 1 && (a.page_size & (a.page_size - 1)) == 0 && a.num_pages >= 1 &&
                                a.S == a.bt_stride * a.page_size),
             "qk_norm_rope: paged cache needs a power-of-two page_size and S = max_pages * page_size");
  EZ_REQUIRE(a.q_out || vec_form(a), "qk_norm_rope: the k / v-only form needs head_dim 64, 128 or 256 and 16-byte rows");
  return EZ_OK;
}

int launch_qk_norm_rope(const QkRopeArgs& a, hipStream_t s) {
  const int rc = check_qk_norm_rope(a);
  if (rc != EZ_OK) return rc;
  const int64_t heads = a.B * (a.q_out ? a.H + a.Hkv : a.Hkv);
  const bool vec = vec_form(a);
  if (vec) {
    const int64_t hpw = kWave / (a.D / 8);
    const unsigned blocks = unsigned((heads + 4 * hpw - 1) / (4 * hpw));
    if (a.D == 64) hipLaunchKernelGGL(qk_norm_rope_vec_kernel<64>, dim3(blocks), dim3(256), 0, s, a);
    else if (a.D == 128) hipLaunchKernelGGL(qk_norm_rope_vec_kernel<128>, dim3(blocks), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(qk_norm_rope_vec_kernel<256>, dim3(blocks), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(unsigned((heads + 3) / 4)), dim3(256), 0, s, a);
  }
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
  EZ_REQUIRE(q_out, "qk_norm_rope: null pointer");
  EZ_REQUIRE(H >= 1 && Hkv >= 1, "qk_norm_rope: num_heads and num_kv_heads must be >= 1");
  EZ_REQUIRE(H % Hkv == 0, "qk_norm_rope: num_heads must be divisible by num_kv_heads");
  EZ_REQUIRE(positions || (position + pos_offset >= 0 && position + pos_offset < S),
             "qk_norm_rope: position out of range");
  return ez::launch_qk_norm_rope(a, stream);
}
