// Prefill (the step before decode): causal GQA flash attention over the KV
// cache for a chunk of new tokens per sequence, and the SwiGLU elementwise
// stage of the batched FFN.
//
// Attention layout on the matrix cores (v_mfma_f32_16x16x32_bf16, lane 16g+i
// holds A[i][8g..8g+7], B[8g..8g+7][i]; C[4g+r][i] in lane 16g+i, reg r):
//   S^T = K Q^T   A = 16 keys x 32 dims of K (LDS, XOR-swizzled rows),
//                 B = Q^T (registers, loaded once), C = S^T[key][query]
//   O^T = V^T P^T A = V^T (LDS, stored transposed), B = P^T straight from the
//                 S^T registers: the k slots 8g..8g+7 of a 32-key step are
//                 keys 4g..4g+3 of its two 16-key tiles, the same slot order
//                 in A and B, so P never leaves the lane.
// Queries sit in the lane column j in both products, so a query's running
// max / sum and its output column share the lane: the only cross-lane step
// is the 4-row reduction over the lanes j, j+16, j+32, j+48.
#include "common.h"
#include "internal.h"
#include "status.h"
#include "../../include/ezops_hip.h"

namespace ez {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kPD = 128;         // head dim
constexpr int kPW = 8;           // waves per block
constexpr int kBK = 64;          // keys per tile
constexpr int kVtStride = kBK + 4;  // transposed V row stride (elements), padded against bank conflicts

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

__device__ __forceinline__ float group4_max(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

// Address of cache row `row` of (sequence b, kv head) for the staging loads.
template <bool PAGED>
__device__ __forceinline__ const uint16_t* cache_row(const PrefillAttnArgs& a, const uint16_t* base, int b, int kvh,
                                                     int64_t row) {
  if constexpr (!PAGED) return base + ((int64_t(b) * a.Hkv + kvh) * a.S + row) * kPD;
  const int sh = __builtin_ctz(unsigned(a.page_size));
  const int64_t pg = row >> sh;
  const uint32_t id = min(uint32_t(a.block_table[int64_t(b) * a.bt_stride + pg]), uint32_t(a.num_pages - 1));
  return base + ((int64_t(id) * a.Hkv + kvh) * a.page_size + (row - (pg << sh))) * kPD;
}

// Block = (query tile, sequence, kv head); wave w serves query head
// kvh*G + w%G, query rows 16*(w/G) .. +15 of the tile (BQ = 16*kPW/G rows).
template <int G, bool PAGED>
__global__ __launch_bounds__(kPW * kWave) void prefill_attn_kernel(PrefillAttnArgs a, int ntq) {
  constexpr int QW = kPW / G;  // 16-row query groups per head
  constexpr int BQ = 16 * QW;
  __shared__ __align__(16) uint16_t Ks[kBK * kPD];        // [key][16B chunk ^ (key & 15)]
  __shared__ __align__(16) uint16_t Vt[kPD * kVtStride];  // [dim][key]

  const int bh = int(a.B * a.Hkv);
  const int qt = ntq - 1 - int(blockIdx.x) / bh;  // longest (last) query tiles first
  const int rem = int(blockIdx.x) % bh;
  const int b = rem / int(a.Hkv), kvh = rem % int(a.Hkv);
  const int64_t q0 = a.cu[b];
  const int64_t qlen0 = int64_t(a.cu[b + 1]) - q0;
  const int64_t past = a.past ? int64_t(a.past[b]) : 0;
  // rows past the cache capacity are neither read nor written
  const int64_t qlen = min(qlen0, a.S - past);
  if (int64_t(qt) * BQ >= qlen) return;

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int g = lane >> 4, j = lane & 15;
  const int hq = kvh * G + wave % G;
  const int64_t qi0 = int64_t(qt) * BQ + (wave / G) * 16;  // first query row (in the sequence) of this wave
  const int64_t qrow = min(qi0 + j, qlen - 1);              // clamped: rows past qlen compute, never store
  const int64_t qpos = past + qrow;                         // its cache position
  const int64_t wave_last = past + min(qi0 + 15, qlen - 1);
  const int64_t kend = past + min(int64_t(qt + 1) * BQ, qlen);  // keys [0, kend) serve this block
  const float sl2 = a.scale * kLog2e;

  bf16x8_t qf[kPD / 32];
  {
    const uint16_t* qp = a.Q + (q0 + qrow) * a.q_rs + int64_t(hq) * kPD;
#pragma unroll
    for (int s = 0; s < kPD / 32; ++s) qf[s] = as_bf16x8(*reinterpret_cast<const uint4*>(qp + 32 * s + 8 * g));
  }

  f32x4_t o[kPD / 16];
#pragma unroll
  for (int d = 0; d < kPD / 16; ++d) o[d] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  // staging assignment: K chunks id = tid + 512c -> key id/16, chunk id%16;
  // V: key pair tid/16, dim chunk tid%16
  uint4 kr[2], vr[2];
  const int vkp = tid >> 4, vcc = tid & 15;
  auto load_tile = [&](int64_t k0) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int id = tid + c * kPW * kWave;
      const int64_t row = min(k0 + (id >> 4), kend - 1);
      kr[c] = *reinterpret_cast<const uint4*>(cache_row<PAGED>(a, a.K, b, kvh, row) + (id & 15) * 8);
      const int64_t vrow = min(k0 + 2 * vkp + c, kend - 1);
      vr[c] = *reinterpret_cast<const uint4*>(cache_row<PAGED>(a, a.V, b, kvh, vrow) + vcc * 8);
    }
  };
  load_tile(0);

  for (int64_t k0 = 0; k0 < kend; k0 += kBK) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int id = tid + c * kPW * kWave;
      const int r = id >> 4, cc = id & 15;
      *reinterpret_cast<uint4*>(&Ks[r * kPD + ((cc ^ (r & 15)) * 8)]) = kr[c];
    }
    {
      const uint32_t* v0 = reinterpret_cast<const uint32_t*>(&vr[0]);
      const uint32_t* v1 = reinterpret_cast<const uint32_t*>(&vr[1]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t lo = (e & 1) ? (v0[e >> 1] >> 16) : (v0[e >> 1] & 0xffffu);
        const uint32_t hi = (e & 1) ? (v1[e >> 1] >> 16) : (v1[e >> 1] & 0xffffu);
        *reinterpret_cast<uint32_t*>(&Vt[(vcc * 8 + e) * kVtStride + 2 * vkp]) = lo | (hi << 16);
      }
    }
    __syncthreads();
    if (k0 + kBK < kend) load_tile(k0 + kBK);  // next tile's global loads overlap this tile's math

    if (k0 <= wave_last) {  // a wave whose queries all precede the tile skips it
      f32x4_t st[kBK / 16];
#pragma unroll
      for (int t = 0; t < kBK / 16; ++t) {
        st[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        const int r = 16 * t + j;  // key row read by this lane (A operand row i = j)
#pragma unroll
        for (int s = 0; s < kPD / 32; ++s) {
          const uint4 kv = *reinterpret_cast<const uint4*>(&Ks[r * kPD + (((4 * s + g) ^ (r & 15)) * 8)]);
          st[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kv), qf[s], st[t], 0, 0, 0);
        }
      }
      // st[t][r] = S[query j][key k0 + 16t + 4g + r]
      float mx = -INFINITY;
#pragma unroll
      for (int t = 0; t < kBK / 16; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t kp = k0 + 16 * t + 4 * g + r;
          const float sv = kp <= qpos ? st[t][r] * sl2 : -INFINITY;
          st[t][r] = sv;
          mx = fmaxf(mx, sv);
        }
      mx = group4_max(mx);
      const float mn = fmaxf(m, mx);  // finite: key 0 is visible to every query
      const float alpha = exp2f(m - mn);
      m = mn;
      l *= alpha;
#pragma unroll
      for (int d = 0; d < kPD / 16; ++d) o[d] *= alpha;
      bf16x8_t pb[kBK / 32];
#pragma unroll
      for (int u = 0; u < kBK / 32; ++u) {
        uint32_t w[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          float p[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[r] = exp2f(st[2 * u + h][r] - mn);
            l += p[r];
          }
          w[2 * h] = pack_bf2(p[0], p[1]);
          w[2 * h + 1] = pack_bf2(p[2], p[3]);
        }
        pb[u] = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
      }
#pragma unroll
      for (int d = 0; d < kPD / 16; ++d) {
        const uint16_t* vrow = &Vt[(16 * d + j) * kVtStride];
#pragma unroll
        for (int u = 0; u < kBK / 32; ++u) {
          const uint2 lo = *reinterpret_cast<const uint2*>(vrow + 32 * u + 4 * g);
          const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 32 * u + 16 + 4 * g);
          o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y)), pb[u],
                                                         o[d], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }

  // l: this lane's share of query j's sum; the four lanes j + 16g add up.
  l = rowgroup_sum<16>(l);
  if (qi0 + j < qlen) {
    const float inv = 1.f / l;
    uint16_t* op = a.Out + (q0 + qi0 + j) * a.o_rs + int64_t(hq) * kPD + 4 * g;
#pragma unroll
    for (int d = 0; d < kPD / 16; ++d) {
      // o[d][r] = O^T[dim 16d + 4g + r][query j]
      *reinterpret_cast<uint2*>(op + 16 * d) =
          make_uint2(pack_bf2(o[d][0] * inv, o[d][1] * inv), pack_bf2(o[d][2] * inv, o[d][3] * inv));
    }
  }
}

// a[t][i] = silu(gu[t][i]) * gu[t][IS + i], bf16 in/out (the batched SwiGLU
// stage between the gate/up and down GEMMs), 8 elements per thread.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* gu, uint16_t* out, int64_t T, int64_t IS) {
  const int64_t n8 = T * IS / 8;
  for (int64_t v = int64_t(blockIdx.x) * 256 + threadIdx.x; v < n8; v += int64_t(gridDim.x) * 256) {
    const int64_t e = v * 8, t = e / IS, i = e - t * IS;
    const uint4 gv = ld16_stream(gu + t * 2 * IS + i), uv = ld16_stream(gu + t * 2 * IS + IS + i);
    float gf[8], uf[8];
    unpack8(gv, gf);
    unpack8(uv, uf);
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // bf16-rounded gate activation, then the product rounded once
      const float a0 = round_bf(silu(gf[2 * k])), a1 = round_bf(silu(gf[2 * k + 1]));
      w[k] = pack_bf2(a0 * uf[2 * k], a1 * uf[2 * k + 1]);
    }
    *reinterpret_cast<uint4*>(out + e) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

}  // namespace

int launch_prefill_attn(const PrefillAttnArgs& a, hipStream_t s) {
  EZ_REQUIRE(a.Q && a.K && a.V && a.Out && a.cu, "prefill_attn: null pointer");
  EZ_REQUIRE(a.B >= 1 && a.H >= 1 && a.Hkv >= 1 && a.S >= 1 && a.max_q >= 0, "prefill_attn: bad shape");
  EZ_REQUIRE(a.D == kPD, "prefill_attn: head_dim must be %d", kPD);
  EZ_REQUIRE(a.H % a.Hkv == 0, "prefill_attn: num_heads must be divisible by num_kv_heads");
  const int64_t G = a.H / a.Hkv;
  EZ_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "prefill_attn: GQA group size must be 1, 2, 4 or 8");
  EZ_REQUIRE(a.q_rs % 8 == 0 && a.o_rs % 4 == 0 && aligned16(a.Q) && aligned16(a.K) && aligned16(a.V),
             "prefill_attn: Q rows and caches must be 16-byte aligned");
  EZ_REQUIRE(!a.block_table || (a.page_size >= 32 && (a.page_size & (a.page_size - 1)) == 0 &&
                                a.S == a.bt_stride * a.page_size && a.num_pages >= 1),
             "prefill_attn: page_size must be a power of two >= 32 and S = max_pages * page_size");
  if (a.max_q == 0) return 0;
  PrefillAttnArgs aa = a;
  if (aa.scale <= 0.f) aa.scale = 1.f / sqrtf(float(kPD));
  const int bq = 16 * kPW / int(G);
  const int ntq = int((a.max_q + bq - 1) / bq);
  const int64_t blocks = int64_t(ntq) * a.B * a.Hkv;
  EZ_REQUIRE(blocks < (int64_t(1) << 31), "prefill_attn: grid too large");
  const dim3 grid{unsigned(blocks)}, block{unsigned(kPW * kWave)};
#define EZ_PF(GG)                                                                                    \
  if (a.block_table) hipLaunchKernelGGL((prefill_attn_kernel<GG, true>), grid, block, 0, s, aa, ntq); \
  else hipLaunchKernelGGL((prefill_attn_kernel<GG, false>), grid, block, 0, s, aa, ntq)
  switch (G) {
    case 1: EZ_PF(1); break;
    case 2: EZ_PF(2); break;
    case 4: EZ_PF(4); break;
    default: EZ_PF(8); break;
  }
#undef EZ_PF
  return launch_status("prefill_attn");
}

int launch_silu_mul(const uint16_t* gu, uint16_t* out, int64_t T, int64_t IS, hipStream_t s) {
  EZ_REQUIRE(gu && out && T >= 1 && IS >= 8 && IS % 8 == 0 && aligned16(gu) && aligned16(out),
             "silu_mul: bad arguments (IS must be a multiple of 8, 16-byte aligned buffers)");
  const int64_t n8 = T * IS / 8;
  const int64_t blocks = std::min<int64_t>((n8 + 255) / 256, 4096);
  hipLaunchKernelGGL(silu_mul_kernel, dim3(unsigned(blocks)), dim3(256), 0, s, gu, out, T, IS);
  return launch_status("silu_mul");
}

}  // namespace ez

extern "C" int ezops_prefill_attn_bf16(const void* Q, const void* K, const void* V, void* Out,
                                       const int32_t* cu_seqlens, const int32_t* past_lens, int64_t B,
                                       int64_t H, int64_t Hkv, int64_t S, int64_t D, int64_t max_q_len,
                                       const int32_t* block_table, int64_t num_pages, int64_t page_size,
                                       float scale, hipStream_t stream) {
  ez::PrefillAttnArgs a{};
  a.Q = static_cast<const uint16_t*>(Q); a.q_rs = H * D;
  a.K = static_cast<const uint16_t*>(K); a.V = static_cast<const uint16_t*>(V);
  a.Out = static_cast<uint16_t*>(Out); a.o_rs = H * D;
  a.cu = cu_seqlens; a.past = past_lens;
  a.B = B; a.H = H; a.Hkv = Hkv; a.S = S; a.D = D; a.max_q = max_q_len;
  a.block_table = block_table;
  if (block_table) {
    EZ_REQUIRE(page_size >= 1 && S % page_size == 0, "prefill_attn: S must be a multiple of page_size");
    a.bt_stride = S / page_size; a.page_size = int(page_size); a.num_pages = num_pages;
  }
  a.scale = scale;
  return ez::launch_prefill_attn(a, stream);
}
