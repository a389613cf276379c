// Split-KV GQA decode attention for gfx950, with an optional fused Qwen3
// prologue (q/k RMSNorm + RoPE + KV-cache write of the decoded token).
//
// Work unit = (sequence b, kv head).  A block of W waves serves one unit
// split; its G = H / Hkv query heads share every K/V byte it loads, so K/V
// cross HBM once per GQA group.  The 32-position tiles of a sequence are
// dealt round-robin: wave w of split s takes tiles s*W + w,
// s*W + w + nsplit*W, ...  The split count is planned on the host's bound
// Lh of the live lengths (the capacity S when no bound is given); the
// lengths themselves are read on the device.
//
// Per wave and tile:
//   * scores S[h, p] = q_h . k_p on MFMA (v_mfma_f32_16x16x32_bf16): A = the
//     G query rows (zero-padded to 16), B = 16 positions of K per sub-tile;
//     a lane loads 16-byte pieces of K rows straight into the B operand
//     (k-slot (lg, e) of step s = head dim 32 s + 8 lg + e, Q uses the same
//     map), so one load instruction reads 64 contiguous bytes of 16 rows.
//   * online softmax in the exp2 domain (scale * log2 e folded into S), the
//     running max wave-uniform, row maxima by DPP.
//   * O += P . V on VALU: V rows are read with fully coalesced 16-byte loads
//     (one wave instruction covers 1 KiB of consecutive rows); P goes through
//     a small LDS slice per wave and is read back as broadcasts.
//   * every tile load is unconditional (rows past the live length read a
//     clamp row): the next tile's K is requested right after the MFMAs and
//     its V right after P.V, and each wait covers only the data it needs.
// The first tile is requested before the length arrives (its addresses only
// need Lh), behind a single scalar load of the length.  The W waves merge
// (max, sum, O) through LDS; with more than one split the blocks write fp32
// partials that attn_combine_kernel merges (the kernel boundary orders the
// hand-off; an in-kernel arrival counter measured no faster on MI355X).
#include "common.h"
#include "internal.h"
#include "prof.h"
#include "status.h"
#include "../../include/ezops_hip.h"

#ifndef EZ_ATTN_TARGET4
#define EZ_ATTN_TARGET4 8  // 4-wave blocks planned per CU
#endif
#ifndef EZ_ATTN_TRACE
#define EZ_ATTN_TRACE 0  // timing experiments only: per-wave phase timestamps
#endif

namespace ez {

EZ_PROF_DEFINE(attn)
namespace {

constexpr int kTile = 32;       // positions per wave iteration
constexpr int kMaxSplits = 32;  // split partials the combine holds per lane
constexpr float kLog2e = 1.4426950408889634f;

#if EZ_ATTN_TRACE
__device__ long long ez_attn_trace[65536 * 8];  // [block][wave][8] s_memrealtime stamps
#define EZ_TRACE(k)                                                                                      \
  do {                                                                                                   \
    if (lane == 0) ez_attn_trace[(blockIdx.x * W + wave) * 8 + (k)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define EZ_TRACE(k) \
  do {              \
  } while (0)
#endif

// Where the cache rows of one (sequence, kv head) unit live.  Contiguous:
// one S x D slab.  Paged: page j of the sequence is pool page bt[j], each
// pool page holding [Hkv][P][D]; P is a multiple of the 32-row tile, so a
// tile never crosses a page and one table lookup serves a whole tile.
template <int D, bool PAGED>
struct KvRows {
  const uint16_t* base;   // contiguous: the unit's slab; paged: the pool
  const int32_t* bt;      // paged: the sequence's block-table row
  int64_t head_off;       // paged: kv head offset inside a page (elements)
  int64_t page_elems;     // paged: Hkv * P * D
  int page_shift;         // paged: log2(P)
  uint32_t last_page;     // paged: pool pages - 1 (ids are clamped into the pool)
  int64_t last_entry;     // paged: block-table row length - 1

  // Block-table entry of the page holding row ts, as a vector load (lane 0
  // reads it; odd lanes read the next entry, clamped to the row) so that its
  // wait is ordered with the tile loads rather than the LDS traffic.
  __device__ __forceinline__ int32_t page_id(int64_t ts, int lane) const {
    if constexpr (!PAGED) return 0;
    int64_t e = (ts >> page_shift) + (lane & 1);
    e = e < last_entry ? e : last_entry;
    return bt[e];
  }
  // First row of the tile starting at row ts, given page_id(ts) (any lane's
  // copy from lane 0).
  __device__ __forceinline__ const uint16_t* at(int64_t ts, int32_t id_v) const {
    if constexpr (!PAGED) return base + ts * D;
    const uint32_t id = min(uint32_t(__builtin_amdgcn_readfirstlane(id_v)), last_page);
    return base + int64_t(id) * page_elems + head_off + (ts & ((int64_t(1) << page_shift) - 1)) * D;
  }
  __device__ __forceinline__ const uint16_t* tile(int64_t ts) const {
    if constexpr (!PAGED) return base + ts * D;
    return at(ts, bt[ts >> page_shift]);
  }
};

// First row of the tile holding rows t0 + r clamped to `last` (a clamped
// tile starts at the tile of `last`).
__device__ __forceinline__ int64_t tile_start(int64_t t0, int64_t last) {
  return t0 <= last ? t0 : (last & ~int64_t(kTile - 1));
}

// K tile rows t0 + 16u + li (clamped to `last`) into the MFMA B operand;
// tb is the first row of the tile at ts = tile_start(t0, last).
template <int D, int NSUB>
__device__ __forceinline__ void load_k_tile(const uint16_t* tb, int64_t ts, int64_t t0, int64_t last, int li,
                                            int lg, uint4 (&kf)[NSUB][D / 32]) {
#pragma unroll
  for (int u = 0; u < NSUB; ++u) {
    int64_t p = t0 + 16 * u + li;
    p = p < last ? p : last;
    const uint16_t* row = tb + (p - ts) * D + lg * 8;
#pragma unroll
    for (int s = 0; s < D / 32; ++s) kf[u][s] = ld16_stream(row + 32 * s);
  }
}

// V rows in row layout: lane (dc, rs) reads rows rs, rs + RPI, ... of the
// tile (clamped to `last`), 16 B at column 8*dc.
template <int D, int NPV>
__device__ __forceinline__ void load_v_tile(const uint16_t* tb, int64_t ts, int64_t t0, int64_t last, int dc,
                                            int rs, uint4 (&vf)[NPV]) {
  constexpr int RPI = kWave / (D / 8);
#pragma unroll
  for (int j = 0; j < NPV; ++j) {
    int64_t p = t0 + rs + RPI * j;
    p = p < last ? p : last;
    vf[j] = ld16_stream(tb + (p - ts) * D + dc * 8);
  }
}

// Qwen3 per-head RMSNorm (fp32 statistics, weight) + half-split RoPE of one
// bf16 head at `src`, rounded once to bf16 into `dst`.  One wave; lane l owns
// the pairs (i, i + D/2), i = l, l + 64, ...  Operation order follows the
// reference (ezops/ops/fused_qk_norm_rope.py:138-147).
template <int D>
__device__ __forceinline__ void norm_rope_head(const uint16_t* src, const uint16_t* w, const uint16_t* crow,
                                               const uint16_t* srow, float eps, uint16_t* dst, int lane) {
  constexpr int HALF = D / 2;
  constexpr int NP = (HALF + kWave - 1) / kWave;
  float x1[NP], x2[NP];
  float ss = 0.f;
#pragma unroll
  for (int t = 0; t < NP; ++t) {
    const int i = lane + t * kWave;
    x1[t] = i < HALF ? bf2f(src[i]) : 0.f;
    x2[t] = i < HALF ? bf2f(src[i + HALF]) : 0.f;
    ss += x1[t] * x1[t] + x2[t] * x2[t];
  }
  const float r = rsqrtf(wave_reduce_uniform<false>(ss) / float(D) + eps);
#pragma unroll
  for (int t = 0; t < NP; ++t) {
    const int i = lane + t * kWave;
    if (i >= HALF) break;
    float y1 = __fmul_rn(x1[t], r), y2 = __fmul_rn(x2[t], r);
    if (w) {
      y1 = __fmul_rn(y1, bf2f(w[i]));
      y2 = __fmul_rn(y2, bf2f(w[i + HALF]));
    }
    float o1 = y1, o2 = y2;
    if (crow) {
      o1 = __fadd_rn(__fmul_rn(y1, bf2f(crow[i])), __fmul_rn(-y2, bf2f(srow[i])));
      o2 = __fadd_rn(__fmul_rn(y2, bf2f(crow[i + HALF])), __fmul_rn(y1, bf2f(srow[i + HALF])));
    }
    dst[i] = f2bf(o1);
    dst[i + HALF] = f2bf(o2);
  }
}

// Output element (query head hq = b*H + h, dim d): row-major [B, H*D], or the
// MFMA-packed layout of that matrix when it feeds the layer's batched o_proj.
__device__ __forceinline__ int64_t out_index(const AttnArgs& a, int64_t hq, int d) {
  if (!a.out_packed) return hq * a.D + d;
  const int64_t b = hq / a.H;
  return packed_index(b, (hq - b * a.H) * a.D + d, a.H * a.D);
}

// Longest-first order of ragged batches: blocks are dispatched in index
// order, so rank r of the grid serves the r-th longest sequence (ties by
// index) and the long sequences never start last.  One wave, B <= 64: lane j
// ranks sequence j against all others, the lane holding rank r is found by
// ballot.
__device__ __forceinline__ int rank_to_seq(const int32_t* lens, int B, int r, int lane) {
  const int32_t Lj = lane < B ? lens[lane] : -1;
  int rank = 0;
  for (int j = 0; j < B; ++j) {
    const int32_t Lo = __builtin_amdgcn_readlane(Lj, j);
    rank += (Lo > Lj) || (Lo == Lj && j < lane);
  }
  const uint64_t hit = __ballot(lane < B && rank == r);
  return hit ? __ffsll(static_cast<unsigned long long>(hit)) - 1 : r;
}

// LAYER: q (and the decoded token's k, v) come from the bf16 QKV projection
// row a.qkv + b*a.qkv_bs, columns [q | k | v]; q and k get the per-head
// RMSNorm and RoPE at position kv_len - 1.  The unit's first block writes
// the token's k, v into the cache slot; no block reads that slot: the token
// enters the softmax as a virtual row from LDS (wave 0 of split 0).
//
// PAGED: the cache is a page pool addressed through a.block_table (see KvRows).
template <int D, int G, int W, bool LAYER, bool PAGED>
__global__ __launch_bounds__(W * kWave) void attn_split_kernel(AttnArgs a, int nsplit, float* opart, float* ml) {
  EZ_PROF_WAVE(kProfAttnSplit);
  constexpr int NS = D / 32;         // MFMA k-steps per 16-position sub-tile
  constexpr int CPR = D / 8;         // 16-byte chunks per K/V row
  constexpr int RPI = kWave / CPR;   // rows covered by one wave-wide V load
  constexpr int NSUB = kTile / 16;   // MFMA sub-tiles per tile
  constexpr int NPV = kTile / RPI;   // V rows per lane per tile
  constexpr int GP = G <= 4 ? 4 : 8; // P row stride in LDS (float4 reads)
  static_assert(G <= 8, "group size");

  __shared__ __align__(16) float Ps[W][kTile][GP];
  __shared__ __align__(16) float Os[W][G][D];
  __shared__ float Ms[W][G], Ls[W][G];
  __shared__ __align__(16) uint16_t Qs[LAYER ? G : 1][D];
  __shared__ __align__(16) uint16_t Kn[LAYER ? D : 1], Vn[LAYER ? D : 1];

  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  EZ_TRACE(0);
  const int li = lane & 15, lg = lane >> 4;
  const int dc = lane % CPR, rs = lane / CPR;
  int split, kvh, b, nsb = nsplit;  // nsb: splits of this block's sequence
  if (a.split_chunk > 0) {
    // Ragged batch (B <= 64), splits in proportion to the lengths: sequence
    // j gets ns_j = ceil(len_j / split_chunk) splits per kv head; blocks run
    // longest sequence first, (kv head, split) within; blocks past the
    // active ones leave before loading anything.  Lane j < B holds
    // sequence j's length, rank and first block.
    const int B = int(a.B);
    int32_t Lj = lane < B ? a.kv_lens[lane] : 0;
    Lj = Lj < 0 ? 0 : (int64_t(Lj) > a.Lh ? int32_t(a.Lh) : Lj);
    int rank = 0;
    for (int m = 0; m < B; ++m) {
      const int32_t Lo = __builtin_amdgcn_readlane(Lj, m);
      rank += (Lo > Lj) || (Lo == Lj && m < lane);
    }
    int ns = int((int64_t(Lj) + a.split_chunk - 1) / a.split_chunk);
    ns = ns < 1 ? 1 : (ns > nsplit ? nsplit : ns);
    int start = 0;
    for (int m = 0; m < B; ++m)
      start += __builtin_amdgcn_readlane(rank, m) < rank ? __builtin_amdgcn_readlane(ns, m) * int(a.Hkv) : 0;
    const int blk = int(blockIdx.x);
    const uint64_t hit = __ballot(lane < B && blk >= start && blk < start + ns * int(a.Hkv));
    if (!hit) return;  // beyond the active blocks (uniform over the block)
    b = __ffsll(static_cast<unsigned long long>(hit)) - 1;
    nsb = __builtin_amdgcn_readlane(ns, b);
    const int off = blk - __builtin_amdgcn_readlane(start, b);
    kvh = off / nsb;
    split = off % nsb;
  } else {
    split = int(blockIdx.x % unsigned(nsplit));
    const int unit = int(blockIdx.x / unsigned(nsplit));
    kvh = unit % int(a.Hkv);
    b = unit / int(a.Hkv);
    if (a.sort_lens) b = rank_to_seq(a.kv_lens, int(a.B), b, lane);
  }
  // The length is requested first, ahead of this wave's tile loads, and
  // unconditionally (a dummy address without kv_lens), so that nothing waits
  // for it before its first use.
  const int32_t Lraw = *(a.kv_lens ? a.kv_lens + b : reinterpret_cast<const int32_t*>(a.K));
  KvRows<D, PAGED> kr{}, vr{};
  if constexpr (PAGED) {
    const int32_t* bt = a.block_table + int64_t(b) * a.bt_stride;
    const int64_t pe = a.Hkv * a.page_size * D, ho = int64_t(kvh) * a.page_size * D;
    const int sh = __builtin_ctz(unsigned(a.page_size));
    const uint32_t lp = uint32_t(a.num_pages - 1);
    kr = {a.K, bt, ho, pe, sh, lp, a.bt_stride - 1};
    vr = {a.V, bt, ho, pe, sh, lp, a.bt_stride - 1};
  } else {
    kr.base = a.K + (int64_t(b) * a.Hkv + kvh) * a.S * D;
    vr.base = a.V + (int64_t(b) * a.Hkv + kvh) * a.S * D;
  }
  const int64_t h0 = int64_t(kvh) * G;  // first query head of the group
  const float sl2 = a.scale * kLog2e;
  const int64_t stride = int64_t(nsb) * W * kTile;  // distance between a wave's tiles

  int64_t t0 = (int64_t(split) * W + wave) * kTile;
  uint4 kf[NSUB][NS], vf[NPV];
  __builtin_amdgcn_sched_barrier(0);
  {
    const int64_t ts = tile_start(t0, a.Lh - 1);
    const int32_t id = kr.page_id(ts, lane);
    load_k_tile<D, NSUB>(kr.at(ts, id), ts, t0, a.Lh - 1, li, lg, kf);
    load_v_tile<D, NPV>(vr.at(ts, id), ts, t0, a.Lh - 1, dc, rs, vf);
  }
  __builtin_amdgcn_sched_barrier(0);

  int64_t L = a.kv_lens ? int64_t(Lraw) : a.S;
  L = L < 0 ? 0 : (L > a.Lh ? a.Lh : L);
  EZ_TRACE(1);
  // Cache rows read here: [0, Lc) (the layer's decoded token is the virtual row).
  const int64_t Lc = LAYER ? (L > 0 ? L - 1 : 0) : L;
  const int64_t cl = Lc > 0 ? Lc - 1 : 0;  // clamp row of later tiles
  // Paged: the table entry of the next tile is read one iteration ahead.
  int32_t id_next = kr.page_id(tile_start(t0 + stride, cl), lane);

  bf16x8_t qf[NS];
  if constexpr (LAYER) {
    const int64_t pos = L - 1;
    const bool publisher = split == 0 && wave == W - 1;
    if (L > 0) {
      const uint16_t* row = a.qkv + int64_t(b) * a.qkv_bs;
      const uint16_t* crow = a.cos ? a.cos + pos * D : nullptr;
      const uint16_t* srow = a.sin ? a.sin + pos * D : nullptr;
      for (int h = wave; h < G; h += W)
        norm_rope_head<D>(row + (h0 + h) * D, a.qw, crow, srow, a.eps, &Qs[h][0], lane);
      if (publisher) {
        norm_rope_head<D>(row + a.H * D + int64_t(kvh) * D, a.kw, crow, srow, a.eps, Kn, lane);
        const uint16_t* vrow = row + (a.H + a.Hkv) * D + int64_t(kvh) * D;
        for (int i = lane; i < D; i += kWave) Vn[i] = vrow[i];
      }
    }
    __syncthreads();  // Qs, Kn, Vn complete
    if (publisher && L > 0) {
      const int64_t ps = pos & ~int64_t(kTile - 1);
      uint16_t* kdst = const_cast<uint16_t*>(kr.tile(ps)) + (pos - ps) * D;
      uint16_t* vdst = const_cast<uint16_t*>(vr.tile(ps)) + (pos - ps) * D;
      for (int i = lane; i < D; i += kWave) {
        kdst[i] = Kn[i];
        vdst[i] = Vn[i];
      }
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (li < G) v = *reinterpret_cast<const uint4*>(&Qs[li][32 * s + lg * 8]);
      qf[s] = as_bf16x8(v);
    }
  } else {
    // Q operand: lane (li, lg) holds Q[h0 + li][s*32 + lg*8 .. +8] for step s.
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (li < G) v = *reinterpret_cast<const uint4*>(a.Q + ((b * a.H + h0 + li) * D) + 32 * s + lg * 8);
      qf[s] = as_bf16x8(v);
    }
  }

  float m_run[G], l_acc[G], o[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m_run[h] = -INFINITY;
    l_acc[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = 0.f;
  }

  EZ_TRACE(2);
  for (int it = 0; t0 < Lc; t0 += stride, ++it) {
    const int64_t tn = t0 + stride;
    // ---- scores: acc[u][j] = S[head 4*lg + j][pos t0 + 16u + li]
    f32x4_t acc[NSUB];
#pragma unroll
    for (int u = 0; u < NSUB; ++u) {
      acc[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s)
        acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf[s], as_bf16x8(kf[u][s]), acc[u], 0, 0, 0);
    }
    if (EZ_ATTN_TRACE && it < 2) {
      if (acc[0][0] == 1.2345e-30f) a.Out[0] = 1;  // the stamp follows the MFMA results
      EZ_TRACE(3 + it);
    }
    const int64_t tsn = tile_start(tn, cl);
    const int32_t id_n = id_next;
    load_k_tile<D, NSUB>(kr.at(tsn, id_n), tsn, tn, cl, li, lg, kf);  // next K while this tile finishes
    id_next = kr.page_id(tile_start(tn + stride, cl), lane);

    float mx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      mx[j] = -INFINITY;
#pragma unroll
      for (int u = 0; u < NSUB; ++u) {
        const bool ok = t0 + 16 * u + li < Lc;
        const float sv = ok ? acc[u][j] * sl2 : -INFINITY;
        acc[u][j] = sv;
        mx[j] = fmaxf(mx[j], sv);
      }
      mx[j] = dpp_row16<true>(mx[j]);
    }
    // ---- wave-uniform running max and rescale factors
    float m_use[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float mt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx[h & 3]), 16 * (h >> 2)));
      const float mn = fmaxf(m_run[h], mt);
      const float alpha = (m_run[h] == -INFINITY) ? 0.f : exp2f(m_run[h] - mn);
      m_run[h] = mn;
      m_use[h] = (mn == -INFINITY) ? 0.f : mn;
      l_acc[h] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[h][e] *= alpha;
    }
    // ---- P = exp2(S - m) into LDS as Ps[pos][head]
    if (lg < GP / 4) {
#pragma unroll
      for (int u = 0; u < NSUB; ++u) {
        float pv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int h = 4 * lg + j;
          float mu = m_use[j < G ? j : 0];
          if constexpr (G > 4) mu = (lg == 1) ? m_use[4 + j] : mu;
          pv[j] = (h < G) ? exp2f(acc[u][j] - mu) : 0.f;
        }
        *reinterpret_cast<float4*>(&Ps[wave][16 * u + li][4 * lg]) = make_float4(pv[0], pv[1], pv[2], pv[3]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- O += P . V
#pragma unroll
    for (int j = 0; j < NPV; ++j) {
      float pr[GP];
#pragma unroll
      for (int q4 = 0; q4 < GP / 4; ++q4) {
        const float4 t = *reinterpret_cast<const float4*>(&Ps[wave][rs + RPI * j][4 * q4]);
        pr[4 * q4 + 0] = t.x; pr[4 * q4 + 1] = t.y; pr[4 * q4 + 2] = t.z; pr[4 * q4 + 3] = t.w;
      }
      float v[8];
      unpack8(vf[j], v);
      if (t0 + rs + RPI * j >= Lc) {  // masked row: its cache bytes may be anything
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        l_acc[h] += pr[h];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = fmaf(pr[h], v[e], o[h][e]);
      }
    }
    load_v_tile<D, NPV>(vr.at(tsn, id_n), tsn, tn, cl, dc, rs, vf);  // next V
    __builtin_amdgcn_wave_barrier();
  }

  if constexpr (LAYER) {
    // The decoded token as one more row of wave 0 of split 0: s_h = q_h . k
    // (fp32 over the bf16 values the cache holds), then the same online
    // update; P and V enter through the row-group-0 lanes only (the row
    // groups are summed below).
    if (split == 0 && wave == 0 && L > 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float d = 0.f;
        for (int i = lane; i < D; i += kWave) d = fmaf(bf2f(Qs[h][i]), bf2f(Kn[i]), d);
        const float sv = wave_reduce_uniform<false>(d) * sl2;
        const float mn = fmaxf(m_run[h], sv);
        const float alpha = (m_run[h] == -INFINITY) ? 0.f : exp2f(m_run[h] - mn);
        const float pv = rs == 0 ? exp2f(sv - mn) : 0.f;
        m_run[h] = mn;
        l_acc[h] = fmaf(l_acc[h], alpha, pv);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = fmaf(o[h][e], alpha, pv * bf2f(Vn[dc * 8 + e]));
      }
    }
  }

  EZ_TRACE(5);
  // ---- merge the row groups of the wave (lanes with equal dc): VALU lane
  // swaps, no LDS round trips
#pragma unroll
  for (int h = 0; h < G; ++h) {
    l_acc[h] = rowgroup_sum<CPR>(l_acc[h]);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[h][e] = rowgroup_sum<CPR>(o[h][e]);
  }
  if (rs == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      *reinterpret_cast<float4*>(&Os[wave][h][dc * 8]) = make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
      *reinterpret_cast<float4*>(&Os[wave][h][dc * 8 + 4]) = make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      Ms[wave][h] = m_run[h];
      Ls[wave][h] = l_acc[h];
    }
  }
  __syncthreads();

  // ---- merge the W waves: thread handles (h, d) pairs
  for (int idx = threadIdx.x; idx < G * D; idx += W * kWave) {
    const int h = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, Ms[w][h]);
    float ov = 0.f, lv = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = (Ms[w][h] == -INFINITY) ? 0.f : exp2f(Ms[w][h] - M);
      ov = fmaf(f, Os[w][h][d], ov);
      lv = fmaf(f, Ls[w][h], lv);
    }
    const int64_t hq = b * a.H + h0 + h;
    if (nsplit == 1) {
      a.Out[out_index(a, hq, d)] = f2bf(lv > 0.f ? ov / lv : 0.f);
    } else {
      opart[(hq * nsplit + split) * D + d] = ov;
      if (d == 0) {
        *reinterpret_cast<float2*>(ml + (hq * nsplit + split) * 2) = make_float2(M, lv);
        // the last split of a sequence with fewer than nsplit marks the
        // unused merge slots empty (weight 0, their partials never read)
        if (split == nsb - 1)
          for (int s2 = nsb; s2 < nsplit; ++s2)
            *reinterpret_cast<float2*>(ml + (hq * nsplit + s2) * 2) = make_float2(-INFINITY, 0.f);
      }
    }
  }
  EZ_TRACE(6);
}

// Merge of one query head (b, h) with one thread per head dim: every thread
// issues its nsplit partial loads at once (they do not depend on the
// weights), while each wave turns the (max, sum) pairs (lane s = split s)
// into normalised weights; one dependent memory round trip in total.
//   out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s
template <int D>
__global__ __launch_bounds__(D) void attn_combine_kernel(AttnArgs a, int nsplit, const float* opart,
                                                         const float* ml) {
  EZ_PROF_WAVE(kProfAttnCombine);
  static_assert(kMaxSplits <= kWave, "one split per lane");
  const int64_t hq = blockIdx.x;
  const int lane = threadIdx.x & (kWave - 1);
  const int d = threadIdx.x;
  const float* op = opart + hq * nsplit * D + d;
  float v[kMaxSplits];
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) v[s] = s < nsplit ? op[s * D] : 0.f;
  const bool ok = lane < nsplit;
  const float2 st = ok ? *reinterpret_cast<const float2*>(ml + hq * nsplit * 2 + 2 * lane)
                       : make_float2(-INFINITY, 0.f);
  const float M = wave_reduce_uniform<true>(st.x);
  const float f = (st.x == -INFINITY) ? 0.f : exp2f(st.x - M);
  const float tot = wave_reduce_uniform<false>(f * st.y);
  const float wgt = tot > 0.f ? f / tot : 0.f;
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) {
    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wgt), s));
    acc = w != 0.f ? fmaf(w, v[s], acc) : acc;  // empty splits: weight 0, partial never used
  }
  a.Out[out_index(a, hq, d)] = f2bf(acc);
}

struct SplitPlan {
  int waves;
  int nsplit;
};

// Splits per (b, kv head), planned on the length bound Lh: enough blocks to
// keep every CU busy, at least one tile per wave at length Lh, and at most
// kMaxSplits partials per merge.
SplitPlan plan_splits(int64_t B, int64_t Hkv, int64_t Lh, int64_t G) {
  const int64_t units = B * Hkv;
  const int64_t cus = num_cus();
  // 8-wave blocks for few units; group 8 keeps 4 waves (its accumulators need
  // the register budget of one wave per SIMD).
  const int waves = (units * 4 <= cus && G <= 4) ? 8 : 4;
  const int64_t target = waves == 8 ? 2 * cus : EZ_ATTN_TARGET4 * cus;  // blocks in flight
  int64_t ns = (target + units - 1) / units;
  const int64_t max_ns = (Lh + int64_t(waves) * kTile - 1) / (int64_t(waves) * kTile);
  if (ns > max_ns) ns = max_ns;
  if (ns > kMaxSplits) ns = kMaxSplits;
  if (ns < 1) ns = 1;
  return {waves, int(ns)};
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

template <int D, bool LAYER, bool PAGED>
void launch_d(const AttnArgs& a, const SplitPlan& pl, float* opart, float* ml, int64_t G, hipStream_t s) {
  const dim3 grid{unsigned(a.B * a.Hkv * pl.nsplit), 1, 1}, block{unsigned(pl.waves * kWave), 1, 1};
#define EZ_LAUNCH(GG, WW) \
  hipLaunchKernelGGL((attn_split_kernel<D, GG, WW, LAYER, PAGED>), grid, block, 0, s, a, pl.nsplit, opart, ml)
  if (G == 8) {
    EZ_LAUNCH(8, 4);
  } else if (pl.waves == 8) {
    if (G == 1) EZ_LAUNCH(1, 8);
    else if (G == 2) EZ_LAUNCH(2, 8);
    else EZ_LAUNCH(4, 8);
  } else {
    if (G == 1) EZ_LAUNCH(1, 4);
    else if (G == 2) EZ_LAUNCH(2, 4);
    else EZ_LAUNCH(4, 4);
  }
#undef EZ_LAUNCH
}

}  // namespace

// The workspace is planned on the capacity S, an upper bound for every Lh.
size_t attn_workspace_size(int64_t B, int64_t H, int64_t Hkv, int64_t S, int64_t D) {
  if (B < 1 || H < 1 || Hkv < 1 || S < 1 || D < 1) return 0;
  const SplitPlan pl = plan_splits(B, Hkv, S, H / Hkv);
  return align256(size_t(B * H * pl.nsplit * D) * 4) + align256(size_t(B * H * pl.nsplit * 2) * 4);
}

int launch_attn(const AttnArgs& a, void* ws, size_t ws_bytes, hipStream_t s) {
  const bool layer = a.Q == nullptr;
  EZ_REQUIRE(a.K && a.V && a.Out && (!layer || a.qkv), "attn_decode: null pointer");
  EZ_REQUIRE(a.B >= 1 && a.H >= 1 && a.Hkv >= 1 && a.S >= 1, "attn_decode: bad shape");
  EZ_REQUIRE(a.B * a.Hkv * kMaxSplits < (int64_t(1) << 31), "attn_decode: too many (batch, kv head) units");
  EZ_REQUIRE(a.H % a.Hkv == 0, "attn_decode: num_heads must be divisible by num_kv_heads");
  const int64_t G = a.H / a.Hkv;
  EZ_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "attn_decode: group size %lld not in {1,2,4,8}", (long long)G);
  EZ_REQUIRE(a.D == 64 || a.D == 128, "attn_decode: head_dim must be 64 or 128");
  EZ_REQUIRE((a.cos == nullptr) == (a.sin == nullptr), "attn_decode: cos and sin go together");
  EZ_REQUIRE(a.Lh >= 0, "attn_decode: max_kv_len must be >= 0");
  EZ_REQUIRE(!a.block_table || (a.page_size >= kTile && (a.page_size & (a.page_size - 1)) == 0 &&
                                a.bt_stride >= 1 && a.S == a.bt_stride * a.page_size),
             "paged attn_decode: page_size must be a power of two >= %d and S = max_pages * page_size", kTile);
  AttnArgs aa = a;
  aa.Lh = (a.Lh == 0 || a.Lh > a.S || !a.kv_lens) ? a.S : a.Lh;
  aa.sort_lens = a.kv_lens && a.B > 1 && a.B <= kWave;
  if (aa.scale <= 0.f) aa.scale = 1.0f / sqrtf(float(a.D));
  const SplitPlan pl = plan_splits(aa.B, aa.Hkv, aa.Lh, G);
  // ragged batches: splits in proportion to each sequence's length
  aa.split_chunk = (aa.sort_lens && pl.nsplit > 1) ? (aa.Lh + pl.nsplit - 1) / pl.nsplit : 0;
  float *opart = nullptr, *ml = nullptr;
  if (pl.nsplit > 1) {
    const size_t need = attn_workspace_size(a.B, a.H, a.Hkv, a.S, a.D);
    EZ_REQUIRE(ws && ws_bytes >= need, "attn_decode: workspace too small (%zu < %zu)", ws_bytes, need);
    opart = static_cast<float*>(ws);
    ml = reinterpret_cast<float*>(static_cast<char*>(ws) + align256(size_t(a.B * a.H * pl.nsplit * a.D) * 4));
  }
  const bool paged = a.block_table != nullptr;
  if (layer) {
    if (paged) {
      if (a.D == 64) launch_d<64, true, true>(aa, pl, opart, ml, G, s);
      else launch_d<128, true, true>(aa, pl, opart, ml, G, s);
    } else {
      if (a.D == 64) launch_d<64, true, false>(aa, pl, opart, ml, G, s);
      else launch_d<128, true, false>(aa, pl, opart, ml, G, s);
    }
  } else {
    if (paged) {
      if (a.D == 64) launch_d<64, false, true>(aa, pl, opart, ml, G, s);
      else launch_d<128, false, true>(aa, pl, opart, ml, G, s);
    } else {
      if (a.D == 64) launch_d<64, false, false>(aa, pl, opart, ml, G, s);
      else launch_d<128, false, false>(aa, pl, opart, ml, G, s);
    }
  }
  if (pl.nsplit > 1) {
    const dim3 grid{unsigned(a.B * a.H), 1, 1}, block{unsigned(a.D), 1, 1};
    if (a.D == 64) hipLaunchKernelGGL(attn_combine_kernel<64>, grid, block, 0, s, aa, pl.nsplit, opart, ml);
    else hipLaunchKernelGGL(attn_combine_kernel<128>, grid, block, 0, s, aa, pl.nsplit, opart, ml);
  }
  return launch_status("attn_decode");
}

}  // namespace ez

#if EZ_ATTN_TRACE
extern "C" int ezops_attn_trace_read(void* host, size_t bytes) {
  if (!host) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(ez::ez_attn_trace)) != hipSuccess) return -1;
    return int(hipMemset(p, 0, bytes));
  }
  return int(hipMemcpyFromSymbol(host, HIP_SYMBOL(ez::ez_attn_trace), bytes, 0, hipMemcpyDeviceToHost));
}
#endif

extern "C" size_t ezops_attn_decode_workspace_size(int64_t B, int64_t H, int64_t Hkv, int64_t S, int64_t D) {
  return ez::attn_workspace_size(B, H, Hkv, S, D);
}

extern "C" int ezops_paged_attn_decode_bf16(const void* Q, const void* K_pages, const void* V_pages, void* Out,
                                            const int32_t* block_table, const int32_t* kv_lens, int64_t B, int64_t H,
                                            int64_t Hkv, int64_t D, int64_t num_pages, int64_t page_size,
                                            int64_t max_pages,
                                            int64_t max_kv_len, float scale, void* ws, size_t ws_bytes,
                                            hipStream_t stream) {
  EZ_REQUIRE(Q && block_table && kv_lens, "paged attn_decode: null pointer");
  EZ_REQUIRE(page_size >= 1 && max_pages >= 1 && num_pages >= 1 && num_pages <= (int64_t(1) << 31),
             "paged attn_decode: bad page geometry");
  ez::AttnArgs a{};
  a.Q = static_cast<const uint16_t*>(Q);
  a.K = static_cast<const uint16_t*>(K_pages);
  a.V = static_cast<const uint16_t*>(V_pages);
  a.Out = static_cast<uint16_t*>(Out);
  a.B = B; a.H = H; a.Hkv = Hkv; a.S = max_pages * page_size; a.D = D;
  a.kv_lens = kv_lens;
  a.block_table = block_table;
  a.bt_stride = max_pages;
  a.page_size = int(page_size);
  a.num_pages = num_pages;
  a.Lh = max_kv_len;
  a.scale = scale;
  return ez::launch_attn(a, ws, ws_bytes, stream);
}

extern "C" int ezops_attn_decode_bf16(const void* Q, const void* K, const void* V, void* Out, int64_t B,
                                      int64_t H, int64_t Hkv, int64_t S, int64_t D, const int32_t* kv_lens,
                                      int64_t max_kv_len, float scale, void* ws, size_t ws_bytes,
                                      hipStream_t stream) {
  EZ_REQUIRE(Q, "attn_decode: null pointer");
  ez::AttnArgs a{};
  a.Q = static_cast<const uint16_t*>(Q);
  a.K = static_cast<const uint16_t*>(K);
  a.V = static_cast<const uint16_t*>(V);
  a.Out = static_cast<uint16_t*>(Out);
  a.B = B; a.H = H; a.Hkv = Hkv; a.S = S; a.D = D;
  a.kv_lens = kv_lens;
  a.Lh = max_kv_len;
  a.scale = scale;
  return ez::launch_attn(a, ws, ws_bytes, stream);
}
