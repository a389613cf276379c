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
// Per wave and tile (both products on v_mfma_f32_16x16x32_bf16):
//   * scores, transposed: S^T = K Q^T with A = 16 positions of K per
//     sub-tile, B = the G query rows (zero-padded to 16 columns).  K rows
//     are read with fully coalesced 16-byte loads into registers, stored
//     into the wave's LDS slab at the top of the tile and read back as the
//     A operand with ds_read_b128 (k-slot (lg, e) of step s = head dim
//     32 s + 8 lg + e, Q uses the same map).  Lane (li, lg) then holds 8
//     scores of query head li.
//   * online softmax in the exp2 domain (scale * log2 e folded into S), one
//     head per lane column: row maxima across the 4 lane groups by lane
//     swaps, the rescale of O skipped when no running max moved.
//   * O^T += V^T P^T: the 8 probabilities of a lane, split into bf16 high
//     and low parts (two MFMAs per fragment), are the B operand as they
//     stand (k-slot 8 lg + e = position 16(e/4) + 4 lg + e%4); V rows are read with fully coalesced 16-byte loads, stored
//     row-major into a per-wave LDS slab and read back as the V^T operand by
//     transposing LDS reads (ds_read_b64_tr_b16), 2 D/16 MFMAs per tile; the
//     slab holds the tile's K first, then its V.
//   * every tile load is unconditional (rows past the live length read a
//     clamp row): the next tile's K is requested right after the score MFMAs
//     and its V right after P.V.
// The first tile is requested before the length arrives (its addresses only
// need Lh), behind a single scalar load of the length.  The W waves merge
// (max, sum, O) through LDS; with more than one split the blocks write fp32
// partials that attn_combine_kernel merges (the kernel boundary orders the
// hand-off; an in-kernel arrival counter measured no faster on MI355X).
#include <mutex>

#include "common.h"
#include "internal.h"
#include "prof.h"
#include "status.h"
#include "../../include/ezops_hip.h"

namespace ez {

EZ_PROF_DEFINE(attn)
namespace {

constexpr int kTile = 32;       // positions per wave iteration
constexpr int kMaxSplits = 32;  // split partials the combine holds per lane
constexpr float kLog2e = 1.4426950408889634f;

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

// K tiles go through the wave's LDS slab: rows read with
// coalesced 16-byte loads (1 KiB per instruction, as V), stored row-major
// with 16-byte chunk c of row p at slot c ^ kswz(p), and read back as MFMA A
// fragments (ds_read_b128, 16 consecutive rows per 16 lanes: the swizzle
// puts them in 16 distinct bank groups of the 64-bank LDS).  Read straight
// into the A operand, each load instruction covers 64-byte pieces of 16 rows;
// a 38 MB burst of that pattern arrives at ~3.2 TB/s against ~4.5 TB/s for
// whole-row reads (same grid, measured on MI355X).
template <int D>
__device__ __forceinline__ int kswz(int p) {
  constexpr int CPR = D / 8;  // 16-byte chunks per row (16 or 8)
  return (p >> (CPR == 16 ? 0 : 1)) & (CPR - 1);
}
template <int D>
__device__ __forceinline__ void load_k_regs(const uint16_t* tb, int64_t ts, int64_t t0, int64_t last, int lane,
                                            uint4 (&k)[kTile * D / 8 / kWave]) {
  constexpr int CPR = D / 8, RPD = kWave / CPR, VI = kTile / RPD;
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const int p = i * RPD + lane / CPR;
    int64_t r = t0 + p;
    r = r < last ? r : last;
    k[i] = ld16_stream(tb + (r - ts) * D + ((lane % CPR) ^ kswz<D>(p)) * 8);
  }
}

// V tiles live in LDS, one slab of kTile rows x D bf16 per wave, row-major
// with 16-byte chunk c of row p at slot c ^ vswz(p): the transposing reads of
// the P.V operand (16 lanes over 4 rows x 32 bytes) then cover all banks.
template <int D>
__device__ __forceinline__ int vswz(int p) {
  return (2 * p) & (D / 8 - 1);
}

// V tile rows t0 + p (clamped to `last`) into registers, in the order of the
// slab's slots: load i of lane l is slot 64i + l = (row p, slot c'), the
// chunk c' ^ vswz(p) of that row (each row still read by CPR lanes as one
// contiguous run).  tb is the first row of the tile at ts = tile_start(t0, last).
template <int D>
__device__ __forceinline__ void load_v_regs(const uint16_t* tb, int64_t ts, int64_t t0, int64_t last, int lane,
                                            uint4 (&v)[kTile * D / 8 / kWave]) {
  constexpr int CPR = D / 8, RPD = kWave / CPR, VI = kTile / RPD;
#pragma unroll
  for (int i = 0; i < VI; ++i) {
    const int p = i * RPD + lane / CPR;
    int64_t r = t0 + p;
    r = r < last ? r : last;
    v[i] = ld16_stream(tb + (r - ts) * D + ((lane % CPR) ^ vswz<D>(p)) * 8);
  }
}

typedef int i32x2_t __attribute__((ext_vector_type(2)));
// Four V^T operand halves by transposing LDS reads (ds_read_b64_tr_b16: in
// each 16-lane group, lane m receives element m%4 of the 8-byte rows that
// lanes m/4, 4 + m/4, 8 + m/4 and 12 + m/4 address): r[2q] from addr[q],
// r[2q+1] from addr[q] + 16 rows.  One asm block with its own wait; the
// caller orders the slab stores before it with a compiler barrier.
template <int ROW16>
__device__ __forceinline__ void vt_read4(const uint32_t* addr, i32x2_t (&r)[8]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8\n\t"
      "ds_read_b64_tr_b16 %1, %8 offset:%12\n\t"
      "ds_read_b64_tr_b16 %2, %9\n\t"
      "ds_read_b64_tr_b16 %3, %9 offset:%12\n\t"
      "ds_read_b64_tr_b16 %4, %10\n\t"
      "ds_read_b64_tr_b16 %5, %10 offset:%12\n\t"
      "ds_read_b64_tr_b16 %6, %11\n\t"
      "ds_read_b64_tr_b16 %7, %11 offset:%12\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
      : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "i"(ROW16));
}

// Qwen3 per-head RMSNorm (fp32 statistics, weight) + half-split RoPE of one
// bf16 head, rounded once to bf16.  One wave; lane l < D/2 owns the pair
// (l, l + D/2).  Split in two so the kernel can request the inputs before
// its first K/V tile (a wave's loads complete in order, so anything
// requested after 16 KB of tile loads waits for them) and finish once they
// have arrived.  Operation order follows the reference
// (ezops/ops/fused_qk_norm_rope.py:138-147); a missing weight is 1 (exact).
struct HeadIn {
  uint16_t x1, x2, w1, w2;  // raw bf16: converting would wait for the loads here
};
template <int D>
__device__ __forceinline__ HeadIn load_head(const uint16_t* src, const uint16_t* w, int lane) {
  static_assert(D <= 2 * kWave, "one pair per lane");
  const int l = lane & (D / 2 - 1);  // lanes past D/2 repeat a pair (unused)
  return HeadIn{src[l], src[l + D / 2], w[l], w[l + D / 2]};
}
struct RopeIn {
  uint16_t c1, c2, s1, s2;
};
template <int D>
__device__ __forceinline__ RopeIn load_rope(const uint16_t* crow, const uint16_t* srow, int lane) {
  const int l = lane & (D / 2 - 1);
  return RopeIn{crow[l], crow[l + D / 2], srow[l], srow[l + D / 2]};
}
// load_rope for a position known only after the tile loads went out: the
// loads and their wait in one asm block, so that the speculative rows'
// registers (requested before the tiles) are all that the merge of the two
// paths waits for.
template <int D>
__device__ __forceinline__ RopeIn load_rope_sync(const uint16_t* crow, const uint16_t* srow, int lane) {
  const int l = lane & (D / 2 - 1);
  uint32_t c1, c2, s1, s2;
  asm volatile(
      "global_load_ushort %0, %4, off\n\t"
      "global_load_ushort %1, %5, off\n\t"
      "global_load_ushort %2, %6, off\n\t"
      "global_load_ushort %3, %7, off\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(c1), "=&v"(c2), "=&v"(s1), "=&v"(s2)
      : "v"(crow + l), "v"(crow + l + D / 2), "v"(srow + l), "v"(srow + l + D / 2)
      : "memory");
  return RopeIn{uint16_t(c1), uint16_t(c2), uint16_t(s1), uint16_t(s2)};
}
template <int D>
__device__ __forceinline__ void finish_head(const HeadIn& in, const RopeIn& ro, bool weighted, bool rope, float eps,
                                            uint16_t* dst, int lane) {
  const bool own = lane < D / 2;
  const float x1 = own ? bf2f(in.x1) : 0.f, x2 = own ? bf2f(in.x2) : 0.f;
  const float r = rsqrtf(wave_reduce_uniform<false>(x1 * x1 + x2 * x2) / float(D) + eps);
  if (!own) return;
  const float w1 = weighted ? bf2f(in.w1) : 1.f, w2 = weighted ? bf2f(in.w2) : 1.f;
  const float y1 = __fmul_rn(__fmul_rn(x1, r), w1), y2 = __fmul_rn(__fmul_rn(x2, r), w2);
  float o1 = y1, o2 = y2;
  if (rope) {
    o1 = __fadd_rn(__fmul_rn(y1, bf2f(ro.c1)), __fmul_rn(-y2, bf2f(ro.s1)));
    o2 = __fadd_rn(__fmul_rn(y2, bf2f(ro.c2)), __fmul_rn(y1, bf2f(ro.s2)));
  }
  dst[lane] = f2bf(o1);
  dst[lane + D / 2] = f2bf(o2);
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
  constexpr int NS = D / 32;          // MFMA k-steps per 16-position sub-tile of S
  constexpr int NSUB = kTile / 16;    // sub-tiles per tile
  constexpr int NDB = D / 16;         // 16-dim blocks of O^T
  constexpr int VI = kTile * D / 8 / kWave;  // 16-byte V loads per lane and tile
  static_assert(G <= 16, "group size: one MFMA column per query head");
  static_assert(kTile == 32 && NDB % 4 == 0, "tile geometry");

  __shared__ __align__(16) uint16_t Vs[W][kTile * D];  // per-wave V tile (vswz layout)
  __shared__ __align__(16) float Os[W][G][D];
  __shared__ float Ms[W][G], Ls[W][G];
  __shared__ __align__(16) uint16_t Qs[LAYER ? G : 1][D];
  __shared__ __align__(16) uint16_t Kn[LAYER ? D : 1], Vn[LAYER ? D : 1];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar tile loop
  const int li = lane & 15, lg = lane >> 4;
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
  // for it before its first use.  It is a vector load (an opaque per-lane
  // zero in the address): a wave's vector loads complete in order, so the
  // first one returns first, whereas a scalar load issued beside the tile
  // flood waited 3.5-10 us for its cache line (per-wave stamps, B = 1).
  int32_t lane0;
  asm volatile("v_mov_b32 %0, 0" : "=v"(lane0));
  const int32_t Lv = (a.kv_lens ? a.kv_lens + b : reinterpret_cast<const int32_t*>(a.K))[lane0];
  __builtin_amdgcn_sched_barrier(0);
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
  // Tiles of this wave: interleaved over the splits (tile s W + w, then every
  // nsb W-th), or with a.tps > 0 the split's own contiguous range (tile
  // s tps + w, then every W-th, below t_end) -- every block then carries the
  // same bytes, which sets the time when there is one block per CU.
  const int64_t stride = (a.tps > 0 ? int64_t(1) : int64_t(nsb)) * W * kTile;  // distance between a wave's tiles
  const int64_t t_end = a.tps > 0 ? min(a.Lh, (int64_t(split) + 1) * a.tps * kTile) : a.Lh;
  uint16_t* slab = &Vs[wave][0];

  int64_t t0 = (a.tps > 0 ? int64_t(split) * a.tps + wave : int64_t(split) * W + wave) * kTile;
  uint4 kn[VI], vn[VI];

  // Layer prologue inputs, requested ahead of the first tile and without
  // branches (a branch join would make the compiler wait for them there):
  // this wave's query heads (h = wave, wave + W, ...; clamped), the k head and
  // v row that split 0's last wave publishes (every wave requests them), and,
  // once the length has arrived (a scalar load), the cos / sin rows of its
  // position.  Absent weights or tables read the q row instead (unused).
  constexpr int NQ = LAYER ? (G + W - 1) / W : 1;
  const bool publisher = LAYER && split == 0 && wave == W - 1;
  HeadIn qin[NQ], kin{};
  RopeIn rin{};
  uint16_t vv1 = 0, vv2 = 0;
  if constexpr (LAYER) {
    const uint16_t* row = a.qkv + int64_t(b) * a.qkv_bs;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const int h = wave + j * W < G ? wave + j * W : G - 1;
      qin[j] = load_head<D>(row + (h0 + h) * D, a.qw ? a.qw : row, lane);
    }
    kin = load_head<D>(row + a.H * D + int64_t(kvh) * D, a.kw ? a.kw : row, lane);
    const uint16_t* vrow = row + (a.H + a.Hkv) * D + int64_t(kvh) * D;
    vv1 = vrow[lane & (D / 2 - 1)];
    vv2 = vrow[(lane & (D / 2 - 1)) + D / 2];
    // The rows of the host's bound Lh - 1, which is the token position
    // whenever the sequence is the longest (B = 1 with an exact bound): no
    // wait for the length before the tile loads go out.  Another position
    // reloads them once the length is in (below).
    const int64_t pos_s = a.Lh > 0 ? a.Lh - 1 : 0;
    rin = load_rope<D>(a.cos ? a.cos + pos_s * D : row, a.sin ? a.sin + pos_s * D : row, lane);
  }
  __builtin_amdgcn_sched_barrier(0);
  {
    const int64_t ts = tile_start(t0, t_end - 1);
    const int32_t id = kr.page_id(ts, lane);
    load_k_regs<D>(kr.at(ts, id), ts, t0, t_end - 1, lane, kn);
    load_v_regs<D>(vr.at(ts, id), ts, t0, t_end - 1, lane, vn);
  }
  __builtin_amdgcn_sched_barrier(0);

  int32_t Lraw;  // read here, behind the tile loads (asm: not hoisted to the load)
  asm volatile("v_readfirstlane_b32 %0, %1" : "=s"(Lraw) : "v"(Lv));
  int64_t L = a.kv_lens ? int64_t(Lraw) : a.S;
  L = L < 0 ? 0 : (L > a.Lh ? a.Lh : L);
  // Cache rows read here: [0, Lc) (the layer's decoded token is the virtual row).
  const int64_t Lc = LAYER ? (L > 0 ? L - 1 : 0) : L;
  const int64_t Le = Lc < t_end ? Lc : t_end;  // this wave's tiles lie below Le
  const int64_t cl = Le > 0 ? Le - 1 : 0;      // clamp row of later tiles
  // Paged: the table entry of the next tile is read one iteration ahead.
  int32_t id_next = kr.page_id(tile_start(t0 + stride, cl), lane);

  bf16x8_t qf[NS];
  if constexpr (LAYER) {
    const int64_t pos = L - 1;
    if (L > 0) {
      const bool rope = a.cos != nullptr;
      if (rope && pos != (a.Lh > 0 ? a.Lh - 1 : 0)) rin = load_rope_sync<D>(a.cos + pos * D, a.sin + pos * D, lane);
#pragma unroll
      for (int j = 0; j < NQ; ++j)
        if (wave + j * W < G) finish_head<D>(qin[j], rin, a.qw != nullptr, rope, a.eps, &Qs[wave + j * W][0], lane);
      if (publisher) {
        finish_head<D>(kin, rin, a.kw != nullptr, rope, a.eps, Kn, lane);
        if (lane < D / 2) {
          Vn[lane] = vv1;
          Vn[lane + D / 2] = vv2;
        }
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

  // Transposing-read addresses (bytes): lane (li, lg) of 16-dim block db
  // reads row 4lg + li/4, dims 16db + 4(li%4) .. +3; the second half of the
  // operand is 16 rows further.
  uint32_t vaddr[NDB];
  {
    const uint32_t sbase = uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint16_t*)slab));
    const int row = 4 * lg + (li >> 2), j = li & 3;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      vaddr[db] = sbase + uint32_t(row * D * 2 + (((2 * db + (j >> 1)) ^ vswz<D>(row)) * 16) + (j & 1) * 8);
  }

  // Lane (li, lg) keeps the state of query head li (heads >= G are padding):
  // running max, its share of the sum, O^T[16db + 4lg + r][li] in o[db][r].
  float m_run = -INFINITY, l_acc = 0.f;
  f32x4_t o[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) o[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int it = 0; t0 < Le; t0 += stride, ++it) {
    const int64_t tn = t0 + stride;
    // ---- S^T = K Q^T: acc[u][r] = S[head li][pos t0 + 16u + 4lg + r]
    // this tile's K from its registers into the slab (the previous tile's
    // V^T reads of it have completed), then the A fragments back out
#pragma unroll
    for (int i = 0; i < VI; ++i) *reinterpret_cast<uint4*>(slab + (i * kWave + lane) * 8) = kn[i];
    uint4 kf[NSUB][NS];
#pragma unroll
    for (int u = 0; u < NSUB; ++u)
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int r = 16 * u + li;
        kf[u][s] = *reinterpret_cast<const uint4*>(slab + r * D + (((4 * s + lg) ^ kswz<D>(r)) * 8));
      }
    f32x4_t acc[NSUB];
#pragma unroll
    for (int u = 0; u < NSUB; ++u) {
      acc[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s)
        acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[u][s]), qf[s], acc[u], 0, 0, 0);
    }
    const int64_t tsn = tile_start(tn, cl);
    const int32_t id_n = id_next;
    load_k_regs<D>(kr.at(tsn, id_n), tsn, tn, cl, lane, kn);  // next K while this tile finishes
    id_next = kr.page_id(tile_start(tn + stride, cl), lane);

    // ---- online softmax in the exp2 domain, one head per lane column
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < NSUB; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = t0 + 16 * u + 4 * lg + r < Lc;
        acc[u][r] = ok ? acc[u][r] * sl2 : -INFINITY;
        mx = fmaxf(mx, acc[u][r]);
      }
    mx = colgroup_max(mx);
    const float mn = fmaxf(m_run, mx);  // finite: position t0 < Lc is in the tile
    const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - mn);
    m_run = mn;
    l_acc *= alpha;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {  // rescale only when some running max moved
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] *= alpha;
    }
    // P^T operand: k-slot 8lg + e = position 16(e/4) + 4lg + e%4, as two
    // bf16 parts p = hi + lo (hi = bf16(p), lo = bf16(p - hi)): the two
    // products against the same V^T fragments carry P to ~16 significant
    // bits, so the value sum matches the fp32 weights of the reference
    // (rounding P to bf16 alone puts a relative error of ~2^-9 on every
    // weight, which the Qwen3 layer's FFN carries to its output).
    uint32_t pw[4], pl[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float p0 = __builtin_amdgcn_exp2f(acc[q >> 1][2 * (q & 1)] - mn);
      const float p1 = __builtin_amdgcn_exp2f(acc[q >> 1][2 * (q & 1) + 1] - mn);
      pw[q] = cvt_bf2(p0, p1);
      pl[q] = cvt_bf2(p0 - bf_lo(pw[q]), p1 - bf_hi(pw[q]));
      l_acc += p0 + p1;
    }
    const bf16x8_t pb = as_bf16x8(make_uint4(pw[0], pw[1], pw[2], pw[3]));
    const bf16x8_t pbl = as_bf16x8(make_uint4(pl[0], pl[1], pl[2], pl[3]));

    // ---- O^T += V^T P^T: this tile's V from its registers into the slab
    // (the previous tile's reads of it have completed), then read transposed.
    // Rows at or past the length get P = 0 but must not hold non-finite
    // values (0 * NaN): a wave's first tile is requested before the length
    // is known and may read such rows; they are zeroed here.
    if (t0 + kTile > Lc) {
#pragma unroll
      for (int i = 0; i < VI; ++i)
        if (t0 + i * (kWave / (D / 8)) + lane / (D / 8) >= Lc) vn[i] = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VI; ++i) *reinterpret_cast<uint4*>(slab + (i * kWave + lane) * 8) = vn[i];
    asm volatile("" ::: "memory");  // the stores stay ahead of the transposing reads
#pragma unroll
    for (int q = 0; q < NDB / 4; ++q) {
      i32x2_t vt[8];
      vt_read4<16 * D * 2>(&vaddr[4 * q], vt);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const bf16x8_t va = __builtin_bit_cast(bf16x8_t, (u32x4_t){uint32_t(vt[2 * k][0]), uint32_t(vt[2 * k][1]),
                                                                   uint32_t(vt[2 * k + 1][0]), uint32_t(vt[2 * k + 1][1])});
        o[4 * q + k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, o[4 * q + k], 0, 0, 0);
        o[4 * q + k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pbl, o[4 * q + k], 0, 0, 0);
      }
    }
    // next V (unconditional like the K loads: past the end every row clamps
    // to the last live row)
    load_v_regs<D>(vr.at(tsn, id_n), tsn, tn, cl, lane, vn);
  }

  // l: the four lanes of a head column hold its partial sums.
  l_acc = rowgroup_sum<16>(l_acc);
  if constexpr (LAYER) {
    // The decoded token as one more row of wave 0 of split 0: s_h = q_h . k
    // (fp32 over the bf16 values the cache holds), then the same online
    // update in fp32, lane column h.
    if (split == 0 && wave == 0 && L > 0) {
      float sv = -INFINITY;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float d = 0.f;
        for (int i = lane; i < D; i += kWave) d = fmaf(bf2f(Qs[h][i]), bf2f(Kn[i]), d);
        const float sh = wave_reduce_uniform<false>(d) * sl2;
        sv = li == h ? sh : sv;
      }
      if (li < G) {
        const float mn = fmaxf(m_run, sv);
        const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - mn);
        const float pv = __builtin_amdgcn_exp2f(sv - mn);
        m_run = mn;
        l_acc = fmaf(l_acc, alpha, pv);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[db][r] = fmaf(o[db][r], alpha, pv * bf2f(Vn[16 * db + 4 * lg + r]));
      }
    }
  }

  if (li < G) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
      *reinterpret_cast<float4*>(&Os[wave][li][16 * db + 4 * lg]) = make_float4(o[db][0], o[db][1], o[db][2], o[db][3]);
    if (lg == 0) {
      Ms[wave][li] = m_run;
      Ls[wave][li] = l_acc;
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
// kMaxSplits partials per merge.  balance: then the fewest splits that keep
// the same maximum of tiles per wave (B=1 at 9291 positions: 19 splits, 2
// tiles on the busiest wave as with 32, and a cheaper merge).  The
// unbalanced plan bounds the balanced one for every Lh up to its own, so the
// workspace is sized with it.
SplitPlan plan_splits(int64_t B, int64_t Hkv, int64_t Lh, int64_t G, bool balance = true) {
  const int64_t units = B * Hkv;
  const int64_t cus = num_cus();
  // 8-wave blocks for few units; groups 8 and 16 keep 4 waves (its accumulators need
  // the register budget of one wave per SIMD).
  const int waves = (units * 4 <= cus && G <= 4) ? 8 : 4;
  const int64_t target = waves == 8 ? 2 * cus : 8 * cus;  // blocks in flight (4-wave: B=16 layer 211/205/205/212/220 us at 4/6/8/12/16 per CU)
  int64_t ns = (target + units - 1) / units;
  const int64_t max_ns = (Lh + int64_t(waves) * kTile - 1) / (int64_t(waves) * kTile);
  if (ns > max_ns) ns = max_ns;
  if (ns > kMaxSplits) ns = kMaxSplits;
  if (ns < 1) ns = 1;
  if (balance) {
    const int64_t tiles = (Lh + kTile - 1) / kTile;
    const int64_t per_wave = (tiles + ns * waves - 1) / (ns * waves);  // tiles on the busiest wave
    if (per_wave > 0) ns = (tiles + per_wave * waves - 1) / (per_wave * waves);
    if (ns < 1) ns = 1;
  }
  return {waves, int(ns)};
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

template <int D, bool LAYER, bool PAGED>
void launch_d(const AttnArgs& a, const SplitPlan& pl, float* opart, float* ml, int64_t G, hipStream_t s) {
  const dim3 grid{unsigned(a.B * a.Hkv * pl.nsplit), 1, 1}, block{unsigned(pl.waves * kWave), 1, 1};
#define EZ_LAUNCH(GG, WW) \
  hipLaunchKernelGGL((attn_split_kernel<D, GG, WW, LAYER, PAGED>), grid, block, 0, s, a, pl.nsplit, opart, ml)
  if (G == 16) {
    EZ_LAUNCH(16, 4);
  } else if (G == 8) {
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
  const SplitPlan pl = plan_splits(B, Hkv, S, H / Hkv, false);
  return align256(size_t(B * H * pl.nsplit * D) * 4) + align256(size_t(B * H * pl.nsplit * 2) * 4);
}

int check_attn(const AttnArgs& a) {
  const bool layer = a.Q == nullptr;
  EZ_REQUIRE(a.K && a.V && a.Out && (!layer || a.qkv), "attn_decode: null pointer");
  EZ_REQUIRE(a.B >= 1 && a.H >= 1 && a.Hkv >= 1 && a.S >= 1, "attn_decode: bad shape");
  EZ_REQUIRE(a.B * a.Hkv * kMaxSplits < (int64_t(1) << 31), "attn_decode: too many (batch, kv head) units");
  EZ_REQUIRE(a.H % a.Hkv == 0, "attn_decode: num_heads must be divisible by num_kv_heads");
  const int64_t G = a.H / a.Hkv;
  EZ_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "attn_decode: group size %lld not in {1,2,4,8,16}",
             (long long)G);
  EZ_REQUIRE(a.D == 64 || a.D == 128, "attn_decode: head_dim must be 64 or 128");
  EZ_REQUIRE((a.cos == nullptr) == (a.sin == nullptr), "attn_decode: cos and sin go together");
  EZ_REQUIRE(a.Lh >= 0, "attn_decode: max_kv_len must be >= 0");
  EZ_REQUIRE(!a.block_table || (a.page_size >= kTile && (a.page_size & (a.page_size - 1)) == 0 &&
                                a.bt_stride >= 1 && a.S == a.bt_stride * a.page_size),
             "paged attn_decode: page_size must be a power of two >= %d and S = max_pages * page_size", kTile);
  return EZ_OK;
}

int launch_attn(const AttnArgs& a, void* ws, size_t ws_bytes, hipStream_t s) {
  const int rc = check_attn(a);
  if (rc != EZ_OK) return rc;
  const bool layer = a.Q == nullptr;
  const int64_t G = a.H / a.Hkv;
  AttnArgs aa = a;
  aa.Lh = (a.Lh == 0 || a.Lh > a.S || !a.kv_lens) ? a.S : a.Lh;
  aa.sort_lens = a.kv_lens && a.B > 1 && a.B <= kWave;
  if (aa.scale <= 0.f) aa.scale = 1.0f / sqrtf(float(a.D));
  SplitPlan pl = plan_splits(aa.B, aa.Hkv, aa.Lh, G);
  // ragged batches: splits in proportion to each sequence's length
  aa.split_chunk = (aa.sort_lens && pl.nsplit > 1) ? (aa.Lh + pl.nsplit - 1) / pl.nsplit : 0;
  aa.tps = 0;
  if (!aa.split_chunk && pl.waves == 8 && (!a.kv_lens || a.Lh > 0)) {
    // Few units (8-wave blocks): one block per CU, each over its own
    // contiguous run of tiles, so that every CU reads the same bytes (the
    // interleaved plan put 16 tiles on some CUs and none on a third of
    // them; a CU streams about 21 GB/s here, so the busiest CU sets the
    // time).  nsplit is then the number of non-empty runs.  Only with a host
    // bound on the lengths (or none to bound): over the capacity S with
    // shorter lengths, the runs past them would leave their CUs idle.
    const int64_t tiles = (aa.Lh + kTile - 1) / kTile;
    const int64_t ws_ns = plan_splits(a.B, a.Hkv, a.S, G, false).nsplit;  // what the workspace holds
    int64_t ns = num_cus() / (aa.B * aa.Hkv);
    ns = ns < ws_ns ? ns : ws_ns;
    ns = ns < (tiles + 7) / 8 ? ns : (tiles + 7) / 8;  // at least a tile per wave
    ns = ns < 1 ? 1 : ns;
    aa.tps = (tiles + ns - 1) / ns;
    pl.nsplit = int((tiles + aa.tps - 1) / aa.tps);
  }
  float *opart = nullptr, *ml = nullptr;
  if (pl.nsplit > 1) {
    const size_t need = attn_workspace_size(a.B, a.H, a.Hkv, a.S, a.D);
    EZ_REQUIRE(ws && ws_bytes >= need, "attn_decode: workspace too small (%zu < %zu)", ws_bytes, need);
    EZ_REQUIRE((reinterpret_cast<uintptr_t>(ws) & 15) == 0, "attn_decode: workspace must be 16-byte aligned");
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

// ---------------------------------------------------------------------------
// Allocation-free entry: the split partials live in a fixed device array
// instead of a caller workspace.  Each GPU holds its own copy of `scratch`
// (at its own address) until the process ends.  `scratch` is a host-side
// stand-in in host code: its device address is looked up once per device
// with hipGetSymbolAddress and only that address reaches a kernel.  Every
// slot the combine reads is written by the same call, so nothing needs
// clearing between calls; calls that overlap in time on one GPU race on it.
constexpr size_t kAttnScratchBytes = size_t(8) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kAttnScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return ez::set_error(int(e), "attn_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return ez::set_error(EZ_EINVAL, "attn_decode_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return ez::set_error(e != hipSuccess ? int(e) : EZ_EINVAL, "attn_decode_noalloc: hipGetSymbolAddress: %s",
                           hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return EZ_OK;
}
}  // namespace

extern "C" size_t ezops_attn_decode_noalloc_max_scratch(void) { return kAttnScratchBytes; }

extern "C" int ezops_attn_decode_noalloc_bf16(const void* Q, const void* K, const void* V, void* Out, int64_t B,
                                              int64_t H, int64_t Hkv, int64_t S, int64_t D, const int32_t* kv_lens,
                                              int64_t max_kv_len, float scale, hipStream_t stream) {
  EZ_REQUIRE(Q, "attn_decode_noalloc: null pointer");
  const size_t need = ez::attn_workspace_size(B, H, Hkv, S, D);
  EZ_REQUIRE(need <= kAttnScratchBytes,
             "attn_decode_noalloc: split partials need %zu bytes, above the %zu-byte device scratch", need,
             kAttnScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != EZ_OK) return rc;
  return ezops_attn_decode_bf16(Q, K, V, Out, B, H, Hkv, S, D, kv_lens, max_kv_len, scale, ws, kAttnScratchBytes,
                                stream);
}

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
