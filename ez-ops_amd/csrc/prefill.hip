// Prefill (the step before decode): causal GQA flash attention over the KV
// cache for a chunk of new tokens per sequence, and the SwiGLU elementwise
// stage of the batched FFN.
//
// Attention layout on the matrix cores (v_mfma_f32_32x32x16_bf16: lane
// 32h+i holds A[i][8h..8h+7] and B[8h..8h+7][i]; reg r of lane 32h+j holds
// C[8(r/4) + 4h + r%4][j]):
//   S^T = K Q^T   A = 32 keys x 16 dims of K (LDS, XOR-swizzled rows),
//                 B = Q^T (registers, loaded once), C = S^T[key][query]
//   O^T = V^T P^T A = V^T (row-major LDS tile, read by transposing
//                 ds_read_b64_tr_b16), B = P^T straight from the
//                 S^T registers: the k slots 8h..8h+7 of a 16-key step are
//                 keys 4h..4h+3 and 8+4h..8+4h+3 of it, the same slot order
//                 in A and B, so P never leaves the lane.
// Probabilities use the hardware v_exp_f32 directly (results below 2^-126 of
// the row maximum flush to zero, far below what the bf16 P operand holds).
// Queries sit in the lane column j in both products, so a query's running
// max / sum and its output column share the lane: the only cross-lane step
// is the swap between the lane halves j and j+32.
#include "common.h"
#include "internal.h"
#include "prof.h"
#include "status.h"
#include "../../include/ezops_hip.h"

namespace ez {

EZ_PROF_DEFINE(prefill)
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.f;        // log2 headroom of the lazily moved softmax max
constexpr int kPD = 128;            // head dim
constexpr int kPW = 8;              // waves per block: 2 per SIMD, all sharing the block's K/V tiles
constexpr int kBK = 64;             // keys per tile
constexpr int kLPT = kBK * kPD / 8 / (kPW * 64);  // 16-byte DMA loads per thread per K or V tile
typedef float f32x16_t __attribute__((ext_vector_type(16)));

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Value of the other lane half (lane l ^ 32) combined with this lane's.
__device__ __forceinline__ float halves_max(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float halves_sum(float v) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
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

typedef unsigned int u32x4v_t __attribute__((ext_vector_type(4)));

typedef int i32x2_t __attribute__((ext_vector_type(2)));

// LDS fragment reads as asm blocks without a memory clobber, issued apart
// from their waits: the compiler's own wait insertion treats any LDS read
// after an LDS DMA as dependent on every outstanding load and would wait
// (vmcnt 0) for the next tile's prefetch; these reads touch the other
// buffer, and the volatile asm keeps its place between the barriers that
// order them against the DMA into that buffer.  A read group is issued one
// step ahead of its use and waited for by lds_wait8 / lds_waitv, which take
// the registers as operands so that no use is scheduled before the wait.
//
// lds_issue8: the 8 K fragments (k-steps) of 32 key rows.
template <int OFF>
__device__ __forceinline__ void lds_issue8(const uint32_t (&addr)[8], u32x4v_t (&r)[8]) {
  asm volatile(
      "ds_read_b128 %0, %8 offset:%16\n\t"
      "ds_read_b128 %1, %9 offset:%16\n\t"
      "ds_read_b128 %2, %10 offset:%16\n\t"
      "ds_read_b128 %3, %11 offset:%16\n\t"
      "ds_read_b128 %4, %12 offset:%16\n\t"
      "ds_read_b128 %5, %13 offset:%16\n\t"
      "ds_read_b128 %6, %14 offset:%16\n\t"
      "ds_read_b128 %7, %15 offset:%16"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
      : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "v"(addr[4]), "v"(addr[5]), "v"(addr[6]),
        "v"(addr[7]), "i"(OFF));
}
static_assert(kPD / 16 == 8, "lds_issue8 reads the 8 k-steps of a 128-dim key row");
// lds_issue_vt4: the 4 V^T operands (dimension blocks d = 0..3) of one
// 16-key step by transposing reads (ds_read_b64_tr_b16: in each 16-lane
// group, lane m receives element m%4 of the 8-byte rows that lanes m/4,
// 4 + m/4, 8 + m/4 and 12 + m/4 address): r[2d] from addr[d] + OFF,
// r[2d+1] 8 key rows further.
template <int OFF>
__device__ __forceinline__ void lds_issue_vt4(const uint32_t (&addr)[4], i32x2_t (&r)[8]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8 offset:%12\n\t"
      "ds_read_b64_tr_b16 %1, %8 offset:%13\n\t"
      "ds_read_b64_tr_b16 %2, %9 offset:%12\n\t"
      "ds_read_b64_tr_b16 %3, %9 offset:%13\n\t"
      "ds_read_b64_tr_b16 %4, %10 offset:%12\n\t"
      "ds_read_b64_tr_b16 %5, %10 offset:%13\n\t"
      "ds_read_b64_tr_b16 %6, %11 offset:%12\n\t"
      "ds_read_b64_tr_b16 %7, %11 offset:%13"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
      : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "i"(OFF), "i"(OFF + 8 * kPD * 2));
}
static_assert(kPD / 32 == 4, "lds_issue_vt4 reads the 4 dimension blocks of a 128-dim head");
// Waits until at most N LDS reads are outstanding (they complete in order).
template <int N>
__device__ __forceinline__ void lds_wait8(u32x4v_t (&r)[8]) {
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7])
               : "i"(N));
}
template <int N>
__device__ __forceinline__ void lds_waitv(i32x2_t (&r)[8]) {
  asm volatile("s_waitcnt lgkmcnt(%8)"
               : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7])
               : "i"(N));
}

// Block = (query tile, sequence, kv head, head group of HPB = min(G, 4) query
// heads); wave w serves query head kvh*G + hb*HPB + w%HPB, query rows
// 32*(w/HPB) .. +31 of the tile (BQ = 32 * kPW/HPB rows).  K/V tiles of 64
// keys are double-buffered in LDS (one barrier per tile) and shared by the
// block's 8 waves: one block per CU, 2 waves per SIMD, so each tile's DMA
// serves twice the queries of a 4-wave block (T=4096: 200 -> 186 us).
template <int G, bool PAGED>
__global__ __launch_bounds__(kPW * kWave) __attribute__((amdgpu_waves_per_eu(2))) void prefill_attn_kernel(PrefillAttnArgs a, int ntq) {
  EZ_PROF_WAVE(kProfPrefillAttn);
  constexpr int HPB = G < 4 ? G : 4;
  constexpr int NHB = G / HPB;  // head groups per kv head
  constexpr int BQ = 32 * (kPW / HPB);
  __shared__ __align__(16) uint16_t Ks[2][kBK * kPD];        // [key][16B chunk ^ (key & 15)]
  __shared__ __align__(16) uint16_t Vs[2][kBK * kPD];        // [key][16B chunk ^ 4(key & 3)]

  const int per_q = int(a.B * a.Hkv) * NHB;
  const int qt = ntq - 1 - int(blockIdx.x) / per_q;  // longest (last) query tiles first
  int rem = int(blockIdx.x) % per_q;
  const int hb = rem % NHB;
  rem /= NHB;
  const int b = rem / int(a.Hkv), kvh = rem % int(a.Hkv);
  // Offsets and lengths come from device memory: clamp them into Q/Out's T
  // rows and the cache capacity so that no access leaves the buffers.
  const int64_t q0 = min(max(int64_t(a.cu[b]), int64_t(0)), a.T);
  const int64_t qlen0 = min(int64_t(a.cu[b + 1]), a.T) - q0;
  const int64_t past = min(max(a.past ? int64_t(a.past[b]) : 0, int64_t(0)), a.S);
  // rows past the cache capacity are neither read nor written
  const int64_t qlen = min(qlen0, a.S - past);
  if (int64_t(qt) * BQ >= qlen) return;

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int h = lane >> 5, j = lane & 31;
  const int hq = kvh * G + hb * HPB + wave % HPB;
  const int64_t qi0 = int64_t(qt) * BQ + (wave / HPB) * 32;  // first query row (in the sequence) of this wave
  const int64_t qrow = min(qi0 + j, qlen - 1);               // clamped: rows past qlen compute, never store
  const int64_t qpos = past + qrow;                          // its cache position
  const int64_t wave_last = past + min(qi0 + 31, qlen - 1);
  const int64_t kend = past + min(int64_t(qt + 1) * BQ, qlen);  // keys [0, kend) serve this block
  const float sl2 = a.scale * kLog2e;

  bf16x8_t qf[kPD / 16];
  {
    const uint16_t* qp = a.Q + (q0 + qrow) * a.q_rs + int64_t(hq) * kPD + 8 * h;
    uint4 qr[kPD / 16];
#pragma unroll
    for (int s = 0; s < kPD / 16; ++s) qr[s] = *reinterpret_cast<const uint4*>(qp + 16 * s);
    if (!a.q_raw) {
#pragma unroll
      for (int s = 0; s < kPD / 16; ++s) qf[s] = as_bf16x8(qr[s]);
    } else {
      // Fragment s of lane half h holds dims 16 s + 8 h .. +7: this lane has
      // 64 of the head's dims, the other half the rest; RoPE partners (i,
      // i + 64) are fragments s and s + 4 of the same lane.  The weight and
      // cos / sin loads go out with the q loads, unconditionally (a missing
      // table reads q's own row and its values are not used).
      const int64_t crow = qpos * kPD + 8 * h;  // cos / sin row of the query's cache position
      const uint16_t* wp = a.qw ? a.qw + 8 * h : qp;
      const uint16_t* cp = a.qcos ? a.qcos + crow : qp;
      const uint16_t* sp = a.qcos ? a.qsin + crow : qp;
      uint4 wr[kPD / 16], cr[kPD / 16], sr[kPD / 16];
#pragma unroll
      for (int s = 0; s < kPD / 16; ++s) {
        wr[s] = *reinterpret_cast<const uint4*>(wp + 16 * s);
        cr[s] = *reinterpret_cast<const uint4*>(cp + 16 * s);
        sr[s] = *reinterpret_cast<const uint4*>(sp + 16 * s);
      }
      float ss = 0.f;
#pragma unroll
      for (int s = 0; s < kPD / 16; ++s) {
        float x[8];
        unpack8(qr[s], x);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
      }
      const float r = rsqrtf(halves_sum(ss) / float(kPD) + a.qeps);
      const bool use_w = a.qw != nullptr, rope = a.qcos != nullptr;
#pragma unroll
      for (int s = 0; s < kPD / 32; ++s) {
        float y1[8], y2[8], w1[8], w2[8], c1[8], c2[8], s1[8], s2[8];
        unpack8(qr[s], y1);
        unpack8(qr[s + 4], y2);
        unpack8(wr[s], w1);
        unpack8(wr[s + 4], w2);
        unpack8(cr[s], c1);
        unpack8(cr[s + 4], c2);
        unpack8(sr[s], s1);
        unpack8(sr[s + 4], s2);
        float o1[8], o2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          y1[e] = __fmul_rn(y1[e], r);
          y2[e] = __fmul_rn(y2[e], r);
          if (use_w) {
            y1[e] = __fmul_rn(y1[e], w1[e]);
            y2[e] = __fmul_rn(y2[e], w2[e]);
          }
          o1[e] = rope ? __fadd_rn(__fmul_rn(y1[e], c1[e]), __fmul_rn(-y2[e], s1[e])) : y1[e];
          o2[e] = rope ? __fadd_rn(__fmul_rn(y2[e], c2[e]), __fmul_rn(y1[e], s2[e])) : y2[e];
        }
        qf[s] = as_bf16x8(make_uint4(pack_bf2(o1[0], o1[1]), pack_bf2(o1[2], o1[3]), pack_bf2(o1[4], o1[5]),
                                     pack_bf2(o1[6], o1[7])));
        qf[s + 4] = as_bf16x8(make_uint4(pack_bf2(o2[0], o2[1]), pack_bf2(o2[2], o2[3]), pack_bf2(o2[4], o2[5]),
                                         pack_bf2(o2[6], o2[7])));
      }
    }
  }

  f32x16_t o[kPD / 32];
#pragma unroll
  for (int d = 0; d < kPD / 32; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.f;
  float m = -INFINITY, l = 0.f;

  // staging: K chunks id = tid + 256c -> key id/16, chunk id%16; V: keys
  // 4*vm .. 4*vm+3 (vm = tid/16), dims 8*vc .. 8*vc+7 (vc = tid%16)
  // contiguous cache: the (sequence, kv head) slabs, rows addressed in 32 bits
  const uint16_t* kslab = a.K + (int64_t(b) * a.Hkv + kvh) * a.S * kPD;
  const uint16_t* vslab = a.V + (int64_t(b) * a.Hkv + kvh) * a.S * kPD;
  const int kend32 = int(kend);
  // K and V go straight to LDS (16-byte LDS DMA loads): load c of wave w
  // fills LDS chunks 256c + 64w .. +63, one per lane, so lane tid writes
  // chunk p = 256c + tid = (key p/16, slot p%16) and reads the global chunk
  // slot ^ (key & 15) of K (conflict-free 16-byte reads of the S operand)
  // and slot ^ 4(key & 3) of V: the transposing reads of the V^T operand
  // take 4 keys x 64 bytes per 32 lanes, each key in its own 64-byte bank
  // block.
  // Contiguous cache: buffer loads over the slab's first kend rows (rows past
  // them read as zeros, which the causal mask hides and which keep P.V
  // finite), per-lane offsets fixed, the tile's row offset in a scalar.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  __amdgpu_buffer_rsrc_t kres, vres;
  uint32_t koff[kLPT], voff[kLPT];
  if constexpr (!PAGED) {
    kres = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kslab), 0, kend32 * kPD * 2, 0x00020000);
    vres = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vslab), 0, kend32 * kPD * 2, 0x00020000);
#pragma unroll
    for (int c = 0; c < kLPT; ++c) {
      const int id = tid + c * kPW * kWave;
      const int r = id >> 4;
      koff[c] = uint32_t(r * kPD + (((id & 15) ^ (r & 15)) * 8)) * 2;
      voff[c] = uint32_t(r * kPD + (((id & 15) ^ (4 * (r & 3))) * 8)) * 2;
    }
  }
  auto load_tile = [&](int64_t k0, int nb) {
    const int k032 = int(k0);
    if constexpr (!PAGED) {
#pragma unroll
      for (int c = 0; c < kLPT; ++c) {
        const int slot = (c * kPW + wave_u) * kWave * 8;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(kres, (__attribute__((address_space(3))) void*)(&Ks[nb][slot]), 16,
                                                 koff[c], uint32_t(k032) * (kPD * 2), 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vres, (__attribute__((address_space(3))) void*)(&Vs[nb][slot]), 16,
                                                 voff[c], uint32_t(k032) * (kPD * 2), 0, 0);
      }
    } else {  // paged: rows through the block table, clamped to kend
#pragma unroll
      for (int c = 0; c < kLPT; ++c) {
        const int id = tid + c * kPW * kWave;
        const int r = id >> 4;
        const int row = min(k032 + r, kend32 - 1);
        const int kc = (id & 15) ^ (r & 15), vc = (id & 15) ^ (4 * (r & 3));
        const uint16_t* kp = cache_row<PAGED>(a, a.K, b, kvh, row) + kc * 8;
        const uint16_t* vp = cache_row<PAGED>(a, a.V, b, kvh, row) + vc * 8;
        const int slot = (c * kPW + wave) * kWave * 8;
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(kp),
                                         (__attribute__((address_space(3))) void*)(&Ks[nb][slot]), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(vp),
                                         (__attribute__((address_space(3))) void*)(&Vs[nb][slot]), 16, 0, 0);
      }
    }
  };
  load_tile(0, 0);
  wait_vm<0>();  // the first tile has landed before the barrier
  __syncthreads();

  // Per-lane LDS addresses in buffer 0, fixed for the whole loop: K row
  // 32kk + j has the swizzle of row j (32kk is a multiple of 16), so the
  // key block, the buffer and the 16-key step are immediate offsets.
  uint32_t kaddr[kPD / 16];
#pragma unroll
  for (int s = 0; s < kPD / 16; ++s)
    kaddr[s] = uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint16_t*)(&Ks[0][0]))) +
               uint32_t(j * kPD + (((2 * s + h) ^ (j & 15)) * 8)) * 2;
  // V^T operand addresses: lane (i = 16(g%2) + m of 16-lane group g, half
  // h) reads key row 4h + m/4 (+ 16-key step, + 8 for the second half),
  // dims 32d + i - m%4 + 4(m%4) .. +3 = 32d + 16(g%2) + 4(m%4) .. +3.
  uint32_t vaddr[kPD / 32];
  {
    const uint32_t vs_base =
        uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint16_t*)(&Vs[0][0])));
    const int mm = lane & 15, g1 = (lane >> 4) & 1;
    const int vrow = 4 * h + (mm >> 2);
#pragma unroll
    for (int d = 0; d < kPD / 32; ++d) {
      const int ch = 4 * d + 2 * g1 + ((mm & 3) >> 1);
      vaddr[d] = vs_base + uint32_t(vrow * kPD * 2 + ((ch ^ (4 * (vrow & 3))) * 16) + (mm & 1) * 8);
    }
  }
  constexpr uint32_t kBufBytes = kBK * kPD * 2;  // one K (or V) buffer
  const bf16x2_t ones = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);

  // One tile in LDS buffer BUF (a compile-time index: the loop below runs
  // two tiles per iteration).
  auto tile = [&](int64_t k0, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    const bool more = k0 + kBK < kend;
    if (more) load_tile(k0 + kBK, BUF ^ 1);  // next tile's global loads overlap this tile's math

    if (k0 <= wave_last) {  // a wave whose queries all precede the tile skips it
      f32x16_t st[kBK / 32];
      {
        u32x4v_t kf0[kPD / 16], kf1[kPD / 16];
        lds_issue8<BUF * kBufBytes>(kaddr, kf0);
        lds_issue8<BUF * kBufBytes + 32 * kPD * 2>(kaddr, kf1);
#pragma unroll
        for (int kk = 0; kk < kBK / 32; ++kk)
#pragma unroll
          for (int r = 0; r < 16; ++r) st[kk][r] = 0.f;
        lds_wait8<8>(kf0);
#pragma unroll
        for (int s = 0; s < kPD / 16; ++s)
          st[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf0[s]), qf[s], st[0], 0, 0, 0);
        lds_wait8<0>(kf1);
#pragma unroll
        for (int s = 0; s < kPD / 16; ++s)
          st[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf1[s]), qf[s], st[1], 0, 0, 0);
      }
      i32x2_t vfa[2 * (kPD / 32)], vfb[2 * (kPD / 32)];
      lds_issue_vt4<BUF * kBufBytes>(vaddr, vfa);  // V^T of the first 16-key step, under the softmax
      // st[kk][r] = S[query j][key k0 + 32kk + 8(r/4) + 4h + r%4] (unscaled)
      if (k0 + kBK - 1 > past + qi0) {  // diagonal tile: causal mask (32-bit offsets)
        const int lim = int(qpos - k0) - 4 * h;
#pragma unroll
        for (int kk = 0; kk < kBK / 32; ++kk)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (32 * kk + 8 * (r >> 2) + (r & 3) > lim) st[kk][r] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kk = 0; kk < kBK / 32; ++kk)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[kk][r]);
      mx = halves_max(mx) * sl2;
      // Lazy rescale: the reference max m moves (and O, l are rescaled) only
      // when some row's tile max exceeds it by more than kLazy, so the
      // probabilities stay <= 2^kLazy (exact in fp32, the same relative
      // precision in the bf16 P operand) and most tiles skip the 64 rescale
      // multiplies.  The first tile always sets m (m = -inf).
      if (__builtin_amdgcn_ballot_w64(mx > m + kLazy)) {
        const float mn = fmaxf(m, mx);  // finite: key 0 is visible to every query
        const float alpha = __builtin_amdgcn_exp2f(m - mn);
        m = mn;
        l *= alpha;
#pragma unroll
        for (int d = 0; d < kPD / 32; ++d) o[d] *= alpha;
      }
      const float mn = m;
#pragma unroll
      for (int kk = 0; kk < kBK / 32; ++kk) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          // k step of 16 keys (k0 + 32kk + 16u ..): slots 8h..8h+7 = regs 8u..8u+7
          uint32_t w[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(st[kk][8 * u + 2 * q], sl2, -mn));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(st[kk][8 * u + 2 * q + 1], sl2, -mn));
            w[q] = cvt_bf2(p0, p1);
            // the denominator sums the bf16 weights the P.V product uses
            l = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w[q]), ones, l, false);
          }
          const bf16x8_t pb = as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
          // keys 32kk + 16u + 4h + 0..3 and + 8..11 of dims 32d + j
          // the next step's V^T reads go out before this step's wait
          const int t = 2 * kk + u;
          if (t == 0) lds_issue_vt4<BUF * kBufBytes + 16 * kPD * 2>(vaddr, vfb);
          else if (t == 1) lds_issue_vt4<BUF * kBufBytes + 32 * kPD * 2>(vaddr, vfa);
          else if (t == 2) lds_issue_vt4<BUF * kBufBytes + 48 * kPD * 2>(vaddr, vfb);
          i32x2_t(&vf)[2 * (kPD / 32)] = (t & 1) ? vfb : vfa;
          if (t < 3) lds_waitv<8>(vf);
          else lds_waitv<0>(vf);
#pragma unroll
          for (int d = 0; d < kPD / 32; ++d) {
            const bf16x8_t va = __builtin_bit_cast(
                bf16x8_t, (u32x4v_t){uint32_t(vf[2 * d][0]), uint32_t(vf[2 * d][1]), uint32_t(vf[2 * d + 1][0]),
                                     uint32_t(vf[2 * d + 1][1])});
            o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb, o[d], 0, 0, 0);
          }
        }
      }
    }
    if (more) wait_vm<0>();  // the next tile's DMA has landed before the barrier
    __syncthreads();
  };
  for (int64_t k0 = 0; k0 < kend; k0 += 2 * kBK) {
    tile(k0, std::integral_constant<int, 0>{});
    if (k0 + kBK < kend) tile(k0 + kBK, std::integral_constant<int, 1>{});
  }

  // l: this lane's share of query j's sum; the two lane halves add up.
  l = halves_sum(l);
  if (qi0 + j < qlen) {
    const float inv = 1.f / l;
    uint16_t* op = a.Out + (q0 + qi0 + j) * a.o_rs + int64_t(hq) * kPD + 4 * h;
#pragma unroll
    for (int d = 0; d < kPD / 32; ++d)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // o[d][4q + e] = O^T[dim 32d + 8q + 4h + e][query j]
        *reinterpret_cast<uint2*>(op + 32 * d + 8 * q) =
            make_uint2(cvt_bf2(o[d][4 * q] * inv, o[d][4 * q + 1] * inv),
                       cvt_bf2(o[d][4 * q + 2] * inv, o[d][4 * q + 3] * inv));
      }
  }
}

// a[t][i] = silu(gu[t][i]) * gu[t][IS + i], bf16 in/out (the batched SwiGLU
// stage between the gate/up and down GEMMs), 8 elements per thread.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* gu, uint16_t* out, int64_t T, int64_t IS) {
  EZ_PROF_WAVE(kProfSiluMul);
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

namespace {
// Grid of the prefill attention: query tiles of bq = 32 kPW / hpb rows
// (hpb = heads per block) per (sequence, kv head, head group).
int prefill_qtiles(const PrefillAttnArgs& a) {
  const int64_t G = a.H / a.Hkv;
  const int hpb = G < 4 ? int(G) : 4;
  const int bq = 32 * kPW / hpb;
  return int((a.max_q + bq - 1) / bq);
}
int64_t prefill_blocks(const PrefillAttnArgs& a) {
  const int64_t G = a.H / a.Hkv;
  const int hpb = G < 4 ? int(G) : 4;
  return int64_t(prefill_qtiles(a)) * a.B * a.Hkv * (G / hpb);
}
}  // namespace

int check_prefill_attn(const PrefillAttnArgs& a) {
  EZ_REQUIRE(a.Q && a.K && a.V && a.Out && a.cu, "prefill_attn: null pointer");
  EZ_REQUIRE(a.B >= 1 && a.T >= 0 && a.H >= 1 && a.Hkv >= 1 && a.S >= 1 && a.max_q >= 0, "prefill_attn: bad shape");
  EZ_REQUIRE(a.D == kPD, "prefill_attn: head_dim must be %d", kPD);
  EZ_REQUIRE(a.S < (int64_t(1) << 23), "prefill_attn: cache capacity must be below 2^23 rows");
  EZ_REQUIRE(a.H % a.Hkv == 0, "prefill_attn: num_heads must be divisible by num_kv_heads");
  const int64_t G = a.H / a.Hkv;
  EZ_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "prefill_attn: GQA group size must be 1, 2, 4 or 8");
  EZ_REQUIRE(a.q_rs % 8 == 0 && a.o_rs % 4 == 0 && aligned16(a.Q) && aligned16(a.K) && aligned16(a.V),
             "prefill_attn: Q rows and caches must be 16-byte aligned");
  EZ_REQUIRE(!a.block_table || (a.page_size >= 32 && (a.page_size & (a.page_size - 1)) == 0 &&
                                a.S == a.bt_stride * a.page_size && a.num_pages >= 1),
             "prefill_attn: page_size must be a power of two >= 32 and S = max_pages * page_size");
  EZ_REQUIRE(!a.q_raw || ((a.qcos == nullptr) == (a.qsin == nullptr) && (!a.qw || aligned16(a.qw)) &&
                          (!a.qcos || (aligned16(a.qcos) && aligned16(a.qsin)))),
             "prefill_attn: q norm weight and cos / sin tables must be 16-byte aligned, cos and sin together");
  EZ_REQUIRE(prefill_blocks(a) < (int64_t(1) << 31), "prefill_attn: grid too large");
  return EZ_OK;
}

int launch_prefill_attn(const PrefillAttnArgs& a, hipStream_t s) {
  const int rc = check_prefill_attn(a);
  if (rc != EZ_OK) return rc;
  if (a.max_q == 0) return 0;
  PrefillAttnArgs aa = a;
  if (aa.scale <= 0.f) aa.scale = 1.f / sqrtf(float(kPD));
  const int64_t G = a.H / a.Hkv;
  const int ntq = prefill_qtiles(a);
  const int64_t blocks = prefill_blocks(a);
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
                                       const int32_t* cu_seqlens, const int32_t* past_lens, int64_t B, int64_t T,
                                       int64_t H, int64_t Hkv, int64_t S, int64_t D, int64_t max_q_len,
                                       const int32_t* block_table, int64_t num_pages, int64_t page_size,
                                       float scale, hipStream_t stream) {
  ez::PrefillAttnArgs a{};
  a.Q = static_cast<const uint16_t*>(Q); a.q_rs = H * D;
  a.K = static_cast<const uint16_t*>(K); a.V = static_cast<const uint16_t*>(V);
  a.Out = static_cast<uint16_t*>(Out); a.o_rs = H * D;
  a.cu = cu_seqlens; a.past = past_lens;
  a.B = B; a.T = T; a.H = H; a.Hkv = Hkv; a.S = S; a.D = D; a.max_q = max_q_len;
  a.block_table = block_table;
  if (block_table) {
    EZ_REQUIRE(page_size >= 1 && S % page_size == 0, "prefill_attn: S must be a multiple of page_size");
    a.bt_stride = S / page_size; a.page_size = int(page_size); a.num_pages = num_pages;
  }
  a.scale = scale;
  return ez::launch_prefill_attn(a, stream);
}
