// bf16 GEMM for the prefill projections on the gfx950 matrix cores:
//   Y[M, N] = X[M, K] W[N, K]^T            (fp32 accumulation, one bf16 rounding)
//   Y[M, N] = bf16(R[M, N] + bf16(X W^T))  with a residual R (same layout as Y;
//                                           R may be Y itself)
// Both operands are K-contiguous rows, the layout of activations [tokens,
// features] and of weights [out, in].
//
// Block tile 256 x 256, K-steps of 64; 8 waves (2 per SIMD), wave (g, wn)
// owning rows 128 g .. +127 and columns 64 wn .. +63 of the tile: 4 x 2
// v_mfma_f32_32x32x16_bf16 accumulators (128 fp32 per lane).  GEMMs with
// fewer tiles than half the CUs use 256 x 128 tiles (waves of 128 x 32).  Operand layout
// of the 32x32x16 MFMA: lane 32h + i holds A[i][8h .. 8h+7] and
// B[8h .. 8h+7][i]; reg r of lane 32h + j holds C[8(r/4) + 4h + r%4][j].  With
// A = X rows and B[k][n] = W[n][k], both operands are 16-byte pieces of K-rows.
//
// Ping-pong schedule: the two waves of a SIMD belong to the two row groups
// (g = 0: waves 0-3, g = 1: waves 4-7) and run the same code, group 1 one
// block barrier behind, so in every interval between barriers one group
// reads a whole K-step's fragments from LDS (24 ds_read_b128 into 96 VGPRs)
// while the other issues that K-step's 32 MFMAs from registers; the matrix
// pipe of each SIMD is fed by one wave at a time with nothing to wait for.
// (With both waves reading and multiplying in step, a double-buffered
// version ran at 0.7 of this.)
//
// The X and W tiles of a K-step (256 rows x 128 bytes each) land in LDS by
// DMA (buffer_load_dwordx4 ... lds: no staging registers; per-lane offsets
// computed once, the K offset and the 32-row stride in a scalar register),
// in two stages.  Issuing a K-step's 64 KiB costs the CU's address unit
// ~1000 cycles, so it is split: group 0 issues X of step j + 1 after its
// reads of step j (into the other stage, which both groups have finished),
// group 1 issues W of step j + 2 after its reads of step j (the stage both
// groups have just finished).  Each group waits for its own DMA before the
// barrier that precedes the first read of that step; issuing all of it from
// group 0 left the MFMA pipes idle while group 0's reads waited behind it
// (0.8x).  Rows are stored with their 16-byte chunks XOR-swizzled by
// (row >> 1) & 7: gfx950's LDS is 64 banks (256 bytes) wide, and a 16-lane
// phase of a fragment read (16 consecutive 128-byte rows) then covers all 16
// bank groups (SQ_LDS_BANK_CONFLICT 0).  The DMA reads the global chunk that
// belongs at each fixed LDS slot; rows past M / N lie past the end of the
// tile's buffer resource and read zeros (never stored).  Fragment reads are
// asm blocks: the compiler would otherwise wait for outstanding DMA (vmcnt 0)
// in front of every LDS read.
//
// Tiles are dealt to the XCDs in contiguous ranges (block b runs on XCD b % 8)
// and, within a range, in groups of 8 M-tiles (M fastest inside a group), so
// the blocks of one XCD share X and W panels in its L2.
#include "common.h"
#include "internal.h"
#include "prof.h"
#include "status.h"

namespace ez {

EZ_PROF_DEFINE(gemm)
namespace {

constexpr int kGM = 256, kGN = 256, kGK = 64;  // block tile
constexpr int kGWaves = 8;
constexpr int kGThreads = kGWaves * kWave;
constexpr int kGRowBytes = kGK * 2;                      // 128 bytes per tile row
constexpr int kGTileBytes = kGM * kGRowBytes;            // 32 KiB per operand tile
constexpr int kGDma = kGTileBytes / 16 / (kGThreads / 2);  // 16-byte DMA loads per thread of one group and tile
constexpr int kGroupM = 8;                                // M-tiles per tile group
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4v_t __attribute__((ext_vector_type(4)));

struct GemmArgs {
  const uint16_t* X; int64_t ldx;
  const uint16_t* W;
  uint16_t* Y; int64_t ldy;
  const uint16_t* R;
  int64_t M, N, K;
  int tm, tn;  // tiles along M and N
  int64_t IS;  // SwiGLU mode: rows [0, IS) of W are gate, [IS, 2 IS) up; Y is [M, IS]
};

// Fragment reads of one 16-k substep: 4 A pieces (the wave's 4 row tiles)
// and 2 B pieces (its 2 column tiles); frag_wait waits for a K-step's 24
// and, taking them as operands, keeps every use after the wait.
__device__ __forceinline__ void frag_issue(const uint32_t (&addr)[6], u32x4v_t* r) {
  asm volatile(
      "ds_read_b128 %0, %6\n\t"
      "ds_read_b128 %1, %7\n\t"
      "ds_read_b128 %2, %8\n\t"
      "ds_read_b128 %3, %9\n\t"
      "ds_read_b128 %4, %10\n\t"
      "ds_read_b128 %5, %11"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5])
      : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "v"(addr[4]), "v"(addr[5]));
}
// The same for 128-column tiles: 4 A pieces and 1 B piece per substep.
__device__ __forceinline__ void frag_issue(const uint32_t (&addr)[5], u32x4v_t* r) {
  asm volatile(
      "ds_read_b128 %0, %5\n\t"
      "ds_read_b128 %1, %6\n\t"
      "ds_read_b128 %2, %7\n\t"
      "ds_read_b128 %3, %8\n\t"
      "ds_read_b128 %4, %9"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4])
      : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "v"(addr[4]));
}
__device__ __forceinline__ void frag_wait(u32x4v_t (&f)[20]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]),
                 "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]), "+v"(f[12]), "+v"(f[13]), "+v"(f[14]),
                 "+v"(f[15]), "+v"(f[16]), "+v"(f[17]), "+v"(f[18]), "+v"(f[19]));
}
__device__ __forceinline__ void frag_wait(u32x4v_t (&f)[24]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]),
                 "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]), "+v"(f[12]), "+v"(f[13]), "+v"(f[14]),
                 "+v"(f[15]), "+v"(f[16]), "+v"(f[17]), "+v"(f[18]), "+v"(f[19]), "+v"(f[20]), "+v"(f[21]),
                 "+v"(f[22]), "+v"(f[23]));
}

// SWIGLU: the tile's 256 W rows are gate rows n0 .. n0 + 127 and the up rows
// IS + n0 .. +127 of the same features (n0 = 128 x tile column), and the
// epilogue writes silu(gate) * up for those 128 features: the prefill's
// SwiGLU without the [M, 2 IS] intermediate.  Rounding as the separate pass:
// gate and up rounded to bf16, the activation rounded, the product rounded.
// NB: 32-column blocks per wave, 2 for 256-column tiles, 1 for 128-column
// tiles (the same schedule and the same per-element accumulation order over
// K, so both widths give bit-identical results; narrow tiles put twice the
// blocks on the CUs when wide ones would leave most of them idle).
template <bool SWIGLU, int NB>
__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(2))) void gemm_bf16_kernel(GemmArgs a) {
  static_assert(NB == 2 || (NB == 1 && !SWIGLU), "tile widths 256 and 128 (SwiGLU: 256)");
  constexpr int BN = 128 * NB, WC = 32 * NB;     // tile columns, columns per wave
  constexpr int kDmaW = kGDma * NB / 2;         // W loads per thread of group 1 and K-step
  EZ_PROF_WAVE(kProfGemm);
  // Two stages of X and W tiles; after the K loop the same 128 KiB holds the
  // block's C tile in bf16 (16 KiB per wave) for row-contiguous stores.
  __shared__ __align__(16) uint16_t lds[2 * (kGM + BN) * kGK];
  uint16_t(*As)[kGM * kGK] = reinterpret_cast<uint16_t(*)[kGM * kGK]>(&lds[0]);
  uint16_t(*Bs)[BN * kGK] = reinterpret_cast<uint16_t(*)[BN * kGK]>(&lds[2 * kGM * kGK]);

  // tile of this block: XCD-contiguous ranges, groups of kGroupM M-tiles
  const int ntiles = a.tm * a.tn;
  int t = int(blockIdx.x);
  if (ntiles % 8 == 0) t = (t % 8) * (ntiles / 8) + t / 8;
  const int grp = t / (kGroupM * a.tn), gi = t % (kGroupM * a.tn);
  const int gm = a.tm - grp * kGroupM < kGroupM ? a.tm - grp * kGroupM : kGroupM;
  const int64_t m0 = int64_t(grp * kGroupM + gi % gm) * kGM, n0 = int64_t(gi / gm) * (SWIGLU ? kGN / 2 : BN);

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar LDS destinations
  const int g = wave >> 2, wn = wave & 3, wg = wave & 3;  // row group, column slot, wave within the group
  const int h = lane >> 5, i = lane & 31;

  // DMA: load c of group wave wg fills LDS chunk p = (c * 4 + wg) * 64 + lane,
  // tile row 32 c + 8 wg + lane / 8, slot lane % 8, which holds the row's
  // logical chunk slot ^ ((row >> 1) & 7).  The per-lane offset does not
  // depend on c (32 c rows go in the scalar offset).
  const int dr = 8 * wg + (lane >> 3), lc = (lane & 7) ^ ((dr >> 1) & 7);
  const uint32_t aoff = uint32_t((dr * a.ldx + lc * 8) * 2), boff = uint32_t((dr * a.K + lc * 8) * 2);
  const int64_t mrows = a.M - m0 < kGM ? a.M - m0 : kGM, nrows = a.N - n0 < BN ? a.N - n0 : BN;
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.X + m0 * a.ldx), 0, int(((mrows - 1) * a.ldx + a.K) * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.W + n0 * a.K), 0, int((SWIGLU ? kGN / 2 : nrows) * a.K * 2), 0x00020000);
  // SwiGLU: tile rows 128 .. 255 (DMA loads c >= kGDma / 2) come from the up block
  const __amdgpu_buffer_rsrc_t ures = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.W + (SWIGLU ? a.IS + n0 : 0) * a.K), 0, int(kGN / 2 * a.K * 2), 0x00020000);
  auto dma_x = [&](int64_t k0, int buf) {
#pragma unroll
    for (int c = 0; c < kGDma; ++c)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (__attribute__((address_space(3))) void*)(&As[buf][(c * 4 + wg) * kWave * 8]),
                                               16, aoff, uint32_t((k0 + int64_t(c) * 32 * a.ldx) * 2), 0, 0);
  };
  auto dma_w = [&](int64_t k0, int buf) {
#pragma unroll
    for (int c = 0; c < kDmaW; ++c) {
      const bool up = SWIGLU && c >= kGDma / 2;
      const int cr = up ? c - kGDma / 2 : c;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(up ? ures : wres,
                                               (__attribute__((address_space(3))) void*)(&Bs[buf][(c * 4 + wg) * kWave * 8]),
                                               16, boff, uint32_t((k0 + int64_t(cr) * 32 * a.K) * 2), 0, 0);
    }
  };

  // Fragment addresses (bytes within a tile): A row 128 g + 32 ra + i, B row
  // 64 wn + 32 rb + i; substep s reads logical chunk 2s + h.
  uint32_t arow[4], brow[NB];
#pragma unroll
  for (int ra = 0; ra < 4; ++ra) arow[ra] = uint32_t(128 * g + 32 * ra + i);
#pragma unroll
  for (int rb = 0; rb < NB; ++rb) brow[rb] = uint32_t(WC * wn + 32 * rb + i);
  const uint32_t abase[2] = {
      uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint16_t*)(&As[0][0]))),
      uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint16_t*)(&As[1][0])))};
  const uint32_t bbase[2] = {
      uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint16_t*)(&Bs[0][0]))),
      uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint16_t*)(&Bs[1][0])))};

  f32x16_t acc[4][NB];
#pragma unroll
  for (int ra = 0; ra < 4; ++ra)
#pragma unroll
    for (int rb = 0; rb < NB; ++rb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[ra][rb][r] = 0.f;

  constexpr int FS = 4 + NB;  // fragments per substep
  u32x4v_t fr[4 * FS];        // one K-step: fr[FS s + ra] A pieces, fr[FS s + 4 + rb] B pieces
  auto read_step = [&](int buf) {
#pragma unroll
    for (int s = 0; s < kGK / 16; ++s) {
      uint32_t addr[FS];
#pragma unroll
      for (int ra = 0; ra < 4; ++ra)
        addr[ra] = abase[buf] + arow[ra] * kGRowBytes + (((2 * s + h) ^ ((arow[ra] >> 1) & 7)) << 4);
#pragma unroll
      for (int rb = 0; rb < NB; ++rb)
        addr[4 + rb] = bbase[buf] + brow[rb] * kGRowBytes + (((2 * s + h) ^ ((brow[rb] >> 1) & 7)) << 4);
      frag_issue(addr, &fr[FS * s]);
    }
    frag_wait(fr);
  };
  // The last K-step of K % 64 != 0: the 16-byte pieces at or past K hold
  // the next row's elements (or zeros past the buffer); both operands'
  // pieces there are zeroed, so they add nothing.
  auto mask_tail = [&](int64_t k0) {
#pragma unroll
    for (int s = 0; s < kGK / 16; ++s)
      if (k0 + (2 * s + h) * 8 >= a.K)
#pragma unroll
        for (int f = 0; f < FS; ++f) fr[FS * s + f] = u32x4v_t{0u, 0u, 0u, 0u};
  };
  auto mult_step = [&]() {
#pragma unroll
    for (int s = 0; s < kGK / 16; ++s)
#pragma unroll
      for (int ra = 0; ra < 4; ++ra)
#pragma unroll
        for (int rb = 0; rb < NB; ++rb)
          acc[ra][rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, fr[FS * s + ra]),
                                                                __builtin_bit_cast(bf16x8_t, fr[FS * s + 4 + rb]),
                                                                acc[ra][rb], 0, 0, 0);
  };
  auto barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };

  const int64_t nk = (a.K + kGK - 1) / kGK;
  const bool ktail = a.K % kGK != 0;
  // Steps 0 and 1 in flight before the loop (group 1 owns W of step 1).
  if (g == 0) {
    dma_x(0, 0);
    dma_w(0, 0);
  } else if (nk > 1) {
    dma_w(kGK, 1);
  }
  wait_vm<0>();
  __syncthreads();
  if (g == 1) barrier();  // group 1 runs one interval behind
  for (int64_t j = 0; j < nk; ++j) {
    const int buf = int(j & 1);
    read_step(buf);
    if (ktail && j + 1 == nk) mask_tail(j * kGK);
    if (g == 0) {
      if (j + 1 < nk) dma_x((j + 1) * kGK, buf ^ 1);
    } else if (j + 2 < nk) {
      dma_w((j + 2) * kGK, buf);
      __builtin_amdgcn_sched_barrier(0);
      wait_vm<kDmaW>();  // W of step j + 1 (the older loads)
    } else {
      __builtin_amdgcn_sched_barrier(0);
      wait_vm<0>();
    }
    barrier();
    mult_step();
    if (g == 0 && j + 1 < nk) {
      __builtin_amdgcn_sched_barrier(0);
      wait_vm<0>();  // X of step j + 1
    }
    barrier();
  }
  if (g == 0) barrier();  // the same barrier count for both groups

  // Epilogue.  Reg r of lane (h, i) in acc[ra][rb] is C[32 ra + 8(r/4) + 4h +
  // r%4][32 rb + i] of the wave's 128 x WC tile: rounded to bf16 into the
  // wave's LDS slot (row-major, 2 WC bytes a row), then read back 16 bytes a
  // lane (64 / (WC / 8) rows per instruction) for 16-byte stores and residual
  // loads.
  __syncthreads();  // every wave is done with the operand tiles
  uint16_t* ct = &lds[wave * 128 * WC];
#pragma unroll
  for (int ra = 0; ra < 4; ++ra)
#pragma unroll
    for (int rb = 0; rb < NB; ++rb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        ct[(32 * ra + 8 * (r >> 2) + 4 * h + (r & 3)) * WC + 32 * rb + i] = f2bf(acc[ra][rb][r]);
  if constexpr (SWIGLU) {
    // Wave (g, wn) of the group finalises rows 128 g + 32 wn .. +31 of the
    // 128 features; gate column c of the tile lives in wave (g, c / 64), up
    // column c in wave (g, 2 + c / 64).
    __syncthreads();
    for (int q = 0; q < 8; ++q) {
      const int rr = 32 * wn + 4 * q + (lane >> 4), cc = (lane & 15) * 8;  // row in the group, feature
      const int64_t row = m0 + 128 * g + rr;
      if (row >= a.M) continue;
      const uint16_t* gp = &lds[(4 * g + (cc >> 6)) * 128 * 64 + rr * 64 + (cc & 63)];
      const uint4 gv = *reinterpret_cast<const uint4*>(gp);
      const uint4 uv = *reinterpret_cast<const uint4*>(gp + 2 * 128 * 64);
      const uint32_t* g32 = reinterpret_cast<const uint32_t*>(&gv);
      const uint32_t* u32 = reinterpret_cast<const uint32_t*>(&uv);
      uint4 out;
      uint32_t* o32 = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a0 = round_bf(silu(__uint_as_float(g32[e] << 16)));
        const float a1 = round_bf(silu(__uint_as_float(g32[e] & 0xffff0000u)));
        o32[e] = pack_bf2(a0 * __uint_as_float(u32[e] << 16), a1 * __uint_as_float(u32[e] & 0xffff0000u));
      }
      *reinterpret_cast<uint4*>(a.Y + row * a.ldy + n0 + cc) = out;
    }
    return;
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's writes are in LDS before its reads
  const bool vec = a.ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(a.Y) & 15) == 0 &&
                   (!a.R || (reinterpret_cast<uintptr_t>(a.R) & 15) == 0);
  constexpr int LPR = WC / 8, RPI = kWave / LPR;  // lanes per row, rows per instruction
  const int lr = lane / LPR, lcb = (lane % LPR) * 8;
#pragma unroll 4
  for (int q = 0; q < 128 / RPI; ++q) {
    const int rr = RPI * q + lr;
    const int64_t row = m0 + 128 * g + rr, col = n0 + WC * wn + lcb;
    if (row >= a.M || col >= a.N) continue;
    const uint4 cv = *reinterpret_cast<const uint4*>(&ct[rr * WC + lcb]);
    uint16_t* y = a.Y + row * a.ldy + col;
    if (vec && col + 8 <= a.N) {
      uint4 out = cv;
      if (a.R) {
        const uint4 rv = *reinterpret_cast<const uint4*>(a.R + row * a.ldy + col);
        const uint32_t* c32 = reinterpret_cast<const uint32_t*>(&cv);
        const uint32_t* r32 = reinterpret_cast<const uint32_t*>(&rv);
        uint32_t* o32 = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = __uint_as_float(r32[e] << 16) + __uint_as_float(c32[e] << 16);
          const float hi = __uint_as_float(r32[e] & 0xffff0000u) + __uint_as_float(c32[e] & 0xffff0000u);
          o32[e] = uint32_t(f2bf(lo)) | (uint32_t(f2bf(hi)) << 16);
        }
      }
      *reinterpret_cast<uint4*>(y) = out;
    } else {
      const uint16_t* c16 = reinterpret_cast<const uint16_t*>(&cv);
      for (int e = 0; e < 8 && col + e < a.N; ++e)
        y[e] = a.R ? f2bf(bf2f(a.R[row * a.ldy + col + e]) + bf2f(c16[e])) : c16[e];
    }
  }
}

}  // namespace

bool gemm_mfma_supported(const uint16_t* X, int64_t ldx, const uint16_t* W, const uint16_t* Y, int64_t ldy,
                         const uint16_t* R, int64_t M, int64_t N, int64_t K) {
  (void)R;  // R shares Y's leading dimension
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  // 16-byte pieces of K-rows (K % 8 == 0; the last K-step may be partial);
  // the DMA addresses operands by 32-bit byte offsets from their base
  return X && W && Y && M >= 1 && N >= 1 && K >= 8 && K % 8 == 0 && ldx >= K && ldx % 8 == 0 && ldy >= N &&
         al16(X) && al16(W) && (M - 1) * ldx * 2 + K * 2 + kGK * 2 < (int64_t(1) << 31) &&
         (N - 1) * K * 2 + K * 2 + kGK * 2 < (int64_t(1) << 31);
}

int gemm_mfma(const uint16_t* X, int64_t ldx, const uint16_t* W, uint16_t* Y, int64_t ldy, const uint16_t* R,
              int64_t M, int64_t N, int64_t K, hipStream_t s) {
  EZ_REQUIRE(gemm_mfma_supported(X, ldx, W, Y, ldy, R, M, N, K), "gemm: shape or alignment not supported by the MFMA kernel");
  // Fewer 256-wide tiles than half the CUs (short prompts): 128-wide tiles,
  // twice the blocks (o_proj at T = 1024: 85 -> 70 us; same results).  A
  // part-filled last round of a longer GEMM gains nothing from narrow tiles
  // (QKV at T = 4096: 180 us either way): a narrow tile takes nearly as long
  // as a wide one, its X stream and fragment reads being the same.
  const int64_t tm = (M + kGM - 1) / kGM, tn = (N + kGN - 1) / kGN, cus = num_cus();
  if (2 * tm * tn <= cus) {
    GemmArgs a{X, ldx, W, Y, ldy, R, M, N, K, int(tm), int((N + 127) / 128), 0};
    hipLaunchKernelGGL((gemm_bf16_kernel<false, 1>), dim3(unsigned(a.tm * a.tn)), dim3(kGThreads), 0, s, a);
  } else {
    GemmArgs a{X, ldx, W, Y, ldy, R, M, N, K, int(tm), int(tn), 0};
    hipLaunchKernelGGL((gemm_bf16_kernel<false, 2>), dim3(unsigned(a.tm * a.tn)), dim3(kGThreads), 0, s, a);
  }
  return launch_status("gemm (MFMA)");
}

bool gemm_swiglu_supported(const uint16_t* X, int64_t ldx, const uint16_t* W, const uint16_t* Y, int64_t ldy,
                           int64_t M, int64_t IS, int64_t K) {
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return IS >= 1 && IS % (kGN / 2) == 0 && ldy % 8 == 0 && al16(Y) && ldy >= IS &&
         gemm_mfma_supported(X, ldx, W, Y, 2 * IS, nullptr, M, 2 * IS, K);
}

int gemm_swiglu(const uint16_t* X, int64_t ldx, const uint16_t* W, uint16_t* Y, int64_t ldy, int64_t M, int64_t IS,
                int64_t K, hipStream_t s) {
  EZ_REQUIRE(gemm_swiglu_supported(X, ldx, W, Y, ldy, M, IS, K),
             "gemm_swiglu: shape or alignment not supported (IS %% 128, K %% 8, ldx >= K, 16-byte rows)");
  GemmArgs a{X, ldx, W, Y, ldy, nullptr, M, 2 * IS, K, int((M + kGM - 1) / kGM), int(IS / (kGN / 2)), IS};
  hipLaunchKernelGGL((gemm_bf16_kernel<true, 2>), dim3(unsigned(a.tm * a.tn)), dim3(kGThreads), 0, s, a);
  return launch_status("gemm_swiglu (MFMA)");
}

// Prefill GEMM entry: the MFMA kernel for 16-byte K-rows (K % 8 == 0,
// aligned operands); any other shape runs the linear-layer kernels of
// gemv.hip (the residual epilogue rounds as here: bf16(R + bf16(X W^T))).
int gemm_bf16(const uint16_t* X, int64_t ldx, const uint16_t* W, uint16_t* Y, int64_t ldy, const uint16_t* R,
              int64_t M, int64_t N, int64_t K, hipStream_t s) {
  EZ_REQUIRE(X && W && Y, "gemm: null pointer");
  EZ_REQUIRE(M >= 1 && N >= 1 && K >= 1 && ldx >= K && ldy >= N, "gemm: bad shape");
  if (gemm_mfma_supported(X, ldx, W, Y, ldy, R, M, N, K)) return gemm_mfma(X, ldx, W, Y, ldy, R, M, N, K, s);
  LinearArgs l{};
  l.X = X; l.ldx = ldx; l.W = W; l.Y = Y; l.ldy = ldy; l.M = M; l.N = N; l.K = K;
  l.res = R; l.ldr = ldy; l.epi = R ? kEpiResid : kEpiStore;
  return launch_linear(l, s);
}

}  // namespace ez

extern "C" size_t ezops_gemm_workspace_size(void) { return 0; }

extern "C" int ezops_gemm_swiglu_bf16(const void* X, int64_t ldx, const void* Wgu, void* Y, int64_t ldy, int64_t M,
                                      int64_t IS, int64_t K, hipStream_t stream) {
  return ez::gemm_swiglu(static_cast<const uint16_t*>(X), ldx, static_cast<const uint16_t*>(Wgu),
                         static_cast<uint16_t*>(Y), ldy, M, IS, K, stream);
}

extern "C" int ezops_gemm_bf16(const void* X, int64_t ldx, const void* W, void* Y, int64_t ldy, const void* R,
                               int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes, hipStream_t stream) {
  (void)ws;  // no workspace: kept for the ABI
  (void)ws_bytes;
  return ez::gemm_bf16(static_cast<const uint16_t*>(X), ldx, static_cast<const uint16_t*>(W),
                       static_cast<uint16_t*>(Y), ldy, static_cast<const uint16_t*>(R), M, N, K, stream);
}
