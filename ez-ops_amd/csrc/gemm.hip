// bf16 GEMM for the prefill projections on the gfx950 matrix cores:
//   Y[M, N] = X[M, K] W[N, K]^T            (fp32 accumulation, one bf16 rounding)
//   Y[M, N] = bf16(R[M, N] + bf16(X W^T))  with a residual R (same layout as Y;
//                                           R may be Y itself)
// Both operands are K-contiguous rows, the layout of activations [tokens,
// features] and of weights [out, in].
//
// Block tile 256 x 256, K-steps of 64; 8 waves (2 per SIMD), wave (wm, wn)
// owning rows 128 wm .. +127 and columns 64 wn .. +63 of the tile: 4 x 2
// v_mfma_f32_32x32x16_bf16 accumulators (128 fp32 per lane).  Operand layout
// of the 32x32x16 MFMA: lane 32h + i holds A[i][8h .. 8h+7] and
// B[8h .. 8h+7][i]; reg r of lane 32h + j holds C[8(r/4) + 4h + r%4][j].  With
// A = X rows and B[k][n] = W[n][k], both operands are 16-byte pieces of K-rows.
//
// The X and W tiles of a K-step (256 rows x 128 bytes each) land in LDS by
// DMA (buffer_load_dwordx4 ... lds: no staging registers; the per-lane
// offsets are computed once and the K offset rides in a scalar register, so
// issuing a K-step's DMA costs no vector address arithmetic), double-
// buffered, one barrier per K-step.  Rows are stored with their 16-byte
// chunks XOR-swizzled by (row >> 1) & 7: gfx950's LDS is 64 banks (256
// bytes) wide, and a 16-lane phase of a fragment read (16 consecutive
// 128-byte rows) then covers all 16 bank groups (SQ_LDS_BANK_CONFLICT 0; the
// swizzle by row & 7 measured 50% conflict cycles).  The DMA reads the
// global chunk that belongs at each fixed LDS slot.
// Fragment reads are asm blocks: the compiler would otherwise wait for the
// next tile's DMA (vmcnt 0) in front of every LDS read.  The reads of K-step
// s + 1 are issued before the MFMAs of step s and waited for after them
// (scheduling barriers keep that order; without them the compiler hoisted
// the MFMAs above the reads and reused their registers, serialising every
// step).
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
constexpr int kGDma = kGTileBytes / 16 / kGThreads;      // 16-byte DMA loads per thread and operand tile
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
};

// Fragment reads of one K-step (16 k): 4 A pieces (the wave's 4 row tiles)
// and 2 B pieces (its 2 column tiles).  frag_issue starts them; frag_wait
// waits for them and, taking the fragments as operands, keeps every use
// after the wait.
__device__ __forceinline__ void frag_issue(const uint32_t (&addr)[6], u32x4v_t (&r)[6]) {
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
__device__ __forceinline__ void frag_wait(u32x4v_t (&r)[6]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]));
}

__global__ __launch_bounds__(kGThreads) __attribute__((amdgpu_waves_per_eu(2))) void gemm_bf16_kernel(GemmArgs a) {
  EZ_PROF_WAVE(kProfGemm);
  __shared__ __align__(16) uint16_t As[2][kGM * kGK];
  __shared__ __align__(16) uint16_t Bs[2][kGN * kGK];

  // tile of this block: XCD-contiguous ranges, groups of kGroupM M-tiles
  const int ntiles = a.tm * a.tn;
  int t = int(blockIdx.x);
  if (ntiles % 8 == 0) t = (t % 8) * (ntiles / 8) + t / 8;
  const int grp = t / (kGroupM * a.tn), gi = t % (kGroupM * a.tn);
  const int gm = a.tm - grp * kGroupM < kGroupM ? a.tm - grp * kGroupM : kGroupM;
  const int64_t m0 = int64_t(grp * kGroupM + gi % gm) * kGM, n0 = int64_t(gi / gm) * kGN;

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int h = lane >> 5, i = lane & 31;

  // DMA sources: load c of wave w fills LDS chunks p = (c * 8 + w) * 64 + lane
  // (row p / 8, slot p % 8), which holds the row's logical chunk
  // slot ^ ((row >> 1) & 7); byte offsets from the operand base.
  const int wv = __builtin_amdgcn_readfirstlane(wave);  // uniform: LDS destinations in scalar registers
  uint32_t aoff[kGDma], boff[kGDma];
#pragma unroll
  for (int c = 0; c < kGDma; ++c) {
    const int p = (c * kGWaves + wave) * kWave + lane;
    const int r = p >> 3, lc = (p & 7) ^ ((r >> 1) & 7);
    const int64_t xr = m0 + r < a.M ? m0 + r : a.M - 1;  // tail rows: a valid row, never stored
    const int64_t wr = n0 + r < a.N ? n0 + r : a.N - 1;
    aoff[c] = uint32_t((xr * a.ldx + lc * 8) * 2);
    boff[c] = uint32_t((wr * a.K + lc * 8) * 2);
  }
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.X), 0, 0x7fffffff,
                                                                        0x00020000);
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.W), 0, 0x7fffffff,
                                                                        0x00020000);
  auto dma = [&](int64_t k0, int buf) {
#pragma unroll
    for (int c = 0; c < kGDma; ++c) {
      const int slot = (c * kGWaves + wv) * kWave * 8;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (__attribute__((address_space(3))) void*)(&As[buf][slot]), 16,
                                               aoff[c], uint32_t(k0 * 2), 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wres, (__attribute__((address_space(3))) void*)(&Bs[buf][slot]), 16,
                                               boff[c], uint32_t(k0 * 2), 0, 0);
    }
  };

  // Fragment addresses (bytes within a tile): A row 128 wm + 32 ra + i, B row
  // 64 wn + 32 rb + i; K-step s reads logical chunk 2s + h.
  uint32_t arow[4], brow[2];
#pragma unroll
  for (int ra = 0; ra < 4; ++ra) arow[ra] = uint32_t(128 * wm + 32 * ra + i);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) brow[rb] = uint32_t(64 * wn + 32 * rb + i);
  const uint32_t abase[2] = {
      uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint16_t*)(&As[0][0]))),
      uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint16_t*)(&As[1][0])))};
  const uint32_t bbase[2] = {
      uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint16_t*)(&Bs[0][0]))),
      uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint16_t*)(&Bs[1][0])))};

  f32x16_t acc[4][2];
#pragma unroll
  for (int ra = 0; ra < 4; ++ra)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[ra][rb][r] = 0.f;

  const int64_t nk = a.K / kGK;
  dma(0, 0);
  wait_vm<0>();
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int buf = int(kt & 1);
    if (kt + 1 < nk) dma((kt + 1) * kGK, buf ^ 1);  // next K-step's tiles land while this one is multiplied
    auto frag_addr = [&](int s, uint32_t (&addr)[6]) {
#pragma unroll
      for (int ra = 0; ra < 4; ++ra)
        addr[ra] = abase[buf] + arow[ra] * kGRowBytes + (((2 * s + h) ^ ((arow[ra] >> 1) & 7)) << 4);
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
        addr[4 + rb] = bbase[buf] + brow[rb] * kGRowBytes + (((2 * s + h) ^ ((brow[rb] >> 1) & 7)) << 4);
    };
    u32x4v_t f[2][6];
    uint32_t addr[6];
    frag_addr(0, addr);
    frag_issue(addr, f[0]);
#pragma unroll
    for (int s = 0; s < kGK / 16; ++s) {
      frag_wait(f[s & 1]);
      if (s + 1 < kGK / 16) {
        frag_addr(s + 1, addr);
        frag_issue(addr, f[(s + 1) & 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ra = 0; ra < 4; ++ra)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
          acc[ra][rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, f[s & 1][ra]),
                                                                __builtin_bit_cast(bf16x8_t, f[s & 1][4 + rb]),
                                                                acc[ra][rb], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vm<0>();     // the next tiles have landed ...
    __syncthreads();  // ... and every wave is done with this buffer
  }

  // epilogue: reg r of lane (h, j = i) is Y[row0 + 8(r/4) + 4h + r%4][col0 + i]
#pragma unroll
  for (int ra = 0; ra < 4; ++ra)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int64_t col = n0 + 64 * wn + 32 * rb + i;
      const int64_t row0 = m0 + 128 * wm + 32 * ra + 4 * h;
      if (col >= a.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row0 + 8 * (r >> 2) + (r & 3);
        if (row >= a.M) continue;
        uint16_t* y = a.Y + row * a.ldy + col;
        const float v = acc[ra][rb][r];
        *y = a.R ? f2bf(bf2f(a.R[row * a.ldy + col]) + round_bf(v)) : f2bf(v);
      }
    }
}

}  // namespace

bool gemm_mfma_supported(const uint16_t* X, int64_t ldx, const uint16_t* W, const uint16_t* Y, int64_t ldy,
                         const uint16_t* R, int64_t M, int64_t N, int64_t K) {
  (void)Y;
  (void)ldy;
  (void)R;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  // the DMA addresses operands by 32-bit byte offsets from their base
  return K % kGK == 0 && ldx % 8 == 0 && al16(X) && al16(W) && M >= 1 && N >= 1 &&
         (M - 1) * ldx * 2 + K * 2 < (int64_t(1) << 31) && (N - 1) * K * 2 + K * 2 < (int64_t(1) << 31);
}

int gemm_mfma(const uint16_t* X, int64_t ldx, const uint16_t* W, uint16_t* Y, int64_t ldy, const uint16_t* R,
              int64_t M, int64_t N, int64_t K, hipStream_t s) {
  EZ_REQUIRE(gemm_mfma_supported(X, ldx, W, Y, ldy, R, M, N, K), "gemm: shape or alignment not supported by the MFMA kernel");
  GemmArgs a{X, ldx, W, Y, ldy, R, M, N, K, int((M + kGM - 1) / kGM), int((N + kGN - 1) / kGN)};
  hipLaunchKernelGGL(gemm_bf16_kernel, dim3(unsigned(a.tm * a.tn)), dim3(kGThreads), 0, s, a);
  return launch_status("gemm (MFMA)");
}

}  // namespace ez
