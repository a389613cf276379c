// bf16 GEMV and skinny linear layers, Y[M, N] = X[M, K] . W[N, K]^T.
//
// Decode-time projections are HBM-bound: every weight byte is read once and
// used M times.  The kernels by batch range:
//   * gemv_rows (M <= 4, K <= 16384): a row group of 64-256 threads owns a
//     few weight rows; each thread holds fixed 16-byte chunks of every row,
//     all issued at once, so one wave instruction reads a fully coalesced
//     1 KiB of a row and every x chunk serves all rows of the group.
//   * gemv_valu (M <= 4, longer rows): one wave per R weight rows streaming
//     16-byte chunks in a loop.
//   * linear_mfma (M > 4): v_mfma_f32_16x16x32_bf16 on 16-row weight tiles
//     against 16 batch rows; the K range is split over the 4 waves of a
//     block and the partial tiles are summed through LDS.
// They fuse the RMSNorm prologue (M <= 4: statistics from the x chunks in
// registers, then the reference's bf16 staging of the normalised input;
// M > 4: one staging pass into the workspace) and the residual / SwiGLU
// epilogues of the decode layer.
#include "common.h"
#include "internal.h"
#include "prof.h"
#include "status.h"
#include "../../include/ezops_hip.h"


namespace ez {

EZ_PROF_DEFINE(gemv)
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kGemvBlock = 256;  // threads per block of the wave-per-row GEMV
constexpr int kGemvWaves = kGemvBlock / kWave;

__device__ __forceinline__ void store_out(const LinearArgs& a, int64_t m, int64_t n, float v,
                                          float v_up) {
  if (a.epi == kEpiStoreF32) {
    reinterpret_cast<float*>(a.Y)[m * a.ldy + n] = v;
    return;
  }
  uint16_t* y = reinterpret_cast<uint16_t*>(a.Y) + (a.y_packed ? packed_index(m, n, a.ldy) : m * a.ldy + n);
  if (a.epi == kEpiStore) {
    *y = f2bf(v);
  } else if (a.epi == kEpiResid) {
    *y = f2bf(bf2f(a.res[m * a.ldr + n]) + round_bf(v));
  } else {  // kEpiSilu: bf16 staging as silu(gate) * up on bf16 tensors
    float g = round_bf(v), u = round_bf(v_up);
    *y = f2bf(round_bf(silu(g)) * u);
  }
}

// ---------------------------------------------------------------------------
// VALU GEMV, M <= 4.  Wave w of block b owns R consecutive weight rows
// (kEpiSilu: R = 2 with gate row n and up row n).  U chunks per lane are in
// flight per loop trip.
template <int M, int R, int U, bool NORM, bool SILU>
__global__ __launch_bounds__(kGemvBlock) void gemv_valu_kernel(LinearArgs a) {
  EZ_PROF_WAVE(kProfGemvValu);
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wrow = int64_t(blockIdx.x) * kGemvWaves + (threadIdx.x >> 6);
  const int64_t n0 = SILU ? wrow : wrow * R;
  if (n0 >= a.N) return;

  const int64_t nchunk = a.K >> 3;
  const uint4* wp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint16_t* base = (SILU && r == 1) ? a.W2 : a.W;
    int64_t row = SILU ? n0 : n0 + r;
    if (row >= a.N) row = a.N - 1;  // tail rows: load a valid row, skip the store
    wp[r] = reinterpret_cast<const uint4*>(base + row * a.K);
  }
  const uint4* xp[M];
#pragma unroll
  for (int m = 0; m < M; ++m) xp[m] = reinterpret_cast<const uint4*>(a.X + m * a.ldx);
  const uint4* nwp = reinterpret_cast<const uint4*>(a.norm_w);

  // The residual is requested with the first weight loads, so the epilogue
  // does not wait on a cold load after the reduction.
  float resv[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = SILU ? n0 : (n0 + r < a.N ? n0 + r : a.N - 1);
      resv[m][r] = (a.epi == kEpiResid) ? bf2f(a.res[m * a.ldr + n]) : 0.f;
    }

  // NORM: the row statistics first (x is L2-resident), so that the input
  // can be staged as the reference stages it, bf16(x * rsqrt(mean x^2 + eps) * w).
  float rs[M];
#pragma unroll
  for (int m = 0; m < M; ++m) rs[m] = 1.f;
  if constexpr (NORM) {
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) ss[m] = 0.f;
    for (int64_t c = lane; c < nchunk; c += kWave) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float x[8];
        unpack8(xp[m][c], x);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss[m] = fmaf(x[e], x[e], ss[m]);
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) rs[m] = rsqrtf(wave_sum(ss[m]) / float(a.K) + a.eps);
  }

  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;

  for (int64_t c0 = lane; c0 < nchunk; c0 += int64_t(kWave) * U) {
    uint4 wv[U][R], xv[U][M], nv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + int64_t(kWave) * u;
      const bool ok = c < nchunk;
#pragma unroll
      for (int r = 0; r < R; ++r) wv[u][r] = ok ? ld16_stream(wp[r] + c) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int m = 0; m < M; ++m) xv[u][m] = ok ? xp[m][c] : make_uint4(0, 0, 0, 0);
      if (NORM) nv[u] = (ok && nwp) ? nwp[c] : make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float nw[8];
      if (NORM) unpack8(nv[u], nw);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float x[8];
        unpack8(xv[u][m], x);
        if (NORM) {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = round_bf(x[e] * rs[m] * nw[e]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          float w[8];
          unpack8(wv[u][r], w);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[m][r] = fmaf(w[e], x[e], acc[m][r]);
        }
      }
    }
  }

#pragma unroll
  for (int m = 0; m < M; ++m) {
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = wave_sum(acc[m][r]);
    if (lane == 0) {
      if (SILU) {
        store_out(a, m, n0, v[0], v[1]);
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (n0 + r >= a.N) continue;
          if (a.epi == kEpiResid)
            reinterpret_cast<uint16_t*>(a.Y)[m * a.ldy + n0 + r] = f2bf(resv[m][r] + round_bf(v[r]));
          else
            store_out(a, m, n0 + r, v[r], 0.f);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA skinny GEMM for M > 4 (blockIdx.y selects a 16-row batch block).  The
// block owns one 16-row weight tile (T = 2: the gate and up tiles of the
// same rows) and NW waves split the K range into contiguous 256-wide chunks.
//
// v_mfma_f32_16x16x32_bf16 operands, lane l = 16 g + i:
//   A (weights):  A[i][8g .. 8g+7]  = W[row0 + i][k0 + 32 s + 8 g + 0..7]
//   B (batch):    B[8g .. 8g+7][i]  = X[m0 + i][k0 + 32 s + 8 g + 0..7]
//   C:            C[4g + j][i]      -> weight row row0 + 4g + j, batch m0 + i
// A register of the A operand spans 16 weight rows, so loading it straight
// from HBM reads 64-byte pieces of 16 rows per instruction.  Instead the
// load unit lands each chunk in LDS (buffer_load_dwordx4 ... lds; the wave
// index is uniform, so the LDS destination needs no per-instruction
// readfirstlane) with 512-byte row-contiguous reads, at 16-byte slot
// (r, c ^ r) for piece c of row r; the
// A fragments are then ds_read_b128 with no bank conflicts (the 16 lanes of
// a read hit 16 distinct slot columns).  Every wave owns a two-stage ring of
// such tiles, so the loop has no block barrier.  X fragments (L2-resident
// activations) are loaded straight into registers, one chunk ahead.
constexpr int kMfmaKC = 256;                     // K elements per chunk
constexpr int kMfmaSteps = kMfmaKC / 32;         // MFMA k-steps per chunk
constexpr int kMfmaSlices = 16 * kMfmaKC / 512;  // 1 KiB DMA slices per 16-row tile and chunk



typedef unsigned int u32x4v_t __attribute__((ext_vector_type(4)));

// Reads the 8 A fragments of one chunk (one per k-step) from a DMA-landed
// LDS tile and waits for them.  Written as one asm block without a memory
// clobber: the compiler's own wait insertion treats any LDS read after an
// LDS DMA as dependent on every outstanding load (vmcnt(0)), which would
// drain the two-stage ring; the caller has already waited for exactly this
// stage's DMA (wait_vm), and the volatile asm keeps its place relative to the
// DMA that later refills the stage.
__device__ __forceinline__ void lds_read_a8(const uint32_t (&addr)[kMfmaSteps], u32x4v_t (&r)[kMfmaSteps]) {
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %9\n\t"
      "ds_read_b128 %2, %10\n\t"
      "ds_read_b128 %3, %11\n\t"
      "ds_read_b128 %4, %12\n\t"
      "ds_read_b128 %5, %13\n\t"
      "ds_read_b128 %6, %14\n\t"
      "ds_read_b128 %7, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]), "=&v"(r[7])
      : "v"(addr[0]), "v"(addr[1]), "v"(addr[2]), "v"(addr[3]), "v"(addr[4]), "v"(addr[5]), "v"(addr[6]),
        "v"(addr[7]));
}
static_assert(kMfmaSteps == 8, "lds_read_a8 reads 8 fragments");

// Marks X fragment registers as redefined here, so no use of them (e.g. the
// K-tail select) is scheduled right behind their loads, which would wait for
// them there.
__device__ __forceinline__ void xfrag_fence(u32x4v_t (&x)[kMfmaSteps]) {
  asm volatile("" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]),
                    "+v"(x[7]));
}

// TPB > 1 (with CPW > 0): the block walks tiles blockIdx.x + k * gridDim.x,
// k < TPB, as one stream of chunks, so the ring's DMAs for a tile's first
// chunks are in flight during the previous tile's epilogue.
// R2 > 0 (T = 2, no SwiGLU): the block owns 16 + R2 consecutive rows, the
// second MFMA tile holding rows 16 .. 16 + R2 - 1 (its other rows are never
// loaded and their outputs never stored); both tiles share each X fragment,
// so a block reads X once for 16 + R2 rows.
template <int T, bool SILU, int CPW, int NW, int TPB, int R2 = 0>
__global__ __launch_bounds__(NW * kWave) void linear_mfma_kernel(LinearArgs a) {
  static_assert(R2 == 0 || (T == 2 && !SILU && TPB == 1 && R2 % 2 == 0 && R2 <= 16), "R2: two row tiles");
  constexpr int kRowsPerBlock = R2 ? 16 + R2 : 16;
  EZ_PROF_WAVE(kProfLinearMfma);
  constexpr int XN = kMfmaSteps;         // X loads per chunk
  constexpr int DN = R2 ? kMfmaSlices + R2 / 2 : T * kMfmaSlices;  // DMA slices per chunk
  // One array per ring stage: distinct LDS objects.
  __shared__ __align__(16) uint4 Wl0[NW][T][kMfmaSlices][kWave];
  __shared__ __align__(16) uint4 Wl1[NW][T][kMfmaSlices][kWave];
  __shared__ float red[NW][T][4][kWave];

  const int lane = threadIdx.x & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int64_t m0 = int64_t(blockIdx.y) * 16;
  const int64_t m = m0 + i;
  int64_t row0 = int64_t(blockIdx.x) * kRowsPerBlock;

  // DMA lane roles: slice q of a chunk holds rows 2q, 2q+1 (lanes 0-31, 32-63);
  // lane piece cs = lane & 31 stores the row's 16-byte piece cs ^ r.
  const int dr = lane >> 5, cs = lane & 31;
  // Buffer resources over the tile's rows (reads past them return zeros)
  // and per-lane byte offsets within the tile; the chunk's K offset is the
  // scalar offset of the load.
  __amdgpu_buffer_rsrc_t wres0, wres1;  // (an array of resources drops the kernel's host stub)
  uint32_t woff[kMfmaSlices];
  auto set_rows = [&](int64_t r0) {
    const int64_t rows = a.N - r0 < 16 ? a.N - r0 : 16;
    wres0 = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.W + r0 * a.K), 0, int(rows * a.K * 2),
                                              0x00020000);
    if constexpr (R2 > 0) {  // rows r0 + 16 .. r0 + 16 + R2 - 1 (past N: none, reads return zeros)
      const int64_t rows1 = a.N - r0 - 16 < R2 ? (a.N - r0 - 16 > 0 ? a.N - r0 - 16 : 0) : R2;
      wres1 = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.W + (rows1 ? r0 + 16 : 0) * a.K), 0,
                                                int(rows1 * a.K * 2), 0x00020000);
    } else {
      wres1 = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>((SILU ? a.W2 : a.W) + r0 * a.K), 0,
                                                int(rows * a.K * 2), 0x00020000);
    }
#pragma unroll
    for (int q = 0; q < kMfmaSlices; ++q) {
      int64_t row = 2 * q + dr;
      if (r0 + row >= a.N) row = a.N - 1 - r0;
      woff[q] = uint32_t((row * a.K + int64_t(cs ^ (2 * q + dr)) * 8) * 2);
    }
  };
  set_rows(row0);
  // Rows past M read row 0: their outputs are never stored.
  const uint16_t* xrow = a.X + (m < a.M ? m : 0) * a.ldx;

  const int64_t nchunks = (a.K + kMfmaKC - 1) / kMfmaKC;
  const int64_t cb = nchunks * wave / NW, ce = nchunks * (wave + 1) / NW;

  auto dma = [&](int64_t c, uint4 (*stage)[kMfmaSlices][kWave]) {
    const uint32_t k0b = uint32_t(c * kMfmaKC * 2);  // past K: the next row's weights or zeros, zeroed at use
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int q = 0; q < (R2 && t ? R2 / 2 : kMfmaSlices); ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(t ? wres1 : wres0, (__attribute__((address_space(3))) void*)(&stage[t][q][0]),
                                                 16, woff[q], k0b, 0, 2);
  };
  // Unconditional loads from clamped addresses: no branch around a pending load.
  // Packed X: the fragment of (batch block, k-step) is 1 KiB at a fixed place.
  const uint16_t* xpk = a.X + int64_t(blockIdx.y) * (a.K >> 5) * 512 + lane * 8;
  auto xload = [&](int64_t c, u32x4v_t (&x)[kMfmaSteps]) {
#pragma unroll
    for (int s = 0; s < kMfmaSteps; ++s) {
      const int64_t k = c * kMfmaKC + 32 * s + 8 * g;
      if (a.x_packed) {
        const int64_t ks = c * kMfmaSteps + s;
        x[s] = *reinterpret_cast<const u32x4v_t*>(xpk + (k < a.K ? ks : 0) * 512);
      } else {
        x[s] = *reinterpret_cast<const u32x4v_t*>(xrow + (k < a.K ? k : 0));
      }
    }
  };

  f32x4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const bool ktail = a.K % kMfmaKC != 0;
  auto compute = [&](int64_t c, const uint4 (*stage)[kMfmaSlices][kWave], u32x4v_t (&x)[kMfmaSteps]) {
    xfrag_fence(x);
    u32x4v_t af[T][kMfmaSteps];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      uint32_t addr[kMfmaSteps];
#pragma unroll
      for (int s = 0; s < kMfmaSteps; ++s)
        addr[s] = uint32_t(reinterpret_cast<uintptr_t>(
            (__attribute__((address_space(3))) const uint4*)(&stage[t][i >> 1][(i & 1) * 32 + ((4 * s + g) ^ i)])));
      lds_read_a8(addr, af[t]);
    }
#pragma unroll
    for (int s = 0; s < kMfmaSteps; ++s) {
      u32x4v_t xv = x[s];
      if (ktail && c * kMfmaKC + 32 * s + 8 * g >= a.K) {  // past K: both operands zero
        xv = u32x4v_t{0u, 0u, 0u, 0u};
#pragma unroll
        for (int t = 0; t < T; ++t) af[t][s] = u32x4v_t{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int t = 0; t < T; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af[t][s]),
                                                         __builtin_bit_cast(bf16x8_t, xv), acc[t], 0, 0, 0);
    }
  };

  // Two-stage ring: chunk c lives in stage (c - cb) % 2 and X buffer xa/xb;
  // after its MFMAs the stage is refilled with chunk c + 2.  Issue order per
  // chunk is [DMA slices][X loads], so waiting for chunk c leaves exactly the
  // next chunk's loads outstanding.  CPW > 0 (chunks per wave known at
  // compile time: the model shapes) unrolls the ring completely.
  u32x4v_t xa[kMfmaSteps], xb[kMfmaSteps];
  auto epilogue = [&](int64_t r0) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave][t][j][lane] = acc[t][j];
    __syncthreads();
    // Thread tid < 256 finalises output (j, l) = (tid / 64, tid % 64).
    if (threadIdx.x < 4 * kWave) {
      const int j = threadIdx.x >> 6, l = threadIdx.x & 63;
      const int64_t mo = m0 + (l & 15);
      const int64_t n = r0 + 4 * (l >> 4) + j;
      if (mo < a.M && n < a.N) {
        float v[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
          float sacc = 0.f;
#pragma unroll
          for (int w = 0; w < NW; ++w) sacc += red[w][t][j][l];
          v[t] = sacc;
        }
        if constexpr (R2 > 0) {
          store_out(a, mo, n, v[0], 0.f);
          if (4 * (l >> 4) + j < R2 && n + 16 < a.N) store_out(a, mo, n + 16, v[1], 0.f);
        } else {
          store_out(a, mo, n, v[0], SILU ? v[1] : 0.f);
        }
      }
    }
  };
  if constexpr (TPB < 0) {
    // Streaming blocks: tiles row0, row0 + stride, ... below N (a run-time
    // count), the two-stage ring running on from one tile's chunks into the
    // next tile's, as in the multi-tile blocks.  CPW is even, so chunk cc
    // always lives in stage cc & 1.
    static_assert(CPW > 0 && CPW % 2 == 0 && R2 == 0, "streaming blocks need an even unrolled ring");
    const int64_t stride = int64_t(gridDim.x) * 16;
    dma(cb, Wl0[wave]);
    xload(cb, xa);
    dma(cb + 1, Wl1[wave]);
    xload(cb + 1, xb);
    for (int64_t r = row0; r < a.N; r += stride) {
      const bool more = r + stride < a.N;
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        if (cc + 1 < CPW || more) wait_vm<DN + XN>(); else wait_vm<0>();
        auto& x = (cc & 1) ? xb : xa;
        auto* stage = (cc & 1) ? Wl1[wave] : Wl0[wave];
        compute(cb + cc, stage, x);
        if (cc + 2 < CPW) {
          dma(cb + cc + 2, stage);
          xload(cb + cc + 2, x);
        } else if (more) {  // the next tile's first two chunks
          if (cc + 2 == CPW) set_rows(r + stride);
          dma(cb + cc + 2 - CPW, stage);
          xload(cb + cc + 2 - CPW, x);
        }
      }
      epilogue(r);
#pragma unroll
      for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      __syncthreads();  // red is rewritten by the next tile
    }
    return;
  }
  if constexpr (TPB > 1) {
    static_assert(CPW > 0, "multi-tile blocks need the unrolled ring");
    constexpr int NC = TPB * CPW;
    const int64_t stride = int64_t(gridDim.x) * 16;
    int64_t rn = row0;  // rows of the chunk the next DMA belongs to
    auto dma_idx = [&](int idx, uint4 (*stage)[kMfmaSlices][kWave]) {
      const int64_t r = row0 + int64_t(idx / CPW) * stride;
      if (r != rn) {
        rn = r;
        set_rows(r);
      }
      dma(cb + idx % CPW, stage);
      xload(cb + idx % CPW, (idx & 1) ? xb : xa);
    };
    dma_idx(0, Wl0[wave]);
    dma_idx(1, Wl1[wave]);
#pragma unroll
    for (int idx = 0; idx < NC; ++idx) {
      if (idx + 1 < NC) wait_vm<DN + XN>(); else wait_vm<0>();
      auto& x = (idx & 1) ? xb : xa;
      auto* stage = (idx & 1) ? Wl1[wave] : Wl0[wave];
      compute(cb + idx % CPW, stage, x);
      if (idx + 2 < NC) dma_idx(idx + 2, stage);
      if (idx % CPW == CPW - 1) {  // tile done: reduce across waves and store
        epilogue(row0 + int64_t(idx / CPW) * stride);
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        __syncthreads();  // red is rewritten by the next tile
      }
    }
    return;
  }
  if constexpr (CPW > 0) {
    dma(cb, Wl0[wave]);
    xload(cb, xa);
    if constexpr (CPW > 1) {
      dma(cb + 1, Wl1[wave]);
      xload(cb + 1, xb);
    }
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      if (cc + 1 < CPW) wait_vm<DN + XN>(); else wait_vm<0>();
      auto& x = (cc & 1) ? xb : xa;
      auto* stage = (cc & 1) ? Wl1[wave] : Wl0[wave];
      compute(cb + cc, stage, x);
      if (cc + 2 < CPW) {
        dma(cb + cc + 2, stage);
        xload(cb + cc + 2, x);
      }
    }
  } else {
    if (cb < ce) {
      dma(cb, Wl0[wave]);
      xload(cb, xa);
    }
    if (cb + 1 < ce) {
      dma(cb + 1, Wl1[wave]);
      xload(cb + 1, xb);
    }
    for (int64_t c = cb; c < ce; c += 2) {
      if (c + 1 < ce) wait_vm<DN + XN>(); else wait_vm<0>();
      compute(c, Wl0[wave], xa);
      if (c + 2 < ce) {
        dma(c + 2, Wl0[wave]);
        xload(c + 2, xa);
      }
      if (c + 1 < ce) {
        if (c + 2 < ce) wait_vm<DN + XN>(); else wait_vm<0>();
        compute(c + 1, Wl1[wave], xb);
        if (c + 3 < ce) {
          dma(c + 3, Wl1[wave]);
          xload(c + 3, xb);
        }
      }
    }
  }

  epilogue(row0);
}

// ---------------------------------------------------------------------------
// X-stationary skinny GEMM (M > 4, K = 1024 * CPW): the linear_mfma layout
// (4 waves split K, weight tiles landed in LDS by DMA through a per-wave
// two-stage ring, v_mfma_f32_16x16x32_bf16) with each wave's K slice of the
// 16 batch rows loaded into registers once, before the ring starts, and
// kept for every tile the block walks (TPB tiles: blockIdx.x + k * gridDim.x;
// R2 > 0: one block of 16 + R2 rows, as in linear_mfma).  X is read once
// per block instead of once per tile.
//
// NORM: the RMSNorm prologue inside the kernel.  X is row-major; each lane
// (row i, k-group g) sums the squares of its stationary elements, the four
// lanes of a row and then the four waves (through LDS) complete the row's
// statistics, and every fragment becomes bf16(x * rsqrt(mean x^2 + eps) * w)
// -- the reference's staging (ezops/ops/fused_o_proj_ffn.py:107-110) --
// as its chunk is first used (the norm weights through LDS), while the ring
// streams on.  This replaces the separate staging pass of the batched path.
template <int T, bool SILU, int CPW, int TPB, int R2, bool NORM>
__global__ __launch_bounds__(4 * kWave) void linear_xs_kernel(LinearArgs a) {
  constexpr int NW = 4;
  static_assert(CPW > 0 && CPW % 2 == 0 && TPB >= 1, "unrolled even ring");
  static_assert(R2 == 0 || (T == 2 && !SILU && TPB == 1 && R2 % 2 == 0 && R2 <= 16), "R2: two row tiles");
  constexpr int kRowsPerBlock = R2 ? 16 + R2 : 16;
  EZ_PROF_WAVE(kProfLinearMfma);
  constexpr int DN = R2 ? kMfmaSlices + R2 / 2 : T * kMfmaSlices;  // DMA slices per chunk
  constexpr int NC = TPB * CPW;
  constexpr int kNormW = 4 * CPW * kMfmaKC / 8 / (NW * kWave);    // 16-byte norm-weight pieces per thread
  __shared__ __align__(16) uint4 Wl0[NW][T][kMfmaSlices][kWave];
  __shared__ __align__(16) uint4 Wl1[NW][T][kMfmaSlices][kWave];
  __shared__ float red[NW][T][4][kWave];
  __shared__ __align__(16) float nst[16][NW];  // read back a row at a time (ds_read_b128)
  __shared__ uint4 wl[NORM ? NW * CPW * kMfmaKC / 8 : 1];  // the norm weights (K bf16)

  const int lane = threadIdx.x & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = lane & 15, g = lane >> 4;
  const int64_t m0 = int64_t(blockIdx.y) * 16;
  const int64_t m = m0 + i;
  const int64_t row0 = int64_t(blockIdx.x) * kRowsPerBlock;
  const int64_t stride = int64_t(gridDim.x) * 16;

  const int dr = lane >> 5, cs = lane & 31;
  __amdgpu_buffer_rsrc_t wres0, wres1;
  uint32_t woff[kMfmaSlices];
  auto set_rows = [&](int64_t r0) {
    const int64_t rows = a.N - r0 < 16 ? a.N - r0 : 16;
    wres0 = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.W + r0 * a.K), 0, int(rows * a.K * 2),
                                              0x00020000);
    if constexpr (R2 > 0) {
      const int64_t rows1 = a.N - r0 - 16 < R2 ? (a.N - r0 - 16 > 0 ? a.N - r0 - 16 : 0) : R2;
      wres1 = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a.W + (rows1 ? r0 + 16 : 0) * a.K), 0,
                                                int(rows1 * a.K * 2), 0x00020000);
    } else {
      wres1 = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>((SILU ? a.W2 : a.W) + r0 * a.K), 0,
                                                int(rows * a.K * 2), 0x00020000);
    }
#pragma unroll
    for (int q = 0; q < kMfmaSlices; ++q) {
      int64_t row = 2 * q + dr;
      if (r0 + row >= a.N) row = a.N - 1 - r0;
      woff[q] = uint32_t((row * a.K + int64_t(cs ^ (2 * q + dr)) * 8) * 2);
    }
  };
  auto dma = [&](int64_t c, uint4 (*stage)[kMfmaSlices][kWave]) {
    const uint32_t k0b = uint32_t(c * kMfmaKC * 2);
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int q = 0; q < (R2 && t ? R2 / 2 : kMfmaSlices); ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(t ? wres1 : wres0, (__attribute__((address_space(3))) void*)(&stage[t][q][0]),
                                                 16, woff[q], k0b, 0, 2);
  };

  // The wave's chunks cb .. cb + CPW - 1 (the host checks K = NW * CPW * 256).
  // The stationary X (and with NORM the norm weights, 16 bytes per thread
  // for LDS) are requested first, then the ring's first two DMAs.  LDS is
  // accessed through asm here: the compiler would make any LDS access
  // behind the DMAs wait for all of them.
  const int64_t cb = int64_t(wave) * CPW;
  u32x4v_t xs[CPW][kMfmaSteps];
  uint4 wv[NORM ? kNormW : 1];
  if constexpr (NORM) {
    // Rows past M read row 0: their outputs are never stored.
    const uint16_t* xrow = a.X + (m < a.M ? m : 0) * a.ldx;
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc)
#pragma unroll
      for (int s2 = 0; s2 < kMfmaSteps; ++s2)
        xs[cc][s2] = *reinterpret_cast<const u32x4v_t*>(xrow + (cb + cc) * kMfmaKC + 32 * s2 + 8 * g);
#pragma unroll
    for (int j = 0; j < kNormW; ++j)
      wv[j] = a.norm_w ? reinterpret_cast<const uint4*>(a.norm_w)[threadIdx.x + NW * kWave * j]
                       : make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
  } else {
    const uint16_t* xpk = a.X + int64_t(blockIdx.y) * (a.K >> 5) * 512 + lane * 8;
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc)
#pragma unroll
      for (int s2 = 0; s2 < kMfmaSteps; ++s2)
        xs[cc][s2] = *reinterpret_cast<const u32x4v_t*>(xpk + ((cb + cc) * kMfmaSteps + s2) * 512);
  }
  set_rows(row0);
  dma(cb, Wl0[wave]);
  dma(cb + 1, Wl1[wave]);
  // every DMA goes out before anything waits for X (the scheduler would
  // otherwise interleave the statistics with the DMA issue, which then
  // waits behind the X loads and part of the first chunk)
  __builtin_amdgcn_sched_barrier(0);

  float rs = 1.f;
  const uint32_t wl_base = uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint4*)&wl[0]));
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < kNormW; ++j)
      asm volatile("ds_write_b128 %0, %1" ::"v"(wl_base + (threadIdx.x + NW * kWave * j) * 16u),
                   "v"(__builtin_bit_cast(u32x4v_t, wv[j])));
    // sum of squares of the lane's elements (row i), then the four lanes of
    // row i (i, i + 16, i + 32, i + 48), then the four waves through LDS
    float ss = 0.f;
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc)
#pragma unroll
      for (int s2 = 0; s2 < kMfmaSteps; ++s2) {
        float f[8];
        unpack8(__builtin_bit_cast(uint4, xs[cc][s2]), f);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
      }
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
    ss = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(ss), __float_as_uint(ss), false, false);
    ss = __uint_as_float(q[0]) + __uint_as_float(q[1]);
    const uint32_t na = uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) float*)&nst[i][0]));
    if (g == 0) asm volatile("ds_write_b32 %0, %1" ::"v"(na + wave * 4u), "v"(ss));
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    f32x4_t parts;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(parts) : "v"(na));
    rs = rsqrtf(((parts[0] + parts[1]) + (parts[2] + parts[3])) / float(a.K) + a.eps);
  }
  // Chunk cc of the stationary X normalised in place just before its first
  // use (the ring streams on meanwhile; normalising every chunk up front,
  // under the first two DMAs, measured slower: gate/up 36.1 -> 37.6 us).
  auto normalise = [&](int cc) {
    uint32_t addr[kMfmaSteps];
#pragma unroll
    for (int s2 = 0; s2 < kMfmaSteps; ++s2)
      addr[s2] = wl_base + uint32_t(((cb + cc) * kMfmaKC + 32 * s2 + 8 * g) * 2);
    u32x4v_t wf[kMfmaSteps];
    lds_read_a8(addr, wf);
#pragma unroll
    for (int s2 = 0; s2 < kMfmaSteps; ++s2) {
      float f[8], w[8];
      unpack8(__builtin_bit_cast(uint4, xs[cc][s2]), f);
      unpack8(__builtin_bit_cast(uint4, wf[s2]), w);
      xs[cc][s2] = u32x4v_t{cvt_bf2(f[0] * rs * w[0], f[1] * rs * w[1]), cvt_bf2(f[2] * rs * w[2], f[3] * rs * w[3]),
                            cvt_bf2(f[4] * rs * w[4], f[5] * rs * w[5]), cvt_bf2(f[6] * rs * w[6], f[7] * rs * w[7])};
    }
  };

  f32x4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](const uint4 (*stage)[kMfmaSlices][kWave], const u32x4v_t* x) {
    u32x4v_t af[T][kMfmaSteps];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      uint32_t addr[kMfmaSteps];
#pragma unroll
      for (int s2 = 0; s2 < kMfmaSteps; ++s2)
        addr[s2] = uint32_t(reinterpret_cast<uintptr_t>(
            (__attribute__((address_space(3))) const uint4*)(&stage[t][i >> 1][(i & 1) * 32 + ((4 * s2 + g) ^ i)])));
      lds_read_a8(addr, af[t]);
    }
#pragma unroll
    for (int s2 = 0; s2 < kMfmaSteps; ++s2)
#pragma unroll
      for (int t = 0; t < T; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, af[t][s2]),
                                                         __builtin_bit_cast(bf16x8_t, x[s2]), acc[t], 0, 0, 0);
  };
  auto epilogue = [&](int64_t r0) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave][t][j][lane] = acc[t][j];
    __syncthreads();
    const int j = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int64_t mo = m0 + (l & 15);
    const int64_t n = r0 + 4 * (l >> 4) + j;
    if (mo < a.M && n < a.N) {
      float v[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        float sacc = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) sacc += red[w][t][j][l];
        v[t] = sacc;
      }
      if constexpr (R2 > 0) {
        store_out(a, mo, n, v[0], 0.f);
        if (4 * (l >> 4) + j < R2 && n + 16 < a.N) store_out(a, mo, n + 16, v[1], 0.f);
      } else {
        store_out(a, mo, n, v[0], SILU ? v[1] : 0.f);
      }
    }
  };

  int64_t rn = row0;  // rows of the tile the next DMA belongs to
#pragma unroll
  for (int idx = 0; idx < NC; ++idx) {
    // outstanding once chunk idx has landed: chunk idx + 1's DMA
    if (idx + 1 < NC) wait_vm<DN>(); else wait_vm<0>();
    const int cc = idx % CPW;
    auto* stage = (idx & 1) ? Wl1[wave] : Wl0[wave];
    if constexpr (NORM) {
      if (idx < CPW) normalise(cc);
    }
    compute(stage, xs[cc]);
    if (idx + 2 < NC) {
      const int64_t r = row0 + int64_t((idx + 2) / CPW) * stride;
      if (r != rn) {
        rn = r;
        set_rows(r);
      }
      dma(cb + (idx + 2) % CPW, stage);
    }
    if (cc == CPW - 1) {  // tile done: reduce across waves and store
      epilogue(row0 + int64_t(idx / CPW) * stride);
#pragma unroll
      for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (idx + 1 < NC) __syncthreads();  // red is rewritten by the next tile
    }
  }
}

// ---------------------------------------------------------------------------
// Row-block GEMV, M <= 4 and K % 8 == 0, K <= 16384.  A block of 256
// threads is split into 256 / TPR row groups of TPR threads; each group owns
// RB output rows (SwiGLU: RB gate rows and the RB matching up rows).  Thread
// t of a group holds the 16-byte chunks t, t + TPR, ... (CH of them, the
// last one masked when K / 8 is not a multiple of TPR) of every row, so each
// wave instruction reads 1 KiB of one row, all weight loads of a thread are
// issued back to back, and every x chunk a thread loads serves all RB rows
// (x traffic through L2 is 1/RB of the weight traffic).  Partial sums are
// reduced per wave (DPP) and across the group's waves through LDS.
//
// NORM: the reference's staging xn = bf16(x * rsqrt(mean x^2 + eps) * w)
// (ezops/ops/fused_o_proj_ffn.py:107-110).  x and the norm weights are
// requested before the weight rows; the sum of squares is reduced across
// the group while the weight loads are in flight, then every x chunk is
// normalised and rounded to bf16 before it meets the weights.
template <int M, int RB, int CH, int TPR, bool NORM, bool SILU, bool TAIL>
__global__ __launch_bounds__(kBlock) void gemv_rows_kernel(LinearArgs a) {
  EZ_PROF_WAVE(kProfGemvRows);
  static_assert(TPR % kWave == 0 && kBlock % TPR == 0, "row group geometry");
  constexpr int NR = SILU ? 2 * RB : RB;  // weight rows per group
  constexpr int RG = kBlock / TPR;        // row groups per block
  constexpr int WPG = TPR / kWave;        // waves per row group
  __shared__ float red[kWavesPerBlock][M * NR];
  __shared__ float sred[NORM ? kWavesPerBlock : 1][M];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int grp = tid / TPR, t = tid % TPR;
  const int64_t n0 = (int64_t(blockIdx.x) * RG + grp) * RB;
  // TAIL: K / 8 is not a multiple of TPR and the last chunk is masked.
  const bool last_ok = !TAIL || t + TPR * (CH - 1) < (a.K >> 3);

  uint4 xv[M][CH], wv[NR][CH];
  auto load_w = [&]() {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const uint16_t* base = (SILU && r >= RB) ? a.W2 : a.W;
      int64_t row = n0 + (r % RB);
      if (row >= a.N) row = a.N - 1;  // tail rows: load a valid row, skip the store
      const uint4* wp = reinterpret_cast<const uint4*>(base + row * a.K) + t;
#pragma unroll
      for (int j = 0; j < CH; ++j)
        wv[r][j] = (j + 1 < CH || last_ok) ? ld16_stream(wp + TPR * j) : make_uint4(0, 0, 0, 0);
    }
  };
  auto load_x = [&]() {
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int j = 0; j < CH; ++j)
        xv[m][j] = (j + 1 < CH || last_ok) ? reinterpret_cast<const uint4*>(a.X + m * a.ldx)[t + TPR * j]
                                           : make_uint4(0, 0, 0, 0);
  };
  // A wave's loads complete in order: with NORM the statistics need x
  // first, so x (and the norm weights) are requested ahead of the weight
  // rows; without it the weight rows go first.
  uint4 nv[NORM ? CH : 1];
  if constexpr (NORM) {
    load_x();
#pragma unroll
    for (int j = 0; j < CH; ++j)
      nv[j] = (a.norm_w && (j + 1 < CH || last_ok)) ? reinterpret_cast<const uint4*>(a.norm_w)[t + TPR * j]
                                                    : make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
    load_w();
  } else {
    load_w();
    load_x();
  }
  // The finishing thread (m, r) of each group fetches its residual with the
  // weight loads.
  uint16_t res_raw = 0;
  if (a.epi == kEpiResid && t < M * RB) {
    const int64_t n = n0 + t % RB;
    if (n < a.N) res_raw = a.res[(t / RB) * a.ldr + n];
  }

  if constexpr (NORM) {
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      ss[m] = 0.f;
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        float x[8];
        unpack8(xv[m][j], x);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss[m] = fmaf(x[e], x[e], ss[m]);
      }
      const float v = wave_reduce_uniform<false>(ss[m]);
      if (lane == 0) sred[wave][m] = v;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float sq = 0.f;
#pragma unroll
      for (int w = 0; w < WPG; ++w) sq += sred[grp * WPG + w][m];
      const float rs = rsqrtf(sq / float(a.K) + a.eps);
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        float x[8], g[8];
        unpack8(xv[m][j], x);
        unpack8(nv[j], g);
        xv[m][j] = make_uint4(pack_bf2(x[0] * rs * g[0], x[1] * rs * g[1]), pack_bf2(x[2] * rs * g[2], x[3] * rs * g[3]),
                              pack_bf2(x[4] * rs * g[4], x[5] * rs * g[5]), pack_bf2(x[6] * rs * g[6], x[7] * rs * g[7]));
      }
    }
  }

  float acc[M][NR];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[m][r] = 0.f;
#pragma unroll
  for (int j = 0; j < CH; ++j) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float x[8];
      unpack8(xv[m][j], x);
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        float w[8];
        unpack8(wv[r][j], w);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][r] = fmaf(w[e], x[e], acc[m][r]);
      }
    }
  }

#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const float v = wave_reduce_uniform<false>(acc[m][r]);
      if (lane == 0) red[wave][m * NR + r] = v;
    }
  __syncthreads();
  if (t >= M * RB) return;
  const int m = t / RB, r = t % RB;
  const int64_t n = n0 + r;
  if (n >= a.N) return;
  float v = 0.f, vu = 0.f;
#pragma unroll
  for (int w = 0; w < WPG; ++w) {
    v += red[grp * WPG + w][m * NR + r];
    if constexpr (SILU) vu += red[grp * WPG + w][m * NR + RB + r];
  }
  if (a.epi == kEpiResid) {
    reinterpret_cast<uint16_t*>(a.Y)[m * a.ldy + n] = f2bf(bf2f(res_raw) + round_bf(v));
  } else {
    store_out(a, m, n, v, vu);
  }
}

// Scalar fallback for K % 8 != 0 or unaligned operands: one wave per output
// row, plain bf16 loads.
__global__ __launch_bounds__(kBlock) void linear_scalar_kernel(LinearArgs a) {
  EZ_PROF_WAVE(kProfLinearScalar);
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t n = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (n >= a.N) return;
  for (int64_t m = 0; m < a.M; ++m) {
    const uint16_t* x = a.X + m * a.ldx;
    float rs = 1.f;
    if (a.norm) {  // statistics first, then the reference's bf16 staging of x * rs * w
      float ss = 0.f;
      for (int64_t k = lane; k < a.K; k += kWave) ss = fmaf(bf2f(x[k]), bf2f(x[k]), ss);
      rs = rsqrtf(wave_sum(ss) / float(a.K) + a.eps);
    }
    float acc = 0.f, acc2 = 0.f;
    for (int64_t k = lane; k < a.K; k += kWave) {
      float xv = bf2f(x[k]);
      if (a.norm) xv = round_bf(xv * rs * (a.norm_w ? bf2f(a.norm_w[k]) : 1.f));
      acc = fmaf(bf2f(a.W[n * a.K + k]), xv, acc);
      if (a.epi == kEpiSilu) acc2 = fmaf(bf2f(a.W2[n * a.K + k]), xv, acc2);
    }
    acc = wave_sum(acc);
    acc2 = wave_sum(acc2);
    if (lane == 0) store_out(a, m, n, acc, acc2);
  }
}

template <int M, bool NORM, bool SILU>
void launch_valu(const LinearArgs& a, hipStream_t s) {
  constexpr int R = SILU ? 2 : (M == 1 ? 2 : 1);  // weight rows per wave
  constexpr int U = M <= 2 ? 8 : 4;               // 16-byte chunks per lane in flight per row
  const int64_t waves = SILU ? a.N : (a.N + R - 1) / R;
  const int64_t blocks = (waves + kGemvWaves - 1) / kGemvWaves;
  hipLaunchKernelGGL((gemv_valu_kernel<M, R, U, NORM, SILU>), dim3(blocks), dim3(kGemvBlock), 0, s, a);
}

// Rows per row group of the row-block GEMV, by chunks per thread (measured
// on the Qwen3-8B stages: K = 4096 four rows, the QKV projection ran
// 10.5 / 11.1 / 12.0 us with 4 / 2 / 1; K = 12288 two rows, the down
// projection 17.8 / 18.4 us with 2 / 1; SwiGLU halves them: two gate and
// two up rows, 32.6 us against 34.5 with one each).  More rows lose at the
// layer level (config L, batch 1, three alternating runs each: 83.4-85.8 us
// per layer; four gate + four up rows 86.4-87.1; four down rows alone
// 86.4-86.7; with eight QKV rows as well 87.6-87.8).
constexpr int rows_per_group(int ch, bool silu) { return silu ? (ch <= 2 ? 2 : 1) : (ch <= 2 ? 4 : 2); }

template <int M, int CH, int TPR, bool NORM, bool SILU, bool TAIL>
void launch_rows_t(const LinearArgs& a, hipStream_t s) {
  constexpr int RB = rows_per_group(CH, SILU);
  constexpr int RG = kBlock / TPR;
  // Small matrices (<= 1024 blocks of RB rows): a quarter of the rows per
  // group, so four times the blocks share the ramp (GEMV 4096 x 4096, RB 4 /
  // 2 / 1: 8.0 / 7.7 / 7.5 us; two rows at K = 6144 and 2048 rows, 1024 or
  // 2048 blocks: 6.20 / 6.24 us).
  if constexpr (RB == 4) {
    if ((a.N + RB * RG - 1) / (RB * RG) <= 1024) {
      const int64_t blocks = (a.N + RG - 1) / RG;
      hipLaunchKernelGGL((gemv_rows_kernel<M, 1, CH, TPR, NORM, SILU, TAIL>), dim3(unsigned(blocks)), dim3(kBlock), 0, s, a);
      return;
    }
  }
  const int64_t blocks = (a.N + RB * RG - 1) / (RB * RG);
  hipLaunchKernelGGL((gemv_rows_kernel<M, RB, CH, TPR, NORM, SILU, TAIL>), dim3(unsigned(blocks)), dim3(kBlock), 0, s, a);
}

template <int M, int CH, int TPR, bool NORM, bool SILU>
void launch_rows(const LinearArgs& a, hipStream_t s) {
  if ((a.K >> 3) % TPR != 0) return launch_rows_t<M, CH, TPR, NORM, SILU, true>(a, s);
  launch_rows_t<M, CH, TPR, NORM, SILU, false>(a, s);
}

template <int M, bool NORM, bool SILU>
void launch_rows_ch(const LinearArgs& a, hipStream_t s) {
  const int64_t nchunk = a.K >> 3;
  if (nchunk <= 64) return launch_rows<M, 1, 64, NORM, SILU>(a, s);
  if (nchunk <= 128) return launch_rows<M, 1, 128, NORM, SILU>(a, s);
  switch ((nchunk + kBlock - 1) / kBlock) {
    case 1: return launch_rows<M, 1, 256, NORM, SILU>(a, s);
    case 2: return launch_rows<M, 2, 256, NORM, SILU>(a, s);
    case 3: return launch_rows<M, 3, 256, NORM, SILU>(a, s);
    case 4: return launch_rows<M, 4, 256, NORM, SILU>(a, s);
    case 5: return launch_rows<M, 5, 256, NORM, SILU>(a, s);
    case 6: return launch_rows<M, 6, 256, NORM, SILU>(a, s);
    case 7: return launch_rows<M, 7, 256, NORM, SILU>(a, s);
    default: return launch_rows<M, 8, 256, NORM, SILU>(a, s);
  }
}

// M <= 4: the row-block kernel for K <= 16384 (every K % 8 == 0 reaching
// here), the wave-per-row kernel for longer rows.
constexpr int64_t kRowsMaxK = 8 * 8 * kBlock;

template <bool NORM, bool SILU>
void launch_valu_m(const LinearArgs& a, hipStream_t s) {
  if (a.K <= kRowsMaxK) {
    switch (a.M) {
      case 1: return launch_rows_ch<1, NORM, SILU>(a, s);
      case 2: return launch_rows_ch<2, NORM, SILU>(a, s);
      case 3: return launch_rows_ch<3, NORM, SILU>(a, s);
      default: return launch_rows_ch<4, NORM, SILU>(a, s);
    }
  }
  switch (a.M) {
    case 1: launch_valu<1, NORM, SILU>(a, s); break;
    case 2: launch_valu<2, NORM, SILU>(a, s); break;
    case 3: launch_valu<3, NORM, SILU>(a, s); break;
    default: launch_valu<4, NORM, SILU>(a, s); break;
  }
}

template <bool SILU, int NW, int TPB = 1>
void launch_mfma_nw(const LinearArgs& a, hipStream_t s) {
  constexpr int T = SILU ? 2 : 1;
  const dim3 grid(unsigned((a.N + 15) / 16), unsigned((a.M + 15) / 16)), block(NW * kWave);
  const int64_t nchunks = (a.K + kMfmaKC - 1) / kMfmaKC;
  const int64_t cpw = nchunks % NW == 0 ? nchunks / NW : 0;
#define EZ_MFMA_LAUNCH(C) hipLaunchKernelGGL((linear_mfma_kernel<T, SILU, C, NW, 1>), grid, block, 0, s, a)
  switch (cpw) {
    case 1: EZ_MFMA_LAUNCH(1); break;
    case 2: EZ_MFMA_LAUNCH(2); break;
    case 4: EZ_MFMA_LAUNCH(4); break;
    case 6: EZ_MFMA_LAUNCH(6); break;
    default: EZ_MFMA_LAUNCH(0); break;
  }
#undef EZ_MFMA_LAUNCH
}

// One block of 16 + R2 rows per CU (M <= 16), the two MFMA tiles sharing X.
template <int R2>
void launch_mfma_r2(const LinearArgs& a, hipStream_t s) {
  const dim3 grid(unsigned((a.N + 15 + R2) / (16 + R2))), block(4 * kWave);
  const int64_t nchunks = (a.K + kMfmaKC - 1) / kMfmaKC;
  const int64_t cpw = nchunks % 4 == 0 ? nchunks / 4 : 0;
#define EZ_MFMA_LAUNCH(C) hipLaunchKernelGGL((linear_mfma_kernel<2, false, C, 4, 1, R2>), grid, block, 0, s, a)
  switch (cpw) {
    case 4: EZ_MFMA_LAUNCH(4); break;
    default: EZ_MFMA_LAUNCH(0); break;
  }
#undef EZ_MFMA_LAUNCH
}

// Many 16-row tiles (at least 4 per CU: an LM head): two 4-wave streaming
// blocks per CU, each walking its tiles with one DMA ring.
void launch_mfma_stream(const LinearArgs& a, int64_t cus, hipStream_t s) {
  const int64_t tn = (a.N + 15) / 16;
  const dim3 grid(unsigned(tn < 2 * cus ? tn : 2 * cus), unsigned((a.M + 15) / 16)), block(4 * kWave);
  hipLaunchKernelGGL((linear_mfma_kernel<1, false, 4, 4, -1>), grid, block, 0, s, a);
}

// Blocks of 16 weight rows (T=2: 16 gate + 16 up).  An 8-wave T=1 block
// holds 136 KB of LDS, one per CU; when the tiles outnumber the CUs but not
// twice over (QKV at 6144 rows: 384 tiles), 4-wave blocks (68 KB) share a CU
// two by two so every tile runs in the first round instead of 1.5 rounds.
template <bool SILU>
void launch_mfma(const LinearArgs& a, hipStream_t s) {
  if constexpr (SILU) {
    // gate/up of the model shapes (K = 4096: 4 chunks per wave): 3 or 2
    // tiles per CU run as multi-tile blocks, one per CU.
    const int64_t tx = (a.N + 15) / 16, cus = num_cus();
    const int64_t nchunks = (a.K + kMfmaKC - 1) / kMfmaKC;
    if (nchunks == 16 && a.K % kMfmaKC == 0 && (tx == 3 * cus || tx == 2 * cus)) {
      const dim3 grid(unsigned(cus), unsigned((a.M + 15) / 16)), block(4 * kWave);
      if (tx == 3 * cus) hipLaunchKernelGGL((linear_mfma_kernel<2, true, 4, 4, 3>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((linear_mfma_kernel<2, true, 4, 4, 2>), grid, block, 0, s, a);
      return;
    }
    launch_mfma_nw<true, 4>(a, s);
  } else {
    const int64_t tiles = ((a.N + 15) / 16) * ((a.M + 15) / 16), cus = num_cus();
    // 16 < rows per CU <= 24 (QKV of the model: 6144 rows, 24 per CU): one
    // 24-row block per CU instead of 16-row tiles two to some CUs.
    const int64_t nchunks = (a.K + kMfmaKC - 1) / kMfmaKC;
    if (a.M <= 16 && a.N > 16 * cus && a.N <= 24 * cus) launch_mfma_r2<8>(a, s);
    else if ((a.N + 15) / 16 >= 4 * cus && nchunks == 16 && a.K % kMfmaKC == 0)
      launch_mfma_stream(a, cus, s);
    else if (tiles > cus && tiles <= 2 * cus) launch_mfma_nw<false, 4>(a, s);
    else launch_mfma_nw<false, 8>(a, s);
  }
}

// The batched stages with the RMSNorm prologue (M > 4, K = 4096: four
// 256-wide chunks per wave) run the X-stationary kernel, which normalises in
// its prologue: gate/up with 2 or 3 tiles per CU as multi-tile blocks, the
// 24-row blocks of a QKV-sized projection, and up to one 16-row tile per CU.
// Larger shapes (an LM head) keep the staging pass and the streaming blocks.
bool launch_xs_norm(const LinearArgs& a, hipStream_t s) {
  if (a.K != 4 * 4 * kMfmaKC || a.x_packed) return false;
  const int64_t cus = num_cus(), tx = (a.N + 15) / 16;
  const unsigned gy = unsigned((a.M + 15) / 16);
  const dim3 block(4 * kWave);
  if (a.epi == kEpiSilu) {
    if (tx == 3 * cus) hipLaunchKernelGGL((linear_xs_kernel<2, true, 4, 3, 0, true>), dim3(unsigned(cus), gy), block, 0, s, a);
    else if (tx == 2 * cus) hipLaunchKernelGGL((linear_xs_kernel<2, true, 4, 2, 0, true>), dim3(unsigned(cus), gy), block, 0, s, a);
    else if (tx * gy <= cus) hipLaunchKernelGGL((linear_xs_kernel<2, true, 4, 1, 0, true>), dim3(unsigned(tx), gy), block, 0, s, a);
    else return false;
    return true;
  }
  if (a.M <= 16 && a.N > 16 * cus && a.N <= 24 * cus) {
    hipLaunchKernelGGL((linear_xs_kernel<2, false, 4, 1, 8, true>), dim3(unsigned((a.N + 23) / 24)), block, 0, s, a);
    return true;
  }
  if (tx * gy <= cus) {
    hipLaunchKernelGGL((linear_xs_kernel<1, false, 4, 1, 0, true>), dim3(unsigned(tx), gy), block, 0, s, a);
    return true;
  }
  return false;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

int launch_linear(const LinearArgs& a, hipStream_t s) {
  EZ_REQUIRE(a.X && a.W && a.Y, "linear: null pointer");
  EZ_REQUIRE(a.M >= 1 && a.N >= 1 && a.K >= 1, "linear: sizes must be >= 1 (M=%lld N=%lld K=%lld)",
             (long long)a.M, (long long)a.N, (long long)a.K);
  EZ_REQUIRE(a.epi != kEpiSilu || a.W2, "linear: SwiGLU epilogue needs the up-projection weights");
  EZ_REQUIRE(a.epi != kEpiResid || a.res, "linear: residual epilogue needs the residual");
  EZ_REQUIRE(a.N < (int64_t(1) << 31) / 16 && a.M < 65536 * 16, "linear: sizes too large");
  // The batched kernels address a 16-row weight tile through a buffer
  // resource with 32-bit extents (16 K bf16 < 2^31 bytes).
  EZ_REQUIRE(a.M <= 4 || a.K < (int64_t(1) << 26), "linear: K must be below 2^26 for batch > 4");
  EZ_REQUIRE(!(a.x_packed || a.y_packed) || a.M > 4, "linear: the packed layouts are for M > 4");
  EZ_REQUIRE(!a.x_packed || a.K % 32 == 0, "linear: packed X needs K %% 32 == 0");
  EZ_REQUIRE(!a.y_packed || (a.N % 32 == 0 && a.ldy == a.N && a.epi != kEpiStoreF32),
             "linear: packed Y needs N %% 32 == 0, ldy == N and a bf16 epilogue");
  const bool silu = a.epi == kEpiSilu;
  const bool vec = (a.K % 8 == 0) && (a.ldx % 8 == 0) && aligned16(a.X) && aligned16(a.W) &&
                   (!silu || aligned16(a.W2)) && (!a.norm_w || aligned16(a.norm_w));
  EZ_REQUIRE(vec || !(a.x_packed || a.y_packed), "linear: the packed layouts need 16-byte aligned operands");
  if (!vec) {
    const int64_t blocks = (a.N + kWavesPerBlock - 1) / kWavesPerBlock;
    hipLaunchKernelGGL(linear_scalar_kernel, dim3(blocks), dim3(kBlock), 0, s, a);
  } else if (a.M <= 4) {
    if (a.norm) {
      silu ? launch_valu_m<true, true>(a, s) : launch_valu_m<true, false>(a, s);
    } else {
      silu ? launch_valu_m<false, true>(a, s) : launch_valu_m<false, false>(a, s);
    }
  } else {
    // M > 4 with the RMSNorm prologue: the X-stationary kernel normalises in
    // its prologue where the shape allows (one block per CU: every block
    // loads X once anyway); otherwise the input is staged once as
    // bf16(x * rsqrt(mean x^2 + eps) * w) (the reference's staging) into the
    // caller's workspace and a plain MFMA GEMM runs on it (normalising inside
    // the per-tile kernel repeats the work in every block of 16 weight rows:
    // measured slower than staging).
    LinearArgs b = a;
    EZ_REQUIRE(!a.norm || (a.xn_ws && aligned16(a.xn_ws)),
               "linear: RMSNorm prologue with M > 4 needs a 16-byte aligned workspace (ezops_linear_stage_workspace_size)");
    EZ_REQUIRE(!a.norm || (!a.x_packed && a.ldx == a.K), "linear: RMSNorm prologue with M > 4 needs contiguous X rows");
    if (a.norm && launch_xs_norm(a, s)) return launch_status("linear");
    if (a.norm) {
      int rc;
      if (a.K % 32 == 0) {  // staged straight into the MFMA-packed layout
        rc = launch_rmsnorm_bf16_packed(a.X, a.norm_w, a.xn_ws, a.M, a.K, a.eps, s);
        b.x_packed = 1;
      } else {
        rc = ezops_rmsnorm_bf16(a.X, a.norm_w, a.xn_ws, a.M, a.K, a.eps, s);
      }
      if (rc) return rc;
      b.X = a.xn_ws;
      b.ldx = a.K;
      b.norm = 0;
    }
    silu ? launch_mfma<true>(b, s) : launch_mfma<false>(b, s);
  }
  return launch_status("linear");
}

}  // namespace ez

extern "C" int ezops_gemv_bf16(const void* A, const void* B, void* C, int64_t N, int64_t K,
                               hipStream_t stream) {
  ez::LinearArgs a{};
  a.X = static_cast<const uint16_t*>(A);
  a.ldx = K;
  a.W = static_cast<const uint16_t*>(B);
  a.Y = C;
  a.ldy = N;
  a.M = 1;
  a.N = N;
  a.K = K;
  a.epi = ez::kEpiStore;
  return ez::launch_linear(a, stream);
}

extern "C" int ezops_linear_bf16(const void* X, int64_t ldx, const void* W, void* Y, int64_t ldy,
                                 int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  EZ_REQUIRE(ldx >= K && ldy >= N, "linear: leading dimensions too small");
  ez::LinearArgs a{};
  a.X = static_cast<const uint16_t*>(X);
  a.ldx = ldx;
  a.W = static_cast<const uint16_t*>(W);
  a.Y = Y;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.epi = ez::kEpiStore;
  return ez::launch_linear(a, stream);
}

extern "C" size_t ezops_linear_stage_workspace_size(int64_t M, int64_t K, int norm) {
  return (norm && M > 4) ? size_t(ez::packed_rows(M) * K) * 2 : 0;
}

extern "C" int ezops_linear_stage_bf16(const void* X, int64_t ldx, const void* W, const void* W2, void* Y,
                                       int64_t ldy, const void* res, int64_t ldr, const void* norm_w, int norm,
                                       float eps, int epilogue, int64_t M, int64_t N, int64_t K, void* workspace,
                                       size_t workspace_bytes, hipStream_t stream) {
  EZ_REQUIRE(workspace_bytes >= ezops_linear_stage_workspace_size(M, K, norm), "linear_stage: workspace too small");
  EZ_REQUIRE(epilogue >= ez::kEpiStore && epilogue <= ez::kEpiStoreF32, "linear_stage: epilogue must be 0..3");
  EZ_REQUIRE(ldx >= K && ldy >= N && (epilogue != ez::kEpiResid || ldr >= N),
             "linear_stage: leading dimensions too small");
  ez::LinearArgs a{};
  a.X = static_cast<const uint16_t*>(X);
  a.ldx = ldx;
  a.W = static_cast<const uint16_t*>(W);
  a.W2 = static_cast<const uint16_t*>(W2);
  a.Y = Y;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.res = static_cast<const uint16_t*>(res);
  a.ldr = ldr;
  a.norm = norm != 0;
  a.norm_w = static_cast<const uint16_t*>(norm_w);
  a.eps = eps;
  a.epi = epilogue;
  a.xn_ws = static_cast<uint16_t*>(workspace);
  return ez::launch_linear(a, stream);
}
