// bf16 GEMV and skinny linear layers, Y[M, N] = X[M, K] . W[N, K]^T.
//
// Decode-time projections are HBM-bound: every weight byte is read once and
// used M times.  Two kernels cover the batch range:
//   * gemv_valu (M <= 4): one wave per R weight rows; each lane streams
//     16-byte (8 x bf16) chunks of the row, so one wave instruction reads a
//     fully coalesced 1 KiB of the row; fp32 FMAs; one wave reduction per
//     output.
//   * linear_mfma (M > 4): v_mfma_f32_16x16x32_bf16 on 16-row weight tiles
//     against 16 batch rows; the K range is split over the 4 waves of a
//     block and the partial tiles are summed through LDS.
// Both can fuse the RMSNorm prologue (statistics from the X chunks already
// in registers) and the residual / SwiGLU epilogues of the decode layer.
#include "common.h"
#include "internal.h"
#include "status.h"
#include "../../include/ezops_hip.h"

// Tunables (defaults chosen by measurement on MI355X).
#ifndef EZ_GEMV_BLOCK
#define EZ_GEMV_BLOCK 256   // threads per block of the VALU GEMV
#endif
#ifndef EZ_GEMV_R1
#define EZ_GEMV_R1 2        // weight rows per wave when M == 1
#endif
#ifndef EZ_GEMV_U
#define EZ_GEMV_U 8         // 16-byte chunks per lane in flight per row (M <= 2)
#endif
#ifndef EZ_MFMA_INTERLEAVE
#define EZ_MFMA_INTERLEAVE 0  // 1: wave w takes 128-wide K chunks w, w+4, ... (else a contiguous quarter)
#endif

namespace ez {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kGemvBlock = EZ_GEMV_BLOCK;
constexpr int kGemvWaves = kGemvBlock / kWave;
#ifndef EZ_GEMV_RES_PREFETCH
#define EZ_GEMV_RES_PREFETCH 1
#endif

__device__ __forceinline__ void store_out(const LinearArgs& a, int64_t m, int64_t n, float v,
                                          float v_up) {
  if (a.epi == kEpiStoreF32) {
    reinterpret_cast<float*>(a.Y)[m * a.ldy + n] = v;
    return;
  }
  uint16_t* y = reinterpret_cast<uint16_t*>(a.Y) + m * a.ldy + n;
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
      resv[m][r] = (EZ_GEMV_RES_PREFETCH && a.epi == kEpiResid) ? bf2f(a.res[m * a.ldr + n]) : 0.f;
    }

  float acc[M][R];
  float ss[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    ss[m] = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.f;
  }

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
          for (int e = 0; e < 8; ++e) {
            ss[m] = fmaf(x[e], x[e], ss[m]);
            x[e] *= nw[e];
          }
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
    float scale = 1.f;
    if (NORM) scale = rsqrtf(wave_sum(ss[m]) / float(a.K) + a.eps);
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = wave_sum(acc[m][r]) * scale;
    if (lane == 0) {
      if (SILU) {
        store_out(a, m, n0, v[0], v[1]);
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (n0 + r >= a.N) continue;
          if (EZ_GEMV_RES_PREFETCH && a.epi == kEpiResid)
            reinterpret_cast<uint16_t*>(a.Y)[m * a.ldy + n0 + r] = f2bf(resv[m][r] + round_bf(v[r]));
          else
            store_out(a, m, n0 + r, v[r], 0.f);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA skinny GEMM for 16 batch rows (blockIdx.y selects the 16-row batch
// block).  Block = 4 waves; the block owns T weight tiles of 16 rows and
// wave w accumulates the w-th quarter of the K range (128-wide chunks).
//
// v_mfma_f32_16x16x32_bf16 operands, lane l = 16*g + i (g = l/16, i = l%16):
//   A (weights):  A[i][g*8 .. g*8+7]   = W[row0 + i][k(g, s, 0..7)]
//   B (batch):    B[g*8 .. g*8+7][i]   = X[m0 + i][k(g, s, 0..7)]
//   C:            C[4*g + j][i], j = 0..3  -> weight row row0+4g+j, batch m0+i
// The k-slot assignment k(g, s, e) = k0 + 32*s + 8*g + e (s = sub-step 0..3
// of a 128-wide chunk) is the same for A and B, so the contraction is
// exact, and each wave load instruction reads 64 contiguous bytes (4 lanes)
// of each of its 16 weight rows.
#ifndef EZ_MFMA_XP
#define EZ_MFMA_XP 0  // timing experiments only
#endif
#ifndef EZ_MFMA_T1
#define EZ_MFMA_T1 1  // 16-row weight tiles per wave (sharing each X fragment), plain epilogues
#endif
#ifndef EZ_MFMA_WAVES
#define EZ_MFMA_WAVES 8   // waves per block of the MFMA kernel (the K range is split over them)
#endif
#ifndef EZ_MFMA_STEPS
#define EZ_MFMA_STEPS 8   // 32-wide k-steps per fragment buffer (two buffers in flight)
#endif
constexpr int kMfmaWaves = EZ_MFMA_WAVES;
constexpr int kMfmaSteps = EZ_MFMA_STEPS;
constexpr int kMfmaChunk = 32 * kMfmaSteps;

template <int T>
struct MfmaFrag {
  uint4 w[T][kMfmaSteps];
  uint4 x[kMfmaSteps];
};

template <int T, bool SILU>
__device__ __forceinline__ void mfma_load(MfmaFrag<T>& f, const uint16_t* const (&wrow)[T], const uint16_t* xrow,
                                          bool mvalid, int64_t c, int g, int64_t K) {
  const int64_t kb = c * kMfmaChunk + g * 8;
#pragma unroll
  for (int s = 0; s < kMfmaSteps; ++s) {
    const int64_t k = kb + s * 32;
    const bool ok = k < K;
#pragma unroll
    for (int t = 0; t < T; ++t) f.w[t][s] = ok ? ld16_stream(wrow[t] + k) : make_uint4(0, 0, 0, 0);
#if EZ_MFMA_XP == 1
    f.x[s] = make_uint4(unsigned(k), 1u, 2u, 3u);
#else
    f.x[s] = (ok && mvalid) ? *reinterpret_cast<const uint4*>(xrow + k) : make_uint4(0, 0, 0, 0);
#endif
  }
}

template <int T>
__device__ __forceinline__ void mfma_step(f32x4_t (&acc)[T], const MfmaFrag<T>& f) {
#pragma unroll
  for (int s = 0; s < kMfmaSteps; ++s) {
    const bf16x8_t bx = as_bf16x8(f.x[s]);
#pragma unroll
    for (int t = 0; t < T; ++t)
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(f.w[t][s]), bx, acc[t], 0, 0, 0);
  }
}

template <int T, bool SILU>
__global__ __launch_bounds__(kMfmaWaves * kWave) void linear_mfma_kernel(LinearArgs a) {
  __shared__ float red[kMfmaWaves][T][4][kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int64_t m0 = int64_t(blockIdx.y) * 16;
  const int64_t m = m0 + i;
  const bool mvalid = m < a.M;

  int64_t tile0[T];
  const uint16_t* wrow[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    tile0[t] = SILU ? int64_t(blockIdx.x) * 16 : (int64_t(blockIdx.x) * T + t) * 16;
    int64_t row = tile0[t] + i;
    if (row >= a.N) row = a.N - 1;
    wrow[t] = ((SILU && t == 1) ? a.W2 : a.W) + row * a.K;
  }
  const uint16_t* xrow = a.X + (mvalid ? m : 0) * a.ldx;

  const int64_t nchunks = (a.K + kMfmaChunk - 1) / kMfmaChunk;
#if EZ_MFMA_INTERLEAVE
  const int64_t cb = 0, ce = (nchunks - wave + kMfmaWaves - 1) / kMfmaWaves;  // local chunk count
  auto chunk = [&](int64_t c) { return c * kMfmaWaves + wave; };
#else
  const int64_t cb = nchunks * wave / kMfmaWaves, ce = nchunks * (wave + 1) / kMfmaWaves;
  auto chunk = [&](int64_t c) { return c; };
#endif

  f32x4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Two fragment buffers: chunk c lives in buffer (c - cb) % 2 and its buffer
  // is refilled with chunk c + 2 right after its MFMAs are issued.
  MfmaFrag<T> fa, fb;
  if (cb < ce) mfma_load<T, SILU>(fa, wrow, xrow, mvalid, chunk(cb), g, a.K);
  if (cb + 1 < ce) mfma_load<T, SILU>(fb, wrow, xrow, mvalid, chunk(cb + 1), g, a.K);
  for (int64_t c = cb; c < ce; c += 2) {
    mfma_step<T>(acc, fa);
    if (c + 2 < ce) mfma_load<T, SILU>(fa, wrow, xrow, mvalid, chunk(c + 2), g, a.K);
    if (c + 1 < ce) {
      mfma_step<T>(acc, fb);
      if (c + 3 < ce) mfma_load<T, SILU>(fb, wrow, xrow, mvalid, chunk(c + 3), g, a.K);
    }
  }

#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][t][j][lane] = acc[t][j];
  __syncthreads();

  // Thread tid < 256 finalises output (j, l) = (tid / 64, tid % 64) of every tile.
  if (threadIdx.x >= 4 * kWave) return;
  const int j = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int64_t mo = m0 + (l & 15);
  if (mo >= a.M) return;
  float v[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float sacc = 0.f;
#pragma unroll
    for (int w = 0; w < kMfmaWaves; ++w) sacc += red[w][t][j][l];
    v[t] = sacc;
  }
  const int rofs = 4 * (l >> 4) + j;
  if (SILU) {
    const int64_t n = tile0[0] + rofs;
    if (n < a.N) store_out(a, mo, n, v[0], v[1]);
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int64_t n = tile0[t] + rofs;
      if (n < a.N) store_out(a, mo, n, v[t], 0.f);
    }
  }
}

// ---------------------------------------------------------------------------
// Row-block GEMV, M <= 4 and K = 2048 * CH.  A block of 256 threads owns RB
// output rows (SwiGLU: RB gate rows and the RB matching up rows); thread t
// holds the 16-byte chunks t, t + 256, ... of every row, so each wave
// instruction reads 1 KiB of one row, all weight loads of a thread are issued
// back to back with no bounds branches, and every x chunk a thread loads
// serves all RB rows (x traffic through L2 is 1/RB of the weight traffic).
// Partial sums are reduced per wave (DPP) and across the 4 waves through LDS.
template <int M, int RB, int CH, bool NORM, bool SILU>
__global__ __launch_bounds__(kBlock) void gemv_rows_kernel(LinearArgs a) {
  constexpr int NR = SILU ? 2 * RB : RB;  // weight rows per block
  constexpr int NQ = M * NR + (NORM ? M : 0);
  __shared__ float red[kWavesPerBlock][NQ];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int64_t n0 = int64_t(blockIdx.x) * RB;

  uint4 wv[NR][CH];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const uint16_t* base = (SILU && r >= RB) ? a.W2 : a.W;
    int64_t row = n0 + (r % RB);
    if (row >= a.N) row = a.N - 1;  // tail rows: load a valid row, skip the store
    const uint4* wp = reinterpret_cast<const uint4*>(base + row * a.K) + tid;
#pragma unroll
    for (int j = 0; j < CH; ++j) wv[r][j] = ld16_stream(wp + kBlock * j);
  }
  uint4 xv[M][CH];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int j = 0; j < CH; ++j) xv[m][j] = reinterpret_cast<const uint4*>(a.X + m * a.ldx)[tid + kBlock * j];
  uint4 nv[NORM ? CH : 1];
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < CH; ++j)
      nv[j] = a.norm_w ? reinterpret_cast<const uint4*>(a.norm_w)[tid + kBlock * j]
                       : make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
  }
  // The finishing thread (m, r) fetches its residual with the weight loads.
  uint16_t res_raw = 0;
  if (a.epi == kEpiResid && tid < M * RB) {
    const int64_t n = n0 + tid % RB;
    if (n < a.N) res_raw = a.res[(tid / RB) * a.ldr + n];
  }

  float acc[M][NR], ss[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    ss[m] = 0.f;
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[m][r] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    float nw[8];
    if constexpr (NORM) unpack8(nv[j], nw);
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float x[8];
      unpack8(xv[m][j], x);
      if constexpr (NORM) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          ss[m] = fmaf(x[e], x[e], ss[m]);
          x[e] *= nw[e];
        }
      }
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
  for (int m = 0; m < M; ++m) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const float v = wave_reduce_uniform<false>(acc[m][r]);
      if (lane == 0) red[wave][m * NR + r] = v;
    }
    if constexpr (NORM) {
      const float v = wave_reduce_uniform<false>(ss[m]);
      if (lane == 0) red[wave][M * NR + m] = v;
    }
  }
  __syncthreads();
  if (tid >= M * RB) return;
  const int m = tid / RB, r = tid % RB;
  const int64_t n = n0 + r;
  if (n >= a.N) return;
  float v = 0.f, vu = 0.f, scale = 1.f;
#pragma unroll
  for (int w = 0; w < kWavesPerBlock; ++w) {
    v += red[w][m * NR + r];
    if constexpr (SILU) vu += red[w][m * NR + RB + r];
  }
  if constexpr (NORM) {
    float sq = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) sq += red[w][M * NR + m];
    scale = rsqrtf(sq / float(a.K) + a.eps);
  }
  v *= scale;
  vu *= scale;
  if (a.epi == kEpiResid) {
    reinterpret_cast<uint16_t*>(a.Y)[m * a.ldy + n] = f2bf(bf2f(res_raw) + round_bf(v));
  } else {
    store_out(a, m, n, v, vu);
  }
}

// ---------------------------------------------------------------------------
// LDS-staged MFMA skinny GEMM (M > 4).  The block owns T 16-row weight tiles
// (T = 2: the gate and up tiles of the same rows) and streams K in 512-wide
// chunks.  Weight rows are read with row-contiguous loads (a wave instruction
// covers 4 rows x 256 B... in 16-byte pieces, 1 KiB of each row per chunk),
// parked in registers while the previous chunk is multiplied, then written to
// LDS, from where the MFMA fragments are read.  The 4 waves split each
// chunk's 16 k-steps (wave w takes steps w, w+4, ...) and their partial tiles
// are summed through LDS at the end.
constexpr int kKC = 512;             // K elements per chunk
constexpr int kRowPad = kKC + 8;     // LDS row stride in bf16 (16 B pad against bank conflicts)
constexpr int kPieces = kKC / 8;     // 16-byte pieces per row per chunk

template <int T>
__global__ __launch_bounds__(kBlock) void linear_mfma_lds_kernel(LinearArgs a) {
  constexpr bool SILU = T == 2;
  constexpr int WROWS = 16 * T;
  constexpr int WP = WROWS * kPieces / kBlock;  // weight pieces per thread per chunk
  constexpr int XP = 16 * kPieces / kBlock;     // activation pieces per thread per chunk
  __shared__ __align__(16) uint16_t Ws[WROWS][kRowPad];
  __shared__ __align__(16) uint16_t Xs[16][kRowPad];
  __shared__ float red[kWavesPerBlock][T][4][kWave];

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int64_t m0 = int64_t(blockIdx.y) * 16;
  const int64_t n0 = int64_t(blockIdx.x) * (SILU ? 16 : WROWS);
  const int64_t nchunks = (a.K + kKC - 1) / kKC;

  // Row bases of the pieces this thread stages (piece p = u*kBlock + tid).
  auto wsrc = [&](int u) -> const uint16_t* {
    const int p = u * kBlock + tid, r = p / kPieces;
    int64_t row = n0 + (SILU ? (r & 15) : r);
    if (row >= a.N) row = a.N - 1;
    return ((SILU && r >= 16) ? a.W2 : a.W) + row * a.K + (p % kPieces) * 8;
  };
  auto xsrc = [&](int u) -> const uint16_t* {
    const int p = u * kBlock + tid, r = p / kPieces;
    const int64_t m = m0 + r < a.M ? m0 + r : a.M - 1;
    return a.X + m * a.ldx + (p % kPieces) * 8;
  };

  uint4 wr[WP], xr[XP];
  auto fetch = [&](int64_t c) {
    const int64_t k0 = c * kKC;
#pragma unroll
    for (int u = 0; u < WP; ++u) {
      const int64_t k = k0 + ((u * kBlock + tid) % kPieces) * 8;
      wr[u] = k < a.K ? ld16_stream(wsrc(u) + k0) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < XP; ++u) {
      const int p = u * kBlock + tid;
      const int64_t k = k0 + (p % kPieces) * 8;
      xr[u] = (k < a.K && m0 + p / kPieces < a.M) ? *reinterpret_cast<const uint4*>(xsrc(u) + k0)
                                                   : make_uint4(0, 0, 0, 0);
    }
  };
  auto park = [&]() {
#pragma unroll
    for (int u = 0; u < WP; ++u) {
      const int p = u * kBlock + tid;
      *reinterpret_cast<uint4*>(&Ws[p / kPieces][(p % kPieces) * 8]) = wr[u];
    }
#pragma unroll
    for (int u = 0; u < XP; ++u) {
      const int p = u * kBlock + tid;
      *reinterpret_cast<uint4*>(&Xs[p / kPieces][(p % kPieces) * 8]) = xr[u];
    }
  };

  f32x4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  if (nchunks > 0) fetch(0);
  for (int64_t c = 0; c < nchunks; ++c) {
    __syncthreads();  // previous chunk's fragments have been read
    park();
    __syncthreads();
    if (c + 1 < nchunks) fetch(c + 1);  // next chunk streams while this one is multiplied
#pragma unroll
    for (int s = wave; s < kKC / 32; s += kWavesPerBlock) {
      const bf16x8_t bx = as_bf16x8(*reinterpret_cast<const uint4*>(&Xs[i][32 * s + 8 * g]));
#pragma unroll
      for (int t = 0; t < T; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(*reinterpret_cast<const uint4*>(&Ws[16 * t + i][32 * s + 8 * g])), bx, acc[t], 0, 0, 0);
    }
  }

#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][t][j][lane] = acc[t][j];
  __syncthreads();

  const int j = tid >> 6, l = tid & 63;
  const int64_t mo = m0 + (l & 15);
  if (mo >= a.M) return;
  float v[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float sacc = 0.f;
#pragma unroll
    for (int w = 0; w < kWavesPerBlock; ++w) sacc += red[w][t][j][l];
    v[t] = sacc;
  }
  const int64_t n = n0 + 4 * (l >> 4) + j;
  if (SILU) {
    if (n < a.N) store_out(a, mo, n, v[0], v[1]);
  } else {
#pragma unroll
    for (int t = 0; t < T; ++t)
      if (n + 16 * t < a.N) store_out(a, mo, n + 16 * t, v[t], 0.f);
  }
}

// Scalar fallback for K % 8 != 0 or unaligned operands: one wave per output
// row, plain bf16 loads.
__global__ __launch_bounds__(kBlock) void linear_scalar_kernel(LinearArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t n = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (n >= a.N) return;
  for (int64_t m = 0; m < a.M; ++m) {
    const uint16_t* x = a.X + m * a.ldx;
    float acc = 0.f, acc2 = 0.f, ss = 0.f;
    for (int64_t k = lane; k < a.K; k += kWave) {
      float xv = bf2f(x[k]);
      if (a.norm) {
        ss = fmaf(xv, xv, ss);
        if (a.norm_w) xv *= bf2f(a.norm_w[k]);
      }
      acc = fmaf(bf2f(a.W[n * a.K + k]), xv, acc);
      if (a.epi == kEpiSilu) acc2 = fmaf(bf2f(a.W2[n * a.K + k]), xv, acc2);
    }
    float scale = a.norm ? rsqrtf(wave_sum(ss) / float(a.K) + a.eps) : 1.f;
    acc = wave_sum(acc) * scale;
    acc2 = wave_sum(acc2) * scale;
    if (lane == 0) store_out(a, m, n, acc, acc2);
  }
}

template <int M, bool NORM, bool SILU>
void launch_valu(const LinearArgs& a, hipStream_t s) {
  constexpr int R = SILU ? 2 : (M == 1 ? EZ_GEMV_R1 : 1);
  constexpr int U = M <= 2 ? EZ_GEMV_U : 4;
  const int64_t waves = SILU ? a.N : (a.N + R - 1) / R;
  const int64_t blocks = (waves + kGemvWaves - 1) / kGemvWaves;
  hipLaunchKernelGGL((gemv_valu_kernel<M, R, U, NORM, SILU>), dim3(blocks), dim3(kGemvBlock), 0, s, a);
}

#ifndef EZ_ROWS_RB4K
#define EZ_ROWS_RB4K 4   // rows per block of the row-block GEMV at K = 4096 (SwiGLU: half)
#endif
#ifndef EZ_ROWS_RB12K
#define EZ_ROWS_RB12K 2  // rows per block at K = 12288
#endif
#ifndef EZ_GEMV_ROWS
#define EZ_GEMV_ROWS 1   // 0: always the wave-per-row kernel
#endif

template <int M, int CH, bool NORM, bool SILU>
void launch_rows(const LinearArgs& a, hipStream_t s) {
  constexpr int RB0 = CH <= 2 ? EZ_ROWS_RB4K : EZ_ROWS_RB12K;
  constexpr int RB = SILU ? (RB0 / 2 > 0 ? RB0 / 2 : 1) : RB0;
  const int64_t blocks = (a.N + RB - 1) / RB;
  hipLaunchKernelGGL((gemv_rows_kernel<M, RB, CH, NORM, SILU>), dim3(unsigned(blocks)), dim3(kBlock), 0, s, a);
}

template <int CH, bool NORM, bool SILU>
void launch_rows_m(const LinearArgs& a, hipStream_t s) {
  switch (a.M) {
    case 1: launch_rows<1, CH, NORM, SILU>(a, s); break;
    case 2: launch_rows<2, CH, NORM, SILU>(a, s); break;
    case 3: launch_rows<3, CH, NORM, SILU>(a, s); break;
    default: launch_rows<4, CH, NORM, SILU>(a, s); break;
  }
}

template <bool NORM, bool SILU>
void launch_valu_m(const LinearArgs& a, hipStream_t s) {
  if (EZ_GEMV_ROWS && a.ldx % 8 == 0 && (a.K == 4096 || a.K == 12288)) {
    if (a.K == 4096) launch_rows_m<2, NORM, SILU>(a, s);
    else launch_rows_m<6, NORM, SILU>(a, s);
    return;
  }
  switch (a.M) {
    case 1: launch_valu<1, NORM, SILU>(a, s); break;
    case 2: launch_valu<2, NORM, SILU>(a, s); break;
    case 3: launch_valu<3, NORM, SILU>(a, s); break;
    default: launch_valu<4, NORM, SILU>(a, s); break;
  }
}

#ifndef EZ_MFMA_LDS
#define EZ_MFMA_LDS 0  // 1: LDS-staged MFMA kernel for M > 4; 0: register-operand kernel
#endif

template <bool SILU>
void launch_mfma(const LinearArgs& a, hipStream_t s) {
  constexpr int T = SILU ? 2 : EZ_MFMA_T1;
  const int64_t blocks = SILU ? (a.N + 15) / 16 : (a.N + 16 * T - 1) / (16 * T);
  dim3 grid(unsigned(blocks), unsigned((a.M + 15) / 16));
  if (EZ_MFMA_LDS) {
    const int64_t lblocks = (a.N + 15) / 16;  // one (or one gate+up pair of) 16-row tile(s) per block
    dim3 lgrid(unsigned(lblocks), unsigned((a.M + 15) / 16));
    hipLaunchKernelGGL((linear_mfma_lds_kernel<T>), lgrid, dim3(kBlock), 0, s, a);
  } else {
    hipLaunchKernelGGL((linear_mfma_kernel<T, SILU>), grid, dim3(kMfmaWaves * kWave), 0, s, a);
  }
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
  const bool silu = a.epi == kEpiSilu;
  const bool vec = (a.K % 8 == 0) && (a.ldx % 8 == 0) && aligned16(a.X) && aligned16(a.W) &&
                   (!silu || aligned16(a.W2)) && (!a.norm_w || aligned16(a.norm_w));
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
    // M > 4: the RMSNorm'd input is staged once as bf16(x * rsqrt(mean x^2 +
    // eps) * w) (the reference's staging) into the caller's workspace, then
    // a plain MFMA GEMM runs on it.
    LinearArgs b = a;
    if (a.norm) {
      EZ_REQUIRE(a.xn_ws, "linear: RMSNorm prologue with M > 4 needs a workspace of M*K bf16");
      EZ_REQUIRE(a.ldx == a.K, "linear: RMSNorm prologue with M > 4 needs contiguous X rows");
      const int rc = ezops_rmsnorm_bf16(a.X, a.norm_w, a.xn_ws, a.M, a.K, a.eps, s);
      if (rc) return rc;
      b.X = a.xn_ws;
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
  return (norm && M > 4) ? size_t(M * K) * 2 : 0;
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
