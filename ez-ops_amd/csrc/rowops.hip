// Row-wise and whole-tensor fp32/bf16 ops: RMSNorm, softmax, full sum, and
// the STREAM probes used to measure the HBM peak.
//
// Row ops keep the whole row in registers (one HBM read, one write): a block
// of BS threads holds VPT float4 per thread.  Rows longer than the register
// budget, or rows that are not 16-byte aligned, take a looped kernel that
// re-reads the row.
#include "common.h"
#include "internal.h"
#include "prof.h"
#include "status.h"
#include "../../include/ezops_hip.h"

namespace ez {

EZ_PROF_DEFINE(rowops)
namespace {

constexpr float kLog2e = 1.4426950408889634f;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ---------------------------------------------------------------- RMSNorm f32
template <int BS, int VPT>
__global__ __launch_bounds__(BS) void rmsnorm_f32_reg_kernel(const float* __restrict__ X,
                                                              float* __restrict__ Out,
                                                              int64_t dim, float eps) {
  EZ_PROF_WAVE(kProfRmsnormF32);
  __shared__ float red[BS / kWave];
  const int64_t row = blockIdx.x;
  const float4* x = reinterpret_cast<const float4*>(X + row * dim);
  float4* o = reinterpret_cast<float4*>(Out + row * dim);
  const int64_t n4 = dim >> 2;
  float4 v[VPT];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t c = threadIdx.x + int64_t(j) * BS;
    v[j] = c < n4 ? x[c] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int j = 0; j < VPT; ++j) ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
  ss = block_reduce<BS / kWave, false>(ss, red);
  const float r = rsqrtf(ss / float(dim) + eps);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t c = threadIdx.x + int64_t(j) * BS;
    if (c < n4) o[c] = make_float4(v[j].x * r, v[j].y * r, v[j].z * r, v[j].w * r);
  }
}

__global__ __launch_bounds__(256) void rmsnorm_f32_loop_kernel(const float* __restrict__ X,
                                                               float* __restrict__ Out,
                                                               int64_t dim, float eps) {
  EZ_PROF_WAVE(kProfRmsnormF32);
  __shared__ float red[4];
  const float* x = X + int64_t(blockIdx.x) * dim;
  float* o = Out + int64_t(blockIdx.x) * dim;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < dim; i += 256) ss = fmaf(x[i], x[i], ss);
  ss = block_reduce<4, false>(ss, red);
  const float r = rsqrtf(ss / float(dim) + eps);
  for (int64_t i = threadIdx.x; i < dim; i += 256) o[i] = x[i] * r;
}

// ------------------------------------------------------ RMSNorm bf16 + weight
// One block per row; VPT chunks of 8 bf16 per thread.  PACKED writes the
// row into the MFMA-packed layout of the skinny GEMM (dim % 32 == 0).
template <int BS, int VPT, bool PACKED = false>
__global__ __launch_bounds__(BS) void rmsnorm_bf16_reg_kernel(const uint16_t* __restrict__ X,
                                                               const uint16_t* __restrict__ W,
                                                               uint16_t* __restrict__ Out,
                                                               int64_t dim, float eps) {
  EZ_PROF_WAVE(kProfRmsnormBf16);
  __shared__ float red[BS / kWave];
  const int64_t row = blockIdx.x;
  const uint4* x = reinterpret_cast<const uint4*>(X + row * dim);
  const uint4* w = reinterpret_cast<const uint4*>(W);
  uint4* o = reinterpret_cast<uint4*>(Out + row * dim);  // row-major output
  const int64_t n8 = dim >> 3;
  uint4 v[VPT], wv[VPT];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t c = threadIdx.x + int64_t(j) * BS;
    v[j] = c < n8 ? x[c] : make_uint4(0, 0, 0, 0);
  }
  // The weight pieces are requested with the row, not after the reduction.
  constexpr uint32_t one2 = 0x3f803f80u;  // two bf16 1.0
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t c = threadIdx.x + int64_t(j) * BS;
    wv[j] = (W && c < n8) ? w[c] : make_uint4(one2, one2, one2, one2);
  }
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    float f[8];
    unpack8(v[j], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
  }
  ss = block_reduce<BS / kWave, false>(ss, red);
  const float r = rsqrtf(ss / float(dim) + eps);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t c = threadIdx.x + int64_t(j) * BS;
    if (c < n8) {
      float f[8], g[8];
      unpack8(v[j], f);
      unpack8(wv[j], g);
      const uint4 y = make_uint4(pack_bf2(f[0] * r * g[0], f[1] * r * g[1]), pack_bf2(f[2] * r * g[2], f[3] * r * g[3]),
                                 pack_bf2(f[4] * r * g[4], f[5] * r * g[5]), pack_bf2(f[6] * r * g[6], f[7] * r * g[7]));
      if constexpr (PACKED) *reinterpret_cast<uint4*>(Out + packed_index(row, 8 * c, dim)) = y;
      else o[c] = y;
    }
  }
}

__global__ __launch_bounds__(256) void rmsnorm_bf16_loop_kernel(const uint16_t* __restrict__ X,
                                                                const uint16_t* __restrict__ W,
                                                                uint16_t* __restrict__ Out,
                                                                int64_t dim, float eps) {
  EZ_PROF_WAVE(kProfRmsnormBf16);
  __shared__ float red[4];
  const uint16_t* x = X + int64_t(blockIdx.x) * dim;
  uint16_t* o = Out + int64_t(blockIdx.x) * dim;
  float ss = 0.f;
  for (int64_t i = threadIdx.x; i < dim; i += 256) {
    const float f = bf2f(x[i]);
    ss = fmaf(f, f, ss);
  }
  ss = block_reduce<4, false>(ss, red);
  const float r = rsqrtf(ss / float(dim) + eps);
  for (int64_t i = threadIdx.x; i < dim; i += 256)
    o[i] = f2bf(bf2f(x[i]) * r * (W ? bf2f(W[i]) : 1.f));
}

// ------------------------------------------------------------------ softmax
template <int BS, int VPT>
__global__ __launch_bounds__(BS) void softmax_reg_kernel(const float* __restrict__ X,
                                                          float* __restrict__ Out, int64_t dim) {
  EZ_PROF_WAVE(kProfSoftmax);
  __shared__ float red[BS / kWave];
  const int64_t row = blockIdx.x;
  const float4* x = reinterpret_cast<const float4*>(X + row * dim);
  float4* o = reinterpret_cast<float4*>(Out + row * dim);
  const int64_t n4 = dim >> 2;
  float4 v[VPT];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t c = threadIdx.x + int64_t(j) * BS;
    v[j] = c < n4 ? x[c] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
  }
#pragma unroll
  for (int j = 0; j < VPT; ++j) mx = fmaxf(mx, fmaxf(fmaxf(v[j].x, v[j].y), fmaxf(v[j].z, v[j].w)));
  mx = block_reduce<BS / kWave, true>(mx, red);
  const float mb = mx * kLog2e;
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    v[j].x = exp2f(fmaf(v[j].x, kLog2e, -mb));
    v[j].y = exp2f(fmaf(v[j].y, kLog2e, -mb));
    v[j].z = exp2f(fmaf(v[j].z, kLog2e, -mb));
    v[j].w = exp2f(fmaf(v[j].w, kLog2e, -mb));
    sum += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  }
  sum = block_reduce<BS / kWave, false>(sum, red);
  const float inv = 1.0f / sum;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int64_t c = threadIdx.x + int64_t(j) * BS;
    if (c < n4) o[c] = make_float4(v[j].x * inv, v[j].y * inv, v[j].z * inv, v[j].w * inv);
  }
}

__global__ __launch_bounds__(1024) void softmax_loop_kernel(const float* __restrict__ X,
                                                            float* __restrict__ Out, int64_t dim) {
  EZ_PROF_WAVE(kProfSoftmax);
  __shared__ float red[16];
  const float* x = X + int64_t(blockIdx.x) * dim;
  float* o = Out + int64_t(blockIdx.x) * dim;
  float mx = -INFINITY;
  for (int64_t i = threadIdx.x; i < dim; i += 1024) mx = fmaxf(mx, x[i]);
  mx = block_reduce<16, true>(mx, red);
  const float mb = mx * kLog2e;
  float sum = 0.f;
  for (int64_t i = threadIdx.x; i < dim; i += 1024) sum += exp2f(fmaf(x[i], kLog2e, -mb));
  sum = block_reduce<16, false>(sum, red);
  const float inv = 1.0f / sum;
  for (int64_t i = threadIdx.x; i < dim; i += 1024) o[i] = exp2f(fmaf(x[i], kLog2e, -mb)) * inv;
}

// --------------------------------------------------------------- full sum
// Stage 1: block b sums a fixed, strided share of the float4s into
// partial[b]; the last block to finish sums partial[0..G) in index order.
// The grid size depends only on n, so the result is bitwise reproducible.
constexpr int kSumBlock = 256;
constexpr int kSumUnroll = 8;
constexpr int kSumMaxBlocks = 1024;

int64_t sum_blocks(int64_t n) {
  const int64_t per_block = int64_t(kSumBlock) * 4 * kSumUnroll;
  int64_t g = (n + per_block - 1) / per_block;
  if (g < 1) g = 1;
  return g > kSumMaxBlocks ? kSumMaxBlocks : g;
}

__global__ __launch_bounds__(kSumBlock) void sum_kernel(const float* __restrict__ A, int64_t n,
                                                        bool vec, float* __restrict__ partial,
                                                        int* counter, float* __restrict__ Out) {
  EZ_PROF_WAVE(kProfSum);
  __shared__ float red[kSumBlock / kWave];
  const int64_t G = gridDim.x;
  const int64_t stride = G * kSumBlock;
  float acc[kSumUnroll];
#pragma unroll
  for (int u = 0; u < kSumUnroll; ++u) acc[u] = 0.f;
  int64_t tail_start = 0;
  if (vec) {
    const float4* a4 = reinterpret_cast<const float4*>(A);
    const int64_t n4 = n >> 2;
    int64_t i = int64_t(blockIdx.x) * kSumBlock + threadIdx.x;
    for (; i + (kSumUnroll - 1) * stride < n4; i += kSumUnroll * stride) {
      float4 v[kSumUnroll];
#pragma unroll
      for (int u = 0; u < kSumUnroll; ++u) v[u] = a4[i + u * stride];
#pragma unroll
      for (int u = 0; u < kSumUnroll; ++u) acc[u] += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    for (; i < n4; i += stride) {
      const float4 v = a4[i];
      acc[0] += (v.x + v.y) + (v.z + v.w);
    }
    tail_start = n4 << 2;
  }
  // scalar remainder (all of it when A is not 16-byte aligned)
  for (int64_t i = tail_start + int64_t(blockIdx.x) * kSumBlock + threadIdx.x; i < n; i += stride)
    acc[1] += A[i];
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < kSumUnroll; ++u) s += acc[u];
  s = block_reduce<kSumBlock / kWave, false>(s, red);
  if (threadIdx.x == 0) st_dev(partial + blockIdx.x, s);
  if (!arrive_last(counter, int(G))) return;
  float t = 0.f;
  for (int64_t i = threadIdx.x; i < G; i += kSumBlock) t += ld_dev(partial + i);
  t = block_reduce<kSumBlock / kWave, false>(t, red);
  if (threadIdx.x == 0) Out[0] = t;
}

// ------------------------------------------------------------ HBM probes
// STREAM kernels, one instantiation per kind (measured shapes):
//   read:            grid-stride, 8 float4 loads in flight per thread;
//   write/copy/triad: each block streams one contiguous range (DRAM page
//                    locality, ~20% faster than grid-striding on MI355X),
//                    8 float4 per thread per trip, non-temporal stores.
constexpr int kProbeUnroll = 8;
typedef float f32x4v_t __attribute__((ext_vector_type(4)));

// Grid-stride read.  NT = 0 allocates in the caches (the cache flush of the
// benchmarks); NT = 1 streams with the non-temporal hint on a 32-blocks-per-CU
// grid, the fastest read pattern measured on MI355X (the read peak).
template <int NT>
__global__ __launch_bounds__(256) void probe_read_kernel(const f32x4v_t* __restrict__ b, int64_t n4,
                                                         f32x4v_t* __restrict__ sink) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  f32x4v_t acc = {0.f, 0.f, 0.f, 0.f};
  for (; i + (kProbeUnroll - 1) * stride < n4; i += kProbeUnroll * stride) {
    f32x4v_t x[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) x[u] = NT ? __builtin_nontemporal_load(b + i + u * stride) : b[i + u * stride];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc += x[u];
  }
  for (; i < n4; i += stride) acc += b[i];
  if (acc.x == 1234.5f) sink[0] = acc;  // keeps the loads alive; practically never stores
}

// One-shot streaming read: block b reads its own contiguous 32 KiB (every
// load issued before any is used, non-temporal), the grid covering the
// array, as the row-block GEMV reads a weight matrix.
__global__ __launch_bounds__(256) void probe_read_blocks_kernel(const f32x4v_t* __restrict__ b, int64_t n4,
                                                                f32x4v_t* __restrict__ sink) {
  const int64_t base = int64_t(blockIdx.x) * 256 * kProbeUnroll + threadIdx.x;
  f32x4v_t x[kProbeUnroll];
#pragma unroll
  for (int u = 0; u < kProbeUnroll; ++u) {
    const int64_t j = base + u * 256;
    x[u] = __builtin_nontemporal_load(b + (j < n4 ? j : n4 - 1));
  }
  f32x4v_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kProbeUnroll; ++u) acc += x[u];
  if (acc.x == 1234.5f) sink[0] = acc;  // keeps the loads alive; practically never stores
}

template <int KIND>  // 1 write, 2 copy, 3 triad
__global__ __launch_bounds__(256) void probe_stream_kernel(f32x4v_t* __restrict__ a, const f32x4v_t* __restrict__ b,
                                                           const f32x4v_t* __restrict__ c, int64_t n4, float s) {
  const int64_t per = (n4 + gridDim.x - 1) / gridDim.x;
  const int64_t beg = int64_t(blockIdx.x) * per;
  const int64_t end = beg + per < n4 ? beg + per : n4;
  for (int64_t i = beg + threadIdx.x; i < end; i += 256 * kProbeUnroll) {
    f32x4v_t x[kProbeUnroll], y[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {
      const int64_t j = i + u * 256;
      if (j < end) {
        if (KIND >= 2) x[u] = b[j];
        if (KIND == 3) y[u] = c[j];
      }
    }
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {
      const int64_t j = i + u * 256;
      if (j >= end) continue;
      if (KIND == 1) __builtin_nontemporal_store(f32x4v_t{s, s, s, s}, a + j);
      else if (KIND == 2) __builtin_nontemporal_store(x[u], a + j);
      else __builtin_nontemporal_store(x[u] + s * y[u], a + j);
    }
  }
}

template <int BS>
void launch_rms_f32(const float* X, float* O, int64_t rows, int64_t dim, float eps, hipStream_t s) {
  const int64_t vpt = (dim / 4 + BS - 1) / BS;
  const dim3 g{unsigned(rows), 1, 1}, b{unsigned(BS), 1, 1};
  if (vpt <= 1) hipLaunchKernelGGL((rmsnorm_f32_reg_kernel<BS, 1>), g, b, 0, s, X, O, dim, eps);
  else if (vpt <= 2) hipLaunchKernelGGL((rmsnorm_f32_reg_kernel<BS, 2>), g, b, 0, s, X, O, dim, eps);
  else if (vpt <= 4) hipLaunchKernelGGL((rmsnorm_f32_reg_kernel<BS, 4>), g, b, 0, s, X, O, dim, eps);
  else hipLaunchKernelGGL((rmsnorm_f32_reg_kernel<BS, 8>), g, b, 0, s, X, O, dim, eps);
}

template <int BS, bool PACKED = false>
void launch_rms_bf16(const uint16_t* X, const uint16_t* W, uint16_t* O, int64_t rows, int64_t dim,
                     float eps, hipStream_t s) {
  const int64_t vpt = (dim / 8 + BS - 1) / BS;
  const dim3 g{unsigned(rows), 1, 1}, b{unsigned(BS), 1, 1};
  if (vpt <= 1) hipLaunchKernelGGL((rmsnorm_bf16_reg_kernel<BS, 1, PACKED>), g, b, 0, s, X, W, O, dim, eps);
  else if (vpt <= 2) hipLaunchKernelGGL((rmsnorm_bf16_reg_kernel<BS, 2, PACKED>), g, b, 0, s, X, W, O, dim, eps);
  else if (vpt <= 4) hipLaunchKernelGGL((rmsnorm_bf16_reg_kernel<BS, 4, PACKED>), g, b, 0, s, X, W, O, dim, eps);
  else hipLaunchKernelGGL((rmsnorm_bf16_reg_kernel<BS, 8, PACKED>), g, b, 0, s, X, W, O, dim, eps);
}

template <int BS>
void launch_softmax(const float* X, float* O, int64_t rows, int64_t dim, hipStream_t s) {
  const int64_t vpt = (dim / 4 + BS - 1) / BS;
  const dim3 g{unsigned(rows), 1, 1}, b{unsigned(BS), 1, 1};
  if (vpt <= 1) hipLaunchKernelGGL((softmax_reg_kernel<BS, 1>), g, b, 0, s, X, O, dim);
  else if (vpt <= 2) hipLaunchKernelGGL((softmax_reg_kernel<BS, 2>), g, b, 0, s, X, O, dim);
  else if (vpt <= 4) hipLaunchKernelGGL((softmax_reg_kernel<BS, 4>), g, b, 0, s, X, O, dim);
  else hipLaunchKernelGGL((softmax_reg_kernel<BS, 8>), g, b, 0, s, X, O, dim);
}

}  // namespace
}  // namespace ez

using namespace ez;

extern "C" int ezops_rmsnorm_f32(const float* X, float* Out, int64_t rows, int64_t dim, float eps,
                                 hipStream_t s) {
  EZ_REQUIRE(X && Out, "rmsnorm_f32: null pointer");
  EZ_REQUIRE(rows >= 1 && dim >= 1 && rows < (int64_t(1) << 31), "rmsnorm_f32: bad shape");
  const bool vec = dim % 4 == 0 && aligned16(X) && aligned16(Out);
  if (!vec || dim > 32768) {
    hipLaunchKernelGGL(rmsnorm_f32_loop_kernel, dim3(unsigned(rows)), dim3(256), 0, s, X, Out, dim, eps);
  } else if (dim <= 2048) {
    launch_rms_f32<64>(X, Out, rows, dim, eps, s);
  } else if (dim <= 8192) {
    launch_rms_f32<256>(X, Out, rows, dim, eps, s);
  } else {
    launch_rms_f32<1024>(X, Out, rows, dim, eps, s);
  }
  return launch_status("rmsnorm_f32");
}

extern "C" int ezops_rmsnorm_bf16(const void* Xv, const void* Wv, void* Ov, int64_t rows, int64_t dim,
                                  float eps, hipStream_t s) {
  auto X = static_cast<const uint16_t*>(Xv);
  auto W = static_cast<const uint16_t*>(Wv);
  auto O = static_cast<uint16_t*>(Ov);
  EZ_REQUIRE(X && O, "rmsnorm_bf16: null pointer");
  EZ_REQUIRE(rows >= 1 && dim >= 1 && rows < (int64_t(1) << 31), "rmsnorm_bf16: bad shape");
  const bool vec = dim % 8 == 0 && aligned16(X) && aligned16(O) && (!W || aligned16(W));
  if (!vec || dim > 65536) {
    hipLaunchKernelGGL(rmsnorm_bf16_loop_kernel, dim3(unsigned(rows)), dim3(256), 0, s, X, W, O, dim, eps);
  } else if (dim <= 1024) {
    launch_rms_bf16<64>(X, W, O, rows, dim, eps, s);
  } else if (dim <= 16384) {
    launch_rms_bf16<256>(X, W, O, rows, dim, eps, s);
  } else {
    launch_rms_bf16<1024>(X, W, O, rows, dim, eps, s);
  }
  return launch_status("rmsnorm_bf16");
}

namespace ez {
int launch_rmsnorm_bf16_packed(const uint16_t* X, const uint16_t* W, uint16_t* O, int64_t rows, int64_t dim,
                               float eps, hipStream_t s) {
  EZ_REQUIRE(X && O, "rmsnorm_bf16_packed: null pointer");
  EZ_REQUIRE(rows >= 1 && dim >= 32 && dim % 32 == 0 && dim <= 16384 && aligned16(X) && aligned16(O) &&
                 (!W || aligned16(W)),
             "rmsnorm_bf16_packed: needs aligned rows, dim %% 32 == 0 and dim <= 16384");
  launch_rms_bf16<256, true>(X, W, O, rows, dim, eps, s);
  return launch_status("rmsnorm_bf16_packed");
}
}  // namespace ez

extern "C" int ezops_softmax_f32(const float* X, float* Out, int64_t rows, int64_t dim, hipStream_t s) {
  EZ_REQUIRE(X && Out, "softmax_f32: null pointer");
  EZ_REQUIRE(rows >= 1 && dim >= 1 && rows < (int64_t(1) << 31), "softmax_f32: bad shape");
  const bool vec = dim % 4 == 0 && aligned16(X) && aligned16(Out);
  if (!vec || dim > 32768) {
    hipLaunchKernelGGL(softmax_loop_kernel, dim3(unsigned(rows)), dim3(1024), 0, s, X, Out, dim);
  } else if (dim <= 2048) {
    launch_softmax<64>(X, Out, rows, dim, s);
  } else if (dim <= 8192) {
    launch_softmax<256>(X, Out, rows, dim, s);
  } else {
    launch_softmax<1024>(X, Out, rows, dim, s);
  }
  return launch_status("softmax_f32");
}

extern "C" size_t ezops_reduce_sum_workspace_size(int64_t n) {
  // one arrival counter in bytes [0, 256), then the partial sums.  The
  // counter's offset does not depend on n, so one workspace serves calls of
  // any length (each call leaves the counter at zero again).
  return size_t(256 + ((sum_blocks(n) * 4 + 255) / 256) * 256);
}

extern "C" int ezops_reduce_sum_f32(const float* A, float* Out, int64_t n, void* ws, size_t ws_bytes,
                                    hipStream_t s) {
  EZ_REQUIRE(A && Out && ws, "reduce_sum_f32: null pointer");
  EZ_REQUIRE(n >= 1, "reduce_sum_f32: n must be >= 1");
  EZ_REQUIRE(ws_bytes >= ezops_reduce_sum_workspace_size(n), "reduce_sum_f32: workspace too small");
  EZ_REQUIRE(aligned16(ws), "reduce_sum_f32: workspace must be 16-byte aligned");
  const int64_t G = sum_blocks(n);
  int* counter = static_cast<int*>(ws);
  float* partial = reinterpret_cast<float*>(static_cast<char*>(ws) + 256);
  hipLaunchKernelGGL(sum_kernel, dim3(unsigned(G)), dim3(kSumBlock), 0, s, A, n, aligned16(A), partial,
                     counter, Out);
  return launch_status("reduce_sum_f32");
}

// MFMA peak probe: every wave keeps 8 independent 16x16x32 accumulator chains
// busy for `iters` rounds (operands built from the lane id, so nothing folds).
// One launch performs blocks * 4 waves * iters * 8 * 16384 flops (kinds 0-2)
// or blocks * 4 * iters * 8 * 2048 (kind 3, fp32 16x16x4).
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
template <int F16>
__global__ __launch_bounds__(256) void probe_mfma_kernel(float* __restrict__ out, int64_t iters) {
  const float lf = float(threadIdx.x & 63) * (1.0f / 64.0f);
  if constexpr (F16 == 3) {  // fp32 v_mfma_f32_16x16x4_f32: 8 chains, 2048 flops per instruction
    f32x4_t acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const float a = lf, b = 1.0f - lf;
    for (int64_t i = 0; i < iters; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j], 0, 0, 0);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
    if (sum == 1234.5f) out[0] = sum;
    return;
  }
  if constexpr (F16 == 2) {  // bf16 32x32x16: 4 chains of 16-float accumulators, same flops per round
    f32x16_t acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;
    bf16x8_t a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) { a[e] = __bf16(lf + e); b[e] = __bf16(1.0f - lf * e); }
    for (int64_t i = 0; i < iters; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[j], 0, 0, 0);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) sum += acc[j][e];
    if (sum == 1234.5f) out[0] = sum;
    return;
  }
  f32x4_t acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if constexpr (F16 == 1) {
    f16x8_t a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) { a[e] = _Float16(lf + e); b[e] = _Float16(1.0f - lf * e); }
    for (int64_t i = 0; i < iters; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
  } else {
    bf16x8_t a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) { a[e] = __bf16(lf + e); b[e] = __bf16(1.0f - lf * e); }
    for (int64_t i = 0; i < iters; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) sum += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  if (sum == 1234.5f) out[0] = sum;  // keeps the chains alive; practically never stores
}

extern "C" int ezops_mfma_probe(int kind, float* out, int64_t blocks, int64_t iters, hipStream_t s) {
  EZ_REQUIRE(kind >= 0 && kind <= 3, "mfma_probe: kind must be 0 (bf16), 1 (fp16), 2 (bf16 32x32x16) or 3 (fp32)");
  EZ_REQUIRE(out && blocks >= 1 && blocks < (int64_t(1) << 31) && iters >= 1, "mfma_probe: bad arguments");
  if (kind == 0) hipLaunchKernelGGL(probe_mfma_kernel<0>, dim3(unsigned(blocks)), dim3(256), 0, s, out, iters);
  else if (kind == 1) hipLaunchKernelGGL(probe_mfma_kernel<1>, dim3(unsigned(blocks)), dim3(256), 0, s, out, iters);
  else if (kind == 2) hipLaunchKernelGGL(probe_mfma_kernel<2>, dim3(unsigned(blocks)), dim3(256), 0, s, out, iters);
  else hipLaunchKernelGGL(probe_mfma_kernel<3>, dim3(unsigned(blocks)), dim3(256), 0, s, out, iters);
  return launch_status("mfma_probe");
}

extern "C" int ezops_hbm_probe(int kind, float* a, const float* b, const float* c, int64_t n, float sc,
                               hipStream_t s) {
  EZ_REQUIRE(kind >= 0 && kind <= 5, "hbm_probe: kind must be 0..5");
  EZ_REQUIRE(a && (kind == 1 || b) && (kind != 3 || c), "hbm_probe: null pointer");
  EZ_REQUIRE(n >= 4 && n % 4 == 0, "hbm_probe: n must be a positive multiple of 4");
  const dim3 grid{unsigned(num_cus() * 16), 1, 1}, block{256, 1, 1};
  auto A = reinterpret_cast<f32x4v_t*>(a);
  auto Bv = reinterpret_cast<const f32x4v_t*>(b);
  auto Cv = reinterpret_cast<const f32x4v_t*>(c);
  switch (kind) {
    case 0: hipLaunchKernelGGL(probe_read_kernel<0>, dim3(unsigned(num_cus() * 4)), block, 0, s, Bv, n / 4, A); break;
    case 4: hipLaunchKernelGGL(probe_read_kernel<1>, dim3(unsigned(num_cus() * 32)), block, 0, s, Bv, n / 4, A); break;
    case 5: {
      const int64_t blocks = (n / 4 + 256 * kProbeUnroll - 1) / (256 * kProbeUnroll);
      EZ_REQUIRE(blocks < (int64_t(1) << 31), "hbm_probe: array too large for one-shot blocks");
      hipLaunchKernelGGL(probe_read_blocks_kernel, dim3(unsigned(blocks)), block, 0, s, Bv, n / 4, A);
      break;
    }
    case 1: hipLaunchKernelGGL(probe_stream_kernel<1>, grid, block, 0, s, A, Bv, Cv, n / 4, sc); break;
    case 2: hipLaunchKernelGGL(probe_stream_kernel<2>, grid, block, 0, s, A, Bv, Cv, n / 4, sc); break;
    default: hipLaunchKernelGGL(probe_stream_kernel<3>, grid, block, 0, s, A, Bv, Cv, n / 4, sc); break;
  }
  return launch_status("hbm_probe");
}
