// Persistent single-launch Qwen3 dense decode layer for small batches (M <= 4).
//
// One block of 8 waves per CU runs the whole layer in five phases separated
// by grid barriers:
//   A  x = bf16(rmsnorm(hidden) * in_norm_w)          (staged in LDS per block)
//      qkv = x . Wqkv^T                               (weight rows streamed once)
//   B  split-KV GQA attention with the q/k RMSNorm + RoPE + KV-slot write
//      prologue (attn_impl.h), splits merged by the last block of each unit
//   C  x2 = hidden + attn . Wo^T
//   D  h = silu(bf16(rmsnorm(x2) * post_norm_w) . Wg^T) * (... . Wu^T)
//   E  out = x2 + h . Wd^T
// Activations between phases (a few KB) go through device-coherent fp32
// stores/loads; every value is rounded to bf16 exactly where the reference
// rounds (ezops/ops/qwen3_dense_decode.py:142-176), and the RMSNorm'd inputs
// are staged as bf16(x * rsqrt(var + eps) * w) like the reference.
//
// Weights do not depend on the previous phase, so before each barrier the
// six "stream" waves of every block issue the loads of their first two
// weight tiles of the next phase; the barrier wait and the activation
// staging then overlap that HBM stream.  On gfx9 loads and stores share one
// in-order completion counter, so the hand-off stores are completed before
// the prefetch is issued, and the barrier polling and activation staging
// are done by the two "staging" waves, which never have weight loads
// outstanding.  Inside a phase, each wave streams its rows with two register
// tiles (16 B per lane per chunk, a wave instruction reads 1 KiB of a row):
// one tile is multiplied while the other is in flight.
//
// The grid barrier is a device-scope counter (relaxed atomics, sc1 polls,
// no cache flushes); its spin is bounded, so a grid that could not become
// co-resident ends with wrong results instead of a hung GPU.  The host only
// launches this kernel when the occupancy query guarantees one block per CU.
#include "attn_impl.h"
#include "internal.h"
#include "status.h"
#include "../../include/ezops_hip.h"

namespace ez {
namespace {

constexpr int kLWaves = 8;                 // waves per block
constexpr int kLThreads = kLWaves * kWave;
constexpr int kStageWaves = 2;             // waves that stage activations and poll barriers
constexpr int kStreamWaves = kLWaves - kStageWaves;
constexpr int kStageThreads = kStageWaves * kWave;
// 16-byte chunks per lane per pass: 8 (a 4096-element row pass) for one or
// two batch rows, 4 for more (register budget of 2 waves per SIMD).
template <int M>
constexpr int chunks_per_pass() { return M <= 2 ? 8 : 4; }
constexpr int kXsMax = 12288;              // largest K staged in LDS (elements per batch row)
constexpr int kSpinLimit = 1 << 22;        // barrier poll bound (seconds, far beyond any real wait)

struct GridBar {
  int gen;        // launches completed
  int release;    // highest released epoch
  int pad[62];
  int flags[1];   // [gridDim.x] arrival epochs
};

struct LayerArgs {
  int64_t B, S, HS, IS, H, Hkv, D, QR, KVR, QKV;
  float eps;
  const uint16_t* hidden;
  uint16_t* Kc; uint16_t* Vc;
  const uint16_t* Wqkv; const uint16_t* Wo; const uint16_t* Wgu; const uint16_t* Wd;
  const uint16_t* in_w; const uint16_t* q_w; const uint16_t* k_w; const uint16_t* post_w;
  const uint16_t* cos; const uint16_t* sin;
  const int32_t* kv_lens;
  uint16_t* out;
  // workspace
  float* qkv_f;   // [B, QKV]
  float* attn_f;  // [B, QR]
  float* x2_f;    // [B, HS]
  float* h_f;     // [B, IS]
  attn::AttnWs aws;
  int64_t nsplit;
  GridBar* bar;
};

// ---------------------------------------------------------------- barrier
// Flag barrier (no same-address atomics: 256 arrivals on one counter
// serialise at the memory side, ~10 us).  Block b publishes the epoch in its
// own slot flags[b]; block 0's control wave polls all slots with one wide
// load per lane and publishes the epoch in `release`; every block polls
// `release`.  Epochs grow across launches (gen * 8 + phase), so nothing has
// to be reset.  Every wave must have completed its device-coherent stores
// (s_waitcnt) before entering.  Only the last wave of a block — a staging
// wave with no loads outstanding — touches the flags.

__device__ __forceinline__ int ld_flag(const int* p) {
  return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_flag(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void grid_barrier(GridBar* bar, int epoch) {
  __syncthreads();
  if ((threadIdx.x >> 6) == kLWaves - 1) {
    const int lane = threadIdx.x & (kWave - 1);
    if (lane == 0) st_flag(&bar->flags[blockIdx.x], epoch);
    if (blockIdx.x == 0) {
      int spins = 0;
      for (;;) {
        int lo = epoch;
        for (int i = lane; i < int(gridDim.x); i += kWave) lo = min(lo, ld_flag(&bar->flags[i]));
#pragma unroll
        for (int off = kWave / 2; off > 0; off >>= 1) lo = min(lo, __shfl_xor(lo, off, kWave));
        if (lo >= epoch || ++spins > kSpinLimit) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (lane == 0) st_flag(&bar->release, epoch);
    }
    if (lane == 0) {
      int spins = 0;
      while (ld_flag(&bar->release) < epoch && spins < kSpinLimit) {
        __builtin_amdgcn_s_sleep(1);
        ++spins;
      }
    }
  }
  __syncthreads();
}

__device__ __forceinline__ bool is_stream_wave() { return (threadIdx.x >> 6) < kStreamWaves; }

// 16-byte device-coherent (sc1) load of fp32 activations written by other
// blocks; reads past `bytes` return zeros.
typedef float f32x4v_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4v_t ld_dev_x4(__amdgpu_buffer_rsrc_t r, int64_t byte_ofs) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, int(byte_ofs), 0, /*sc1*/ 16);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const float* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, int(bytes), 0x00020000);
}

// ---------------------------------------------------------------- staging
// xs[m][k] (bf16, LDS), m < M, k < K, staged by the two staging waves from a
// bf16 global source or an fp32 device-coherent source; with `norm`,
// xs = bf16(x * rsqrt(mean(x^2) + eps) * w) exactly as the reference stages
// it.  Called by every thread of the block (it contains block barriers).
template <int M>
__device__ __forceinline__ void stage_x(uint16_t* xs, const uint16_t* src_bf, const float* src_f, int64_t ld, int64_t K, bool norm,
                        const uint16_t* w, float eps, float* red) {
  const int st = int(threadIdx.x) - kStreamWaves * kWave;  // staging thread index, < 0 for stream waves
  float ss[M];
#pragma unroll
  for (int m = 0; m < M; ++m) ss[m] = 0.f;
  if (st >= 0) {
    if (src_bf) {
      for (int64_t c = st; c < K / 8; c += kStageThreads) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint4 v = *reinterpret_cast<const uint4*>(src_bf + m * ld + c * 8);
          float f[8];
          unpack8(v, f);
#pragma unroll
          for (int e = 0; e < 8; ++e) ss[m] = fmaf(f[e], f[e], ss[m]);
          *reinterpret_cast<uint4*>(xs + m * kXsMax + c * 8) = v;
        }
      }
    } else {
      constexpr int U = M <= 2 ? 8 : 2;  // 16-byte loads in flight per thread (register budget)
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const __amdgpu_buffer_rsrc_t r = dev_rsrc(src_f + m * ld, K * 4);
        for (int64_t c0 = st; c0 < K / 4; c0 += int64_t(kStageThreads) * U) {
          f32x4v_t v[U];
#pragma unroll
          for (int u = 0; u < U; ++u) v[u] = ld_dev_x4(r, (c0 + int64_t(u) * kStageThreads) * 16);
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int64_t c = c0 + int64_t(u) * kStageThreads;
            if (c < K / 4) {
              ss[m] += v[u].x * v[u].x + v[u].y * v[u].y + v[u].z * v[u].z + v[u].w * v[u].w;
              *reinterpret_cast<uint2*>(xs + m * kXsMax + c * 4) =
                  make_uint2(pack_bf2(v[u].x, v[u].y), pack_bf2(v[u].z, v[u].w));
            }
          }
        }
      }
    }
  }
  if (!norm) {
    __syncthreads();
    return;
  }
  float r[M];
#pragma unroll
  for (int m = 0; m < M; ++m) r[m] = rsqrtf(block_reduce<kLWaves, false>(ss[m], red) / float(K) + eps);
  if (st >= 0) {
    // 8-element chunks; the weight chunks of a trip are loaded together
    constexpr int U = 4;
    for (int64_t c0 = st; c0 < K / 8; c0 += int64_t(kStageThreads) * U) {
      uint4 wv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + int64_t(u) * kStageThreads;
        wv[u] = (w && c < K / 8) ? *reinterpret_cast<const uint4*>(w + c * 8)
                                 : make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t c = c0 + int64_t(u) * kStageThreads;
        if (c >= K / 8) break;
        float wf[8];
        unpack8(wv[u], wf);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          uint4* px = reinterpret_cast<uint4*>(xs + m * kXsMax + c * 8);
          float x[8];
          unpack8(*px, x);
          float y[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] = w ? (x[e] * r[m]) * wf[e] : x[e] * r[m];
          *px = make_uint4(pack_bf2(y[0], y[1]), pack_bf2(y[2], y[3]), pack_bf2(y[4], y[5]), pack_bf2(y[6], y[7]));
        }
      }
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------- GEMV streaming
// A register tile: RT weight rows x kCH chunks per lane of one K pass.
template <int RT, int CH>
struct WTile {
  uint4 v[RT][CH];
};

// PAIR: the tile's two rows are row `row` of W (gate) and of W2 (up).
template <int RT, int CH, bool PAIR>
__device__ __forceinline__ void load_tile(WTile<RT, CH>& t, const uint16_t* W, const uint16_t* W2, int64_t row,
                                          int64_t K, int pass, int lane) {
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const uint16_t* base = PAIR ? ((r == 0 ? W : W2) + row * K) : (W + (row + r) * K);
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int64_t k = int64_t(pass) * (CH * kWave * 8) + (j * kWave + lane) * 8;
      t.v[r][j] = k < K ? ld16_stream(base + k) : make_uint4(0, 0, 0, 0);
    }
  }
}

template <int M, int RT, int CH>
__device__ __forceinline__ void fma_tile(float (&acc)[M][RT], const WTile<RT, CH>& t, const uint16_t* xs, int64_t K,
                                         int pass, int lane) {
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const int64_t k = int64_t(pass) * (CH * kWave * 8) + (j * kWave + lane) * 8;
    if (k >= K) break;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float x[8];
      unpack8(*reinterpret_cast<const uint4*>(xs + m * kXsMax + k), x);
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        float w[8];
        unpack8(t.v[r][j], w);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[m][r] = fmaf(w[e], x[e], acc[m][r]);
      }
    }
  }
}

// Rows [0, N) in groups of RT (PAIR: one gate/up pair per group) are split
// contiguously over all waves of the grid.
struct GroupRange {
  int64_t g0, g1;
};
__device__ __forceinline__ GroupRange wave_groups(int64_t ngroups) {
  const int64_t nw = int64_t(gridDim.x) * kLWaves;
  const int64_t gw = int64_t(blockIdx.x) * kLWaves + (threadIdx.x >> 6);
  return {gw * ngroups / nw, (gw + 1) * ngroups / nw};
}

// Two register tiles: tile i of the wave's (group, pass) sequence lives in
// buffer i % 2.
template <int RT, int CH>
struct WPair {
  WTile<RT, CH> t[2];
};

template <int RT, int CH, bool PAIR>
__device__ __forceinline__ void load_tile_idx(WTile<RT, CH>& t, const uint16_t* W, const uint16_t* W2, int64_t K,
                                              GroupRange gr, int npass, int64_t idx) {
  const int64_t g = gr.g0 + idx / npass;
  load_tile<RT, CH, PAIR>(t, W, W2, PAIR ? g : g * RT, K, int(idx % npass), threadIdx.x & (kWave - 1));
}

template <int RT, int CH>
__device__ __forceinline__ int passes(int64_t K) {
  return int((K + int64_t(CH) * kWave * 8 - 1) / (int64_t(CH) * kWave * 8));
}

// Issue the first two tiles of a phase (done before the barrier by stream
// waves, after staging by staging waves).
template <int RT, int CH, bool PAIR>
__device__ __forceinline__ void prefetch2(WPair<RT, CH>& w, const uint16_t* W, const uint16_t* W2, int64_t K,
                                          GroupRange gr) {
  const int npass = passes<RT, CH>(K);
  const int64_t ntiles = (gr.g1 - gr.g0) * npass;
  if (ntiles > 0) load_tile_idx<RT, CH, PAIR>(w.t[0], W, W2, K, gr, npass, 0);
  if (ntiles > 1) load_tile_idx<RT, CH, PAIR>(w.t[1], W, W2, K, gr, npass, 1);
}

// Streams the wave's row groups; tiles 0 and 1 are already in flight in `w`.
// After multiplying tile i, its buffer is refilled with tile i + 2.
// Epi(m, row, acc, acc_up) finishes one output (called by lane 0).
template <int M, int RT, int CH, bool PAIR, class Epi>
__device__ __forceinline__ void gemv_phase(const uint16_t* W, const uint16_t* W2, int64_t K, const uint16_t* xs, GroupRange gr,
                           WPair<RT, CH>& w, Epi epi) {
  const int lane = threadIdx.x & (kWave - 1);
  const int npass = passes<RT, CH>(K);
  const int64_t ntiles = (gr.g1 - gr.g0) * npass;
  float acc[M][RT];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[m][r] = 0.f;

  auto step = [&](int64_t idx, WTile<RT, CH>& cur) {
    const int64_t g = gr.g0 + idx / npass;
    const int pass = int(idx % npass);
    fma_tile<M, RT, CH>(acc, cur, xs, K, pass, lane);
    if (idx + 2 < ntiles) load_tile_idx<RT, CH, PAIR>(cur, W, W2, K, gr, npass, idx + 2);
    if (pass == npass - 1) {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float v[RT];
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          v[r] = wave_reduce_uniform<false>(acc[m][r]);
          acc[m][r] = 0.f;
        }
        if (lane == 0) {
          if (PAIR) {
            epi(m, g, v[0], v[RT - 1]);
          } else {
#pragma unroll
            for (int r = 0; r < RT; ++r) epi(m, g * RT + r, v[r], 0.f);
          }
        }
      }
    }
  };
  for (int64_t idx = 0; idx < ntiles; idx += 2) {
    step(idx, w.t[0]);
    if (idx + 1 < ntiles) step(idx + 1, w.t[1]);
  }
}

// End of a phase: complete this wave's hand-off stores, let the stream waves
// issue the next phase's first two weight tiles, then the grid barrier.
template <int RT, int CH, bool PAIR>
__device__ __forceinline__ void phase_end(WPair<RT, CH>& w, const uint16_t* W, const uint16_t* W2, int64_t K,
                                          GroupRange gr, GridBar* bar, int epoch) {
  __builtin_amdgcn_s_waitcnt(0);
  if (is_stream_wave()) prefetch2<RT, CH, PAIR>(w, W, W2, K, gr);
  grid_barrier(bar, epoch);
}

// ---------------------------------------------------------------- the layer
template <int M, int G>
__global__ __launch_bounds__(kLThreads) void qwen3_layer_persistent(LayerArgs p) {
  __shared__ __align__(16) uint16_t xs[M * kXsMax];
  __shared__ float red[kLWaves];
  constexpr int CH = chunks_per_pass<M>();
  const int nb = int(gridDim.x);
  const int e0 = ld_flag(&p.bar->gen) * 8;  // this launch's epochs: e0 + 1 .. e0 + 4
  const uint16_t* Wg = p.Wgu;
  const uint16_t* Wu = p.Wgu + p.IS * p.HS;

  // ---- A: RMSNorm + QKV projection (qkv_f holds bf16-rounded values)
  constexpr int RTA = 1;
  const GroupRange ga = wave_groups(p.QKV / RTA);
  WPair<RTA, CH> wa;
  if (is_stream_wave()) prefetch2<RTA, CH, false>(wa, p.Wqkv, nullptr, p.HS, ga);
  stage_x<M>(xs, p.hidden, nullptr, p.HS, p.HS, true, p.in_w, p.eps, red);
  if (!is_stream_wave()) prefetch2<RTA, CH, false>(wa, p.Wqkv, nullptr, p.HS, ga);
  gemv_phase<M, RTA, CH, false>(p.Wqkv, nullptr, p.HS, xs, ga, wa, [&](int m, int64_t n, float v, float) {
    st_dev(p.qkv_f + m * p.QKV + n, round_bf(v));
  });
  __builtin_amdgcn_s_waitcnt(0);
  grid_barrier(p.bar, e0 + 1);

  // ---- B: attention (q/k norm + RoPE + KV write in its prologue)
  {
    AttnArgs a{};
    a.Q = nullptr;
    a.K = p.Kc; a.V = p.Vc; a.Out = nullptr;
    a.B = p.B; a.H = p.H; a.Hkv = p.Hkv; a.S = p.S; a.D = 128;
    a.kv_lens = p.kv_lens;
    a.scale = 1.0f / sqrtf(128.f);
    a.qkv_bs = p.QKV;
    a.qw = p.q_w; a.kw = p.k_w; a.cos = p.cos; a.sin = p.sin; a.eps = p.eps;
    a.qkv_f = p.qkv_f;
    a.out_f = p.attn_f;
    const int64_t items = p.B * p.Hkv * p.nsplit;
    for (int64_t it = blockIdx.x; it < items; it += nb) {
      attn::attn_block<128, G, kLWaves, attn::kQFromQkvF32, attn::kOutF32Dev, true>(a, it % p.nsplit, it / p.nsplit,
                                                                             p.nsplit, p.aws);
      __syncthreads();
    }
  }
  constexpr int RTC = 2;
  const GroupRange gc = wave_groups(p.HS / RTC);
  WPair<RTC, CH> wc;
  phase_end<RTC, CH, false>(wc, p.Wo, nullptr, p.QR, gc, p.bar, e0 + 2);

  // ---- C: o_proj + residual
  stage_x<M>(xs, nullptr, p.attn_f, p.QR, p.QR, false, nullptr, p.eps, red);
  if (!is_stream_wave()) prefetch2<RTC, CH, false>(wc, p.Wo, nullptr, p.QR, gc);
  gemv_phase<M, RTC, CH, false>(p.Wo, nullptr, p.QR, xs, gc, wc, [&](int m, int64_t n, float v, float) {
    st_dev(p.x2_f + m * p.HS + n, round_bf(bf2f(p.hidden[m * p.HS + n]) + round_bf(v)));
  });
  const GroupRange gd = wave_groups(p.IS);
  WPair<2, CH> wd;
  phase_end<2, CH, true>(wd, Wg, Wu, p.HS, gd, p.bar, e0 + 3);

  // ---- D: post-attention RMSNorm + gate/up + SwiGLU
  stage_x<M>(xs, nullptr, p.x2_f, p.HS, p.HS, true, p.post_w, p.eps, red);
  if (!is_stream_wave()) prefetch2<2, CH, true>(wd, Wg, Wu, p.HS, gd);
  gemv_phase<M, 2, CH, true>(Wg, Wu, p.HS, xs, gd, wd, [&](int m, int64_t n, float g, float u) {
    st_dev(p.h_f + m * p.IS + n, round_bf(round_bf(silu(round_bf(g))) * round_bf(u)));
  });
  constexpr int RTE = 2;
  const GroupRange ge = wave_groups(p.HS / RTE);
  WPair<RTE, CH> we;
  phase_end<RTE, CH, false>(we, p.Wd, nullptr, p.IS, ge, p.bar, e0 + 4);

  // ---- E: down projection + residual
  stage_x<M>(xs, nullptr, p.h_f, p.IS, p.IS, false, nullptr, p.eps, red);
  if (!is_stream_wave()) prefetch2<RTE, CH, false>(we, p.Wd, nullptr, p.IS, ge);
  gemv_phase<M, RTE, CH, false>(p.Wd, nullptr, p.IS, xs, ge, we, [&](int m, int64_t n, float v, float) {
    p.out[m * p.HS + n] = f2bf(ld_dev(p.x2_f + m * p.HS + n) + round_bf(v));
  });

  // ---- block 0 advances the generation once every block has read it
  // (all blocks passed the first barrier, after reading `gen`).
  if (blockIdx.x == 0 && threadIdx.x == 0) st_flag(&p.bar->gen, e0 / 8 + 1);
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

int grid_blocks() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
  }
  return cus;
}

struct MkPlan {
  int64_t nsplit;
};

MkPlan mk_plan(const ezops_qwen3_layer& L) {
  const int64_t units = L.B * L.Hkv;
  int64_t ns = grid_blocks() / units;
  const int64_t min_chunk = int64_t(kLWaves) * attn::kTile;
  const int64_t max_ns = (L.S + min_chunk - 1) / min_chunk;
  if (ns > max_ns) ns = max_ns;
  if (ns > attn::kMaxSplits) ns = attn::kMaxSplits;
  if (ns < 1) ns = 1;
  return {ns};
}

template <int M, int G>
const void* kernel_ptr() {
  return reinterpret_cast<const void*>(&qwen3_layer_persistent<M, G>);
}

const void* pick_kernel(int64_t M, int64_t G) {
  if (G == 2) {
    switch (M) {
      case 1: return kernel_ptr<1, 2>();
      case 2: return kernel_ptr<2, 2>();
      case 3: return kernel_ptr<3, 2>();
      case 4: return kernel_ptr<4, 2>();
    }
  } else if (G == 4) {
    switch (M) {
      case 1: return kernel_ptr<1, 4>();
      case 2: return kernel_ptr<2, 4>();
      case 3: return kernel_ptr<3, 4>();
      case 4: return kernel_ptr<4, 4>();
    }
  }
  return nullptr;
}

}  // namespace

bool layer_persistent_supported(const ezops_qwen3_layer& L) {
  const int64_t G = L.H / L.Hkv;
  const int64_t QR = L.H * L.D;
  if (L.B < 1 || L.B > 4 || L.D != 128 || (G != 2 && G != 4)) return false;
  if (L.HS > kXsMax || QR > kXsMax || L.IS > kXsMax) return false;
  if (L.HS % 8 || L.IS % 8 || QR % 8 || L.HS % 2) return false;
  const void* k = pick_kernel(L.B, G);
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, kLThreads, 0) != hipSuccess) return false;
  return per_cu >= 1;
}

size_t layer_persistent_ws(const ezops_qwen3_layer& L) {
  const int64_t QR = L.H * L.D, KVR = L.Hkv * L.D, QKV = QR + 2 * KVR;
  const MkPlan pl = mk_plan(L);
  return align256(size_t(L.B * QKV) * 4) + align256(size_t(L.B * QR) * 4) + align256(size_t(L.B * L.HS) * 4) +
         align256(size_t(L.B * L.IS) * 4) + align256(size_t(L.B * L.H * pl.nsplit * L.D) * 4) +
         align256(size_t(L.B * L.H * pl.nsplit * 2) * 4) + align256(size_t(L.B * L.Hkv) * 4) +
         align256(sizeof(GridBar) + sizeof(int) * size_t(grid_blocks()));
}

int launch_layer_persistent(const ezops_qwen3_layer& L, void* ws, hipStream_t s) {
  LayerArgs p{};
  p.B = L.B; p.S = L.S; p.HS = L.HS; p.IS = L.IS; p.H = L.H; p.Hkv = L.Hkv; p.D = L.D;
  p.QR = L.H * L.D; p.KVR = L.Hkv * L.D; p.QKV = p.QR + 2 * p.KVR;
  p.eps = L.eps;
  p.hidden = static_cast<const uint16_t*>(L.hidden);
  p.Kc = static_cast<uint16_t*>(L.K_cache);
  p.Vc = static_cast<uint16_t*>(L.V_cache);
  p.Wqkv = static_cast<const uint16_t*>(L.Wqkv);
  p.Wo = static_cast<const uint16_t*>(L.Wo);
  p.Wgu = static_cast<const uint16_t*>(L.Wgu);
  p.Wd = static_cast<const uint16_t*>(L.Wd);
  p.in_w = static_cast<const uint16_t*>(L.in_norm_w);
  p.q_w = static_cast<const uint16_t*>(L.q_norm_w);
  p.k_w = static_cast<const uint16_t*>(L.k_norm_w);
  p.post_w = static_cast<const uint16_t*>(L.post_norm_w);
  p.cos = static_cast<const uint16_t*>(L.cos);
  p.sin = static_cast<const uint16_t*>(L.sin);
  p.kv_lens = L.kv_lens;
  p.out = static_cast<uint16_t*>(L.out);
  const MkPlan pl = mk_plan(L);
  p.nsplit = pl.nsplit;
  char* c = static_cast<char*>(ws);
  auto take = [&](size_t bytes) {
    char* r = c;
    c += align256(bytes);
    return r;
  };
  p.qkv_f = reinterpret_cast<float*>(take(size_t(p.B * p.QKV) * 4));
  p.attn_f = reinterpret_cast<float*>(take(size_t(p.B * p.QR) * 4));
  p.x2_f = reinterpret_cast<float*>(take(size_t(p.B * p.HS) * 4));
  p.h_f = reinterpret_cast<float*>(take(size_t(p.B * p.IS) * 4));
  p.aws.opart = reinterpret_cast<float*>(take(size_t(p.B * p.H * pl.nsplit * p.D) * 4));
  p.aws.ml = reinterpret_cast<float*>(take(size_t(p.B * p.H * pl.nsplit * 2) * 4));
  p.aws.counters = reinterpret_cast<int*>(take(size_t(p.B * p.Hkv) * 4));
  p.bar = reinterpret_cast<GridBar*>(take(sizeof(GridBar) + sizeof(int) * size_t(grid_blocks())));

  const int64_t G = L.H / L.Hkv;
  const dim3 grid{unsigned(grid_blocks()), 1, 1}, block{kLThreads, 1, 1};
  switch (G * 10 + L.B) {
    case 21: hipLaunchKernelGGL((qwen3_layer_persistent<1, 2>), grid, block, 0, s, p); break;
    case 22: hipLaunchKernelGGL((qwen3_layer_persistent<2, 2>), grid, block, 0, s, p); break;
    case 23: hipLaunchKernelGGL((qwen3_layer_persistent<3, 2>), grid, block, 0, s, p); break;
    case 24: hipLaunchKernelGGL((qwen3_layer_persistent<4, 2>), grid, block, 0, s, p); break;
    case 41: hipLaunchKernelGGL((qwen3_layer_persistent<1, 4>), grid, block, 0, s, p); break;
    case 42: hipLaunchKernelGGL((qwen3_layer_persistent<2, 4>), grid, block, 0, s, p); break;
    case 43: hipLaunchKernelGGL((qwen3_layer_persistent<3, 4>), grid, block, 0, s, p); break;
    case 44: hipLaunchKernelGGL((qwen3_layer_persistent<4, 4>), grid, block, 0, s, p); break;
    default: return set_error(EZ_EINVAL, "qwen3 persistent layer: unsupported batch/group");
  }
  return launch_status("qwen3_layer_persistent");
}

}  // namespace ez
