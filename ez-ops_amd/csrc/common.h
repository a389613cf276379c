// Shared device helpers for the gfx950 (CDNA4, wave64) kernels of libezops_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ez {

constexpr int kWave = 64;

// MFMA operand/result vectors (v_mfma_f32_16x16x32_bf16: 8 bf16 per lane in,
// 4 fp32 per lane out).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// ---- bf16 <-> fp32 -------------------------------------------------------
// bf16 is carried as raw uint16 bits; a uint32 word holds two of them with
// the lower-indexed element in the low half.
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return uint32_t(f2bf(lo)) | (uint32_t(f2bf(hi)) << 16);
}

// Unpack 8 bf16 held in a uint4 into fp32.
__device__ __forceinline__ void unpack8(const uint4& v, float (&f)[8]) {
  f[0] = bf_lo(v.x); f[1] = bf_hi(v.x);
  f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
  f[4] = bf_lo(v.z); f[5] = bf_hi(v.z);
  f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}

// 16-byte global load with the non-temporal hint: streamed weights / KV are read once and should not
// displace reused lines.  Measured on MI355X: a 4 GiB streaming read reaches
// 6.7 TB/s with the hint against 6.1 TB/s without, and the RMSNorm + gate/up
// GEMV drops from 36 to 32 us.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8_t, v); }

// ---- wave / block reductions (fixed butterfly order => deterministic,
// and every lane ends with the bit-identical result) ----------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
// Reductions inside each 16-lane row of the wave.
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// DPP reductions inside each 16-lane row: quad_perm [1,0,3,2], quad_perm
// [2,3,0,1], row_half_mirror, row_mirror.  Every lane of the row ends with the
// row's result (the combination order is the same for all lanes up to
// commutation, so the values are bit-identical).
template <bool MAX>
__device__ __forceinline__ float dpp_row16(float v) {
#define EZ_DPP_STEP(ctrl)                                                                 \
  {                                                                                       \
    const float o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, true)); \
    v = MAX ? fmaxf(v, o) : v + o;                                                        \
  }
  EZ_DPP_STEP(0xB1)
  EZ_DPP_STEP(0x4E)
  EZ_DPP_STEP(0x141)
  EZ_DPP_STEP(0x140)
#undef EZ_DPP_STEP
  return v;
}

// Sum over the lanes that share lane % CPR (CPR = 8 or 16): DPP row_ror:8
// pairs lanes l and l ^ 8 inside a 16-lane row, then the gfx950 lane swaps
// v_permlane16_swap (rows 0<->1, 2<->3) and v_permlane32_swap (halves) add
// the four rows.  Every lane ends with the bit-identical sum.
template <int CPR>
__device__ __forceinline__ float rowgroup_sum(float v) {
  static_assert(CPR == 8 || CPR == 16, "row group width");
  if constexpr (CPR == 8) v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Max over the four lanes that share lane % 16 (lanes l, l ^ 16, l ^ 32,
// l ^ 48) through the gfx950 lane swaps; every lane ends with the result.
__device__ __forceinline__ float colgroup_max(float v) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
// Two fp32 -> packed bf16 in one hardware convert (round to nearest even).
__device__ __forceinline__ uint32_t cvt_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// s_waitcnt with vmcnt = N and the other counters unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wave-uniform sum/max: DPP inside the four 16-lane rows, then the four row
// results combined in a fixed order through readlane.
template <bool MAX>
__device__ __forceinline__ float wave_reduce_uniform(float v) {
  v = dpp_row16<MAX>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return MAX ? fmaxf(fmaxf(r0, r1), fmaxf(r2, r3)) : (r0 + r1) + (r2 + r3);
}

// Block-wide reduction; `red` must hold NWAVES floats of LDS.  Every thread
// gets the result.  Contains __syncthreads().
template <int NWAVES, bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* red) {
  v = MAX ? wave_max(v) : wave_sum(v);
  if constexpr (NWAVES == 1) {
    return v;
  } else {
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
    __syncthreads();  // protect `red` from a previous use
    if (lane == 0) red[w] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < NWAVES; ++i) r = MAX ? fmaxf(r, red[i]) : r + red[i];
    return r;
  }
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

// ---- cross-block hand-off without cache maintenance ---------------------
// gfx950 has one L2 per XCD and the L2s are not coherent with each other.
// A device-scope fence (__threadfence) therefore writes back and
// invalidates the whole L2 of the XCD (buffer_wbl2 / buffer_inv), which costs
// about a microsecond and serialises per XCD.  Data handed from one block to
// another is instead written and read with device-scope atomic accesses
// (global_store/global_load with the sc1 bit), which are coherent at device
// scope by themselves; only completion ordering is then needed.
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrival counter for "last block finishes" reductions.  Precondition: every
// thread's hand-off data was written with st_dev.  Waits until those stores
// have completed, counts the block's arrival, and tells every thread whether
// this block is the last of `expected`.  The last block resets the counter
// to zero, so the next launch (or graph replay) starts clean.  The last
// block must read the hand-off data with ld_dev.
__device__ __forceinline__ bool arrive_last(int* counter, int expected) {
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's sc1 stores are complete
  __syncthreads();                 // ... and so are every other thread's
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev == expected - 1;
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  return s_last != 0;
}

}  // namespace ez
