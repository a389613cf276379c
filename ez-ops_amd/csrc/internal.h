// Host-side launchers shared between the translation units of libezops_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ezops_hip.h"

namespace ez {

// "MFMA-packed" activation layout for the skinny GEMM (M > 4): batch rows
// in blocks of 16, each 32-wide k-step of a block stored as the 1 KiB B
// operand of v_mfma_f32_16x16x32_bf16 (lane 16 g + i holds row i, k-slots
// 8 g .. 8 g + 7), so every fragment load is one contiguous 1 KiB read.
// Element (m, k) of an [M, K] matrix (K % 32 == 0; M padded to 16) sits at:
__host__ __device__ __forceinline__ int64_t packed_index(int64_t m, int64_t k, int64_t K) {
  return (((m >> 4) * (K >> 5) + (k >> 5)) * 64 + ((k >> 3) & 3) * 16 + (m & 15)) * 8 + (k & 7);
}
__host__ __device__ __forceinline__ int64_t packed_rows(int64_t M) { return (M + 15) / 16 * 16; }

enum Epilogue : int {
  kEpiStore = 0,   // Y = bf16(acc)
  kEpiResid = 1,   // Y = bf16(res + bf16(acc))            (o_proj / down_proj + residual)
  kEpiSilu = 2,    // Y = bf16(bf16(silu(bf16(g))) * bf16(u)), g from W row n, u from W2 row n
  kEpiStoreF32 = 3 // Y = acc (fp32)
};

// Y[m, n] = epilogue( sum_k Xn[m, k] * W[n, k] ), m < M, n < N, where
// Xn = X, or with `norm` set Xn = X * rsqrt(mean(X^2) + eps) * norm_w
// (the RMSNorm prologue, statistics over the full K row of X).
struct LinearArgs {
  const uint16_t* X; int64_t ldx;
  const uint16_t* W;
  const uint16_t* W2;          // kEpiSilu: up-projection rows
  void* Y; int64_t ldy;
  int64_t M, N, K;
  const uint16_t* res; int64_t ldr;  // kEpiResid
  int norm;                    // apply the RMSNorm prologue
  const uint16_t* norm_w;      // NULL = unit weight
  float eps;
  int epi;
  uint16_t* xn_ws;             // M > 4 with `norm`: packed_rows(M)*K bf16 scratch for the staged input
  int x_packed;                // X is in the MFMA-packed layout (M > 4, K % 32 == 0; ldx unused)
  int y_packed;                // Y is written in the MFMA-packed layout (M > 4, ldy = N, N % 32 == 0)
};

int launch_linear(const LinearArgs& a, hipStream_t s);

// Out = bf16(X * rsqrt(mean(X^2) + eps) * W) per row, written in the
// MFMA-packed layout (rowops.hip); dim % 32 == 0, Out holds packed_rows(rows)*dim.
int launch_rmsnorm_bf16_packed(const uint16_t* X, const uint16_t* W, uint16_t* Out, int64_t rows, int64_t dim,
                               float eps, hipStream_t s);

struct QkRopeArgs {
  const uint16_t* q; int64_t q_bs;
  const uint16_t* k; int64_t k_bs;
  const uint16_t* v; int64_t v_bs;
  const uint16_t* qw; const uint16_t* kw;
  const uint16_t* cos; const uint16_t* sin;
  uint16_t* Kc; uint16_t* Vc;
  uint16_t* q_out; uint16_t* k_out;  // q_out NULL: the k / v heads only (q is left to its consumer)
  int64_t B, H, Hkv, D, S;
  int64_t position; const int32_t* positions; int64_t pos_offset;
  float eps;
  // Prefill rows (cu != NULL): row t (t < B) is a token of sequence s with
  // cu[s] <= t < cu[s+1] (nseq sequences) at cache position past[s] + t - cu[s].
  const int32_t* cu; const int32_t* past; int64_t nseq;
  // Paged cache (block_table != NULL): Kc / Vc are pools [pages, Hkv, page_size, D].
  const int32_t* block_table; int64_t bt_stride; int page_size; int64_t num_pages;
};
// check_*: the launcher's argument checks alone (EZ_OK or EZOPS_EINVAL with
// the error text set), for callers that validate every stage before launching any.
int check_qk_norm_rope(const QkRopeArgs& a);
int launch_qk_norm_rope(const QkRopeArgs& a, hipStream_t s);

struct AttnArgs {
  const uint16_t* Q;  // [B, H, D]; NULL selects the fused layer prologue below
  const uint16_t* K; const uint16_t* V;  // [B, Hkv, S, D], or page pools [pages, Hkv, page_size, D]
  // Paged cache (block_table != NULL): logical page j of sequence b is pool
  // page block_table[b * bt_stride + j]; S = bt_stride * page_size.
  const int32_t* block_table; int64_t bt_stride; int page_size; int64_t num_pages;
  uint16_t* Out;      // [B, H, D]
  int64_t B, H, Hkv, S, D;
  const int32_t* kv_lens;
  int out_packed;     // Out in the MFMA-packed layout of [B, H*D] (the layer's o_proj input)
  int sort_lens;      // set by the launcher: serve the sequences longest first
  int64_t split_chunk;  // set by the launcher: > 0 = ragged batch, ceil(len / split_chunk) splits per sequence
  int64_t tps;          // set by the launcher: > 0 = split s owns the contiguous tiles [s tps, (s + 1) tps)
  int64_t Lh;         // bound on the live lengths for planning (0 = S); lengths above it are cut to it
  float scale;
  // Fused layer prologue (Q == NULL): q/k/v of the decoded token come from
  // the bf16 QKV projection (row b at qkv + b*qkv_bs, columns [q | k | v]);
  // q and k get the per-head RMSNorm (weights qw/kw, NULL = unit) and RoPE
  // (cos/sin rows at the token position, NULL = none), and the block whose
  // split holds the token position writes k and v into the cache slot.
  const uint16_t* qkv; int64_t qkv_bs;
  const uint16_t* qw; const uint16_t* kw;
  const uint16_t* cos; const uint16_t* sin;
  float eps;
};
size_t attn_workspace_size(int64_t B, int64_t H, int64_t Hkv, int64_t S, int64_t D);
int check_attn(const AttnArgs& a);
int launch_attn(const AttnArgs& a, void* ws, size_t ws_bytes, hipStream_t s);

// Prefill attention: new tokens of sequence b are rows cu[b] .. cu[b+1]-1 of
// Q / Out (row strides q_rs / o_rs, head h at + h*D) and sit at cache rows
// past[b] + i; each attends cache rows [0, its row] (causal).
struct PrefillAttnArgs {
  const uint16_t* Q; int64_t q_rs;
  const uint16_t* K; const uint16_t* V;  // [B, Hkv, S, D] or pools [pages, Hkv, page_size, D]
  uint16_t* Out; int64_t o_rs;
  const int32_t* cu; const int32_t* past;  // [B + 1], [B] (NULL = 0)
  const int32_t* block_table; int64_t bt_stride; int page_size; int64_t num_pages;
  int64_t B, T, H, Hkv, S, D, max_q;  // T: rows of Q / Out
  float scale;
  // Raw q (q_raw != 0, the layer's QKV rows): each query head gets the
  // per-head RMSNorm (weight qw, NULL = unit; eps) and the half-split RoPE
  // at its cache position (cos / sin rows, NULL = none) as it is loaded,
  // rounded to bf16 as the separate QK-norm + RoPE stage rounds it.
  int q_raw; const uint16_t* qw; const uint16_t* qcos; const uint16_t* qsin; float qeps;
};
int check_prefill_attn(const PrefillAttnArgs& a);
int launch_prefill_attn(const PrefillAttnArgs& a, hipStream_t s);
int launch_silu_mul(const uint16_t* gu, uint16_t* out, int64_t T, int64_t IS, hipStream_t s);

// Own MFMA GEMM (gemm.hip): Y[M,N] = X[M,K] W[N,K]^T, or bf16(R + bf16(X W^T))
// with R (same layout as Y, may be Y); needs K % 8 == 0, ldx % 8 == 0,
// ldx >= K, ldy >= N and 16-byte aligned X and W.
bool gemm_mfma_supported(const uint16_t* X, int64_t ldx, const uint16_t* W, const uint16_t* Y, int64_t ldy,
                         const uint16_t* R, int64_t M, int64_t N, int64_t K);
int gemm_mfma(const uint16_t* X, int64_t ldx, const uint16_t* W, uint16_t* Y, int64_t ldy, const uint16_t* R,
              int64_t M, int64_t N, int64_t K, hipStream_t s);
// Gate/up projection fused with SwiGLU: Y[M, IS] = silu(X Wg^T) * (X Wu^T),
// W = [Wg; Wu] as [2 IS, K]; rounding as GEMM then the separate SwiGLU pass.
bool gemm_swiglu_supported(const uint16_t* X, int64_t ldx, const uint16_t* W, const uint16_t* Y, int64_t ldy,
                           int64_t M, int64_t IS, int64_t K);
int gemm_swiglu(const uint16_t* X, int64_t ldx, const uint16_t* W, uint16_t* Y, int64_t ldy, int64_t M, int64_t IS,
                int64_t K, hipStream_t s);
// Any shape: the MFMA kernel where supported, else the linear-layer kernels.
int gemm_bf16(const uint16_t* X, int64_t ldx, const uint16_t* W, uint16_t* Y, int64_t ldy, const uint16_t* R,
              int64_t M, int64_t N, int64_t K, hipStream_t s);


}  // namespace ez
