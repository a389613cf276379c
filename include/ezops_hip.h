/*
 * ezops_hip.h - C ABI of libezops_hip.so, the MI355X (gfx950) operator
 * backend for the ez-ops decode hot path.
 *
 * Conventions shared by every entry point:
 *   - Tensors are raw device pointers to contiguous row-major memory.  bf16
 *     tensors are passed as `void*` (2-byte elements), fp32 as `float*`.
 *   - Sizes are int64_t element counts.
 *   - Work is enqueued on `stream`; nothing synchronises, allocates or reads
 *     device memory back, so every call can be captured into a HIP graph.
 *   - Scratch memory is caller-owned: `*_workspace_size` gives the byte count
 *     and the caller passes a zero-filled, 16-byte aligned buffer of at least
 *     that size once;
 *     the kernels leave their counters at zero again after every call, so
 *     the same workspace serves later calls on the same stream.  Calls that
 *     overlap in time must not share a workspace.
 *   - Return value: 0 on success, EZOPS_EINVAL (-22) for rejected arguments,
 *     or the hipError_t of a failed launch; ezops_hip_last_error() describes
 *     the last failure of the calling thread.
 *
 * Each entry point names the reference (coffee0224/ez-ops) interface it
 * replaces as a drop-in behind the reference's op/registry API.
 */
#ifndef EZOPS_HIP_H
#define EZOPS_HIP_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EZOPS_HIP_ABI_VERSION 2
#define EZOPS_EINVAL (-22)
#define EZOPS_ENOSYS (-38) /* feature not compiled into this build */

int ezops_hip_abi_version(void);
const char* ezops_hip_last_error(void);

/* bf16 GEMV: C[n] = sum_k A[k] * B[n, k], fp32 accumulation, one bf16 rounding.
 * A [K], B [N, K], C [N].  Any N >= 1, K >= 1.
 * Replaces: gemv_cu(A, B, C) (ezops/kernels/gemv/gemv_cu.cu:71-87), reached
 * through GemvOp.forward (ezops/ops/gemv.py:25-26). */
int ezops_gemv_bf16(const void* A, const void* B, void* C, int64_t N, int64_t K,
                    hipStream_t stream);

/* Skinny bf16 linear layer: Y[m, n] = sum_k X[m, k] * W[n, k] for m < M.
 * X [M, K] (row stride ldx), W [N, K], Y [M, N] (row stride ldy); M >= 1.
 * Rows are processed 16 at a time with MFMA when M > 4.
 * Replaces: the `x @ W.T` projections inside the fused decode kernels
 * (ezops/kernels/fused_o_proj_ffn/fused_o_proj_ffn_triton.py:31-231,
 * ezops/kernels/qwen3_dense_decode/qwen3_dense_decode_triton.py:37-271). */
int ezops_linear_bf16(const void* X, int64_t ldx, const void* W, void* Y, int64_t ldy,
                      int64_t M, int64_t N, int64_t K, hipStream_t stream);

/* One projection stage of the fused decode ops, with its fused prologue and
 * epilogue: Y[m, n] = epi(sum_k Xn[m, k] * W[n, k]), m < M, n < N, where
 * Xn = X, or with norm != 0, Xn = X * rsqrt(mean(X^2) + eps) * norm_w
 * (norm_w NULL = unit).  epilogue 0: Y = bf16(acc); 1: Y = bf16(res + bf16(acc));
 * 2: SwiGLU, W2 holds the up rows: Y = bf16(bf16(silu(bf16(g))) * bf16(u));
 * 3: Y = acc as fp32.  With norm and M > 4 the normalised input is staged in
 * the workspace (ezops_linear_stage_workspace_size bytes, 16-byte aligned;
 * X rows contiguous).
 * Replaces: the per-stage kernels of the reference's multi-launch fused
 * variants (ezops/kernels/fused_o_proj_ffn/fused_o_proj_ffn_tl.py:49-250,
 * ezops/kernels/qwen3_dense_decode/qwen3_dense_decode_multilaunch_tl.py:68-588). */
size_t ezops_linear_stage_workspace_size(int64_t M, int64_t K, int norm);
int ezops_linear_stage_bf16(const void* X, int64_t ldx, const void* W, const void* W2, void* Y,
                            int64_t ldy, const void* res, int64_t ldr, const void* norm_w, int norm,
                            float eps, int epilogue, int64_t M, int64_t N, int64_t K, void* workspace,
                            size_t workspace_bytes, hipStream_t stream);

/* fp32 RMSNorm without weight: Out = X * rsqrt(mean(X^2) + eps), per row.
 * X, Out [rows, dim].
 * Replaces: rmsnorm_kernel host launch (ezops/kernels/rmsnorm/rmsnorm_cu.cu:51-63)
 * behind RmsNormOp (ezops/ops/rmsnorm.py:7-36). */
int ezops_rmsnorm_f32(const float* X, float* Out, int64_t rows, int64_t dim, float eps,
                      hipStream_t stream);

/* bf16 Qwen3 RMSNorm with weight: Out = bf16(x * rsqrt(mean(x^2) + eps) * w),
 * fp32 statistics.  X, Out [rows, dim]; W [dim] (NULL = unit weight).
 * Replaces: FusedOProjFfnOp._rmsnorm / Qwen3DenseDecodeOp._rmsnorm
 * (ezops/ops/fused_o_proj_ffn.py:107-110, ezops/ops/qwen3_dense_decode.py:137-140). */
int ezops_rmsnorm_bf16(const void* X, const void* W, void* Out, int64_t rows, int64_t dim,
                       float eps, hipStream_t stream);

/* fp32 row softmax over the last dim; X, Out [rows, dim].
 * Replaces: softmax_kernel host launch (ezops/kernels/softmax/softmax_cu.cu:78-89)
 * behind SoftmaxOp (ezops/ops/softmax.py:7-34). */
int ezops_softmax_f32(const float* X, float* Out, int64_t rows, int64_t dim, hipStream_t stream);

/* Deterministic fp32 full sum: Out[0] = sum(A[0:n]).
 * Replaces: reduce_cu (ezops/kernels/reduce/reduce_cu.cu:233-282) behind
 * ReduceOp (ezops/ops/reduce.py:7-31).  Two-stage, fixed order, no float atomics. */
size_t ezops_reduce_sum_workspace_size(int64_t n);
int ezops_reduce_sum_f32(const float* A, float* Out, int64_t n, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);

/* Split-KV GQA decode attention, one query token per sequence.
 * Q [B, H, D] (== [B, H, 1, D]), K/V [B, Hkv, S, D], Out [B, H, D]; bf16.
 * H % Hkv == 0, H / Hkv in {1, 2, 4, 8, 16}, D in {64, 128}.  kv_lens [B] int32 (NULL = S
 * for every sequence) limits sequence b to slots [0, kv_lens[b]).
 * max_kv_len: the caller's bound on the kv_lens entries (0 = S), used to plan
 * the split-KV grid and to request the first K/V tiles before the lengths
 * are read; entries above it are treated as max_kv_len.  Ignored without
 * kv_lens.  scale <= 0 selects 1/sqrt(D).
 * Replaces: flash_decode_tilelang_gqa_split (+ combine)
 * (ezops/kernels/attn_decode/attn_decode_tl.py:316-470, 617-627) and
 * attn_decode_cu (ezops/kernels/attn_decode/attn_decode_cu.cu:140-181)
 * behind AttnDecodeOp (ezops/ops/attn_decode.py:9-67). */
size_t ezops_attn_decode_workspace_size(int64_t B, int64_t H, int64_t Hkv, int64_t S, int64_t D);
int ezops_attn_decode_bf16(const void* Q, const void* K, const void* V, void* Out, int64_t B,
                           int64_t H, int64_t Hkv, int64_t S, int64_t D, const int32_t* kv_lens,
                           int64_t max_kv_len, float scale, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);

/* The same decode attention without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture that may not
 * call hipMalloc, tight serving loops, harnesses that forbid allocation).
 * No counterpart in the reference.  The split partials live in a fixed
 * device array of ezops_attn_decode_noalloc_max_scratch() bytes (8 MiB),
 * one per GPU, held until the process ends; shapes whose partials need more
 * (ezops_attn_decode_workspace_size above that) return EZOPS_EINVAL.  Nothing
 * is allocated, and every result equals ezops_attn_decode_bf16 bit for bit.
 * Calls that overlap in time on one GPU share the array and race: order
 * them on one stream.  The first call on a device looks up the array's
 * address (not capturable: make it once eagerly before a graph capture). */
size_t ezops_attn_decode_noalloc_max_scratch(void);
int ezops_attn_decode_noalloc_bf16(const void* Q, const void* K, const void* V, void* Out, int64_t B,
                                   int64_t H, int64_t Hkv, int64_t S, int64_t D, const int32_t* kv_lens,
                                   int64_t max_kv_len, float scale, hipStream_t stream);

/* The same decode attention over a paged KV cache (block tables).
 * K_pages / V_pages [num_pages, Hkv, page_size, D] bf16 page pools;
 * block_table [B, max_pages] int32: logical page j of sequence b (cache rows
 * [j*page_size, (j+1)*page_size)) is pool page block_table[b*max_pages + j].
 * page_size a power of two >= 32.  kv_lens [B] int32 (required) and
 * max_kv_len as in ezops_attn_decode_bf16 with S = max_pages * page_size.
 * Only the entries below ceil(max_kv_len / page_size) are read; ids outside
 * [0, num_pages) are clamped into the pool, never dereferenced out of it.
 * Workspace: ezops_attn_decode_workspace_size(B, H, Hkv, max_pages*page_size, D).
 * Results equal ezops_attn_decode_bf16 on the gathered contiguous cache.
 * No counterpart in the reference, whose cache is one contiguous
 * [B, Hkv, S, D] tensor (ezops/ops/attn_decode.py:60-61); it extends
 * AttnDecodeOp (ezops/ops/attn_decode.py:9-67) to vLLM-style page pools. */
int ezops_paged_attn_decode_bf16(const void* Q, const void* K_pages, const void* V_pages, void* Out,
                                 const int32_t* block_table, const int32_t* kv_lens, int64_t B,
                                 int64_t H, int64_t Hkv, int64_t D, int64_t num_pages,
                                 int64_t page_size, int64_t max_pages, int64_t max_kv_len,
                                 float scale, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream);

/* Prefill attention: causal GQA flash attention for a chunk of new tokens.
 * Sequence b's new tokens are rows cu_seqlens[b] .. cu_seqlens[b+1]-1 of
 * Q / Out ([T, H, D] bf16, T = cu_seqlens[B]); they already sit in the cache
 * at rows past_lens[b] + i (past_lens NULL = 0), and token i attends cache
 * rows [0, past_lens[b] + i].  Cache K/V [B, Hkv, S, D], or page pools
 * [num_pages, Hkv, page_size, D] with block_table [B, S / page_size] when
 * block_table != NULL.  max_q_len: host bound on the per-sequence token
 * counts (grid size).  D = 128; H / Hkv in {1, 2, 4, 8}; S < 2^23 (cache
 * offsets are 32-bit); scale <= 0 selects 1/sqrt(D).  T: rows of Q / Out.  Offsets and lengths are clamped into
 * [0, T] rows and [0, S] cache rows on the device; rows at or beyond S are
 * skipped (left unwritten).
 * No counterpart in the reference (decode only, ezops/ops/attn_decode.py:9-67):
 * the step before the decode path, writing the cache it reads. */
int ezops_prefill_attn_bf16(const void* Q, const void* K, const void* V, void* Out,
                            const int32_t* cu_seqlens, const int32_t* past_lens, int64_t B, int64_t T,
                            int64_t H, int64_t Hkv, int64_t S, int64_t D, int64_t max_q_len,
                            const int32_t* block_table, int64_t num_pages, int64_t page_size,
                            float scale, hipStream_t stream);

/* Qwen3 per-head QK RMSNorm + half-split RoPE + KV-cache write, one decode step.
 * q [B, H, D] (batch stride q_bstride elements), k/v [B, Hkv, D] (strides
 * k_bstride / v_bstride), q_norm_w / k_norm_w [D] (NULL = unit), cos/sin
 * [S, D] HF tables (both NULL = no RoPE), caches [B, Hkv, S, D].
 * Position of sequence b: (positions ? positions[b] : position) + pos_offset.
 * Writes q_out [B, H, D], k_out [B, Hkv, D] (k_out may be NULL) and the cache slot.
 * Replaces: FusedQkNormRopeOp backends (ezops/kernels/fused_qk_norm_rope/
 * fused_qk_norm_rope_triton.py:23-190, fused_qk_norm_rope_tl.py:32-165). */
int ezops_qk_norm_rope_bf16(const void* q, int64_t q_bstride, const void* k, int64_t k_bstride,
                            const void* v, int64_t v_bstride, const void* q_norm_w,
                            const void* k_norm_w, const void* cos, const void* sin,
                            void* K_cache, void* V_cache, void* q_out, void* k_out, int64_t B,
                            int64_t H, int64_t Hkv, int64_t D, int64_t S, int64_t position,
                            const int32_t* positions, int64_t pos_offset, float eps,
                            hipStream_t stream);

/* Fused o_proj + post-norm + SwiGLU FFN (batch x 1 token), bf16:
 *   x2 = residual + attn @ Wo^T ; xn = rmsnorm(x2) * post_norm_w
 *   out = x2 + (silu(xn @ Wg^T) * (xn @ Wu^T)) @ Wd^T
 * attn [B, QR], residual/out [B, HS], Wo [HS, QR], post_norm_w [HS],
 * Wg/Wu [IS, HS], Wd [HS, IS].  Wu may equal Wg + IS*HS (fused [gate|up]).
 * Replaces: FusedOProjFfnOp backends (ezops/kernels/fused_o_proj_ffn/
 * fused_o_proj_ffn_persistent_tl.py:56-286, fused_o_proj_ffn_triton.py:31-231). */
size_t ezops_o_proj_ffn_workspace_size(int64_t B, int64_t HS, int64_t IS, int64_t QR);
int ezops_o_proj_ffn_bf16(const void* attn, const void* residual, const void* Wo,
                          const void* post_norm_w, const void* Wg, const void* Wu, const void* Wd,
                          void* out, int64_t B, int64_t HS, int64_t IS, int64_t QR, float eps,
                          void* workspace, size_t workspace_bytes, hipStream_t stream);

/* One Qwen3 dense decoder-layer decode step (see ezops/ops/qwen3_dense_decode.py).
 * The attention stage has the limits of ezops_attn_decode_bf16: H / Hkv in
 * {1, 2, 4, 8, 16} and D in {64, 128} (EZOPS_EINVAL otherwise); the same holds
 * for the paged layer and the multi-layer step below.
 * Replaces: Qwen3DenseDecodeOp backends (ezops/kernels/qwen3_dense_decode/
 * qwen3_dense_decode_triton.py:273-384, qwen3_dense_decode_persistent_tl.py:566-609). */
typedef struct ezops_qwen3_layer {
  /* shapes */
  int64_t B, S, HS, IS, H, Hkv, D;
  float eps;
  /* inputs (bf16 unless noted) */
  const void* hidden;       /* [B, HS] */
  void* K_cache;            /* [B, Hkv, S, D], slot kv_len-1 written */
  void* V_cache;            /* [B, Hkv, S, D], slot kv_len-1 written */
  const void* Wqkv;         /* [H*D + 2*Hkv*D, HS], rows [q | k | v] */
  const void* Wo;           /* [HS, H*D] */
  const void* Wgu;          /* [2*IS, HS], rows [gate | up] */
  const void* Wd;           /* [HS, IS] */
  const void* in_norm_w;    /* [HS] or NULL (unit) */
  const void* q_norm_w;     /* [D] or NULL */
  const void* k_norm_w;     /* [D] or NULL */
  const void* post_norm_w;  /* [HS] or NULL */
  const void* cos;          /* [S, D] or NULL (no RoPE) */
  const void* sin;          /* [S, D] or NULL */
  const int32_t* kv_lens;   /* [B] int32 or NULL (= S for every sequence) */
  int64_t max_kv_len;       /* bound on the kv_lens entries, 0 = S (see ezops_attn_decode_bf16) */
  /* output */
  void* out;                /* [B, HS] */
} ezops_qwen3_layer;

size_t ezops_qwen3_layer_workspace_size(const ezops_qwen3_layer* p);
int ezops_qwen3_dense_decode_bf16(const ezops_qwen3_layer* p, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream);

/* The same layer step over a paged KV cache: K_cache / V_cache are page pools
 * [num_pages, Hkv, page_size, D]; block_table [B, S / page_size] int32 maps
 * logical page j of sequence b to a pool page (layout and clamping as in
 * ezops_paged_attn_decode_bf16).  kv_lens is required; the decoded token's
 * k/v go to row kv_lens[b]-1 of the sequence (pool page
 * block_table[b][(kv_lens[b]-1) / page_size]).  page_size: power of two >= 32
 * dividing S.  Workspace: ezops_qwen3_layer_workspace_size(p).
 * No counterpart in the reference (its cache is contiguous,
 * ezops/ops/qwen3_dense_decode.py:142-176); extends Qwen3DenseDecodeOp. */
int ezops_qwen3_dense_decode_paged_bf16(const ezops_qwen3_layer* p, const int32_t* block_table,
                                        int64_t num_pages, int64_t page_size, void* workspace,
                                        size_t workspace_bytes, hipStream_t stream);

/* A multi-layer decode step: n_layers layer steps (same shapes, each with its
 * own weights and cache) chained on one stream, then, if vocab > 0, the final
 * RMSNorm (final_norm_w [HS] or NULL = unit) and the LM head
 * (lm_head [vocab, HS]) into logits [B, vocab] bf16.
 * Input: layers[0].hidden.  Output hidden state: layers[n_layers-1].out.  The
 * other hidden/out fields are ignored (the hidden state moves through the
 * workspace).  block_table != NULL: every layer's cache is a page pool with
 * the same block table, page_size and num_pages (as in
 * ezops_qwen3_dense_decode_paged_bf16).  Allocation-free and stream-ordered:
 * the whole step can be captured in one HIP graph.
 * No counterpart in the reference, which stops at one layer
 * (ezops/ops/qwen3_dense_decode.py:9-176); it is that layer's caller. */
size_t ezops_qwen3_decode_step_workspace_size(const ezops_qwen3_layer* layers, int64_t n_layers,
                                              int64_t vocab);
int ezops_qwen3_decode_step_bf16(const ezops_qwen3_layer* layers, int64_t n_layers,
                                 const int32_t* block_table, int64_t num_pages, int64_t page_size,
                                 const void* final_norm_w, const void* lm_head, int64_t vocab,
                                 void* logits, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream);

/* Prefill of one Qwen3 dense layer for a chunk of new tokens.
 * p->hidden / p->out: [T, HS] bf16, the sequences' new tokens back to back
 * (sequence b owns rows cu_seqlens[b] .. cu_seqlens[b+1]-1, p->B sequences);
 * p->kv_lens: rows already cached per sequence before the chunk (NULL = 0);
 * token i of sequence b is written to cache row kv_lens[b] + i (after q/k
 * norm + RoPE at that position) and attends rows [0, kv_lens[b] + i].
 * p->max_kv_len is unused.  block_table != NULL: paged caches as in
 * ezops_qwen3_dense_decode_paged_bf16.  max_q_len: host bound on the
 * per-sequence token counts.  D = 128, IS % 8 == 0.  The projections run
 * the library's own GEMM (see ezops_gemm_bf16): deterministic,
 * allocation-free and graph-capturable for every shape.
 * No counterpart in the reference (decode only,
 * ezops/ops/qwen3_dense_decode.py:9-176): the step that fills the cache the
 * decode layer reads. */
size_t ezops_qwen3_prefill_workspace_size(const ezops_qwen3_layer* p, int64_t T);
int ezops_qwen3_prefill_bf16(const ezops_qwen3_layer* p, int64_t T, const int32_t* cu_seqlens,
                             int64_t max_q_len, const int32_t* block_table, int64_t num_pages,
                             int64_t page_size, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);

/* GEMM used by prefill: Y[M, N] = X[M, K] W[N, K]^T, and with R != NULL
 * (R [M, N], same leading dimension as Y; may be Y) Y = bf16(R + bf16(X W^T));
 * bf16 in/out, fp32 accumulation.  K % 8 == 0 with ldx % 8 == 0 and 16-byte
 * aligned X and W runs the MFMA kernel (a partial last K-step is masked);
 * other shapes run the library's linear-layer kernels, with the same
 * rounding.  No workspace is used: ezops_gemm_workspace_size() returns 0
 * and `workspace` may be NULL (kept for the ABI).
 * No counterpart in the reference (its GEMMs are decode GEMVs). */
size_t ezops_gemm_workspace_size(void);
int ezops_gemm_bf16(const void* X, int64_t ldx, const void* W, void* Y, int64_t ldy, const void* R,
                    int64_t M, int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                    hipStream_t stream);

/* Prefill gate/up projection fused with SwiGLU:
 * Y[M, IS] = bf16(bf16(silu(bf16(X Wg^T))) * bf16(X Wu^T)) with Wgu = [Wg; Wu]
 * as [2 IS, K] (the layer's gate/up weight), bit-identical to
 * ezops_gemm_bf16 into [M, 2 IS] followed by the SwiGLU pass.  Requires
 * IS % 128 == 0, K % 8 == 0, ldx >= K, ldx % 8 == 0, ldy % 8 == 0, ldy >= IS
 * and non-null, 16-byte aligned X, Wgu, Y (EZOPS_EINVAL otherwise).
 * No counterpart in the reference (its FFN is the decode GEMV chain). */
int ezops_gemm_swiglu_bf16(const void* X, int64_t ldx, const void* Wgu, void* Y, int64_t ldy, int64_t M,
                           int64_t IS, int64_t K, hipStream_t stream);

/* Wave-level kernel timelines (a library built with -DEZ_PROFILE=1; the
 * production build returns EZOPS_ENOSYS).  Every wave of the instrumented
 * kernels (GEMV/GEMM, decode and prefill attention, combine, norms, softmax,
 * sum, qk-norm/RoPE, SwiGLU) appends one 32-byte record when it ends:
 *   uint64 t0, t1   s_memrealtime ticks (100 MHz) at wave begin / end
 *   uint32 hw_id    HW_ID register (wave slot 3:0, SIMD 5:4, CU 11:8, SH 12, SE 15:13)
 *   uint32 xcc_id   XCC_ID register (XCD in bits 3:0)
 *   uint16 kernel   kernel id (1 gemv_rows, 2 gemv_valu, 3 linear_scalar, 4 linear_mfma,
 *                   5 attn_split, 6 attn_combine, 7 prefill_attn, 8 silu_mul,
 *                   9 qk_norm_rope, 10 rmsnorm_f32, 11 rmsnorm_bf16, 12 softmax, 13 sum,
 *                   14 gemm)
 *   uint16 wave     wave index in its block;  uint32 block  blockIdx.x
 * ezops_profile_reset clears the buffers; ezops_profile_read copies up to
 * `capacity` records to host memory and returns how many (both synchronise
 * the device).  Up to 512 records per CU and kernel source file are kept.
 * Replaces: the reference's advertised SM-level profiling with Perfetto
 * export (README.md:13), which its tree does not implement (its profiling is
 * scripts/ncu_profile.py, an Nsight Compute wrapper). */
int64_t ezops_profile_read(void* records, int64_t capacity);
int ezops_profile_reset(void);

/* STREAM-style HBM probes used to measure the chip's bandwidth peak
 * (replaces benchmarks/hardware/memory/hbm_saturation.cu:49-90):
 * kind 0 = read (sum into out[0..]; allocates in the caches, used as the
 * cache flush), 1 = write, 2 = copy, 3 = triad a = b + s*c, 4 = streaming read
 * (non-temporal hint, 32 blocks per CU looping over the array), 5 = streaming
 * read in one-shot blocks (each block reads its own contiguous 32 KiB, the
 * grid covering the array).  n = float count per array. */
int ezops_hbm_probe(int kind, float* a, const float* b, const float* c, int64_t n, float s,
                    hipStream_t stream);

/* MFMA peak probe for the hardware profile (replaces the torch-matmul sweep of
 * benchmarks/hardware/compute/matmul_peak.py, used by
 * scripts/roofline_profile.py:171-199): kind 0 = bf16, 1 = fp16
 * v_mfma_f32_16x16x32 chains, 2 = bf16 v_mfma_f32_32x32x16 chains (each
 * blocks * 4 * iters * 8 * 16384 flops per launch), 3 = fp32
 * v_mfma_f32_16x16x4_f32 chains (blocks * 4 * iters * 8 * 2048 flops). */
int ezops_mfma_probe(int kind, float* out, int64_t blocks, int64_t iters, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* EZOPS_HIP_H */
