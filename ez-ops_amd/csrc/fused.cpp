// Host-side composition of the fused decode ops from the kernels of
// gemv.hip, qk_rope.hip and attn.hip, all enqueued on the caller's stream.
//
//   o_proj + FFN:  x2 = residual + attn.Wo^T         (linear, residual epilogue)
//                  h  = silu(n(x2).Wg^T) * n(x2).Wu^T (linear, RMSNorm prologue,
//                                                       SwiGLU epilogue)
//                  out = x2 + h.Wd^T                 (linear, residual epilogue)
//   layer:         qkv = n(hidden).Wqkv^T            (linear, RMSNorm prologue)
//                  attn = gqa_decode(norm_rope(q), K/V cache + this token's
//                         norm_rope(k), v), one kernel (attn.hip)
//                  out = o_proj + FFN(attn, hidden)
#include <hip/hip_runtime.h>

#include <algorithm>


#include "internal.h"
#include "status.h"
#include "../../include/ezops_hip.h"

namespace ez {
namespace {

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

struct Carve {
  char* p;
  template <typename T>
  T* take(size_t bytes) {
    T* r = reinterpret_cast<T*>(p);
    p += align256(bytes);
    return r;
  }
};

// Batched (B > 4) stages hand activations to the next MFMA GEMM in its
// packed operand layout when the width allows it and the stages on both
// sides take their vector path (16-byte aligned weights, rows of whole
// 16-byte chunks); otherwise row-major, so no stage can reject the layout
// after earlier stages have run.
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool packable(int64_t B, int64_t K) { return B > 4 && K % 32 == 0; }

size_t ffn_ws(int64_t B, int64_t HS, int64_t IS) {
  const int64_t Bp = packed_rows(B);
  return align256(size_t(B * HS) * 2) + align256(size_t(Bp * IS) * 2) + align256(size_t(Bp * HS) * 2);
}

// attn_packed: `attn` is in the packed layout (the layer's attention output).
int run_ffn(const uint16_t* attn, bool attn_packed, const uint16_t* residual, const uint16_t* Wo,
            const uint16_t* post_w, const uint16_t* Wg, const uint16_t* Wu, const uint16_t* Wd, uint16_t* out,
            int64_t B, int64_t HS, int64_t IS, int64_t QR, float eps, char* ws, hipStream_t s) {
  Carve c{ws};
  uint16_t* x2 = c.take<uint16_t>(size_t(B * HS) * 2);
  uint16_t* h = c.take<uint16_t>(size_t(packed_rows(B) * IS) * 2);
  uint16_t* xn = c.take<uint16_t>(size_t(packed_rows(B) * HS) * 2);  // staged RMSNorm input (batch > 4)
  const bool hp = packable(B, IS) && HS % 8 == 0 && al16(Wg) && al16(Wu) && al16(Wd) && (!post_w || al16(post_w));

  LinearArgs o{};
  o.X = attn; o.ldx = QR; o.x_packed = attn_packed; o.W = Wo; o.Y = x2; o.ldy = HS;
  o.M = B; o.N = HS; o.K = QR; o.res = residual; o.ldr = HS; o.epi = kEpiResid;
  int rc = launch_linear(o, s);
  if (rc) return rc;

  LinearArgs gu{};
  gu.X = x2; gu.ldx = HS; gu.W = Wg; gu.W2 = Wu; gu.Y = h; gu.ldy = IS; gu.y_packed = hp;
  gu.M = B; gu.N = IS; gu.K = HS; gu.norm = 1; gu.norm_w = post_w; gu.eps = eps; gu.epi = kEpiSilu;
  gu.xn_ws = xn;
  rc = launch_linear(gu, s);
  if (rc) return rc;

  LinearArgs dn{};
  dn.X = h; dn.ldx = IS; dn.x_packed = hp; dn.W = Wd; dn.Y = out; dn.ldy = HS;
  dn.M = B; dn.N = HS; dn.K = IS; dn.res = x2; dn.ldr = HS; dn.epi = kEpiResid;
  return launch_linear(dn, s);
}

}  // namespace
}  // namespace ez

using namespace ez;

extern "C" size_t ezops_o_proj_ffn_workspace_size(int64_t B, int64_t HS, int64_t IS, int64_t QR) {
  (void)QR;
  return ffn_ws(B, HS, IS);
}

extern "C" int ezops_o_proj_ffn_bf16(const void* attn, const void* residual, const void* Wo,
                                     const void* post_norm_w, const void* Wg, const void* Wu,
                                     const void* Wd, void* out, int64_t B, int64_t HS, int64_t IS,
                                     int64_t QR, float eps, void* ws, size_t ws_bytes, hipStream_t s) {
  EZ_REQUIRE(attn && residual && Wo && Wg && Wu && Wd && out && ws, "o_proj_ffn: null pointer");
  EZ_REQUIRE(B >= 1 && HS >= 1 && IS >= 1 && QR >= 1, "o_proj_ffn: bad shape");
  EZ_REQUIRE(ws_bytes >= ffn_ws(B, HS, IS) && al16(ws), "o_proj_ffn: workspace too small or not 16-byte aligned");
  return run_ffn(static_cast<const uint16_t*>(attn), false, static_cast<const uint16_t*>(residual),
                 static_cast<const uint16_t*>(Wo), static_cast<const uint16_t*>(post_norm_w),
                 static_cast<const uint16_t*>(Wg), static_cast<const uint16_t*>(Wu),
                 static_cast<const uint16_t*>(Wd), static_cast<uint16_t*>(out), B, HS, IS, QR, eps,
                 static_cast<char*>(ws), s);
}

namespace {
size_t multi_kernel_ws(const ezops_qwen3_layer* p) {
  const int64_t QR = p->H * p->D, KVR = p->Hkv * p->D;
  const int64_t Bp = packed_rows(p->B);
  return align256(size_t(Bp * p->HS) * 2)                // staged RMSNorm input (batch > 4)
         + align256(size_t(p->B * (QR + 2 * KVR)) * 2)   // qkv
         + align256(size_t(Bp * QR) * 2)                 // attention output
         + align256(attn_workspace_size(p->B, p->H, p->Hkv, p->S, p->D)) + ffn_ws(p->B, p->HS, p->IS);
}
}  // namespace

extern "C" size_t ezops_qwen3_layer_workspace_size(const ezops_qwen3_layer* p) {
  if (!p || p->B < 1 || p->H < 1 || p->Hkv < 1 || p->D < 1) return 0;
  return multi_kernel_ws(p);
}

namespace {
// One layer step; block_table != NULL selects the paged cache (K_cache /
// V_cache are page pools, S = max_pages * page_size).
int run_layer(const ezops_qwen3_layer* p, const int32_t* block_table, int64_t num_pages, int64_t page_size,
              void* ws, size_t ws_bytes, hipStream_t s) {
  EZ_REQUIRE(p, "qwen3_dense_decode: null parameter block");
  EZ_REQUIRE(p->hidden && p->K_cache && p->V_cache && p->Wqkv && p->Wo && p->Wgu && p->Wd && p->out && ws,
             "qwen3_dense_decode: null pointer");
  EZ_REQUIRE(p->B >= 1 && p->S >= 1 && p->HS >= 1 && p->IS >= 1 && p->H >= 1 && p->Hkv >= 1 && p->D >= 2,
             "qwen3_dense_decode: bad shape");
  EZ_REQUIRE(p->H % p->Hkv == 0, "qwen3_dense_decode: num_heads must be divisible by num_kv_heads");
  EZ_REQUIRE((p->cos == nullptr) == (p->sin == nullptr), "qwen3_dense_decode: cos and sin go together");
  EZ_REQUIRE(ws_bytes >= ezops_qwen3_layer_workspace_size(p) && al16(ws),
             "qwen3_dense_decode: workspace too small or not 16-byte aligned");
  const int64_t QR = p->H * p->D, KVR = p->Hkv * p->D, QKV = QR + 2 * KVR;
  Carve c{static_cast<char*>(ws)};
  uint16_t* xn = c.take<uint16_t>(size_t(packed_rows(p->B) * p->HS) * 2);
  uint16_t* qkv = c.take<uint16_t>(size_t(p->B * QKV) * 2);
  uint16_t* att = c.take<uint16_t>(size_t(packed_rows(p->B) * QR) * 2);
  const bool att_packed = packable(p->B, QR) && al16(p->Wo);
  char* attn_ws = c.take<char>(attn_workspace_size(p->B, p->H, p->Hkv, p->S, p->D));
  char* ffn = c.p;

  const uint16_t* hidden = static_cast<const uint16_t*>(p->hidden);
  LinearArgs l{};
  l.X = hidden; l.ldx = p->HS; l.W = static_cast<const uint16_t*>(p->Wqkv); l.Y = qkv; l.ldy = QKV;
  l.M = p->B; l.N = QKV; l.K = p->HS; l.norm = 1; l.norm_w = static_cast<const uint16_t*>(p->in_norm_w);
  l.eps = p->eps; l.epi = kEpiStore; l.xn_ws = xn;
  // q/k RMSNorm + RoPE and the K/V-cache write of the decoded token run in
  // the attention kernel's prologue (attn.hip), reading the bf16 QKV row.
  AttnArgs a{};
  a.Q = nullptr;
  a.K = static_cast<const uint16_t*>(p->K_cache);
  a.V = static_cast<const uint16_t*>(p->V_cache);
  a.Out = att;
  a.out_packed = att_packed;
  a.B = p->B; a.H = p->H; a.Hkv = p->Hkv; a.S = p->S; a.D = p->D;
  a.kv_lens = p->kv_lens;
  a.Lh = p->max_kv_len;
  if (block_table) {
    a.block_table = block_table;
    a.page_size = int(page_size);
    a.bt_stride = p->S / page_size;
    a.num_pages = num_pages;
  }
  a.scale = 0.f;
  a.qkv = qkv; a.qkv_bs = QKV;
  a.qw = static_cast<const uint16_t*>(p->q_norm_w);
  a.kw = static_cast<const uint16_t*>(p->k_norm_w);
  a.cos = static_cast<const uint16_t*>(p->cos);
  a.sin = static_cast<const uint16_t*>(p->sin);
  a.eps = p->eps;
  // The attention stage's checks before the first launch: a rejected call
  // leaves nothing queued on the stream.
  int rc = check_attn(a);
  if (!rc) rc = launch_linear(l, s);
  if (!rc) rc = launch_attn(a, attn_ws, attn_workspace_size(p->B, p->H, p->Hkv, p->S, p->D), s);
  if (rc) return rc;

  const uint16_t* Wgu = static_cast<const uint16_t*>(p->Wgu);
  return run_ffn(att, att_packed, hidden, static_cast<const uint16_t*>(p->Wo), static_cast<const uint16_t*>(p->post_norm_w),
                 Wgu, Wgu + p->IS * p->HS, static_cast<const uint16_t*>(p->Wd), static_cast<uint16_t*>(p->out),
                 p->B, p->HS, p->IS, QR, p->eps, ffn, s);
}
}  // namespace

extern "C" int ezops_qwen3_dense_decode_bf16(const ezops_qwen3_layer* p, void* ws, size_t ws_bytes,
                                             hipStream_t s) {
  return run_layer(p, nullptr, 0, 0, ws, ws_bytes, s);
}

extern "C" int ezops_qwen3_dense_decode_paged_bf16(const ezops_qwen3_layer* p, const int32_t* block_table,
                                                   int64_t num_pages, int64_t page_size, void* ws, size_t ws_bytes,
                                                   hipStream_t s) {
  EZ_REQUIRE(p && block_table && p->kv_lens, "qwen3_dense_decode_paged: null pointer (block_table and kv_lens are required)");
  EZ_REQUIRE(page_size >= 32 && (page_size & (page_size - 1)) == 0 && p->S % page_size == 0,
             "qwen3_dense_decode_paged: page_size must be a power of two >= 32 dividing S");
  EZ_REQUIRE(num_pages >= 1 && num_pages <= (int64_t(1) << 31), "qwen3_dense_decode_paged: bad num_pages");
  return run_layer(p, block_table, num_pages, page_size, ws, ws_bytes, s);
}

// ---------------------------------------------------------------------------
// Multi-layer decode step: n_layers layer steps chained on one stream, the
// hidden state ping-ponging through the workspace, then the optional final
// RMSNorm + LM head.  Every launch is stream-ordered and allocation-free, so
// a caller captures the whole step in one HIP graph.
namespace {
bool same_shape(const ezops_qwen3_layer& a, const ezops_qwen3_layer& b) {
  return a.B == b.B && a.S == b.S && a.HS == b.HS && a.IS == b.IS && a.H == b.H && a.Hkv == b.Hkv && a.D == b.D;
}
size_t step_ws(const ezops_qwen3_layer* l0, int64_t vocab) {
  const size_t hid = align256(size_t(l0->B * l0->HS) * 2);
  const size_t head = vocab > 0 ? align256(ezops_linear_stage_workspace_size(l0->B, l0->HS, 1)) : 0;
  return 2 * hid + std::max(align256(multi_kernel_ws(l0)), head);
}
}  // namespace

extern "C" size_t ezops_qwen3_decode_step_workspace_size(const ezops_qwen3_layer* layers, int64_t n_layers,
                                                         int64_t vocab) {
  if (!layers || n_layers < 1 || !ezops_qwen3_layer_workspace_size(layers)) return 0;
  return step_ws(layers, vocab);
}

extern "C" int ezops_qwen3_decode_step_bf16(const ezops_qwen3_layer* layers, int64_t n_layers,
                                            const int32_t* block_table, int64_t num_pages, int64_t page_size,
                                            const void* final_norm_w, const void* lm_head, int64_t vocab,
                                            void* logits, void* ws, size_t ws_bytes, hipStream_t s) {
  EZ_REQUIRE(layers && n_layers >= 1 && ws, "qwen3_decode_step: null pointer or no layers");
  const ezops_qwen3_layer& l0 = layers[0];
  EZ_REQUIRE(l0.hidden && layers[n_layers - 1].out, "qwen3_decode_step: layers[0].hidden and the last out are required");
  EZ_REQUIRE(vocab >= 0 && (vocab == 0 || (lm_head && logits)), "qwen3_decode_step: lm_head and logits go with vocab > 0");
  for (int64_t i = 1; i < n_layers; ++i)
    EZ_REQUIRE(same_shape(l0, layers[i]), "qwen3_decode_step: layer %lld shape differs from layer 0", (long long)i);
  EZ_REQUIRE(ws_bytes >= ezops_qwen3_decode_step_workspace_size(layers, n_layers, vocab) && al16(ws),
             "qwen3_decode_step: workspace too small or not 16-byte aligned");
  if (block_table) {
    EZ_REQUIRE(page_size >= 32 && (page_size & (page_size - 1)) == 0 && l0.S % page_size == 0 && num_pages >= 1 &&
                   num_pages <= (int64_t(1) << 31),
               "qwen3_decode_step: page_size must be a power of two >= 32 dividing S");
  }
  for (int64_t i = 0; i < n_layers; ++i)
    EZ_REQUIRE(!block_table || layers[i].kv_lens, "qwen3_decode_step: a paged cache requires kv_lens");
  Carve c{static_cast<char*>(ws)};
  uint16_t* hbuf[2] = {c.take<uint16_t>(size_t(l0.B * l0.HS) * 2), c.take<uint16_t>(size_t(l0.B * l0.HS) * 2)};
  void* lws = c.p;
  const size_t lws_bytes = ws_bytes - size_t(c.p - static_cast<char*>(ws));
  const void* h = l0.hidden;
  for (int64_t i = 0; i < n_layers; ++i) {
    ezops_qwen3_layer p = layers[i];
    p.hidden = h;
    if (i + 1 < n_layers) p.out = hbuf[i & 1];
    const int rc = run_layer(&p, block_table, num_pages, page_size, lws, lws_bytes, s);
    if (rc) return rc;
    h = p.out;
  }
  if (vocab == 0) return 0;
  LinearArgs l{};
  l.X = static_cast<const uint16_t*>(h); l.ldx = l0.HS;
  l.W = static_cast<const uint16_t*>(lm_head);
  l.Y = static_cast<uint16_t*>(logits); l.ldy = vocab;
  l.M = l0.B; l.N = vocab; l.K = l0.HS;
  l.norm = 1; l.norm_w = static_cast<const uint16_t*>(final_norm_w); l.eps = l0.eps;
  l.epi = kEpiStore; l.xn_ws = static_cast<uint16_t*>(lws);
  return launch_linear(l, s);
}

// ---------------------------------------------------------------------------
// Prefill of one Qwen3 dense layer: T new tokens (the sequences' chunks back
// to back) through RMSNorm -> QKV GEMM -> k norm + RoPE + cache write of k and
// v -> causal flash attention (q norm + RoPE as it loads q from the QKV rows)
// -> o_proj GEMM (+residual) -> RMSNorm -> gate/up GEMM -> SwiGLU -> down
// GEMM (+residual).
namespace {
struct PrefillBufs {
  uint16_t *xn, *qkv, *att, *h, *gu, *act;
};
size_t prefill_ws(const ezops_qwen3_layer* p, int64_t T, PrefillBufs* b, char* base) {
  const int64_t QR = p->H * p->D, QKV = QR + 2 * p->Hkv * p->D;
  Carve c{base};
  auto take = [&](int64_t elems) { return c.take<uint16_t>(size_t(elems) * 2); };
  PrefillBufs t{};
  t.xn = take(T * p->HS);
  t.qkv = take(T * QKV);
  t.att = take(T * QR);
  t.h = take(T * p->HS);
  t.gu = take(T * 2 * p->IS);
  t.act = take(T * p->IS);
  if (b) *b = t;
  return size_t(c.p - base);
}
}  // namespace

extern "C" size_t ezops_qwen3_prefill_workspace_size(const ezops_qwen3_layer* p, int64_t T) {
  if (!p || T < 1 || p->H < 1 || p->Hkv < 1 || p->D < 1) return 0;
  return prefill_ws(p, T, nullptr, nullptr);
}

extern "C" int ezops_qwen3_prefill_bf16(const ezops_qwen3_layer* p, int64_t T, const int32_t* cu_seqlens,
                                        int64_t max_q_len, const int32_t* block_table, int64_t num_pages,
                                        int64_t page_size, void* ws, size_t ws_bytes, hipStream_t s) {
  EZ_REQUIRE(p && cu_seqlens && ws, "qwen3_prefill: null pointer");
  EZ_REQUIRE(p->hidden && p->K_cache && p->V_cache && p->Wqkv && p->Wo && p->Wgu && p->Wd && p->out,
             "qwen3_prefill: null pointer");
  EZ_REQUIRE(T >= 1 && p->B >= 1 && p->S >= 1 && p->HS >= 1 && p->IS >= 8 && p->IS % 8 == 0 && p->H >= 1 &&
                 p->Hkv >= 1 && p->H % p->Hkv == 0 && max_q_len >= 1,
             "qwen3_prefill: bad shape");
  EZ_REQUIRE((p->cos == nullptr) == (p->sin == nullptr), "qwen3_prefill: cos and sin go together");
  EZ_REQUIRE(ws_bytes >= ezops_qwen3_prefill_workspace_size(p, T) && al16(ws),
             "qwen3_prefill: workspace too small or not 16-byte aligned");
  if (block_table)
    EZ_REQUIRE(page_size >= 32 && (page_size & (page_size - 1)) == 0 && p->S % page_size == 0 && num_pages >= 1,
               "qwen3_prefill: page_size must be a power of two >= 32 dividing S");
  const int64_t QR = p->H * p->D, KVR = p->Hkv * p->D, QKV = QR + 2 * KVR, HS = p->HS, IS = p->IS;
  PrefillBufs w{};
  prefill_ws(p, T, &w, static_cast<char*>(ws));
  const uint16_t* hidden = static_cast<const uint16_t*>(p->hidden);
  auto W = [](const void* q) { return static_cast<const uint16_t*>(q); };

  QkRopeArgs r{};
  r.q = w.qkv; r.q_bs = QKV;
  r.k = w.qkv + QR; r.k_bs = QKV;
  r.v = w.qkv + QR + KVR; r.v_bs = QKV;
  r.qw = W(p->q_norm_w); r.kw = W(p->k_norm_w);
  r.cos = W(p->cos); r.sin = W(p->sin);
  r.Kc = static_cast<uint16_t*>(p->K_cache); r.Vc = static_cast<uint16_t*>(p->V_cache);
  r.q_out = nullptr;  // k / v only: the attention normalises and rotates q as it loads it
  r.B = T; r.H = p->H; r.Hkv = p->Hkv; r.D = p->D; r.S = p->S;
  r.cu = cu_seqlens; r.past = p->kv_lens; r.nseq = p->B;
  r.eps = p->eps;
  if (block_table) {
    r.block_table = block_table; r.bt_stride = p->S / page_size; r.page_size = int(page_size);
    r.num_pages = num_pages;
  }

  PrefillAttnArgs a{};
  a.Q = w.qkv; a.q_rs = QKV;
  a.q_raw = 1; a.qw = r.qw; a.qcos = r.cos; a.qsin = r.sin; a.qeps = p->eps;
  a.K = r.Kc; a.V = r.Vc;
  a.Out = w.att; a.o_rs = QR;
  a.cu = cu_seqlens; a.past = p->kv_lens;
  a.block_table = block_table; a.bt_stride = r.bt_stride; a.page_size = r.page_size; a.num_pages = num_pages;
  a.B = p->B; a.T = T; a.H = p->H; a.Hkv = p->Hkv; a.S = p->S; a.D = p->D; a.max_q = max_q_len;
  a.scale = 0.f;
  // Both stages' checks before the first launch: a rejected call leaves
  // the cache and the stream untouched.
  int rc = check_qk_norm_rope(r);
  if (!rc) rc = check_prefill_attn(a);
  if (rc) return rc;

  rc = ezops_rmsnorm_bf16(hidden, p->in_norm_w, w.xn, T, HS, p->eps, s);
  if (!rc) rc = gemm_bf16(w.xn, HS, W(p->Wqkv), w.qkv, QKV, nullptr, T, QKV, HS, s);
  if (!rc) rc = launch_qk_norm_rope(r, s);
  if (!rc) rc = launch_prefill_attn(a, s);
  if (!rc) rc = gemm_bf16(w.att, QR, W(p->Wo), w.h, HS, hidden, T, HS, QR, s);
  if (!rc) rc = ezops_rmsnorm_bf16(w.h, p->post_norm_w, w.xn, T, HS, p->eps, s);
  if (!rc) {
    if (gemm_swiglu_supported(w.xn, HS, W(p->Wgu), w.act, IS, T, IS, HS)) {
      rc = gemm_swiglu(w.xn, HS, W(p->Wgu), w.act, IS, T, IS, HS, s);
    } else {
      rc = gemm_bf16(w.xn, HS, W(p->Wgu), w.gu, 2 * IS, nullptr, T, 2 * IS, HS, s);
      if (!rc) rc = launch_silu_mul(w.gu, w.act, T, IS, s);
    }
  }
  if (!rc)
    rc = gemm_bf16(w.act, IS, W(p->Wd), static_cast<uint16_t*>(p->out), HS, w.h, T, HS, IS, s);
  return rc;
}
