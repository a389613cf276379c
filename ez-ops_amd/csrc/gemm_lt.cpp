// bf16 GEMMs of the prefill stage:
//   Y[M, N] = X[M, K] W[N, K]^T (+ R[M, N]), fp32 accumulation, bf16 out.
// Shapes with K % 64 == 0 and 16-byte aligned operands (every transformer
// projection) run the own MFMA kernel (gemm.hip); the others fall back to a
// hipBLASLt library GEMM, set up here, whose residual add rides on the
// GEMM's beta * C term (one rounding instead of the MFMA kernel's two).
//
// hipBLASLt is column-major: the row-major Y^T is D (N x M, ld ldy), computed
// as op(A) B with A = W viewed as a K x N column-major matrix (op T) and
// B = X^T viewed as K x M (ld ldx).
//
// One handle per device and one algorithm per shape are set up on first use
// and cached: the first eager call of a shape times up to kTune candidates
// from hipBLASLt's heuristic on the caller's stream (a one-time host wait)
// and keeps the fastest; a first call under graph capture, or with the
// residual aliasing the output, takes the heuristic's first choice.  A
// caller that captures a graph runs the shape once eagerly first.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "internal.h"
#include "status.h"
#include "../../include/ezops_hip.h"

namespace ez {
namespace {

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t ws = 0;
};

constexpr int kTune = 8;
using Key = std::tuple<int, int64_t, int64_t, int64_t, int64_t, int64_t, bool, size_t>;
std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<Key, Plan> g_plans;

#define EZ_LT(call)                                                                  \
  do {                                                                               \
    const hipblasStatus_t st_ = (call);                                              \
    EZ_REQUIRE(st_ == HIPBLAS_STATUS_SUCCESS, "gemm: %s failed (status %d)", #call, int(st_)); \
  } while (0)

// Time one candidate: a warm-up and 3 runs between events on the stream.
float time_algo(hipblasLtHandle_t h, const Plan& p, const hipblasLtMatmulAlgo_t& algo, size_t ws_need,
                const uint16_t* X, const uint16_t* W, uint16_t* Y, const uint16_t* R, void* ws, hipStream_t s) {
  const float alpha = 1.f, beta = R ? 1.f : 0.f;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.f;
  float ms = -1.f;
  bool ok = hipblasLtMatmul(h, p.desc, &alpha, W, p.a, X, p.b, &beta, R ? R : Y, p.c, Y, p.c, &algo,
                            ws_need ? ws : nullptr, ws_need, s) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipEventRecord(e0, s) == hipSuccess;
  for (int i = 0; ok && i < 3; ++i)
    ok = hipblasLtMatmul(h, p.desc, &alpha, W, p.a, X, p.b, &beta, R ? R : Y, p.c, Y, p.c, &algo,
                         ws_need ? ws : nullptr, ws_need, s) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
  ok = ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return ok ? ms : -1.f;
}

int get_plan(int dev, int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, bool resid, size_t ws_cap,
             hipblasLtHandle_t* h, const Plan** out, const uint16_t* X, const uint16_t* W, uint16_t* Y,
             const uint16_t* R, void* ws, hipStream_t s) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto hit = g_handles.find(dev);
  if (hit == g_handles.end()) {
    hipblasLtHandle_t nh = nullptr;
    EZ_LT(hipblasLtCreate(&nh));
    hit = g_handles.emplace(dev, nh).first;
  }
  *h = hit->second;
  const Key key{dev, M, N, K, ldx, ldy, resid, ws_cap};
  auto it = g_plans.find(key);
  if (it != g_plans.end()) {
    *out = &it->second;
    return 0;
  }
  Plan p;
  EZ_LT(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F));
  const int32_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  EZ_LT(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)));
  EZ_LT(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)));
  EZ_LT(hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, uint64_t(K), uint64_t(N), K));
  EZ_LT(hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, uint64_t(K), uint64_t(M), ldx));
  EZ_LT(hipblasLtMatrixLayoutCreate(&p.c, HIP_R_16BF, uint64_t(N), uint64_t(M), ldy));
  hipblasLtMatmulPreference_t pref = nullptr;
  EZ_LT(hipblasLtMatmulPreferenceCreate(&pref));
  const uint64_t cap = ws_cap;
  EZ_LT(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &cap, sizeof(cap)));
  hipblasLtMatmulHeuristicResult_t res[kTune];
  int n = 0;
  const hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(*h, p.desc, p.a, p.b, p.c, p.c, pref, kTune, res, &n);
  hipblasLtMatmulPreferenceDestroy(pref);
  EZ_REQUIRE(st == HIPBLAS_STATUS_SUCCESS && n >= 1, "gemm: no hipBLASLt algorithm for M=%lld N=%lld K=%lld",
             (long long)M, (long long)N, (long long)K);
  int best = 0;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  const bool tune =
      n > 1 && R != Y && hipStreamIsCapturing(s, &capture) == hipSuccess && capture == hipStreamCaptureStatusNone;
  if (tune) {
    float best_ms = -1.f;
    for (int i = 0; i < n; ++i) {
      if (res[i].state != HIPBLAS_STATUS_SUCCESS || res[i].workspaceSize > ws_cap) continue;
      const float ms = time_algo(*h, p, res[i].algo, res[i].workspaceSize, X, W, Y, R, ws, s);
      if (ms > 0.f && (best_ms < 0.f || ms < best_ms)) {
        best_ms = ms;
        best = i;
      }
    }
  }
  p.algo = res[best].algo;
  p.ws = res[best].workspaceSize;
  *out = &g_plans.emplace(key, p).first->second;
  return 0;
}

}  // namespace

int gemm_bf16(const uint16_t* X, int64_t ldx, const uint16_t* W, uint16_t* Y, int64_t ldy, const uint16_t* R,
              int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes, hipStream_t s) {
  EZ_REQUIRE(X && W && Y, "gemm: null pointer");
  EZ_REQUIRE(M >= 1 && N >= 1 && K >= 1 && ldx >= K && ldy >= N, "gemm: bad shape");
  if (gemm_mfma_supported(X, ldx, W, Y, ldy, R, M, N, K)) return gemm_mfma(X, ldx, W, Y, ldy, R, M, N, K, s);
  int dev = 0;
  EZ_REQUIRE(hipGetDevice(&dev) == hipSuccess, "gemm: no current device");
  hipblasLtHandle_t h = nullptr;
  const Plan* p = nullptr;
  const int rc = get_plan(dev, M, N, K, ldx, ldy, R != nullptr, ws ? ws_bytes : 0, &h, &p, X, W, Y, R, ws, s);
  if (rc) return rc;
  const float alpha = 1.f, beta = R ? 1.f : 0.f;
  EZ_LT(hipblasLtMatmul(h, p->desc, &alpha, W, p->a, X, p->b, &beta, R ? R : Y, p->c, Y, p->c, &p->algo,
                        p->ws ? ws : nullptr, p->ws, s));
  return launch_status("gemm");
}

}  // namespace ez

extern "C" size_t ezops_gemm_workspace_size(void) { return ez::kGemmWorkspace; }

extern "C" int ezops_gemm_swiglu_bf16(const void* X, int64_t ldx, const void* Wgu, void* Y, int64_t ldy, int64_t M,
                                      int64_t IS, int64_t K, hipStream_t stream) {
  return ez::gemm_swiglu(static_cast<const uint16_t*>(X), ldx, static_cast<const uint16_t*>(Wgu),
                         static_cast<uint16_t*>(Y), ldy, M, IS, K, stream);
}

extern "C" int ezops_gemm_bf16(const void* X, int64_t ldx, const void* W, void* Y, int64_t ldy, const void* R,
                               int64_t M, int64_t N, int64_t K, void* ws, size_t ws_bytes, hipStream_t stream) {
  return ez::gemm_bf16(static_cast<const uint16_t*>(X), ldx, static_cast<const uint16_t*>(W),
                       static_cast<uint16_t*>(Y), ldy, static_cast<const uint16_t*>(R), M, N, K, ws, ws_bytes, stream);
}
