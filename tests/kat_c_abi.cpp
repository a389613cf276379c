// Known-answer checks of the C ABI from C++ (no Python): tiny inputs whose
// results are exact in bf16 / fp32, run through libezops_hip.so on the
// current HIP device.  Built next to the library (ez-ops_amd/build.py) and
// run by tests/test_hip_c_abi.py; exit status 0 = every check passed.
//
//   gemv:     W[n][k] = n - 3, x[k] = k % 3 - 1 (K = 16): y[n] = (n - 3) * sum(x)
//   attn:     q = 0 (uniform softmax over the live rows), V rows of 3s, 6s,
//             9s: the output is 6 everywhere (exact in bf16), with a length
//             of 3 inside a larger cache whose other rows hold 1000
//   prefill:  q = 0 over 16 new tokens: token i averages V rows 0..i
//   rmsnorm:  rows of +-2: x * rsqrt(4 + eps) = +-1 within 1e-6
//   errors:   N = 0 is rejected with EZOPS_EINVAL and a message
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../include/ezops_hip.h"

namespace {

int failures = 0;

void check(bool ok, const char* what) {
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
  if (!ok) ++failures;
}

uint16_t bf(float f) {  // exact for the small integers used here
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return uint16_t(u >> 16);
}
float fb(uint16_t h) {
  const uint32_t u = uint32_t(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

template <typename T>
T* dev(const std::vector<T>& h) {
  T* d = nullptr;
  if (hipMalloc(&d, h.size() * sizeof(T)) != hipSuccess) return nullptr;
  if (hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
  return d;
}
template <typename T>
std::vector<T> host(const T* d, size_t n) {
  std::vector<T> h(n);
  if (hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess) h.clear();
  return h;
}

void kat_gemv() {
  const int64_t N = 8, K = 16;
  std::vector<uint16_t> W(N * K), x(K), y(N, 0);
  float sx = 0.f;
  for (int64_t k = 0; k < K; ++k) {
    x[k] = bf(float(k % 3 - 1));
    sx += float(k % 3 - 1);
  }
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) W[n * K + k] = bf(float(n - 3));
  uint16_t *dx = dev(x), *dW = dev(W), *dy = dev(y);
  const int rc = ezops_gemv_bf16(dx, dW, dy, N, K, nullptr);
  check(rc == 0 && hipDeviceSynchronize() == hipSuccess, "gemv returns 0");
  const auto out = host(dy, N);
  bool ok = out.size() == size_t(N);
  for (int64_t n = 0; ok && n < N; ++n) ok = fb(out[n]) == float(n - 3) * sx;
  check(ok, "gemv y[n] = (n - 3) * sum(x), exact");
  (void)hipFree(dx);
  (void)hipFree(dW);
  (void)hipFree(dy);
}

void kat_attn() {
  const int64_t B = 1, H = 4, Hkv = 1, S = 40, D = 64, L = 3;
  std::vector<uint16_t> Q(B * H * D, bf(0.f)), K(B * Hkv * S * D, bf(1000.f)), V(B * Hkv * S * D, bf(1000.f));
  for (int64_t s = 0; s < L; ++s)
    for (int64_t d = 0; d < D; ++d) {
      K[s * D + d] = bf(float(d % 5));
      V[s * D + d] = bf(float(3 * (s + 1)));
    }
  std::vector<uint16_t> O(B * H * D, 0);
  const std::vector<int32_t> lens{int32_t(L)};
  const size_t ws_bytes = ezops_attn_decode_workspace_size(B, H, Hkv, S, D);
  std::vector<uint8_t> ws(ws_bytes > 0 ? ws_bytes : 1, 0);
  uint16_t *dQ = dev(Q), *dK = dev(K), *dV = dev(V), *dO = dev(O);
  int32_t* dl = dev(lens);
  uint8_t* dws = dev(ws);
  const int rc = ezops_attn_decode_bf16(dQ, dK, dV, dO, B, H, Hkv, S, D, dl, 0, 0.f, dws, ws.size(), nullptr);
  check(rc == 0 && hipDeviceSynchronize() == hipSuccess, "attn_decode returns 0");
  const auto out = host(dO, size_t(B * H * D));
  bool ok = out.size() == size_t(B * H * D);
  for (size_t i = 0; ok && i < out.size(); ++i) ok = fb(out[i]) == 6.f;
  check(ok, "attn_decode: uniform softmax over 3 live rows gives their mean 6, exact");
  (void)hipFree(dQ);
  (void)hipFree(dK);
  (void)hipFree(dV);
  (void)hipFree(dO);
  (void)hipFree(dl);
  (void)hipFree(dws);
}

void kat_prefill_attn() {
  // q = 0: token i attends keys 0..i uniformly; V row r holds 3(r + 1), so
  // every output of token i is 3(i + 2) / 2 (exact in bf16 for i < 16).
  const int64_t B = 1, T = 16, H = 4, Hkv = 1, S = 16, D = 128;
  std::vector<uint16_t> Q(T * H * D, bf(0.f)), K(B * Hkv * S * D), V(B * Hkv * S * D), O(T * H * D, 0);
  for (int64_t r = 0; r < S; ++r)
    for (int64_t d = 0; d < D; ++d) {
      K[r * D + d] = bf(float((r + d) % 7) - 3.f);
      V[r * D + d] = bf(float(3 * (r + 1)));
    }
  const std::vector<int32_t> cu{0, int32_t(T)};
  uint16_t *dQ = dev(Q), *dK = dev(K), *dV = dev(V), *dO = dev(O);
  int32_t* dcu = dev(cu);
  const int rc = ezops_prefill_attn_bf16(dQ, dK, dV, dO, dcu, nullptr, B, T, H, Hkv, S, D, T, nullptr, 0, 0, 0.f,
                                         nullptr);
  check(rc == 0 && hipDeviceSynchronize() == hipSuccess, "prefill_attn returns 0");
  const auto out = host(dO, size_t(T * H * D));
  bool ok = out.size() == size_t(T * H * D);
  for (int64_t i = 0; ok && i < T; ++i)
    for (int64_t j = 0; ok && j < H * D; ++j) ok = fb(out[i * H * D + j]) == 1.5f * float(i + 2);
  check(ok, "prefill_attn: token i averages V rows 0..i, 3(i + 2) / 2, exact");
  (void)hipFree(dQ);
  (void)hipFree(dK);
  (void)hipFree(dV);
  (void)hipFree(dO);
  (void)hipFree(dcu);
}

void kat_rmsnorm() {
  const int64_t rows = 3, dim = 100;
  std::vector<float> X(rows * dim), Out(rows * dim, 0.f);
  for (int64_t i = 0; i < rows * dim; ++i) X[i] = (i % 2) ? 2.f : -2.f;
  float *dX = dev(X), *dOut = dev(Out);
  const int rc = ezops_rmsnorm_f32(dX, dOut, rows, dim, 1e-6f, nullptr);
  check(rc == 0 && hipDeviceSynchronize() == hipSuccess, "rmsnorm_f32 returns 0");
  const auto out = host(dOut, size_t(rows * dim));
  bool ok = out.size() == size_t(rows * dim);
  for (int64_t i = 0; ok && i < rows * dim; ++i) ok = std::fabs(out[i] - ((i % 2) ? 1.f : -1.f)) <= 1e-6f;
  check(ok, "rmsnorm_f32 of +-2 rows is +-1 within 1e-6");
  (void)hipFree(dX);
  (void)hipFree(dOut);
}

void kat_errors() {
  const int rc = ezops_gemv_bf16(nullptr, nullptr, nullptr, 0, 16, nullptr);
  const char* msg = ezops_hip_last_error();
  check(rc == EZOPS_EINVAL && msg && std::strlen(msg) > 0, "gemv N = 0 -> EZOPS_EINVAL with a message");
}

}  // namespace

int main() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
    std::printf("no HIP device\n");
    return 2;
  }
  std::printf("abi version %d\n", ezops_hip_abi_version());
  kat_gemv();
  kat_attn();
  kat_prefill_attn();
  kat_rmsnorm();
  kat_errors();
  std::printf(failures ? "KAT FAILED (%d)\n" : "KAT OK\n", failures);
  return failures ? 1 : 0;
}
