// Torch-free check of the C ABI (include/co_alibi.h): device buffers from hipMalloc, the
// launches of co_alibi_fwd / co_alibi_bwd / co_alibi_decode on a stream, results against the
// plain-C oracle (oracle/co_alibi_ref.c, double precision), and the error paths.  It is what a
// C or C++ caller of the library does; tests/test_gpu_capi.py runs it on the GPU and
// tests/capi/build.py builds it.
//
// Bars: max-abs <= 1e-4 in fp32, <= 2e-2 in fp16 (O, LSE, dQ, dK, dV), as the Python tests.
// Exit status 0 when every check passes; one line per check on stdout.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/co_alibi.h"
#include "../../oracle/co_alibi_ref.h"

namespace {

int g_failures = 0;

void report(const char* what, double err, double tol) {
  const bool ok = err <= tol;
  std::printf("%-52s max-abs %.3e (tol %.0e) %s\n", what, err, tol, ok ? "ok" : "FAIL");
  std::fflush(stdout);
  if (!ok) ++g_failures;
}

void expect(const char* what, bool ok) {
  std::printf("%-52s %s\n", what, ok ? "ok" : "FAIL");
  std::fflush(stdout);
  if (!ok) ++g_failures;
}

#define HIP_OK(x)                                                                   \
  do {                                                                              \
    const hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                         \
      std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      std::exit(2);                                                                 \
    }                                                                               \
  } while (0)

// Deterministic N(0,1)-ish values (sum of uniforms, LCG) scaled by `scale`.
std::vector<double> randn(size_t n, uint64_t seed, double scale) {
  std::vector<double> x(n);
  uint64_t s = seed * 6364136223846793005ull + 1442695040888963407ull;
  for (size_t i = 0; i < n; ++i) {
    double acc = 0.0;
    for (int r = 0; r < 4; ++r) {
      s = s * 6364136223846793005ull + 1442695040888963407ull;
      acc += (double)(s >> 11) * (1.0 / 9007199254740992.0) - 0.5;
    }
    x[i] = scale * acc * std::sqrt(3.0);
  }
  return x;
}

// The slope table of co_alibi_attn.py:11-22, times 2 (co_alibi_attn.py:147).
std::vector<double> slopes(int H, double bias_max) {
  int n = 1;
  while (n * 2 <= H) n *= 2;
  std::vector<double> s;
  for (int h = 1; h <= n; ++h) s.push_back(2.0 * std::pow(std::pow(2.0, -bias_max / n), h));
  for (int t = 1; (int)s.size() < H; t += 2) s.push_back(2.0 * std::pow(std::pow(2.0, -(bias_max / 2) / n), t));
  return s;
}

// Host values in the element type of `dtype` (fp32 or fp16) and back.
struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
  int dtype = CO_ALIBI_F32;
  DevBuf(size_t n_, int dt) : n(n_), dtype(dt) { HIP_OK(hipMalloc(&p, bytes() ? bytes() : 16)); }
  ~DevBuf() { (void)hipFree(p); }
  size_t elem() const { return dtype == CO_ALIBI_F32 ? 4 : 2; }
  size_t bytes() const { return n * elem(); }
  // Upload x rounded to the element type; returns the rounded values as doubles.
  std::vector<double> upload(const std::vector<double>& x) {
    std::vector<double> r(n);
    if (dtype == CO_ALIBI_F32) {
      std::vector<float> h(n);
      for (size_t i = 0; i < n; ++i) r[i] = h[i] = (float)x[i];
      HIP_OK(hipMemcpy(p, h.data(), bytes(), hipMemcpyHostToDevice));
    } else {
      std::vector<_Float16> h(n);
      for (size_t i = 0; i < n; ++i) r[i] = (double)(h[i] = (_Float16)x[i]);
      HIP_OK(hipMemcpy(p, h.data(), bytes(), hipMemcpyHostToDevice));
    }
    return r;
  }
  std::vector<double> download() const {
    std::vector<double> r(n);
    if (dtype == CO_ALIBI_F32) {
      std::vector<float> h(n);
      HIP_OK(hipMemcpy(h.data(), p, bytes(), hipMemcpyDeviceToHost));
      for (size_t i = 0; i < n; ++i) r[i] = h[i];
    } else {
      std::vector<_Float16> h(n);
      HIP_OK(hipMemcpy(h.data(), p, bytes(), hipMemcpyDeviceToHost));
      for (size_t i = 0; i < n; ++i) r[i] = (double)h[i];
    }
    return r;
  }
};

double max_abs(const std::vector<double>& a, const std::vector<double>& b) {
  double m = 0.0;
  for (size_t i = 0; i < a.size(); ++i) {
    const double d = std::fabs(a[i] - b[i]);
    if (!(d <= m)) m = d;  // NaN propagates as a failure
  }
  return m;
}

// Forward + backward through the C ABI against the oracle.
void check_attention(const char* name, int dtype, int B, int Hq, int Hkv, int Sq, int Skv, int D, int causal,
                     hipStream_t stream) {
  const double tol = dtype == CO_ALIBI_F32 ? 1e-4 : 2e-2;
  const double scale = 1.0 / std::sqrt((double)D);
  const size_t nq = (size_t)B * Hq * Sq * D, nkv = (size_t)B * Hkv * Skv * D, nrow = (size_t)B * Hq * Sq;
  DevBuf q(nq, dtype), k(nkv, dtype), v(nkv, dtype), dout(nq, dtype), o(nq, dtype), dq(nq, dtype), dk(nkv, dtype),
      dv(nkv, dtype), lse(nrow, CO_ALIBI_F32), stats(co_alibi_stats_numel(B, Hq, Sq, Skv), CO_ALIBI_F32),
      sl(Hq, CO_ALIBI_F32);
  const std::vector<double> hq = q.upload(randn(nq, 1, 0.5)), hk = k.upload(randn(nkv, 2, 0.5)),
                            hv = v.upload(randn(nkv, 3, 0.5)), hdo = dout.upload(randn(nq, 4, 1.0));
  // The slopes are rounded to the input type first, as co_alibi_attn.py:147 does.
  std::vector<double> hs = slopes(Hq, 8.0);
  {
    DevBuf tmp(Hq, dtype);
    hs = tmp.upload(hs);
  }
  sl.upload(hs);
  const size_t ws_bytes = co_alibi_bwd_workspace_bytes(B, Hq, Sq, Skv);
  void* ws = nullptr;
  HIP_OK(hipMalloc(&ws, ws_bytes));

  int rc = co_alibi_fwd(dtype, q.p, k.p, v.p, (const float*)sl.p, o.p, (float*)lse.p, (float*)stats.p, B, Hq, Hkv, Sq,
                        Skv, D, causal, (float)scale, stream);
  if (rc == CO_ALIBI_OK)
    rc = co_alibi_bwd(dtype, dout.p, q.p, k.p, v.p, o.p, (const float*)lse.p, (const float*)stats.p,
                      (const float*)sl.p, dq.p, dk.p, dv.p, ws, ws_bytes, B, Hq, Hkv, Sq, Skv, D, causal,
                      (float)scale, stream);
  HIP_OK(hipStreamSynchronize(stream));
  char label[160];
  std::snprintf(label, sizeof label, "%s: launches", name);
  expect(label, rc == CO_ALIBI_OK);
  if (rc != CO_ALIBI_OK) std::printf("  %s\n", co_alibi_last_error());

  std::vector<double> ro(nq), rlse(nrow), rdq(nq), rdk(nkv), rdv(nkv);
  co_alibi_ref_forward(B, Hq, Hkv, Sq, Skv, D, causal, scale, hs.data(), hq.data(), hk.data(), hv.data(), ro.data(),
                       rlse.data());
  co_alibi_ref_backward(B, Hq, Hkv, Sq, Skv, D, causal, scale, hs.data(), hq.data(), hk.data(), hv.data(),
                        hdo.data(), rdq.data(), rdk.data(), rdv.data());
  const struct {
    const char* n;
    const DevBuf* got;
    const std::vector<double>* want;
  } outs[] = {{"o", &o, &ro}, {"lse", &lse, &rlse}, {"dq", &dq, &rdq}, {"dk", &dk, &rdk}, {"dv", &dv, &rdv}};
  for (const auto& e : outs) {
    std::snprintf(label, sizeof label, "%s: %s", name, e.n);
    report(label, max_abs(e.got->download(), *e.want), tol);
  }
  (void)hipFree(ws);
}

// One decode step against the oracle forward (non-causal, Sq = 1, the first L cache rows).
void check_decode(const char* name, int dtype, int B, int Hq, int Hkv, int L, int cap, int D, hipStream_t stream) {
  const double tol = dtype == CO_ALIBI_F32 ? 1e-4 : 2e-2;
  const double scale = 1.0 / std::sqrt((double)D);
  const size_t nq = (size_t)B * Hq * D, ncache = (size_t)B * Hkv * cap * D;
  DevBuf q(nq, dtype), kc(ncache, dtype), vc(ncache, dtype), o(nq, dtype), lse((size_t)B * Hq, CO_ALIBI_F32),
      sl(Hq, CO_ALIBI_F32);
  const std::vector<double> hq = q.upload(randn(nq, 5, 0.5)), hk = kc.upload(randn(ncache, 6, 0.5)),
                            hv = vc.upload(randn(ncache, 7, 0.5));
  std::vector<double> hs = slopes(Hq, 8.0);
  {
    DevBuf tmp(Hq, dtype);
    hs = tmp.upload(hs);
  }
  sl.upload(hs);
  const size_t ws_bytes = co_alibi_decode_workspace_bytes(B, Hq, L, D);
  void* ws = nullptr;
  HIP_OK(hipMalloc(&ws, ws_bytes));
  const int rc = co_alibi_decode(dtype, q.p, kc.p, vc.p, (const float*)sl.p, nullptr, o.p, (float*)lse.p, ws,
                                 ws_bytes, B, Hq, Hkv, L, cap, D, (float)scale, stream);
  HIP_OK(hipStreamSynchronize(stream));
  char label[160];
  std::snprintf(label, sizeof label, "%s: launches", name);
  expect(label, rc == CO_ALIBI_OK);
  if (rc != CO_ALIBI_OK) std::printf("  %s\n", co_alibi_last_error());
  // The oracle sees the first L rows of every cache head.
  std::vector<double> kL((size_t)B * Hkv * L * D), vL(kL.size()), ro(nq), rlse((size_t)B * Hq);
  for (int bh = 0; bh < B * Hkv; ++bh)
    for (size_t e = 0; e < (size_t)L * D; ++e) {
      kL[(size_t)bh * L * D + e] = hk[(size_t)bh * cap * D + e];
      vL[(size_t)bh * L * D + e] = hv[(size_t)bh * cap * D + e];
    }
  co_alibi_ref_forward(B, Hq, Hkv, 1, L, D, 0, scale, hs.data(), hq.data(), kL.data(), vL.data(), ro.data(),
                       rlse.data());
  std::snprintf(label, sizeof label, "%s: o", name);
  report(label, max_abs(o.download(), ro), tol);
  std::snprintf(label, sizeof label, "%s: lse", name);
  report(label, max_abs(lse.download(), rlse), tol);
  (void)hipFree(ws);
}

void check_errors(hipStream_t stream) {
  DevBuf q(2 * 8 * 64, CO_ALIBI_F32), o(2 * 8 * 64, CO_ALIBI_F32), sl(2, CO_ALIBI_F32);
  const int bad_dtype = co_alibi_fwd(7, q.p, q.p, q.p, (const float*)sl.p, o.p, nullptr, nullptr, 1, 2, 2, 8, 8, 64,
                                     1, 0.125f, stream);
  expect("error: unknown dtype is EUNSUPPORTED with a message",
         bad_dtype == CO_ALIBI_EUNSUPPORTED && std::strlen(co_alibi_last_error()) > 0);
  const int bad_dim = co_alibi_fwd(CO_ALIBI_F32, q.p, q.p, q.p, (const float*)sl.p, o.p, nullptr, nullptr, 1, 2, 2,
                                   8, 8, 48, 1, 0.125f, stream);
  expect("error: head_dim 48 is EUNSUPPORTED", bad_dim == CO_ALIBI_EUNSUPPORTED);
  const int misaligned = co_alibi_fwd(CO_ALIBI_F32, (const char*)q.p + 4, q.p, q.p, (const float*)sl.p, o.p, nullptr,
                                      nullptr, 1, 2, 2, 8, 8, 64, 1, 0.125f, stream);
  expect("error: misaligned q is EINVAL", misaligned == CO_ALIBI_EINVAL);
  const int groups = co_alibi_fwd(CO_ALIBI_F32, q.p, q.p, q.p, (const float*)sl.p, o.p, nullptr, nullptr, 1, 3, 2, 8,
                                  8, 64, 1, 0.125f, stream);
  expect("error: 3 query heads over 2 kv heads is EINVAL", groups == CO_ALIBI_EINVAL);
  DevBuf ws(64, CO_ALIBI_F32);  // hipMalloc'd, so 256-byte aligned: only its size is wrong
  const int small_ws = co_alibi_bwd(CO_ALIBI_F32, q.p, q.p, q.p, q.p, o.p, (const float*)sl.p, (const float*)sl.p,
                                    (const float*)sl.p, o.p, o.p, o.p, ws.p, 0, 1, 2, 2, 8, 8, 64, 1, 0.125f, stream);
  expect("error: a workspace of 0 bytes is EINVAL", small_ws == CO_ALIBI_EINVAL &&
                                                        std::strstr(co_alibi_last_error(), "workspace") != nullptr);
  expect("abi version 6", co_alibi_abi_version() == 6);
}

}  // namespace

int main() {
  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));
  check_attention("fwd+bwd fp32 causal B1 Hq4/2 S70 D64", CO_ALIBI_F32, 1, 4, 2, 70, 70, 64, 1, stream);
  check_attention("fwd+bwd fp32 non-causal B2 Hq2/1 Sq33 Skv100 D32", CO_ALIBI_F32, 2, 2, 1, 33, 100, 32, 0, stream);
  check_attention("fwd+bwd fp16 causal B1 Hq6/3 S150 D128", CO_ALIBI_F16, 1, 6, 3, 150, 150, 128, 1, stream);
  check_decode("decode fp32 B2 Hq8/2 L300 cap320 D64", CO_ALIBI_F32, 2, 8, 2, 300, 320, 64, stream);
  check_decode("decode fp16 B1 Hq4/4 L1000 D128", CO_ALIBI_F16, 1, 4, 4, 1000, 1000, 128, stream);
  check_errors(stream);
  HIP_OK(hipStreamDestroy(stream));
  std::printf("%s: %d failure(s)\n", g_failures ? "FAILED" : "PASSED", g_failures);
  return g_failures ? 1 : 0;
}
