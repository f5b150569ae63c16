// Native host harness for libneso_amd.so: drives the C ABI from C++ with no
// Python, the role of the reference's kernel harness (macos/harness.rs:
// test() at :201-290, bench() at :292-366).
//
//   neso_harness test    known-answer tests through the C entry points
//   neso_harness bench   FA2 N sweep (one head, d = 64) and the headline
//                        shape, median of 20 timed launches after 10
//
// The known answers are closed forms, computed here without any attention
// or matmul code:
//   * FA2 with Q = K = 0: every score is 0, so each output row is the column
//     mean of V (the reference harness's own check, :247-268, tolerance
//     2e-3), at N = 64 (d = 64 and 128) and at the ragged N = 100 with 3
//     heads;
//   * int4 W4A16 with one-hot X rows: Y[m][n] = (code(n, k_m) - 8) *
//     scale(n, k_m / 32) exactly (small integers times an fp16 scale, one
//     rounding), at M = 1 (GEMV) and M = 3 (MFMA kernels);
//   * a rejected call (head_dim 48) returns NESO_EUNSUPPORTED and sets
//     neso_last_error().
// Exit status 0 when every check passes.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "neso_amd.h"

namespace {

#define HIP_OK(x)                                                                  \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      exit(2);                                                                     \
    }                                                                              \
  } while (0)

uint16_t to_half(float f) {
  const _Float16 h = (_Float16)f;
  uint16_t u;
  memcpy(&u, &h, 2);
  return u;
}
float from_half(uint16_t u) {
  _Float16 h;
  memcpy(&h, &u, 2);
  return (float)h;
}

template <typename T>
T* upload(const std::vector<T>& v) {
  T* d = nullptr;
  HIP_OK(hipMalloc(&d, std::max<size_t>(v.size(), 1) * sizeof(T)));
  if (!v.empty()) HIP_OK(hipMemcpy(d, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
  return d;
}
template <typename T>
std::vector<T> download(const T* d, size_t n) {
  std::vector<T> v(n);
  HIP_OK(hipMemcpy(v.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
  return v;
}

// The reference harness's value patterns (:171-183), exactly representable
// in fp16.
float pattern_v(size_t i) { return ((float)(i % 17) - 8.f) * 0.125f; }
float pattern_q(size_t i) { return ((float)(i % 29) - 14.f) * 0.01f; }
float pattern_k(size_t i) { return ((float)(i % 31) - 15.f) * 0.01f; }

int check_status(int st, const char* what) {
  if (st != NESO_OK) {
    fprintf(stderr, "FAIL %s: %s (%s)\n", what, neso_status_string(st), neso_last_error());
    return 1;
  }
  return 0;
}

int fa2_mean_kat(int n, int d, int heads) {
  const size_t cnt = (size_t)heads * n * d;
  std::vector<uint16_t> zero(cnt, to_half(0.f)), v(cnt);
  for (size_t i = 0; i < cnt; ++i) v[i] = to_half(pattern_v(i));
  uint16_t *dq = upload(zero), *dk = upload(zero), *dv = upload(v);
  float* dout = nullptr;
  HIP_OK(hipMalloc(&dout, cnt * sizeof(float)));
  const int st = neso_flash_attention_fwd(dq, dk, dv, dout, n, d, d, 1.f / sqrtf((float)d), d,
                                          heads, (int64_t)n * d, (int64_t)n * d, 0, nullptr);
  int bad = check_status(st, "neso_flash_attention_fwd");
  if (!bad) {
    HIP_OK(hipDeviceSynchronize());
    const std::vector<float> out = download(dout, cnt);
    float worst = 0.f;
    for (int h = 0; h < heads; ++h)
      for (int c = 0; c < d; ++c) {
        double mean = 0;
        for (int r = 0; r < n; ++r) mean += from_half(v[((size_t)h * n + r) * d + c]);
        mean /= n;
        for (int r = 0; r < n; ++r)
          worst = std::max(worst, (float)fabs(out[((size_t)h * n + r) * d + c] - mean));
      }
    bad = worst > 2e-3f;
    printf("%s flash_attention_fwd Q=K=0 -> column mean of V (f16, N=%d, d=%d, heads=%d): "
           "max error %.3g\n", bad ? "FAIL" : "PASS", n, d, heads, worst);
  }
  HIP_OK(hipFree(dq));
  HIP_OK(hipFree(dk));
  HIP_OK(hipFree(dv));
  HIP_OK(hipFree(dout));
  return bad;
}

int w4a16_onehot_kat(int m) {
  const int n = 300, k = 256, groups = k / 32;
  // Codes and scales from a fixed pattern; X row r is one-hot at k_r.
  std::vector<int32_t> words((size_t)n * k / 8, 0);
  std::vector<uint16_t> scales((size_t)n * groups), x((size_t)m * k, to_half(0.f));
  auto code = [&](int nn, int kk) { return (nn * 7 + kk * 3) % 16; };
  for (int nn = 0; nn < n; ++nn) {
    for (int kk = 0; kk < k; ++kk)
      words[(size_t)nn * (k / 8) + kk / 8] |= code(nn, kk) << (4 * (kk % 8));
    for (int g = 0; g < groups; ++g) scales[(size_t)nn * groups + g] = to_half(0.0625f * (1 + (nn + g) % 5));
  }
  std::vector<int> hot(m);
  for (int r = 0; r < m; ++r) {
    hot[r] = (37 + 61 * r) % k;
    x[(size_t)r * k + hot[r]] = to_half(1.f);
  }
  uint16_t *dx = upload(x), *ds = upload(scales), *dy = nullptr;
  int32_t* dw = upload(words);
  HIP_OK(hipMalloc(&dy, (size_t)m * n * 2));
  const int st = neso_w4a16_matmul(dx, dw, ds, dy, m, n, k, k, n, 32, 8, nullptr);
  int bad = check_status(st, "neso_w4a16_matmul");
  if (!bad) {
    HIP_OK(hipDeviceSynchronize());
    const std::vector<uint16_t> y = download(dy, (size_t)m * n);
    int wrong = 0;
    for (int r = 0; r < m; ++r)
      for (int nn = 0; nn < n; ++nn) {
        const float want = (float)(code(nn, hot[r]) - 8) *
                           from_half(scales[(size_t)nn * groups + hot[r] / 32]);
        wrong += from_half(y[(size_t)r * n + nn]) != (float)(_Float16)want;
      }
    bad = wrong != 0;
    printf("%s w4a16_matmul one-hot X -> (code - 8) * scale exactly (M=%d, N=%d, K=%d): "
           "%d of %d wrong\n", bad ? "FAIL" : "PASS", m, n, k, wrong, m * n);
  }
  HIP_OK(hipFree(dx));
  HIP_OK(hipFree(ds));
  HIP_OK(hipFree(dw));
  HIP_OK(hipFree(dy));
  return bad;
}

int rejected_call() {
  // Valid buffers, unsupported head_dim: rejected before any launch.
  float* buf = nullptr;
  HIP_OK(hipMalloc(&buf, 64 * 48 * sizeof(float)));
  const int st = neso_flash_attention_fwd(buf, buf, buf, buf, 64, 48, 48, 0.1f, 48, 1, 0, 0, 0,
                                          nullptr);
  HIP_OK(hipFree(buf));
  const bool ok = st == NESO_EUNSUPPORTED && neso_last_error()[0] != '\0';
  printf("%s head_dim 48 rejected: %s (%s)\n", ok ? "PASS" : "FAIL", neso_status_string(st),
         neso_last_error());
  return ok ? 0 : 1;
}

int test() {
  printf("neso_amd ABI version %d, manifest %zu bytes\n", neso_abi_version(),
         strlen(neso_kernel_manifest()));
  int bad = 0;
  bad += fa2_mean_kat(64, 64, 1);
  bad += fa2_mean_kat(100, 64, 3);
  bad += fa2_mean_kat(64, 128, 2);
  bad += w4a16_onehot_kat(1);
  bad += w4a16_onehot_kat(3);
  bad += rejected_call();
  printf("%s\n", bad ? "FAILED" : "ALL PASSED");
  return bad ? 1 : 0;
}

// Median of `iters` launches, each timed with its own pair of HIP events,
// after `warmup` untimed ones (the reference's measure(), :297-311).
template <typename F>
float median_ms(F launch, int warmup, int iters, hipStream_t s) {
  for (int i = 0; i < warmup; ++i) launch();
  HIP_OK(hipStreamSynchronize(s));
  std::vector<float> t(iters);
  hipEvent_t a, b;
  HIP_OK(hipEventCreate(&a));
  HIP_OK(hipEventCreate(&b));
  for (int i = 0; i < iters; ++i) {
    HIP_OK(hipEventRecord(a, s));
    launch();
    HIP_OK(hipEventRecord(b, s));
    HIP_OK(hipEventSynchronize(b));
    HIP_OK(hipEventElapsedTime(&t[i], a, b));
  }
  HIP_OK(hipEventDestroy(a));
  HIP_OK(hipEventDestroy(b));
  std::sort(t.begin(), t.end());
  return t[iters / 2];
}

int bench() {
  const int d = 64, nmax = 2048, heads_max = 16;
  const size_t cnt = (size_t)heads_max * nmax * d;
  std::vector<uint16_t> q(cnt), k(cnt), v(cnt);
  for (size_t i = 0; i < cnt; ++i) {
    q[i] = to_half(pattern_q(i));
    k[i] = to_half(pattern_k(i));
    v[i] = to_half(pattern_v(i));
  }
  uint16_t *dq = upload(q), *dk = upload(k), *dv = upload(v);
  float* dout = nullptr;
  HIP_OK(hipMalloc(&dout, cnt * sizeof(float)));
  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  int bad = 0;
  auto run = [&](int n, int heads) {
    int st = NESO_OK;
    const float ms = median_ms(
        [&] {
          st = neso_flash_attention_fwd(dq, dk, dv, dout, n, d, d, 0.125f, d, heads,
                                        (int64_t)n * d, (int64_t)n * d, 0, s);
        },
        10, 20, s);
    bad += check_status(st, "neso_flash_attention_fwd");
    const double flops = 4.0 * heads * (double)n * n * d;
    printf("flash_attn2 f16 N=%4d d=%d heads=%2d  %8.4f ms  %9.2f GFLOP/s (median of 20, one "
           "launch per sample)\n", n, d, heads, ms, flops / (ms * 1e-3) / 1e9);
  };
  for (int n : {128, 256, 512, 1024, 2048}) run(n, 1);
  run(2048, heads_max);
  HIP_OK(hipStreamDestroy(s));
  HIP_OK(hipFree(dq));
  HIP_OK(hipFree(dk));
  HIP_OK(hipFree(dv));
  HIP_OK(hipFree(dout));
  return bad ? 1 : 0;
}

}  // namespace

int main(int argc, char** argv) {
  const char* mode = argc > 1 ? argv[1] : "";
  if (!strcmp(mode, "test")) return test();
  if (!strcmp(mode, "bench")) return bench();
  fprintf(stderr, "usage: neso_harness <test|bench>\n");
  return 2;
}
