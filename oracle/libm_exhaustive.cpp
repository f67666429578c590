// libm_exhaustive.cpp - CPU check that the device float math in
// uncertain-gpt_amd/csrc/ugk_libm.h equals the host glibc bit for bit.
//
// Test infrastructure only (it links the host libm as the reference). For
// every one of the 2^32 binary32 inputs in [lo, hi) with the given stride it
// compares ugk_<fn>(x) against glibc <fn>(x); two NaNs count as equal.
//
// usage: libm_exhaustive <fn> [stride] [threads]
//   fn in expf0 expf1 expf2 expf log1pf expm1f tanhf softplus, and
//   logf_normal[0] (ugk_logf_normal_t on normal finite x > 0, glibc's logf
//   elsewhere) and cosf_small[0] (ugk_cosf_small_t on |x| < 120, glibc's cosf
//   elsewhere), with fused (default) or unfused (0) multiply-adds; logf
//   (ugk_logf, every input)
// Prints "<fn> checked=<n> mismatches=<m>" and up to 8 mismatching inputs;
// exits 1 if any mismatch.
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <thread>
#include <vector>

#include "../uncertain-gpt_amd/csrc/ugk_libm.h"

typedef float (*fn_t)(float);

static float glibc_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }
static float e0(float x) { return ugk_expf_v<0>(x); }
static float e1(float x) { return ugk_expf_v<1>(x); }
static float e2(float x) { return ugk_expf_v<2>(x); }
static float mine_log1pf(float x) { return ugk_log1pf(x); }
static float mine_expm1f(float x) { return ugk_expm1f(x); }
static float mine_tanhf(float x) { return ugk_tanhf(x); }
static float mine_expf(float x) { return ugk_expf(x); }
static float mine_softplus(float x) { return ugk_softplusf(x); }
static float g_expf(float x) { return expf(x); }
static float g_log1pf(float x) { return log1pf(x); }
static float g_expm1f(float x) { return expm1f(x); }
static float g_tanhf(float x) { return tanhf(x); }
static bool logf_dom(float x) { return x >= 0x1p-126f && x <= 0x1.fffffep127f; }
static bool cosf_dom(float x) { return fabsf(x) < 120.0f; }
static float mine_logf1(float x) { return logf_dom(x) ? ugk_logf_normal_t<1>(x, UgkLogfTable{}) : logf(x); }
static float mine_logf0(float x) { return logf_dom(x) ? ugk_logf_normal_t<0>(x, UgkLogfTable{}) : logf(x); }
static float mine_cosf1(float x) { return cosf_dom(x) ? ugk_cosf_small_t<1>(x) : cosf(x); }
static float mine_cosf0(float x) { return cosf_dom(x) ? ugk_cosf_small_t<0>(x) : cosf(x); }
static float g_logf(float x) { return logf(x); }
static float mine_logf_all(float x) { return ugk_logf(x); }
static float g_cosf(float x) { return cosf(x); }

int main(int argc, char **argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: %s fn [stride] [threads]\n", argv[0]);
    return 2;
  }
  const char *name = argv[1];
  const uint64_t stride = argc > 2 ? strtoull(argv[2], 0, 0) : 1;
  const int nthreads = argc > 3 ? atoi(argv[3]) : 8;
  fn_t mine = 0, ref = 0;
  if (!strcmp(name, "expf0")) { mine = e0; ref = g_expf; }
  else if (!strcmp(name, "expf1")) { mine = e1; ref = g_expf; }
  else if (!strcmp(name, "expf2")) { mine = e2; ref = g_expf; }
  else if (!strcmp(name, "expf")) { mine = mine_expf; ref = g_expf; }
  else if (!strcmp(name, "log1pf")) { mine = mine_log1pf; ref = g_log1pf; }
  else if (!strcmp(name, "expm1f")) { mine = mine_expm1f; ref = g_expm1f; }
  else if (!strcmp(name, "tanhf")) { mine = mine_tanhf; ref = g_tanhf; }
  else if (!strcmp(name, "softplus")) { mine = mine_softplus; ref = glibc_softplus; }
  else if (!strcmp(name, "logf_normal")) { mine = mine_logf1; ref = g_logf; }
  else if (!strcmp(name, "logf")) { mine = mine_logf_all; ref = g_logf; }
  else if (!strcmp(name, "logf_normal0")) { mine = mine_logf0; ref = g_logf; }
  else if (!strcmp(name, "cosf_small")) { mine = mine_cosf1; ref = g_cosf; }
  else if (!strcmp(name, "cosf_small0")) { mine = mine_cosf0; ref = g_cosf; }
  else { fprintf(stderr, "unknown fn %s\n", name); return 2; }

  std::atomic<uint64_t> bad{0}, checked{0};
  std::vector<uint32_t> examples[64];
  std::vector<std::thread> th;
  const uint64_t total = 1ull << 32;
  for (int t = 0; t < nthreads; t++) {
    th.emplace_back([&, t]() {
      uint64_t nb = 0, nc = 0;
      for (uint64_t i = (uint64_t)t * stride; i < total; i += (uint64_t)nthreads * stride) {
        const float x = ugk_u2f((uint32_t)i);
        const float a = mine(x), b = ref(x);
        nc++;
        if (ugk_f2u(a) != ugk_f2u(b) && !(a != a && b != b)) {
          nb++;
          if (examples[t].size() < 8) examples[t].push_back((uint32_t)i);
        }
      }
      bad += nb;
      checked += nc;
    });
  }
  for (auto &x : th) x.join();
  printf("%s checked=%llu mismatches=%llu\n", name, (unsigned long long)checked.load(),
         (unsigned long long)bad.load());
  int shown = 0;
  for (int t = 0; t < nthreads && shown < 8; t++)
    for (uint32_t u : examples[t]) {
      if (shown++ >= 8) break;
      const float x = ugk_u2f(u);
      printf("  x=%a (0x%08x) mine=%a ref=%a\n", x, u, mine(x), ref(x));
    }
  return bad.load() ? 1 : 0;
}
