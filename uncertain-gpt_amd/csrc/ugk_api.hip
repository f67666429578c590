// ugk_api.hip - the C-ABI of libugk.so: argument checks, error reporting,
// stream and scratch management, and the GPT-2 layer-kernel step driver.
//
// Every entry point validates its arguments on the host before it touches the
// HIP runtime, so invalid calls are reported (UGK_EINVAL + message) without a
// GPU, and no kernel is ever launched with a shape it does not expect.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>
#include <climits>
#include <mutex>
#include <vector>

#include "../../include/ugk.h"
#include "ugk_internal.h"

namespace ugk {

namespace {
thread_local char g_err[512] = "";
std::atomic<hipStream_t> g_stream{nullptr};
std::mutex g_mu;
constexpr int kMaxDevices = 64;
constexpr size_t kAlign = 256;
size_t align_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }
const char *const kRegionName[kNumRegions] = {"LayerNorm partial rows", "encoder bucket state", "KL partial sums",
                                              "softmax row statistics"};

// Per device: the library's own region allocations, or the caller's workspace
// and the offset and capacity of each region in it.
struct DevWorkspace {
  void *own[kNumRegions] = {};
  size_t own_bytes[kNumRegions] = {};
  char *user = nullptr;
  size_t user_bytes = 0;
  size_t off[kNumRegions] = {}, cap[kNumRegions] = {};
  bool fresh[kNumRegions] = {true, true, true, true};
};
DevWorkspace g_ws[kMaxDevices];

int current_device(const char *what) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return -1;
  }
  (void)what;
  return dev;
}

// Region sizes for every entry point at shapes up to cfg: the step driver's
// 2L+1 LayerNorm slots (at least the one slot of a per-op call), the encoder
// state, the KL partial sums and the softmax statistics of B*T rows.
void region_sizes(const ugk_config &cfg, size_t out[kNumRegions]) {
  const int rows = cfg.B * cfg.T;
  const size_t slot = align_up(layernorm_backward_scratch(rows, cfg.C));
  out[kRegLn] = slot * (size_t)(2 * (cfg.L > 0 ? cfg.L : 0) + 1);
  out[kRegEncoder] = encoder_backward_scratch();
  out[kRegKl] = kl_forward_scratch();
  out[kRegSoftmax] = softmax_scratch(rows, cfg.V);
}

// Grow the library-owned region r of device dev to `bytes` (lock held).
void *own_region(DevWorkspace &w, Region r, size_t bytes) {
  if (w.own[r] && w.own_bytes[r] >= bytes) return w.own[r];
  if (w.own[r]) {
    // kernels queued earlier, on this or another stream, may still use the old buffer
    (void)hipDeviceSynchronize();
    (void)hipFree(w.own[r]);
    w.own[r] = nullptr;
    w.own_bytes[r] = 0;
  }
  const size_t want = align_up(bytes < ((size_t)1 << 16) ? ((size_t)1 << 16) : bytes);
  if (hipMalloc(&w.own[r], want) != hipSuccess) {
    (void)hipGetLastError();
    w.own[r] = nullptr;
    set_error(UGK_ENOMEM, "workspace: cannot allocate %zu bytes for the %s", want, kRegionName[r]);
    return nullptr;
  }
  w.own_bytes[r] = want;
  w.fresh[r] = true;
  return w.own[r];
}

// Per device, one double of pinned host memory that ugk_kl_forward's last
// kernel writes its total into (held until the process ends).
volatile double *g_kl_slot[kMaxDevices] = {};

volatile double *kl_result_slot() {
  const int dev = current_device("ugk_kl_forward");
  if (dev < 0) {
    set_error(UGK_EHIP, "ugk_kl_forward: hipGetDevice failed");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_kl_slot[dev]) {
    void *p = nullptr;
    if (hipHostMalloc(&p, kAlign, hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      set_error(UGK_ENOMEM, "ugk_kl_forward: cannot allocate the pinned result slot");
      return nullptr;
    }
    g_kl_slot[dev] = static_cast<volatile double *>(p);
  }
  return g_kl_slot[dev];
}

void free_own(DevWorkspace &w) {
  bool any = false;
  for (int r = 0; r < kNumRegions; r++) any = any || w.own[r];
  if (!any) return;
  (void)hipDeviceSynchronize();
  for (int r = 0; r < kNumRegions; r++) {
    if (w.own[r]) (void)hipFree(w.own[r]);
    w.own[r] = nullptr;
    w.own_bytes[r] = 0;
    w.fresh[r] = true;
  }
}
}  // namespace

hipStream_t stream() { return g_stream.load(std::memory_order_relaxed); }

LaunchEvents *&armed_events() {
  thread_local LaunchEvents *armed = nullptr;
  return armed;
}

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(UGK_EHIP, "%s: %s", what, hipGetErrorString(e));
  return UGK_OK;
}

bool stream_capturing() {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream(), &st) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return st != hipStreamCaptureStatusNone;
}

void *workspace(Region r, size_t bytes, bool *fresh, bool keep_fresh) {
  const int dev = current_device("workspace");
  if (dev < 0) {
    set_error(UGK_EHIP, "workspace: hipGetDevice failed");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  DevWorkspace &w = g_ws[dev];
  void *p;
  if (w.user) {
    if (bytes > w.cap[r]) {
      set_error(UGK_ENOMEM,
                "workspace: the %s need %zu bytes, the caller's workspace holds %zu for them (size it with "
                "ugk_workspace_bytes for the largest shape)",
                kRegionName[r], bytes, w.cap[r]);
      return nullptr;
    }
    p = w.user + w.off[r];
  } else {
    if (!(w.own[r] && w.own_bytes[r] >= bytes) && stream_capturing()) {
      // hipMalloc (and the wait before a regrowth) cannot be part of a graph
      set_error(UGK_ENOMEM,
                "workspace: the %s need %zu bytes, which must be allocated before graph capture "
                "(ugk_reserve_config, ugk_set_workspace, or one call at this shape outside the capture)",
                kRegionName[r], bytes);
      return nullptr;
    }
    p = own_region(w, r, bytes);
    if (!p) return nullptr;
  }
  if (fresh) {  // the fresh mark is for the region's user, not for ugk_reserve*
    *fresh = w.fresh[r];
    if (!keep_fresh) w.fresh[r] = false;
  }
  return p;
}

size_t workspace_bytes_current() {
  const int dev = current_device("ugk_scratch_bytes");
  if (dev < 0) return 0;
  std::lock_guard<std::mutex> lock(g_mu);
  const DevWorkspace &w = g_ws[dev];
  if (w.user) return w.user_bytes;
  size_t t = 0;
  for (int r = 0; r < kNumRegions; r++) t += w.own_bytes[r];
  return t;
}

}  // namespace ugk

using namespace ugk;

namespace {

int ok() {
  g_err[0] = '\0';
  return UGK_OK;
}

int bad(const char *fn, const char *what) { return set_error(UGK_EINVAL, "%s: %s", fn, what); }

// B, T, C >= 0 and B*T*C addressable; B*T fits an int (the reference indexes
// rows with int).
int check_btc(const char *fn, int B, int T, int C) {
  if (B < 0 || T < 0 || C < 0) return bad(fn, "B, T and C must be >= 0");
  if ((long long)B * T > INT_MAX) return bad(fn, "B*T exceeds INT_MAX");
  return UGK_OK;
}

bool any_null(std::initializer_list<const void *> ps) {
  for (const void *p : ps)
    if (!p) return true;
  return false;
}

// Buffers one call writes must be distinct (the CPU loops would otherwise see
// each other's stores within an element).
bool any_same(std::initializer_list<const void *> ps) {
  for (auto a = ps.begin(); a != ps.end(); ++a)
    for (auto b = a + 1; b != ps.end(); ++b)
      if (*a == *b) return true;
  return false;
}

}  // namespace

extern "C" {

int ugk_encoder_forward(float *out, const int *inp, const float *wte, const float *wpe, int B, int T,
                        int C) {
  const char *fn = "ugk_encoder_forward";
  if (int e = check_btc(fn, B, T, C)) return e;
  if ((long long)B * T * C == 0) return ok();
  if (any_null({out, inp, wte, wpe})) return bad(fn, "NULL pointer");
  if (int e = launch_encoder_forward(out, inp, wte, wpe, B, T, C)) return e;
  return ok();
}

int ugk_encoder_backward(float *dwte, float *dwpe, const float *dout, const int *inp, int B, int T,
                         int C) {
  const char *fn = "ugk_encoder_backward";
  if (int e = check_btc(fn, B, T, C)) return e;
  if ((long long)B * T * C == 0) return ok();
  if (any_null({dwte, dwpe, dout, inp})) return bad(fn, "NULL pointer");
  if (int e = launch_encoder_backward(dwte, dwpe, dout, inp, B, T, C)) return e;
  return ok();
}

int ugk_layernorm_forward(float *out, float *mean, float *rstd, const float *inp, const float *weight,
                          const float *bias, int B, int T, int C) {
  const char *fn = "ugk_layernorm_forward";
  if (int e = check_btc(fn, B, T, C)) return e;
  if ((long long)B * T == 0) return ok();
  if (C == 0) return bad(fn, "C must be > 0 when B*T > 0 (mean over an empty row)");
  if (any_null({out, mean, rstd, inp, weight, bias})) return bad(fn, "NULL pointer");
  if (int e = launch_layernorm_forward(out, mean, rstd, inp, weight, bias, B * T, C)) return e;
  return ok();
}

int ugk_layernorm_backward(float *dinp, float *dweight, float *dbias, const float *dout,
                           const float *inp, const float *weight, const float *mean, const float *rstd,
                           int B, int T, int C) {
  const char *fn = "ugk_layernorm_backward";
  if (int e = check_btc(fn, B, T, C)) return e;
  if ((long long)B * T * C == 0) return ok();
  if (any_null({dinp, dweight, dbias, dout, inp, weight, mean, rstd})) return bad(fn, "NULL pointer");
  if (int e = launch_layernorm_backward(dinp, dweight, dbias, dout, inp, weight, mean, rstd, B * T, C))
    return e;
  return ok();
}

int ugk_layernorm_backward_noalloc(float *dinp, float *dweight, float *dbias, const float *dout,
                                   const float *inp, const float *weight, const float *mean, const float *rstd,
                                   int B, int T, int C) {
  const char *fn = "ugk_layernorm_backward_noalloc";
  if (int e = check_btc(fn, B, T, C)) return e;
  if ((long long)B * T * C == 0) return ok();
  if (any_null({dinp, dweight, dbias, dout, inp, weight, mean, rstd})) return bad(fn, "NULL pointer");
  if (noalloc_max_blocks(C) < 1)
    return set_error(UGK_EINVAL, "%s: C = %d needs more than the %zu bytes of scratch (at most %zu channels)", fn, C,
                     kNoAllocScratchBytes, kNoAllocScratchBytes / (2 * sizeof(float)));
  float *partial = noalloc_scratch();
  if (!partial) return UGK_EHIP;
  if (int e = launch_layernorm_residual_backward_into(partial, noalloc_max_blocks(C), dinp, dweight, dbias, nullptr,
                                                      nullptr, dout, inp, weight, mean, rstd, B * T, C))
    return e;
  return ok();
}

int ugk_encoder_layernorm_forward(float *enc, float *out, float *mean, float *rstd, const int *inp,
                                  const float *wte, const float *wpe, const float *weight, const float *bias, int B,
                                  int T, int C) {
  const char *fn = "ugk_encoder_layernorm_forward";
  if (int e = check_btc(fn, B, T, C)) return e;
  if ((long long)B * T == 0) return ok();
  if (C == 0) return bad(fn, "C must be > 0 when B*T > 0 (mean over an empty row)");
  if (any_null({enc, out, mean, rstd, inp, wte, wpe, weight, bias})) return bad(fn, "NULL pointer");
  if (int e = launch_encoder_layernorm_forward(enc, out, mean, rstd, inp, wte, wpe, weight, bias, B, T, C))
    return e;
  return ok();
}

int ugk_residual_layernorm_forward(float *res, float *out, float *mean, float *rstd, const float *x,
                                   const float *y, const float *weight, const float *bias, int B, int T,
                                   int C) {
  const char *fn = "ugk_residual_layernorm_forward";
  if (int e = check_btc(fn, B, T, C)) return e;
  if ((long long)B * T == 0) return ok();
  if (C == 0) return bad(fn, "C must be > 0 when B*T > 0 (mean over an empty row)");
  if (any_null({res, out, mean, rstd, x, y, weight, bias})) return bad(fn, "NULL pointer");
  if (int e = launch_residual_layernorm_forward(res, out, mean, rstd, x, y, weight, bias, B * T, C)) return e;
  return ok();
}

int ugk_layernorm_residual_backward(float *dinp, float *dweight, float *dbias, float *dx, float *dy,
                                    const float *dout, const float *inp, const float *weight,
                                    const float *mean, const float *rstd, int B, int T, int C) {
  const char *fn = "ugk_layernorm_residual_backward";
  if (int e = check_btc(fn, B, T, C)) return e;
  if ((long long)B * T * C == 0) return ok();
  if (any_null({dinp, dweight, dbias, dx, dy, dout, inp, weight, mean, rstd})) return bad(fn, "NULL pointer");
  if (dinp == dx || dinp == dy) return bad(fn, "dinp must be distinct from dx and dy");
  if (int e = launch_layernorm_residual_backward(dinp, dweight, dbias, dx, dy, dout, inp, weight, mean, rstd,
                                                 B * T, C))
    return e;
  return ok();
}

int ugk_gelu_forward(float *out, const float *inp, int N) {
  const char *fn = "ugk_gelu_forward";
  if (N < 0) return bad(fn, "N must be >= 0");
  if (N == 0) return ok();
  if (any_null({out, inp})) return bad(fn, "NULL pointer");
  if (int e = launch_gelu_forward(out, inp, (size_t)N)) return e;
  return ok();
}

int ugk_gelu_backward(float *dinp, const float *inp, const float *dout, int N) {
  const char *fn = "ugk_gelu_backward";
  if (N < 0) return bad(fn, "N must be >= 0");
  if (N == 0) return ok();
  if (any_null({dinp, inp, dout})) return bad(fn, "NULL pointer");
  if (int e = launch_gelu_backward(dinp, inp, dout, (size_t)N)) return e;
  return ok();
}

int ugk_residual_forward(float *out, const float *x, const float *y, int N) {
  const char *fn = "ugk_residual_forward";
  if (N < 0) return bad(fn, "N must be >= 0");
  if (N == 0) return ok();
  if (any_null({out, x, y})) return bad(fn, "NULL pointer");
  if (int e = launch_residual_forward(out, x, y, (size_t)N)) return e;
  return ok();
}

int ugk_residual_backward(float *dx, float *dy, const float *dout, int N) {
  const char *fn = "ugk_residual_backward";
  if (N < 0) return bad(fn, "N must be >= 0");
  if (N == 0) return ok();
  if (any_null({dx, dy, dout})) return bad(fn, "NULL pointer");
  if (int e = launch_residual_backward(dx, dy, dout, (size_t)N)) return e;
  return ok();
}

int ugk_bayes_materialize(float *w, const float *mu, const float *rho, const float *eps, size_t n) {
  const char *fn = "ugk_bayes_materialize";
  if (n == 0) return ok();
  if (any_null({w, mu, rho, eps})) return bad(fn, "NULL pointer");
  if (int e = launch_bayes_materialize(w, mu, rho, eps, n)) return e;
  return ok();
}

int ugk_softmax_crossentropy(float *losses, float *probs, const float *logits, const int *targets, int B, int T,
                             int V) {
  const char *fn = "ugk_softmax_crossentropy";
  if (int e = check_btc(fn, B, T, V)) return e;
  if ((long long)B * T == 0) return ok();
  if (V == 0) return bad(fn, "V must be > 0 when B*T > 0 (the target indexes the row)");
  if (any_null({losses, probs, logits, targets})) return bad(fn, "NULL pointer");
  if ((const void *)probs == (const void *)logits) return bad(fn, "probs and logits must be distinct buffers");
  if (int e = launch_softmax_crossentropy(losses, probs, logits, targets, B * T, V)) return e;
  return ok();
}

namespace {
int xent_backward(const char *fn, bool zeroed, float *dlogits, const float *probs, const int *targets, int B, int T,
                  int V) {
  if (int e = check_btc(fn, B, T, V)) return e;
  if ((long long)B * T * V == 0) return ok();
  if (any_null({dlogits, probs, targets})) return bad(fn, "NULL pointer");
  const float dloss = 1.0f / (B * T);  // train_bnn.c:360
  if (int e = launch_crossentropy_softmax_backward(dlogits, probs, targets, B * T, V, dloss, zeroed)) return e;
  return ok();
}
}  // namespace

int ugk_crossentropy_softmax_backward(float *dlogits, const float *probs, const int *targets, int B, int T, int V) {
  return xent_backward("ugk_crossentropy_softmax_backward", false, dlogits, probs, targets, B, T, V);
}

int ugk_crossentropy_softmax_backward_zeroed(float *dlogits, const float *probs, const int *targets, int B, int T,
                                             int V) {
  return xent_backward("ugk_crossentropy_softmax_backward_zeroed", true, dlogits, probs, targets, B, T, V);
}

int ugk_bayes_sample(float *w, float *eps, const float *mu, const float *rho, size_t n,
                     unsigned long long seed, int step) {
  const char *fn = "ugk_bayes_sample";
  if (n == 0) return ok();
  if (any_null({w, mu, rho})) return bad(fn, "NULL pointer");
  if (eps && w == eps) return bad(fn, "w and eps must be distinct buffers");
  if (int e = launch_bayes_sample(w, eps, mu, rho, n, seed, step)) return e;
  return ok();
}

int ugk_bayes_backward(float *dmu, float *drho, const float *dw, const float *eps, const float *rho,
                       size_t n) {
  const char *fn = "ugk_bayes_backward";
  if (n == 0) return ok();
  if (any_null({dmu, drho, dw, eps, rho})) return bad(fn, "NULL pointer");
  if (dmu == drho) return bad(fn, "dmu and drho must be distinct buffers");
  if (int e = launch_bayes_backward(dmu, drho, dw, eps, rho, n)) return e;
  return ok();
}

int ugk_bayes_backward_philox(float *dmu, float *drho, const float *dw, const float *rho, size_t n,
                              unsigned long long seed, int step) {
  const char *fn = "ugk_bayes_backward_philox";
  if (n == 0) return ok();
  if (any_null({dmu, drho, dw, rho})) return bad(fn, "NULL pointer");
  if (dmu == drho) return bad(fn, "dmu and drho must be distinct buffers");
  if (int e = launch_bayes_backward_philox(dmu, drho, dw, rho, n, seed, step)) return e;
  return ok();
}

int ugk_kl_forward(double *kl, const float *mu, const float *rho, size_t n, float sigma_prior) {
  const char *fn = "ugk_kl_forward";
  if (!kl) return bad(fn, "NULL result pointer");
  if (n == 0) {
    *kl = 0.0;
    return ok();
  }
  if (any_null({mu, rho})) return bad(fn, "NULL pointer");
  double *buf = static_cast<double *>(workspace(kRegKl, kl_forward_scratch()));
  if (!buf) return UGK_ENOMEM;
  volatile double *slot = kl_result_slot();
  if (!slot) return UGK_ENOMEM;
  // the final-sum kernel stores the total straight into the pinned slot: no copy to wait for
  if (int e = launch_kl_forward(const_cast<double *>(slot), buf, mu, rho, n, sigma_prior)) return e;
  if (hipStreamSynchronize(stream()) != hipSuccess) {
    const hipError_t err = hipGetLastError();
    return set_error(UGK_EHIP, "%s: %s", fn, hipGetErrorString(err));
  }
  *kl = *slot;
  return ok();
}

int ugk_kl_backward(float *dmu, float *drho, const float *mu, const float *rho, size_t n,
                    float sigma_prior, float weight) {
  const char *fn = "ugk_kl_backward";
  if (n == 0) return ok();
  if (any_null({dmu, drho, mu, rho})) return bad(fn, "NULL pointer");
  if (dmu == drho) return bad(fn, "dmu and drho must be distinct buffers");
  if (int e = launch_kl_backward(dmu, drho, mu, rho, n, sigma_prior, weight)) return e;
  return ok();
}

int ugk_adamw_update(float *params, const float *grads, float *m, float *v, size_t n, int t, float lr,
                     float beta1, float beta2, float eps, float wd) {
  const char *fn = "ugk_adamw_update";
  if (t < 1) return bad(fn, "t must be >= 1");
  if (n == 0) return ok();
  if (any_null({params, grads, m, v})) return bad(fn, "NULL pointer");
  if (any_same({params, m, v})) return bad(fn, "params, m and v must be distinct buffers");
  // train_bnn.c:704-705, on the host as there.
  const float bc1 = 1.0f - powf(beta1, (float)t);
  const float bc2 = 1.0f - powf(beta2, (float)t);
  if (int e = launch_adamw(params, grads, m, v, n, lr, beta1, beta2, eps, wd, bc1, bc2)) return e;
  return ok();
}

int ugk_bbb_step_fused(float *mu, float *rho, float *m_mu, float *v_mu, float *m_rho, float *v_rho,
                       float *w, float *dw, size_t n, unsigned long long seed, int step, float sp,
                       float klw, float bc1, float bc2, float lr, float beta1, float beta2, float aeps,
                       float wd) {
  const char *fn = "ugk_bbb_step_fused";
  if (n == 0) return ok();
  if (any_null({mu, rho, m_mu, v_mu, m_rho, v_rho, w, dw})) return bad(fn, "NULL pointer");
  if (any_same({mu, rho, m_mu, v_mu, m_rho, v_rho, w, dw})) return bad(fn, "the eight buffers must be distinct");
  if (int e = launch_bbb_step_fused(mu, rho, m_mu, v_mu, m_rho, v_rho, w, dw, n, seed, step, sp, klw, bc1,
                                    bc2, lr, beta1, beta2, aeps, wd))
    return e;
  return ok();
}

int ugk_set_gelu_exact(int exact) {
  set_gelu_exact(exact);
  return ok();
}

int ugk_get_gelu_exact(void) { return gelu_exact(); }

int ugk_set_philox_exact(int exact) {
  set_philox_exact(exact);
  return ok();
}

int ugk_get_philox_exact(void) { return philox_exact(); }

int ugk_set_kl_exact(int exact) {
  set_kl_exact(exact);
  return ok();
}

int ugk_get_kl_exact(void) { return kl_exact(); }

int ugk_set_softmax_exact(int exact) {
  set_softmax_exact(exact);
  return ok();
}

int ugk_get_softmax_exact(void) { return softmax_exact(); }

int ugk_set_layernorm_exact(int exact) {
  set_layernorm_exact(exact);
  return ok();
}

int ugk_get_layernorm_exact(void) { return layernorm_exact(); }

int ugk_set_encoder_exact(int exact) {
  set_encoder_exact(exact);
  return ok();
}

int ugk_get_encoder_exact(void) { return encoder_exact(); }

const char *ugk_last_error(void) { return g_err; }

int ugk_set_stream(void *s) {
  const hipStream_t next = static_cast<hipStream_t>(s);
  const hipStream_t prev = g_stream.exchange(next);
  // kernels still queued on the previous stream may use the workspace, which
  // the new stream's work would then share
  if (prev != next && hipStreamSynchronize(prev) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(UGK_EHIP, "ugk_set_stream: waiting for the previous stream failed");
  }
  return ok();
}

void *ugk_get_stream(void) { return g_stream.load(); }

int ugk_reserve(int rows, int C) {
  if (rows < 0 || C < 0) return bad("ugk_reserve", "rows and C must be >= 0");
  ugk_config cfg{1, rows, C, 1, 1, rows, 0};
  return ugk_reserve_config(cfg);
}

size_t ugk_workspace_bytes(ugk_config cfg) {
  if (cfg.B < 0 || cfg.T < 0 || cfg.C < 0 || cfg.V < 0 || cfg.L < 0 || (long long)cfg.B * cfg.T > INT_MAX) return 0;
  size_t sz[kNumRegions];
  region_sizes(cfg, sz);
  size_t t = 0;
  for (int r = 0; r < kNumRegions; r++) t += align_up(sz[r]);
  return t;
}

int ugk_reserve_config(ugk_config cfg) {
  const char *fn = "ugk_reserve_config";
  if (cfg.B < 0 || cfg.T < 0 || cfg.C < 0 || cfg.V < 0 || cfg.L < 0) return bad(fn, "negative size in config");
  if ((long long)cfg.B * cfg.T > INT_MAX) return bad(fn, "B*T exceeds INT_MAX");
  size_t sz[kNumRegions];
  region_sizes(cfg, sz);
  for (int r = 0; r < kNumRegions; r++) {
    bool fresh = false;
    void *p = workspace(static_cast<Region>(r), sz[r], r == kRegEncoder ? &fresh : nullptr);
    if (!p) return UGK_ENOMEM;
    // the encoder backward's state is cleared now, so that its first call may be captured
    if (fresh)
      if (int e = launch_encoder_state_init(p)) return e;
  }
  return ok();
}

int ugk_set_workspace(void *ptr, size_t bytes, ugk_config cfg) {
  const char *fn = "ugk_set_workspace";
  if (ptr && ((uintptr_t)ptr % kAlign) != 0) return bad(fn, "the workspace must be 256-byte aligned");
  size_t sz[kNumRegions];
  if (ptr) {
    if (cfg.B < 0 || cfg.T < 0 || cfg.C < 0 || cfg.V < 0 || cfg.L < 0 || (long long)cfg.B * cfg.T > INT_MAX)
      return bad(fn, "invalid config");
    region_sizes(cfg, sz);
    size_t need = 0;
    for (int r = 0; r < kNumRegions; r++) need += align_up(sz[r]);
    if (bytes < need) return set_error(UGK_EINVAL, "%s: %zu bytes given, the config needs %zu", fn, bytes, need);
  }
  const int dev = current_device(fn);
  if (dev < 0) return set_error(UGK_EHIP, "%s: hipGetDevice failed", fn);
  // work queued on the library stream may still use the current workspace
  if (hipStreamSynchronize(stream()) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(UGK_EHIP, "%s: waiting for the stream failed", fn);
  }
  std::lock_guard<std::mutex> lock(g_mu);
  DevWorkspace &w = g_ws[dev];
  free_own(w);
  w.user = static_cast<char *>(ptr);
  w.user_bytes = ptr ? bytes : 0;
  size_t o = 0;
  for (int r = 0; r < kNumRegions; r++) {
    w.off[r] = o;
    w.cap[r] = ptr ? align_up(sz[r]) : 0;
    o += w.cap[r];
    w.fresh[r] = true;
  }
  if (ptr) {  // the encoder backward's state is cleared now, so that its first call may be captured
    if (int e = launch_encoder_state_init(w.user + w.off[kRegEncoder])) return e;
    w.fresh[kRegEncoder] = false;
  }
  return ok();
}

size_t ugk_scratch_bytes(void) { return workspace_bytes_current(); }

namespace {
const char *ids_op_name(int code) {
  switch (code) {
    case UGK_IDS_ENCODER_FORWARD: return "encoder_forward";
    case UGK_IDS_ENCODER_BACKWARD: return "encoder_backward";
    case UGK_IDS_ENCODER_LAYERNORM_FORWARD: return "encoder_layernorm_forward";
    case UGK_IDS_SOFTMAX_CROSSENTROPY: return "softmax_crossentropy";
    case UGK_IDS_CROSSENTROPY_BACKWARD: return "crossentropy_softmax_backward";
    default: return "a guarded call";
  }
}
}  // namespace

int ugk_ids_guard(int *ids, int n, int bound, int fill, int code) {
  const char *fn = "ugk_ids_guard";
  if (n < 0 || bound < 0) return bad(fn, "n and bound must be >= 0");
  if (code <= 0) return bad(fn, "code must be > 0");
  if (n == 0) return ok();
  if (!ids) return bad(fn, "NULL pointer");
  if (int e = launch_ids_guard(ids, n, bound, fill, code)) return e;
  return ok();
}

int ugk_synchronize(void) {
  const hipError_t e = hipStreamSynchronize(stream());
  if (e != hipSuccess) return set_error(UGK_EHIP, "ugk_synchronize: %s", hipGetErrorString(e));
  int *word = ids_error_word();
  if (!word) return UGK_EHIP;
  int code = 0;
  const int zero = 0;
  if (hipMemcpyAsync(&code, word, sizeof code, hipMemcpyDeviceToHost, stream()) != hipSuccess ||
      hipStreamSynchronize(stream()) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(UGK_EHIP, "ugk_synchronize: reading the id error word failed");
  }
  if (code != 0) {
    if (hipMemcpyAsync(word, &zero, sizeof zero, hipMemcpyHostToDevice, stream()) != hipSuccess ||
        hipStreamSynchronize(stream()) != hipSuccess) {
      (void)hipGetLastError();
      return set_error(UGK_EHIP, "ugk_synchronize: clearing the id error word failed");
    }
    return set_error(UGK_EINVAL,
                     "ugk_synchronize: %s was given an id outside its table (found on the device by "
                     "ugk_ids_guard; the out-of-range ids were replaced, so its results are not meaningful)",
                     ids_op_name(code));
  }
  return ok();
}

int ugk_version(void) { return 100; }

}  // extern "C"

// ---- GPT-2 layer-kernel step driver -----------------------------------------
namespace {

// Offsets of the reference's flat parameter buffer (gpt2_kernels.cuh:656-685).
struct POff {
  size_t wte, wpe, blk0, bstride;
  size_t lng, lnb, qw, qb, pw, pb, ln2g, ln2b, w1, b1, w2, b2;
  size_t flng, flnb, hw, hb, total;
};

// Offsets of the reference's flat activation buffer (gpt2_kernels.cuh:687-719).
struct AOff {
  size_t enc, blk0, bstride;
  size_t lno, lnm, lnr, qkv, atty, apr, resa, ln2o, ln2m, ln2r, fch, gelu, mlpo, res1;
  size_t flo, flm, flr, log, prb, los, total;
};

POff poff(const ugk_config &c) {
  const size_t C = c.C, V = c.V, maxT = c.maxT;
  POff p{};
  p.wte = 0;
  p.wpe = V * C;
  p.blk0 = p.wpe + maxT * C;
  size_t o = 0;
  p.lng = o; o += C;
  p.lnb = o; o += C;
  p.qw = o; o += C * 3 * C;
  p.qb = o; o += 3 * C;
  p.pw = o; o += C * C;
  p.pb = o; o += C;
  p.ln2g = o; o += C;
  p.ln2b = o; o += C;
  p.w1 = o; o += C * 4 * C;
  p.b1 = o; o += 4 * C;
  p.w2 = o; o += 4 * C * C;
  p.b2 = o; o += C;
  p.bstride = o;
  const size_t after = p.blk0 + (size_t)c.L * p.bstride;
  p.flng = after;
  p.flnb = p.flng + C;
  p.hw = p.flnb + C;
  p.hb = p.hw + C * V;
  p.total = p.hb + V;
  return p;
}

AOff aoff(const ugk_config &c) {
  const size_t BT = (size_t)c.B * c.T, C = c.C, V = c.V;
  AOff a{};
  a.enc = 0;
  a.blk0 = BT * C;
  size_t o = 0;
  a.lno = o; o += BT * C;
  a.lnm = o; o += BT;
  a.lnr = o; o += BT;
  a.qkv = o; o += BT * 3 * C;
  a.atty = o; o += BT * C;
  a.apr = o; o += BT * C;
  a.resa = o; o += BT * C;
  a.ln2o = o; o += BT * C;
  a.ln2m = o; o += BT;
  a.ln2r = o; o += BT;
  a.fch = o; o += BT * 4 * C;
  a.gelu = o; o += BT * 4 * C;
  a.mlpo = o; o += BT * C;
  a.res1 = o; o += BT * C;
  a.bstride = o;
  const size_t after = a.blk0 + (size_t)c.L * a.bstride;
  a.flo = after;
  a.flm = a.flo + BT * C;
  a.flr = a.flm + BT;
  a.log = a.flr + BT;
  a.prb = a.log + BT * V;
  a.los = a.prb + BT * V;
  a.total = a.los + BT;
  return a;
}

int check_cfg(const char *fn, const ugk_config &c) {
  if (c.B < 0 || c.T < 0 || c.C <= 0 || c.V <= 0 || c.L < 0 || c.maxT < c.T)
    return bad(fn, "config needs B,T,L >= 0, C,V > 0 and maxT >= T");
  if ((long long)c.B * c.T * 4 * c.C > INT_MAX)
    return bad(fn, "B*T*4C exceeds INT_MAX (the element counts are int, as in train_bnn.c)");
  return UGK_OK;
}

#define UGK_TRY(x) \
  do {             \
    int e_ = (x);  \
    if (e_) return e_; \
  } while (0)

int dense(int rc, const char *what) {
  return rc ? set_error(rc, "dense op callback %s returned %d", what, rc) : UGK_OK;
}

// Per-op timer of the step driver. An op's event pair is recorded by its
// dispatches themselves (from its first kernel's start to its last kernel's
// end); the encoder backward, whose three kernels are launched directly, is
// bracketed by two event records on the stream.
struct OpTimer {
  std::vector<hipEvent_t> ev;
  std::vector<LaunchEvents> pair;
  std::vector<int> op;
  int n = 0;
  bool on = false;
};
OpTimer g_timer;

template <class F>
int timed(int op, F &&f) {
  OpTimer &t = g_timer;
  if (!t.on || t.n >= (int)t.op.size()) return f();
  const int i = t.n++;
  t.op[i] = op;
  if (op == UGK_OP_ENCODER_BACKWARD) {
    if (hipEventRecord(t.ev[2 * i], stream()) != hipSuccess) {
      (void)hipGetLastError();
      t.n--;
      return set_error(UGK_EHIP, "op timer: hipEventRecord failed");
    }
    const int rc = f();
    if (hipEventRecord(t.ev[2 * i + 1], stream()) != hipSuccess) {
      (void)hipGetLastError();
      return set_error(UGK_EHIP, "op timer: hipEventRecord failed");
    }
    return rc;
  }
  t.pair[i] = {t.ev[2 * i], t.ev[2 * i + 1], false};
  armed_events() = &t.pair[i];
  const int rc = f();
  armed_events() = nullptr;
  if (!t.pair[i].started) t.n--;  // nothing was launched (an empty op): no record
  return rc;
}

}  // namespace

extern "C" {

size_t ugk_param_count(ugk_config cfg) { return poff(cfg).total; }
size_t ugk_act_count(ugk_config cfg) { return aoff(cfg).total; }

// gpt2_kernels.cuh:756-813
int ugk_gpt2_layers_forward(float *acts, const float *params, const int *inputs, ugk_config cfg,
                            const ugk_dense_ops *ops) {
  const char *fn = "ugk_gpt2_layers_forward";
  UGK_TRY(check_cfg(fn, cfg));
  if (any_null({acts, params, inputs})) return bad(fn, "NULL pointer");
  const POff p = poff(cfg);
  const AOff a = aoff(cfg);
  const int B = cfg.B, T = cfg.T, C = cfg.C, M = B * T;
  const int NBTC = M * C;
  auto A = [&](size_t l, size_t rel) { return acts + a.blk0 + l * a.bstride + rel; };
  auto P = [&](size_t l, size_t rel) { return params + p.blk0 + l * p.bstride + rel; };
  // The encoder_forward and every residual_forward are followed at once by a
  // layernorm_forward of their output (block 0's LN1 or the final LN, the
  // next block's LN1): those pairs run as one pass each,
  // ugk_encoder_layernorm_forward and ugk_residual_layernorm_forward.
  // Buffers and values are the reference's.
  UGK_TRY(timed(UGK_OP_ENCODER_LAYERNORM_FORWARD, [&] {
    return cfg.L > 0 ? ugk_encoder_layernorm_forward(acts + a.enc, A(0, a.lno), A(0, a.lnm), A(0, a.lnr), inputs,
                                                     params + p.wte, params + p.wpe, P(0, p.lng), P(0, p.lnb), B,
                                                     T, C)
                     : ugk_encoder_layernorm_forward(acts + a.enc, acts + a.flo, acts + a.flm, acts + a.flr, inputs,
                                                     params + p.wte, params + p.wpe, params + p.flng,
                                                     params + p.flnb, B, T, C);
  }));
  const float *stream_in = acts + a.enc;
  for (int l = 0; l < cfg.L; l++) {
    if (ops && ops->matmul_forward)
      UGK_TRY(dense(ops->matmul_forward(ops->ctx, A(l, a.qkv), A(l, a.lno), P(l, p.qw), P(l, p.qb), M, C,
                                        3 * C), "matmul_forward(qkv)"));
    if (ops && ops->attention_forward)
      UGK_TRY(dense(ops->attention_forward(ops->ctx, A(l, a.atty), A(l, a.qkv), B, T, C, cfg.NH),
                    "attention_forward"));
    if (ops && ops->matmul_forward)
      UGK_TRY(dense(ops->matmul_forward(ops->ctx, A(l, a.apr), A(l, a.atty), P(l, p.pw), P(l, p.pb), M, C, C),
                    "matmul_forward(proj)"));
    UGK_TRY(timed(UGK_OP_RESIDUAL_LAYERNORM_FORWARD, [&] {
      return ugk_residual_layernorm_forward(A(l, a.resa), A(l, a.ln2o), A(l, a.ln2m), A(l, a.ln2r), stream_in,
                                            A(l, a.apr), P(l, p.ln2g), P(l, p.ln2b), B, T, C);
    }));
    if (ops && ops->matmul_forward)
      UGK_TRY(dense(ops->matmul_forward(ops->ctx, A(l, a.fch), A(l, a.ln2o), P(l, p.w1), P(l, p.b1), M, C,
                                        4 * C), "matmul_forward(fc)"));
    UGK_TRY(timed(UGK_OP_GELU_FORWARD, [&] { return ugk_gelu_forward(A(l, a.gelu), A(l, a.fch), NBTC * 4); }));
    if (ops && ops->matmul_forward)
      UGK_TRY(dense(ops->matmul_forward(ops->ctx, A(l, a.mlpo), A(l, a.gelu), P(l, p.w2), P(l, p.b2), M,
                                        4 * C, C), "matmul_forward(fc2)"));
    if (l + 1 < cfg.L)
      UGK_TRY(timed(UGK_OP_RESIDUAL_LAYERNORM_FORWARD, [&] {
        return ugk_residual_layernorm_forward(A(l, a.res1), A(l + 1, a.lno), A(l + 1, a.lnm), A(l + 1, a.lnr),
                                              A(l, a.resa), A(l, a.mlpo), P(l + 1, p.lng), P(l + 1, p.lnb), B, T,
                                              C);
      }));
    else
      UGK_TRY(timed(UGK_OP_RESIDUAL_LAYERNORM_FORWARD, [&] {
        return ugk_residual_layernorm_forward(A(l, a.res1), acts + a.flo, acts + a.flm, acts + a.flr,
                                              A(l, a.resa), A(l, a.mlpo), params + p.flng, params + p.flnb, B, T,
                                              C);
      }));
    stream_in = A(l, a.res1);
  }
  return ok();
}

// gpt2_kernels.cuh:846-894. zeroed: grads_acts is zero outside flo on entry
// (the arms' memset, train_bnn_gpu.cu:475), so the buffers this pass writes
// first are written without being read: GELU backward's dinp (fch), the
// residual splits' dx and dy (resa, mlpo, res1, apr) and the final
// LayerNorm's dinp (res1 of the last block).
namespace {
int layers_backward(const char *fn, bool zeroed, float *grads, float *grads_acts, const float *acts,
                    const float *params, const int *inputs, ugk_config cfg, const ugk_dense_ops *ops) {
  UGK_TRY(check_cfg(fn, cfg));
  if (any_null({grads, grads_acts, acts, params, inputs})) return bad(fn, "NULL pointer");
  const POff p = poff(cfg);
  const AOff a = aoff(cfg);
  const int B = cfg.B, T = cfg.T, C = cfg.C, M = B * T;
  const int NBTC = M * C;
  auto A = [&](size_t l, size_t rel) { return a.blk0 + l * a.bstride + rel; };
  auto P = [&](size_t l, size_t rel) { return p.blk0 + l * p.bstride + rel; };
  // Every layernorm_backward but the last is followed at once by a
  // residual_backward whose dout is that LN's dinp (the block's first
  // residual_backward consumes the LN1 gradient of the block above, or the
  // final LN's): those pairs run as one pass, ugk_layernorm_residual_backward.
  // The 2L+1 LayerNorm backwards write their dweight/dbias partial rows to
  // separate slots of the workspace; one batched launch at the end adds them
  // (nothing in between reads those gradients), instead of a reduce launch
  // after each.
  const size_t slot = align_up(layernorm_backward_scratch(M, C));
  const int slot_rows = layernorm_backward_blocks_bound(M, C);  // partial rows a slot holds
  const int nln = 2 * cfg.L + 1;
  char *pbase = static_cast<char *>(workspace(kRegLn, slot * (size_t)nln));
  if (!pbase) return UGK_ENOMEM;
  std::vector<LnReduceJob> jobs;
  jobs.reserve((size_t)nln);
  const bool exact = layernorm_exact() != 0;
  auto ln_bwd = [&](float *dinp, float *dw, float *db, float *dx, float *dy, const float *dout, const float *inp,
                    const float *w, const float *mean, const float *rstd, int dinp_mode = kDinpRead) -> int {
    if (exact)  // the reference's LayerNorm backward then residual_backward, each in its own order
      return timed(dx ? UGK_OP_LAYERNORM_RESIDUAL_BACKWARD_MAIN : UGK_OP_LAYERNORM_BACKWARD_MAIN, [&] {
        return launch_layernorm_residual_backward(dinp, dw, db, dx, dy, dout, inp, w, mean, rstd, M, C);
      });
    float *part = reinterpret_cast<float *>(pbase + slot * jobs.size());
    int nblk = 0;
    // A pair's dinp is read (the LayerNorm adds to it) but not written back:
    // in gpt2_backward nothing reads it after the residual_backward that
    // splits it into dx and dy (res1 of every block and each block's resa).
    if (int e = timed(dx ? UGK_OP_LAYERNORM_RESIDUAL_BACKWARD_MAIN : UGK_OP_LAYERNORM_BACKWARD_MAIN, [&] {
          return launch_layernorm_backward_partials(dinp, part, dx, dy, dout, inp, w, mean, rstd, M, C, slot_rows,
                                                    &nblk, dx ? dinp_mode : kDinpRw, zeroed && dx != nullptr);
        }))
      return e;
    jobs.push_back({part, dw, db, nblk});
    return 0;
  };
  const size_t last = cfg.L > 0 ? A(cfg.L - 1, a.res1) : a.enc;
  if (cfg.L > 0)
    UGK_TRY(ln_bwd(grads_acts + last, grads + p.flng, grads + p.flnb, grads_acts + A(cfg.L - 1, a.resa),
                   grads_acts + A(cfg.L - 1, a.mlpo), grads_acts + a.flo, acts + last, params + p.flng,
                   acts + a.flm, acts + a.flr, zeroed ? kDinpNone : kDinpRead));
  else
    UGK_TRY(ln_bwd(grads_acts + last, grads + p.flng, grads + p.flnb, nullptr, nullptr, grads_acts + a.flo,
                   acts + last, params + p.flng, acts + a.flm, acts + a.flr));
  for (int l = cfg.L - 1; l >= 0; l--) {
    const size_t st = (l == 0) ? a.enc : A(l - 1, a.res1);
    if (ops && ops->matmul_backward)
      UGK_TRY(dense(ops->matmul_backward(ops->ctx, grads_acts + A(l, a.gelu), grads + P(l, p.w2),
                                         grads + P(l, p.b2), acts + A(l, a.gelu), params + P(l, p.w2),
                                         grads_acts + A(l, a.mlpo), M, 4 * C, C), "matmul_backward(fc2)"));
    UGK_TRY(timed(UGK_OP_GELU_BACKWARD, [&] {
      float *dfch = grads_acts + A(l, a.fch);
      const float *fch = acts + A(l, a.fch), *dgelu = grads_acts + A(l, a.gelu);
      return zeroed ? launch_gelu_backward_zero(dfch, fch, dgelu, (size_t)NBTC * 4)
                    : launch_gelu_backward(dfch, fch, dgelu, (size_t)NBTC * 4);
    }));
    if (ops && ops->matmul_backward)
      UGK_TRY(dense(ops->matmul_backward(ops->ctx, grads_acts + A(l, a.ln2o), grads + P(l, p.w1),
                                         grads + P(l, p.b1), acts + A(l, a.ln2o), params + P(l, p.w1),
                                         grads_acts + A(l, a.fch), M, C, 4 * C), "matmul_backward(fc)"));
    UGK_TRY(ln_bwd(grads_acts + A(l, a.resa), grads + P(l, p.ln2g), grads + P(l, p.ln2b), grads_acts + st,
                   grads_acts + A(l, a.apr), grads_acts + A(l, a.ln2o), acts + A(l, a.resa),
                   params + P(l, p.ln2g), acts + A(l, a.ln2m), acts + A(l, a.ln2r)));
    if (ops && ops->matmul_backward)
      UGK_TRY(dense(ops->matmul_backward(ops->ctx, grads_acts + A(l, a.atty), grads + P(l, p.pw),
                                         grads + P(l, p.pb), acts + A(l, a.atty), params + P(l, p.pw),
                                         grads_acts + A(l, a.apr), M, C, C), "matmul_backward(proj)"));
    if (ops && ops->attention_backward)
      UGK_TRY(dense(ops->attention_backward(ops->ctx, grads_acts + A(l, a.qkv), grads_acts + A(l, a.atty),
                                            acts + A(l, a.qkv), B, T, C, cfg.NH), "attention_backward"));
    if (ops && ops->matmul_backward)
      UGK_TRY(dense(ops->matmul_backward(ops->ctx, grads_acts + A(l, a.lno), grads + P(l, p.qw),
                                         grads + P(l, p.qb), acts + A(l, a.lno), params + P(l, p.qw),
                                         grads_acts + A(l, a.qkv), M, C, 3 * C), "matmul_backward(qkv)"));
    if (l > 0)
      UGK_TRY(ln_bwd(grads_acts + st, grads + P(l, p.lng), grads + P(l, p.lnb), grads_acts + A(l - 1, a.resa),
                     grads_acts + A(l - 1, a.mlpo), grads_acts + A(l, a.lno), acts + st, params + P(l, p.lng),
                     acts + A(l, a.lnm), acts + A(l, a.lnr)));
    else
      UGK_TRY(ln_bwd(grads_acts + st, grads + P(l, p.lng), grads + P(l, p.lnb), nullptr, nullptr,
                     grads_acts + A(l, a.lno), acts + st, params + P(l, p.lng), acts + A(l, a.lnm),
                     acts + A(l, a.lnr)));
  }
  if (!jobs.empty())
    UGK_TRY(timed(UGK_OP_LAYERNORM_COLUMN_SUMS,
                  [&] { return launch_layernorm_reduce(jobs.data(), (int)jobs.size(), C); }));
  UGK_TRY(timed(UGK_OP_ENCODER_BACKWARD, [&] {
    return ugk_encoder_backward(grads + p.wte, grads + p.wpe, grads_acts + a.enc, inputs, B, T, C);
  }));
  return ok();
}
}  // namespace

int ugk_gpt2_layers_backward(float *grads, float *grads_acts, const float *acts, const float *params,
                             const int *inputs, ugk_config cfg, const ugk_dense_ops *ops) {
  return layers_backward("ugk_gpt2_layers_backward", false, grads, grads_acts, acts, params, inputs, cfg, ops);
}

int ugk_gpt2_layers_backward_zeroed(float *grads, float *grads_acts, const float *acts, const float *params,
                                    const int *inputs, ugk_config cfg, const ugk_dense_ops *ops) {
  return layers_backward("ugk_gpt2_layers_backward_zeroed", true, grads, grads_acts, acts, params, inputs, cfg,
                         ops);
}

int ugk_op_timer_start(int capacity) {
  const char *fn = "ugk_op_timer_start";
  if (capacity < 0) return bad(fn, "capacity must be >= 0");
  OpTimer &t = g_timer;
  for (hipEvent_t e : t.ev) (void)hipEventDestroy(e);
  t.ev.assign(2 * (size_t)capacity, nullptr);
  t.pair.assign((size_t)capacity, LaunchEvents{nullptr, nullptr, false});
  t.op.assign((size_t)capacity, 0);
  t.n = 0;
  t.on = false;
  for (auto &e : t.ev)
    if (hipEventCreate(&e) != hipSuccess) {
      (void)hipGetLastError();
      return set_error(UGK_EHIP, "%s: hipEventCreate failed", fn);
    }
  t.on = true;
  return ok();
}

int ugk_op_timer_read(float *ms, int *ops, int capacity, int *count) {
  const char *fn = "ugk_op_timer_read";
  if (!count || (capacity > 0 && (!ms || !ops))) return bad(fn, "NULL pointer");
  OpTimer &t = g_timer;
  t.on = false;
  const int n = t.n < capacity ? t.n : capacity;
  if (t.n > 0 && hipEventSynchronize(t.ev[2 * (t.n - 1) + 1]) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(UGK_EHIP, "%s: waiting for the events failed", fn);
  }
  for (int i = 0; i < n; i++) {
    float v = 0.0f;
    if (hipEventElapsedTime(&v, t.ev[2 * i], t.ev[2 * i + 1]) != hipSuccess) {
      (void)hipGetLastError();
      return set_error(UGK_EHIP, "%s: hipEventElapsedTime failed", fn);
    }
    ms[i] = v;
    ops[i] = t.op[i];
  }
  *count = n;
  t.n = 0;
  return ok();
}

}  // extern "C"
