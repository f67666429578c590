// ugk_bayes.hip - the O(P) posterior path around the layer kernels: Philox
// sampling of w, the data-term backward onto (mu, rho), the KL term and its
// gradient, AdamW, and the fused Bayes-by-Backprop step.
//
// All are streams over flat fp32 parameter vectors (ugk_map.h). Arithmetic
// follows train_bnn.c operation by operation (built with -ffp-contract=off),
// with expf/log1pf exact to glibc (ugk_libm_dev.h) and IEEE division and
// square root, so every op that is given its eps is bit-identical to the CPU
// oracle. The Philox ops draw eps on the fly (ugk_philox.h): their integer
// stream is exact, their Box-Muller transform uses the device logf/cosf.
#include <atomic>

#include "ugk_map.h"
#include "ugk_philox.h"

namespace ugk {
namespace {

__device__ __forceinline__ float expf_lds(float x, const uint64_t *tab) {
  return ugk_expf_t<UGK_EXPF_CONTRACT>(x, UgkExp2Lds{tab});
}

// train_bnn.c:820-822 (sigmoidf_), gpt2_kernels.cuh:199-201 (d_sigmoid).
__device__ __forceinline__ float sigmoid_lds(float x, const uint64_t *tab) {
  return ugk_dev_recip_ge1(1.0f + expf_lds(-x, tab));
}

// The Philox ops' softplus and sigmoid: the hardware-transcendental forms by
// default (kFast; within a few ulp of glibc's and within 1e-6 absolute / 1e-5
// relative on every input, ugk_diag.hip fn 66 and 67), or the glibc-exact
// forms of the eps-taking ops (bit-identical to train_bnn.c given the same
// eps), selected by ugk_set_philox_exact.
template <bool kFast>
__device__ __forceinline__ float softplus_of(float x, const uint64_t *tab) {
  if constexpr (kFast)
    return ugk_fast_softplus(x);
  else
    return ugk_dev_softplusf_lds(x, tab);
}
template <bool kFast>
__device__ __forceinline__ float sigmoid_of(float x, const uint64_t *tab) {
  if constexpr (kFast)
    return ugk_fast_sigmoid(x);
  else
    return sigmoid_lds(x, tab);
}

struct PhiloxParams {
  unsigned long long seed;
  int step;
};

// eps(seed, step, i) in the op's form: the hardware radius in the default form,
// glibc's logf and cosf and the correctly rounded square root in the
// glibc-exact one.
template <bool kFast>
__device__ __forceinline__ float draw(unsigned long long seed, int step, size_t i) {
  return kFast ? ugk_dev_philox_normal_fast(seed, step, i) : ugk_dev_philox_normal(seed, step, i);
}

// train_bnn_gpu.cu:93-97 (k_bayes_sample): w = mu + softplus(rho) * eps(seed,
// step, i). Loads mu, rho.
template <bool kFast>
struct BayesSample : MapOp {
  static constexpr int kLoads = 2, kStores = 1;
  static constexpr bool kTable = !kFast;
  static constexpr int kUnroll = 1;
  // eps for all four of a thread's elements while mu and rho load: with the
  // branches of the fast softplus, 296-299 against 349 us (select form, eps in
  // place) over 124.4M; the glibc-exact form 402 against 427 us
  static constexpr bool kPre = true;
  typedef float Pre;
  typedef PhiloxParams Params;
  __device__ static float pre(size_t i, const Params &p) { return draw<kFast>(p.seed, p.step, i); }
  __device__ static void apply_pre(const float *ld, float *st, const uint64_t *tab, size_t, const Params &,
                                   float eps) {
    st[0] = ld[0] + softplus_of<kFast>(ld[1], tab) * eps;
  }
};

// The same draw, also storing eps (train_bnn.c:841-845's bayes_sample keeps eps
// for the backward). Stores w, eps.
template <bool kFast>
struct BayesSampleEps : BayesSample<kFast> {
  static constexpr int kStores = 2;
  typedef PhiloxParams Params;
  __device__ static void apply_pre(const float *ld, float *st, const uint64_t *tab, size_t, const Params &,
                                   float eps) {
    st[0] = ld[0] + softplus_of<kFast>(ld[1], tab) * eps;
    st[1] = eps;
  }
};

// train_bnn.c:855-861: dmu += dw; drho += dw * eps * sigmoid(rho).
// Loads dw, eps, rho, dmu, drho; stores dmu, drho.
struct BayesBackward : MapOp {
  static constexpr int kLoads = 5, kStores = 2;
  static constexpr int kUnroll = 1, kThreads = 1024;  // measured best of the map shapes
  static constexpr bool kTable = true;
  __device__ static void apply(const float *ld, float *st, const uint64_t *tab, size_t, Params) {
    st[0] = ld[3] + ld[0];
    st[1] = ld[4] + ld[0] * ld[1] * sigmoid_lds(ld[2], tab);
  }
};

// train_bnn_gpu.cu:99-109 (k_bayes_backward): the same with eps regenerated.
// Loads dw, rho, dmu, drho; stores dmu, drho.
template <bool kFast>
struct BayesBackwardPhilox : MapOp {
  static constexpr int kLoads = 4, kStores = 2;
  // measured best of the map shapes: 512 threads for the glibc-exact form, 1024
  // for the fast one (506 us at 512, 515 at 256, 484 at 1024 over 124.4M)
  static constexpr int kUnroll = 1, kThreads = kFast ? 1024 : 512;
  static constexpr bool kTable = !kFast;
  // eps drawn in place: drawing all four of a thread's eps while the streams
  // load (kPre) measured 488-510 against 483-496 us.
  typedef PhiloxParams Params;
  __device__ static void apply(const float *ld, float *st, const uint64_t *tab, size_t i, const Params &p) {
    const float g = ld[0];
    const float eps = draw<kFast>(p.seed, p.step, i);
    st[0] = ld[2] + g;
    st[1] = ld[3] + g * eps * sigmoid_of<kFast>(ld[1], tab);
  }
};

// train_bnn.c:966-979: dmu += weight * (mu / sp2);
// drho += weight * (sigma / sp2 - 1 / sigma) * sigmoid(rho), sigma = softplus(rho).
// Loads mu, rho, dmu, drho; stores dmu, drho.
// A launch-wide divisor with its reciprocal (1.0f / b, correctly rounded) and
// whether the reciprocal form of the quotient applies to it.
struct SharedDivisor {
  float b, y;
  bool ok;
  static SharedDivisor of(float b) { return SharedDivisor{b, 1.0f / b, ugk_div_shared_ok(b)}; }
};

__device__ __forceinline__ float div_by(float a, const SharedDivisor &d) { return ugk_div_shared(a, d.b, d.y, d.ok); }

struct KlBackward : MapOp {
  static constexpr int kLoads = 4, kStores = 2;
  static constexpr int kUnroll = 1, kThreads = 256;  // measured best of the map shapes
  static constexpr bool kTable = true;
  struct Params {
    SharedDivisor sp2;
    float weight;
  };
  __device__ static void apply(const float *ld, float *st, const uint64_t *tab, size_t, const Params &p) {
    const float r = ld[1];
    const float sigma = ugk_dev_softplusf_lds(r, tab);
    st[0] = ld[2] + p.weight * div_by(ld[0], p.sp2);
    const float dsigma = div_by(sigma, p.sp2) - 1.0f / sigma;
    st[1] = ld[3] + p.weight * dsigma * sigmoid_lds(r, tab);
  }
};

struct AdamParams {
  float lr, beta1, beta2, eps, wd;
  SharedDivisor bc1, bc2;
};

// One AdamW update of (param, m, v) by gradient g; train_bnn.c:704-716 and
// gpt2_kernels.cuh:973-984 evaluate the same expression (the quotients by
// the bias corrections and the square root are the correctly rounded ones).
__device__ __forceinline__ float adamw_one(float param, float g, float &m, float &v, const AdamParams &a) {
  m = a.beta1 * m + (1.0f - a.beta1) * g;
  v = a.beta2 * v + (1.0f - a.beta2) * g * g;
  const float m_hat = div_by(m, a.bc1);
  const float v_hat = div_by(v, a.bc2);
  return param - a.lr * (m_hat / (ugk_dev_sqrtf(v_hat) + a.eps) + a.wd * param);
}

// train_bnn.c:699-717. Loads params, grads, m, v; stores params, m, v.
struct AdamW : MapOp {
  static constexpr int kLoads = 4, kStores = 3;
  static constexpr int kUnroll = 1, kThreads = 1024;  // measured best of the map shapes
  typedef AdamParams Params;
  __device__ static void apply(const float *ld, float *st, const uint64_t *, size_t, const Params &p) {
    float m = ld[2], v = ld[3];
    st[0] = adamw_one(ld[0], ld[1], m, v, p);
    st[1] = m;
    st[2] = v;
  }
};

// train_bnn_gpu.cu:173-217 (k_bbb_step_fused): bayes_backward with
// eps(step), kl_backward when klw > 0, AdamW on mu and on rho, dw cleared,
// and w drawn for step + 1 from the updated parameters.
// Loads dw, rho, mu, m_mu, v_mu, m_rho, v_rho;
// stores dw, mu, rho, m_mu, v_mu, m_rho, v_rho, w.
template <bool kFast>
struct BbbStepFused : MapOp {
  static constexpr int kLoads = 7, kStores = 8;
  static constexpr bool kTable = !kFast;
  static constexpr int kUnroll = 1;
  // The fast form fits 8 wavefronts per SIMD in its registers but runs best at
  // 6 (24 KiB of LDS per 256-thread workgroup leaves room for 6 per CU):
  // 1338-1419 us at 8, 1327-1407 at 7, 1325-1345 at 6, 1337-1345 at 5 and
  // 1355 at 4 over 124.4M (cold, two boxes). The glibc-exact form is best
  // at 8 (1422 us; 1444 at 6).
  static constexpr unsigned kLdsReserve = kFast ? 24576u : 0u;
  struct Params {
    unsigned long long seed;
    int step;
    SharedDivisor sp2;  // the prior variance sp * sp
    float klw;
    AdamParams adam;
  };
  // Both draws while the streams load (kPre) in the glibc-exact form: 1407
  // against 1436 us in place; the fast form draws in place (1324-1378 against
  // 1339-1391 us with kPre).
  static constexpr bool kPre = !kFast;
  struct Pre {
    float eps, eps_next;
  };
  __device__ static Pre pre(size_t i, const Params &p) {
    return Pre{draw<kFast>(p.seed, p.step, i), draw<kFast>(p.seed, p.step + 1, i)};
  }
  // The step, with eps(k) the draw for step + k (k = 0 the gradient's, 1 the
  // next sample's), evaluated where the step uses it.
  template <class Eps>
  __device__ static void body(const float *ld, float *st, const uint64_t *tab, const Params &p, Eps eps) {
    const float g = ld[0], r = ld[1], mm = ld[2];
    const float sg = sigmoid_of<kFast>(r, tab);
    float gmu = g;
    float grho = g * eps(0) * sg;
    if (p.klw > 0.0f) {
      const float sigma = softplus_of<kFast>(r, tab);
      gmu += p.klw * div_by(mm, p.sp2);
      grho += p.klw * (div_by(sigma, p.sp2) - 1.0f / sigma) * sg;
    }
    float m1 = ld[3], v1 = ld[4], m2 = ld[5], v2 = ld[6];
    const float mu_new = adamw_one(mm, gmu, m1, v1, p.adam);
    const float rho_new = adamw_one(r, grho, m2, v2, p.adam);
    st[0] = 0.0f;
    st[1] = mu_new;
    st[2] = rho_new;
    st[3] = m1;
    st[4] = v1;
    st[5] = m2;
    st[6] = v2;
    st[7] = mu_new + softplus_of<kFast>(rho_new, tab) * eps(1);
  }
  __device__ static void apply_pre(const float *ld, float *st, const uint64_t *tab, size_t, const Params &p,
                                   const Pre &e) {
    body(ld, st, tab, p, [&](int k) { return k ? e.eps_next : e.eps; });
  }
  __device__ static void apply(const float *ld, float *st, const uint64_t *tab, size_t i, const Params &p) {
    body(ld, st, tab, p, [&](int k) { return draw<kFast>(p.seed, p.step + k, i); });
  }
};

// ---- KL total (train_bnn.c:941-957) -----------------------------------------
// Each term in double: log(sp / sigma) + (sigma^2 + mu^2) / (2 sp^2) - 1/2.
// Summed without a logarithm per term: sum_i log sigma_i = log prod_i sigma_i,
// the product kept as a double mantissa M and a binary exponent E (an integer
// sum). M takes each sigma (exact as a double; the product rounds once, which
// moves the logarithm by at most 2^-53, as a per-term logarithm's own rounding
// would) and gives its exponent to E after every float4 of sigma: four factors
// in [2^-149, 2^128] keep M inside the double range, subnormal sigma included.
// sigma^2 + mu^2 is summed as it comes and scaled by 1/(2 sp^2) at the end, and
// the constant log sp - 1/2 is counted, so a thread's share is
//   k (log sp - 1/2) - (E ln 2 + log M) + Q / (2 sp^2),
// one double logarithm per thread. The terms of sigma = 0, +inf or NaN are not
// finite and are not evaluated: +inf for sigma = 0 (the log of sp/0), NaN for
// +inf (-inf + inf) and for NaN, as train_bnn.c's evaluation gives. They go to
// a separate sum (a branch, rarely taken), which then decides the total.
// Summed in a fixed order: every thread over a fixed stride of float4 slots,
// then a wavefront butterfly, then the block's waves in order, then one block
// over the per-block partials. Deterministic for a given n; it differs from the
// CPU's sequential sum of terms by the rounding of a double sum in another
// order.
constexpr int kKlBlocks = 2048;

// The KL's sigma = softplus(rho): the glibc-exact form, or (kFast) the
// hardware-transcendental form while rho >= -80, where sigma is a normal float
// and that form is within 8 ulp of the exact one (ugk_diag.hip fn 66 over every
// float input), so each term moves by at most 8 * 2^-23 * (1 + sigma^2/sp^2).
// Below -80 sigma nears the subnormal range, where a few ulp are a large share
// of sigma and of its logarithm, so the exact form is taken there (a branch,
// rarely taken).
template <bool kFast>
__device__ __forceinline__ float kl_softplus(float rho, const uint64_t *tab) {
  if (!kFast) return ugk_dev_softplusf_lds(rho, tab);
  float s = ugk_fast_softplus(rho);
  if (rho < -80.0f) {
    asm volatile("");  // a branch, not both forms and a select
    s = ugk_dev_softplusf_lds(rho, tab);
  }
  return s;
}

// One thread's share of the KL total. The exponent sum stays within 150 per
// element, far inside an int for any n that fits in memory.
struct KlAcc {
  double q = 0.0;     // sum of sigma^2 + mu^2 over the product's elements
  double m = 1.0;     // mantissa product
  double cnt = 0.0;   // elements in the product
  double rare = 0.0;  // the terms of sigma = 0, +inf, NaN (+inf or NaN)
  int e = 0;          // exponent sum

  __device__ __forceinline__ void add(float mu, float sigma_f) {
    if (sigma_f > 0.0f && sigma_f < __builtin_huge_valf()) {
      const double s = (double)sigma_f, u = (double)mu;
      q += s * s + u * u;
      m *= s;
      cnt += 1.0;
    } else {
      asm volatile("");  // a branch, rarely taken
      rare += sigma_f == 0.0f ? __builtin_huge_val() : __builtin_nan("");
    }
  }
  // M's exponent into E; M to [1, 2)
  __device__ __forceinline__ void renorm() {
    const uint64_t b = ugk_d2u(m);
    e += (int)((b >> 52) & 0x7ff) - 1023;
    m = ugk_u2d((b & 0x800fffffffffffffull) | 0x3ff0000000000000ull);
  }
  __device__ __forceinline__ double total(double log_sp, double inv_two_sp2) {
    renorm();
    return cnt * (log_sp - 0.5) - __builtin_fma((double)e, 0.69314718055994530942, log(m)) +
           q * inv_two_sp2 + rare;
  }
};

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ double block_sum_d(double v, double *lds) {
  v = wave_sum_d(v);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  double t = 0.0;
  if (threadIdx.x == 0)
    for (int w = 0; w < kBlock / kWave; w++) t += lds[w];
  return t;
}

template <bool kFast>
__global__ __launch_bounds__(kBlock) void k_kl_partial(double *part, const float *mu, const float *rho,
                                                       size_t n, float sigma_prior, float sp2) {
  __shared__ uint64_t tab[32];
  __shared__ double lds[kBlock / kWave];
  ugk_exp2_stage(tab);
  __syncthreads();
  const double log_sp = log((double)sigma_prior), inv_two_sp2 = 1.0 / (2.0 * (double)sp2);
  KlAcc acc;
  const size_t stride = (size_t)gridDim.x * kBlock;
  const bool vec = aligned16(mu) && aligned16(rho);
  const size_t n4 = vec ? n / 4 : 0;
  // (issuing the next slot's loads before the current slot's terms was slower: 192 against 176 us
  // per call at n = 124,439,808, the result's wait included)
  for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
    const float4 m = ld_nt(reinterpret_cast<const float4 *>(mu) + i);
    const float4 r = ld_nt(reinterpret_cast<const float4 *>(rho) + i);
    acc.add(m.x, kl_softplus<kFast>(r.x, tab));
    acc.add(m.y, kl_softplus<kFast>(r.y, tab));
    acc.add(m.z, kl_softplus<kFast>(r.z, tab));
    acc.add(m.w, kl_softplus<kFast>(r.w, tab));
    acc.renorm();
  }
  for (size_t i = 4 * n4 + (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
    acc.add(mu[i], kl_softplus<kFast>(rho[i], tab));
    acc.renorm();
  }
  const double t = block_sum_d(acc.total(log_sp, inv_two_sp2), lds);
  if (threadIdx.x == 0) part[blockIdx.x] = t;
}

// The per-block partials, summed by one block: thread k adds partials k,
// k + 256, ... in that order (all its loads in flight at once), then the
// block's sum as above. out may be host memory mapped for the device.
static_assert(kKlBlocks % kBlock == 0, "whole rounds of partials per thread");
__global__ __launch_bounds__(kBlock) void k_kl_final(double *out, const double *part, int nparts) {
  __shared__ double lds[kBlock / kWave];
  constexpr int kPer = kKlBlocks / kBlock;
  double v[kPer];
#pragma unroll
  for (int k = 0; k < kPer; k++) v[k] = part[min((int)threadIdx.x + k * kBlock, nparts - 1)];
  double acc = 0.0;
#pragma unroll
  for (int k = 0; k < kPer; k++)
    if ((int)threadIdx.x + k * kBlock < nparts) acc += v[k];
  const double t = block_sum_d(acc, lds);
  if (threadIdx.x == 0) out[0] = t;
}

}  // namespace

namespace {
std::atomic<int> g_philox_exact{0};
std::atomic<int> g_kl_exact{0};
}  // namespace

void set_philox_exact(int exact) { g_philox_exact.store(exact ? 1 : 0); }
int philox_exact() { return g_philox_exact.load(); }
void set_kl_exact(int exact) { g_kl_exact.store(exact ? 1 : 0); }
int kl_exact() { return g_kl_exact.load(); }

namespace {
template <bool kFast>
int sample(float *w, float *eps, const float *mu, const float *rho, size_t n, unsigned long long seed, int step) {
  if (eps) {
    Streams<BayesSampleEps<kFast>> s{{mu, rho}, {w, eps}, {seed, step}};
    return run_map(s, n, "bayes_sample");
  }
  Streams<BayesSample<kFast>> s{{mu, rho}, {w}, {seed, step}};
  return run_map(s, n, "bayes_sample");
}
}  // namespace

int launch_bayes_sample(float *w, float *eps, const float *mu, const float *rho, size_t n,
                        unsigned long long seed, int step) {
  return philox_exact() ? sample<false>(w, eps, mu, rho, n, seed, step) : sample<true>(w, eps, mu, rho, n, seed, step);
}

int launch_bayes_backward(float *dmu, float *drho, const float *dw, const float *eps,
                          const float *rho, size_t n) {
  Streams<BayesBackward> s{{dw, eps, rho, dmu, drho}, {dmu, drho}, {}};
  return run_map(s, n, "bayes_backward");
}

int launch_bayes_backward_philox(float *dmu, float *drho, const float *dw, const float *rho,
                                 size_t n, unsigned long long seed, int step) {
  if (philox_exact()) {
    Streams<BayesBackwardPhilox<false>> s{{dw, rho, dmu, drho}, {dmu, drho}, {seed, step}};
    return run_map(s, n, "bayes_backward_philox");
  }
  Streams<BayesBackwardPhilox<true>> s{{dw, rho, dmu, drho}, {dmu, drho}, {seed, step}};
  return run_map(s, n, "bayes_backward_philox");
}

int launch_kl_backward(float *dmu, float *drho, const float *mu, const float *rho, size_t n,
                       float sigma_prior, float weight) {
  Streams<KlBackward> s{{mu, rho, dmu, drho}, {dmu, drho}, {SharedDivisor::of(sigma_prior * sigma_prior), weight}};
  return run_map(s, n, "kl_backward");
}

int launch_adamw(float *params, const float *grads, float *m, float *v, size_t n, float lr,
                 float beta1, float beta2, float eps, float wd, float bc1, float bc2) {
  Streams<AdamW> s{{params, grads, m, v},
                   {params, m, v},
                   {lr, beta1, beta2, eps, wd, SharedDivisor::of(bc1), SharedDivisor::of(bc2)}};
  return run_map(s, n, "adamw_update");
}

int launch_bbb_step_fused(float *mu, float *rho, float *m_mu, float *v_mu, float *m_rho, float *v_rho,
                          float *w, float *dw, size_t n, unsigned long long seed, int step, float sp,
                          float klw, float bc1, float bc2, float lr, float beta1, float beta2,
                          float aeps, float wd) {
  const typename BbbStepFused<true>::Params p{
      seed, step, SharedDivisor::of(sp * sp), klw,
      {lr, beta1, beta2, aeps, wd, SharedDivisor::of(bc1), SharedDivisor::of(bc2)}};
  if (philox_exact()) {
    Streams<BbbStepFused<false>> s{{dw, rho, mu, m_mu, v_mu, m_rho, v_rho}, {dw, mu, rho, m_mu, v_mu, m_rho, v_rho, w},
                                   {p.seed, p.step, p.sp2, p.klw, p.adam}};
    return run_map(s, n, "bbb_step_fused");
  }
  Streams<BbbStepFused<true>> s{{dw, rho, mu, m_mu, v_mu, m_rho, v_rho}, {dw, mu, rho, m_mu, v_mu, m_rho, v_rho, w}, p};
  return run_map(s, n, "bbb_step_fused");
}

size_t kl_forward_scratch() { return kKlBlocks * sizeof(double); }

int launch_kl_forward(double *out, double *part, const float *mu, const float *rho, size_t n,
                      float sigma_prior) {
  const float sp2 = sigma_prior * sigma_prior;
  size_t want = (n + 4ull * kBlock - 1) / (4ull * kBlock);
  const int blocks = (int)(want < 1 ? 1 : (want > (size_t)kKlBlocks ? (size_t)kKlBlocks : want));
  if (kl_exact())
    hipLaunchKernelGGL(k_kl_partial<false>, dim3(blocks), dim3(kBlock), 0, stream(), part, mu, rho, n,
                       sigma_prior, sp2);
  else
    hipLaunchKernelGGL(k_kl_partial<true>, dim3(blocks), dim3(kBlock), 0, stream(), part, mu, rho, n,
                       sigma_prior, sp2);
  hipLaunchKernelGGL(k_kl_final, dim3(1), dim3(kBlock), 0, stream(), out, part, blocks);
  return check_launch("kl_forward");
}

}  // namespace ugk
