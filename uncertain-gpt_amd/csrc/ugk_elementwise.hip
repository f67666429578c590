// ugk_elementwise.hip - streaming elementwise kernels: residual fwd/bwd,
// GELU fwd/bwd and bayes_materialize.
//
// All five are maps over flat fp32 arrays through the streaming map of
// ugk_map.h.
//
// Arithmetic follows train_bnn.c operation by operation (the library is built
// with -ffp-contract=off) and the transcendental functions come from
// ugk_libm_dev.h, which equals the host glibc on every input, so every result
// is bit-identical to the CPU oracle -- except GELU's default form, which
// evaluates the same function through the hardware exponential and
// reciprocal (ugk_fast_gelu*: within 1e-5 relative / 1e-6 absolute of the CPU
// on every input, and memory-bound where the glibc-exact tanhf made the
// forward VALU-bound); ugk_set_gelu_exact(1) selects the bit-exact kernels.
#include <atomic>

#include "ugk_map.h"

namespace ugk {
namespace {

// ---- per-element operators ------------------------------------------------
// `ld` are the loaded operands in the order of the launcher's load list, `st`
// the stored values in the order of its store list.

struct ResidualFwd : MapOp {  // train_bnn.c:182-186
  static constexpr int kLoads = 2, kStores = 1;
  static constexpr int kUnroll = 1, kThreads = 512;  // measured best of the map shapes
  __device__ static void apply(const float *ld, float *st, const uint64_t *, size_t, Params) { st[0] = ld[0] + ld[1]; }
};

struct ResidualBwd : MapOp {  // train_bnn.c:491-496; loads dout, dx, dy
  static constexpr int kLoads = 3, kStores = 2;
  static constexpr int kUnroll = 1, kThreads = 512;
  __device__ static void apply(const float *ld, float *st, const uint64_t *, size_t, Params) {
    st[0] = ld[1] + ld[0];
    st[1] = ld[2] + ld[0];
  }
};

// dx and dy are the same buffer: the CPU loop then adds dout twice, in order.
struct ResidualBwdSame : MapOp {  // loads dout, dx
  static constexpr int kLoads = 2, kStores = 1;
  static constexpr int kUnroll = 1, kThreads = 512;
  __device__ static void apply(const float *ld, float *st, const uint64_t *, size_t, Params) { st[0] = (ld[1] + ld[0]) + ld[0]; }
};

struct GeluFwd : MapOp {  // train_bnn.c:163-170
  static constexpr int kLoads = 1, kStores = 1;
  __device__ static void apply(const float *ld, float *st, const uint64_t *, size_t, Params) {
    st[0] = ugk_dev_gelu(ld[0]);
  }
};

struct GeluFwdFast : MapOp {  // train_bnn.c:163-170, logistic form
  static constexpr int kLoads = 1, kStores = 1;
  static constexpr int kUnroll = 1, kThreads = 512;  // measured best of the map shapes
  __device__ static void apply(const float *ld, float *st, const uint64_t *, size_t, Params) {
    st[0] = ugk_fast_gelu(ld[0]);
  }
};

struct GeluBwdFast : MapOp {  // train_bnn.c:520-533, logistic form; loads inp, dout, dinp
  static constexpr int kLoads = 3, kStores = 1;
  static constexpr int kUnroll = 1, kThreads = 1024;  // measured best of the map shapes
  __device__ static void apply(const float *ld, float *st, const uint64_t *, size_t, Params) {
    st[0] = ld[2] + ugk_fast_gelu_grad(ld[0]) * ld[1];
  }
};

struct GeluBwd : MapOp {  // train_bnn.c:520-533; loads inp, dout, dinp
  static constexpr int kLoads = 3, kStores = 1;
  static constexpr int kUnroll = 1, kThreads = 512;  // measured best of the map shapes
  __device__ static void apply(const float *ld, float *st, const uint64_t *, size_t, Params) {
    st[0] = ld[2] + ugk_dev_gelu_grad(ld[0]) * ld[1];
  }
};

// The same two with dinp taken as +0.0 instead of read (the zeroed-gradient
// step driver, where GELU backward is the first writer of its dinp): +0.0 + x
// gives the bits that the read of a zero buffer would give.
struct GeluBwdFastZero : MapOp {  // loads inp, dout
  static constexpr int kLoads = 2, kStores = 1;
  static constexpr int kUnroll = 1, kThreads = 1024;
  __device__ static void apply(const float *ld, float *st, const uint64_t *, size_t, Params) {
    st[0] = 0.0f + ugk_fast_gelu_grad(ld[0]) * ld[1];
  }
};

struct GeluBwdZero : MapOp {  // loads inp, dout
  static constexpr int kLoads = 2, kStores = 1;
  static constexpr int kUnroll = 1, kThreads = 512;
  __device__ static void apply(const float *ld, float *st, const uint64_t *, size_t, Params) {
    st[0] = 0.0f + ugk_dev_gelu_grad(ld[0]) * ld[1];
  }
};

struct Materialize : MapOp {  // train_bnn.c:831-835; loads mu, rho, eps
  static constexpr int kLoads = 3, kStores = 1;
  static constexpr int kUnroll = 1, kThreads = 256;  // measured best of the map shapes
  static constexpr bool kTable = true;  // expf's 2^(i/32) table staged in LDS
  __device__ static void apply(const float *ld, float *st, const uint64_t *tab, size_t, Params) {
    st[0] = ld[0] + ugk_dev_softplusf_lds(ld[1], tab) * ld[2];
  }
};

}  // namespace

int launch_residual_forward(float *out, const float *x, const float *y, size_t n) {
  Streams<ResidualFwd> s{{x, y}, {out}, {}};
  return run_map(s, n, "residual_forward");
}

int launch_residual_backward(float *dx, float *dy, const float *dout, size_t n) {
  if (dx == dy) {
    Streams<ResidualBwdSame> s{{dout, dx}, {dx}, {}};
    return run_map(s, n, "residual_backward");
  }
  Streams<ResidualBwd> s{{dout, dx, dy}, {dx, dy}, {}};
  return run_map(s, n, "residual_backward");
}

namespace {
std::atomic<int> g_gelu_exact{0};
}  // namespace

void set_gelu_exact(int exact) { g_gelu_exact.store(exact ? 1 : 0); }
int gelu_exact() { return g_gelu_exact.load(); }

int launch_gelu_forward(float *out, const float *inp, size_t n) {
  if (gelu_exact()) {
    Streams<GeluFwd> s{{inp}, {out}, {}};
    return run_map(s, n, "gelu_forward");
  }
  Streams<GeluFwdFast> s{{inp}, {out}, {}};
  return run_map(s, n, "gelu_forward");
}

int launch_gelu_backward(float *dinp, const float *inp, const float *dout, size_t n) {
  if (gelu_exact()) {
    Streams<GeluBwd> s{{inp, dout, dinp}, {dinp}, {}};
    return run_map(s, n, "gelu_backward");
  }
  Streams<GeluBwdFast> s{{inp, dout, dinp}, {dinp}, {}};
  return run_map(s, n, "gelu_backward");
}

int launch_gelu_backward_zero(float *dinp, const float *inp, const float *dout, size_t n) {
  if (gelu_exact()) {
    Streams<GeluBwdZero> s{{inp, dout}, {dinp}, {}};
    return run_map(s, n, "gelu_backward");
  }
  Streams<GeluBwdFastZero> s{{inp, dout}, {dinp}, {}};
  return run_map(s, n, "gelu_backward");
}

int launch_bayes_materialize(float *w, const float *mu, const float *rho,
                             const float *eps, size_t n) {
  Streams<Materialize> s{{mu, rho, eps}, {w}, {}};
  return run_map(s, n, "bayes_materialize");
}

}  // namespace ugk
