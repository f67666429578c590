// ugk_elementwise.hip - streaming elementwise kernels: residual fwd/bwd,
// GELU fwd/bwd and bayes_materialize.
//
// All five are maps over flat fp32 arrays. Each thread owns kUnroll float4
// (16-byte) slots strided by the workgroup size, so every load and store
// instruction of a wavefront covers one contiguous 1 KiB span, all of a
// thread's loads are issued before its first arithmetic instruction, and every
// access is non-temporal (each byte is touched once). A launch-shape sweep on
// MI355X (unroll 1-8, 256-1024 threads, flat or grid-stride, with and without
// nt) put unroll 1-2 of 256 threads with nt loads and stores on top.
// Arrays whose pointers are not all 16-byte aligned, and the n % 4 tail, take
// a scalar grid-stride path with identical arithmetic.
//
// Arithmetic follows train_bnn.c operation by operation (the library is built
// with -ffp-contract=off) and the transcendental functions come from
// ugk_libm_dev.h, which equals the host glibc on every input, so every result
// is bit-identical to the CPU oracle.
#include "ugk_internal.h"
#include "ugk_libm_dev.h"

namespace ugk {
namespace {

constexpr int kUnroll = 2;

// ---- per-element operators ------------------------------------------------
// `ld` are the loaded operands in the order of the launcher's load list, `st`
// the stored values in the order of its store list.

struct ResidualFwd {  // train_bnn.c:182-186
  static constexpr int kLoads = 2, kStores = 1;
  static constexpr bool kTable = false;
  __device__ static void apply(const float *ld, float *st, const uint64_t *) { st[0] = ld[0] + ld[1]; }
};

struct ResidualBwd {  // train_bnn.c:491-496; loads dout, dx, dy
  static constexpr int kLoads = 3, kStores = 2;
  static constexpr bool kTable = false;
  __device__ static void apply(const float *ld, float *st, const uint64_t *) {
    st[0] = ld[1] + ld[0];
    st[1] = ld[2] + ld[0];
  }
};

// dx and dy are the same buffer: the CPU loop then adds dout twice, in order.
struct ResidualBwdSame {  // loads dout, dx
  static constexpr int kLoads = 2, kStores = 1;
  static constexpr bool kTable = false;
  __device__ static void apply(const float *ld, float *st, const uint64_t *) { st[0] = (ld[1] + ld[0]) + ld[0]; }
};

struct GeluFwd {  // train_bnn.c:163-170
  static constexpr int kLoads = 1, kStores = 1;
  static constexpr bool kTable = false;
  __device__ static void apply(const float *ld, float *st, const uint64_t *) {
    const float k = 0.7978845608f;
    const float x = ld[0];
    const float inner = k * (x + 0.044715f * x * x * x);
    st[0] = 0.5f * x * (1.0f + ugk_dev_tanhf(inner));
  }
};

struct GeluBwd {  // train_bnn.c:520-533; loads inp, dout, dinp
  static constexpr int kLoads = 3, kStores = 1;
  static constexpr bool kTable = false;
  __device__ static void apply(const float *ld, float *st, const uint64_t *) {
    const float k = 0.7978845608f;
    const float x = ld[0];
    const float u = k * (x + 0.044715f * x * x * x);
    const float tanh_u = ugk_dev_tanhf(u);
    const float sech2 = 1.0f - tanh_u * tanh_u;
    const float du_dx = k * (1.0f + 3.0f * 0.044715f * x * x);
    const float local_grad = 0.5f * (1.0f + tanh_u) + 0.5f * x * sech2 * du_dx;
    st[0] = ld[2] + local_grad * ld[1];
  }
};

struct Materialize {  // train_bnn.c:831-835; loads mu, rho, eps
  static constexpr int kLoads = 3, kStores = 1;
  static constexpr bool kTable = true;  // expf's 2^(i/32) table staged in LDS
  __device__ static void apply(const float *ld, float *st, const uint64_t *tab) {
    st[0] = ld[0] + ugk_dev_softplusf_lds(ld[1], tab) * ld[2];
  }
};

template <class Op>
struct Streams {
  const float *ld[Op::kLoads];
  float *st[Op::kStores];
};

template <class Op>
__global__ __launch_bounds__(kBlock) void k_map_vec4(Streams<Op> s, size_t n4) {
  __shared__ uint64_t tab[Op::kTable ? 32 : 1];
  if (Op::kTable) {
    ugk_exp2_stage(tab);
    __syncthreads();
  }
  const size_t base = (size_t)blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
  float4 v[kUnroll][Op::kLoads];
#pragma unroll
  for (int u = 0; u < kUnroll; u++) {
    const size_t i = base + (size_t)u * kBlock;
    if (i < n4) {
#pragma unroll
      for (int l = 0; l < Op::kLoads; l++) v[u][l] = ld_nt(reinterpret_cast<const float4 *>(s.ld[l]) + i);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; u++) {
    const size_t i = base + (size_t)u * kBlock;
    if (i < n4) {
      float in[4][Op::kLoads], out[4][Op::kStores];
#pragma unroll
      for (int l = 0; l < Op::kLoads; l++) {
        in[0][l] = v[u][l].x; in[1][l] = v[u][l].y;
        in[2][l] = v[u][l].z; in[3][l] = v[u][l].w;
      }
#pragma unroll
      for (int e = 0; e < 4; e++) Op::apply(in[e], out[e], tab);
#pragma unroll
      for (int o = 0; o < Op::kStores; o++)
        st_nt(reinterpret_cast<float4 *>(s.st[o]) + i, make_float4(out[0][o], out[1][o], out[2][o], out[3][o]));
    }
  }
}

template <class Op>
__global__ __launch_bounds__(kBlock) void k_map_scalar(Streams<Op> s, size_t begin, size_t n) {
  __shared__ uint64_t tab[Op::kTable ? 32 : 1];
  if (Op::kTable) {
    ugk_exp2_stage(tab);
    __syncthreads();
  }
  for (size_t i = begin + (size_t)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (size_t)gridDim.x * kBlock) {
    float in[Op::kLoads], out[Op::kStores];
#pragma unroll
    for (int l = 0; l < Op::kLoads; l++) in[l] = s.ld[l][i];
    Op::apply(in, out, tab);
#pragma unroll
    for (int o = 0; o < Op::kStores; o++) s.st[o][i] = out[o];
  }
}

template <class Op>
int run_map(const Streams<Op> &s, size_t n, const char *name) {
  if (n == 0) return 0;
  bool vec = true;
  for (int l = 0; l < Op::kLoads; l++) vec = vec && aligned16(s.ld[l]);
  for (int o = 0; o < Op::kStores; o++) vec = vec && aligned16(s.st[o]);
  size_t done = 0;
  if (vec && n >= 4) {
    const size_t n4 = n / 4;
    hipLaunchKernelGGL(k_map_vec4<Op>, dim3(grid_for(n4, (size_t)kBlock * kUnroll)),
                       dim3(kBlock), 0, stream(), s, n4);
    done = n4 * 4;
  }
  if (done < n) {
    const size_t rest = n - done;
    unsigned g = grid_for(rest, kBlock);
    if (g > 65536u) g = 65536u;
    hipLaunchKernelGGL(k_map_scalar<Op>, dim3(g), dim3(kBlock), 0, stream(), s, done, n);
  }
  return check_launch(name);
}

}  // namespace

int launch_residual_forward(float *out, const float *x, const float *y, size_t n) {
  Streams<ResidualFwd> s{{x, y}, {out}};
  return run_map(s, n, "residual_forward");
}

int launch_residual_backward(float *dx, float *dy, const float *dout, size_t n) {
  if (dx == dy) {
    Streams<ResidualBwdSame> s{{dout, dx}, {dx}};
    return run_map(s, n, "residual_backward");
  }
  Streams<ResidualBwd> s{{dout, dx, dy}, {dx, dy}};
  return run_map(s, n, "residual_backward");
}

int launch_gelu_forward(float *out, const float *inp, size_t n) {
  Streams<GeluFwd> s{{inp}, {out}};
  return run_map(s, n, "gelu_forward");
}

int launch_gelu_backward(float *dinp, const float *inp, const float *dout, size_t n) {
  Streams<GeluBwd> s{{inp, dout, dinp}, {dinp}};
  return run_map(s, n, "gelu_backward");
}

int launch_bayes_materialize(float *w, const float *mu, const float *rho,
                             const float *eps, size_t n) {
  Streams<Materialize> s{{mu, rho, eps}, {w}};
  return run_map(s, n, "bayes_materialize");
}

}  // namespace ugk
