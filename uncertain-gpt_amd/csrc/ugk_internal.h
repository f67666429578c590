// ugk_internal.h - shared by the libugk translation units (not installed).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "ugk.h"  // status codes

namespace ugk {

constexpr int kWave = 64;      // CDNA wavefront width
constexpr int kBlock = 256;    // 4 waves per workgroup for streaming kernels

// Library state, defined in ugk_api.hip.
hipStream_t stream();
int set_error(int code, const char *fmt, ...);
int check_launch(const char *what);

// Device workspace, one region per purpose, so that a kernel's scratch is
// never another's: the LayerNorm-backward partial rows (one slot per call, or
// 2L+1 slots for the step driver), the encoder backward's bucket state (kept
// between calls), the KL total's partial sums and the long-row softmax's row
// statistics. Each region is the library's own allocation, grown when a
// larger shape arrives (after waiting for the device), or a fixed part of a
// workspace the caller handed over with ugk_set_workspace, which then never
// grows. workspace() returns at least `bytes` of region r on the current
// device, or nullptr with the error set; *fresh (if given) tells whether the
// region's memory is new since its last use (its contents are undefined).
// With keep_fresh the fresh mark is reported but left set (for a caller that
// cannot prepare the memory now, e.g. under graph capture).
enum Region { kRegLn = 0, kRegEncoder = 1, kRegKl = 2, kRegSoftmax = 3, kNumRegions = 4 };
void *workspace(Region r, size_t bytes, bool *fresh = nullptr, bool keep_fresh = false);
// Whether the library stream is being captured into a graph (false if the
// query fails).
bool stream_capturing();

// The step driver's op timer arms an event pair for the kernel launches of
// an op; launch() then records them with the dispatches themselves
// (hipExtLaunchKernelGGL, no marker packets between kernels): the start with
// the op's first kernel, the stop with each of its kernels, so that the pair
// spans from the first kernel's start to the last one's end. Unarmed,
// launch() is a plain launch on stream().
struct LaunchEvents {
  hipEvent_t start, stop;
  bool started;  // the start has been recorded (a kernel of the op was launched)
};
LaunchEvents *&armed_events();

template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, unsigned shmem, Args... args) {
  LaunchEvents *ev = armed_events();
  if (ev) {
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream(), ev->started ? nullptr : ev->start, ev->stop, 0u,
                          static_cast<KArgs>(args)...);
    ev->started = true;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shmem, stream(), static_cast<KArgs>(args)...);
  }
}

__host__ __device__ inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

inline unsigned grid_for(size_t work, size_t per_block) {
  return (unsigned)((work + per_block - 1) / per_block);
}

// Streaming access: loads and stores of data touched once per kernel use the
// non-temporal (nt) cache policy, which on MI355X measured 5-12% more
// bandwidth than the default policy for read-read-write streams.
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld_nt(const float4 *p) {
  const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(float4 *p, float4 v) {
  const v4f w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<v4f *>(p));
}
__device__ __forceinline__ float ld_nt(const float *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_nt(float *p, float v) { __builtin_nontemporal_store(v, p); }

// v from lane dpp(i) of the same row of 16 (kCtrl: a DPP lane pattern).
template <int kCtrl>
__device__ __forceinline__ float dpp_lane(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
constexpr int kDppQuadSwap1 = 0xb1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4e;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror: lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;     // row_mirror: lane i <-> 15 - i within 16

// Sum over the 64 lanes of a wavefront, all lanes active; every lane gets the
// same bits. Within each row of 16 lanes, four DPP steps each add the value
// of a partner lane (partners then hold the same two operands, so the same
// sum); the four row sums are read into scalar registers and added as
// (r0 + r1) + (r2 + r3). No LDS round trips, unlike a shuffle butterfly.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_lane<kDppQuadSwap1>(v);
  v += dpp_lane<kDppQuadSwap2>(v);
  v += dpp_lane<kDppHalfMirror>(v);
  v += dpp_lane<kDppMirror>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Serial float sums in a fixed order (the CPU loops' order), one chain per
// lane, fed from LDS four terms at a time:
// s = (((s + t[0]) + t[1]) + ...) + t[4 n4 - 1] for each of kArr chains, the
// terms of chain a at t[a]; n4 float4 reads per chain, a multiple of 2 kB.
// The reads of a batch (kB float4 per chain) are issued before the additions
// of the batch before, which cover the LDS latency; the scheduling barriers
// keep the compiler from sinking the reads down to their use.
template <int kArr, int kB>
__device__ __forceinline__ void chain_add4(float (&s)[kArr], const float4 *const (&t)[kArr], int n4) {
  float4 a[kArr][kB], b[kArr][kB];
#pragma unroll
  for (int r = 0; r < kArr; r++)
#pragma unroll
    for (int k = 0; k < kB; k++) a[r][k] = t[r][k];
  for (int q = 0; q < n4; q += 2 * kB) {
#pragma unroll
    for (int r = 0; r < kArr; r++)
#pragma unroll
      for (int k = 0; k < kB; k++) b[r][k] = t[r][q + kB + k];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < kB; k++)
#pragma unroll
      for (int r = 0; r < kArr; r++) s[r] = (((s[r] + a[r][k].x) + a[r][k].y) + a[r][k].z) + a[r][k].w;
    __builtin_amdgcn_sched_barrier(0);
    if (q + 2 * kB < n4) {
#pragma unroll
      for (int r = 0; r < kArr; r++)
#pragma unroll
        for (int k = 0; k < kB; k++) a[r][k] = t[r][q + 2 * kB + k];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < kB; k++)
#pragma unroll
      for (int r = 0; r < kArr; r++) s[r] = (((s[r] + b[r][k].x) + b[r][k].y) + b[r][k].z) + b[r][k].w;
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Launchers, one per kernel family. Each validates nothing (ugk_api.hip does)
// and returns the launch status through check_launch.
int launch_residual_forward(float *out, const float *x, const float *y, size_t n);
int launch_residual_backward(float *dx, float *dy, const float *dout, size_t n);
// GELU form: 0 (default) the logistic form through the hardware exponential,
// 1 the glibc-exact tanhf (bit-identical to train_bnn.c).
void set_gelu_exact(int exact);
int gelu_exact();
int launch_gelu_forward(float *out, const float *inp, size_t n);
int launch_gelu_backward(float *dinp, const float *inp, const float *dout, size_t n);
// dinp = gelu'(inp) * dout, as launch_gelu_backward on a dinp of zeros (not read)
int launch_gelu_backward_zero(float *dinp, const float *inp, const float *dout, size_t n);
// Philox ops' softplus/sigmoid: 0 (default) the hardware-transcendental forms,
// 1 the glibc-exact forms of the eps-taking ops.
void set_philox_exact(int exact);
int philox_exact();
// kl_forward's softplus: 0 (default) the hardware-transcendental form where
// sigma is a normal float, 1 the glibc-exact form throughout.
void set_kl_exact(int exact);
int kl_exact();
int launch_bayes_materialize(float *w, const float *mu, const float *rho,
                             const float *eps, size_t n);
int launch_bayes_sample(float *w, float *eps, const float *mu, const float *rho, size_t n,
                        unsigned long long seed, int step);
int launch_bayes_backward(float *dmu, float *drho, const float *dw, const float *eps,
                          const float *rho, size_t n);
int launch_bayes_backward_philox(float *dmu, float *drho, const float *dw, const float *rho,
                                 size_t n, unsigned long long seed, int step);
int launch_kl_backward(float *dmu, float *drho, const float *mu, const float *rho, size_t n,
                       float sigma_prior, float weight);
int launch_adamw(float *params, const float *grads, float *m, float *v, size_t n, float lr,
                 float beta1, float beta2, float eps, float wd, float bc1, float bc2);
int launch_bbb_step_fused(float *mu, float *rho, float *m_mu, float *v_mu, float *m_rho, float *v_rho,
                          float *w, float *dw, size_t n, unsigned long long seed, int step, float sp,
                          float klw, float bc1, float bc2, float lr, float beta1, float beta2,
                          float aeps, float wd);
// KL total into out[0] (device memory, or host memory mapped for the device);
// part holds kl_forward_scratch() bytes.
int launch_kl_forward(double *out, double *part, const float *mu, const float *rho, size_t n,
                      float sigma_prior);
int launch_layernorm_forward(float *out, float *mean, float *rstd, const float *inp,
                             const float *weight, const float *bias, int rows, int C);
int launch_layernorm_backward(float *dinp, float *dweight, float *dbias,
                              const float *dout, const float *inp, const float *weight,
                              const float *mean, const float *rstd, int rows, int C);
// residual_forward then layernorm_forward of its output, in one pass when the
// float4 path applies (two launches otherwise).
int launch_encoder_layernorm_forward(float *enc, float *out, float *mean, float *rstd, const int *inp,
                                     const float *wte, const float *wpe, const float *weight, const float *bias,
                                     int B, int T, int C);
int launch_residual_layernorm_forward(float *res, float *out, float *mean, float *rstd, const float *x,
                                      const float *y, const float *weight, const float *bias, int rows,
                                      int C);
// layernorm_backward then residual_backward(dx, dy, dinp), likewise (dx, dy
// null: layernorm_backward alone).
int launch_layernorm_residual_backward(float *dinp, float *dweight, float *dbias, float *dx, float *dy,
                                       const float *dout, const float *inp, const float *weight,
                                       const float *mean, const float *rstd, int rows, int C);
// The LayerNorm backward split in two: the main pass writes dinp (and, with dx
// non-null, applies residual_backward(dx, dy, dinp)) and *nblk partial rows
// of the dweight/dbias column sums to `partial`; launch_layernorm_reduce then
// adds each job's column totals into its dweight/dbias, many jobs per launch.
struct LnReduceJob {
  const float *partial;
  float *dweight, *dbias;
  int nblk;
};
// What a fused LayerNorm -> residual backward does with its dinp (the
// float4 path; the scalar path always reads and writes it):
enum LnDinp {
  kDinpRw = 0,    // read (the LayerNorm adds to it) and written
  kDinpRead = 1,  // read, not written back (nothing reads it after the residual split)
  kDinpNone = 2,  // neither: taken as +0.0 (the zeroed-gradient driver's first pair)
};
// At most max_blocks partial rows (the float4 path takes up to 1024, the
// scalar path up to 512). With dx non-null, dinp_mode says what happens to
// dinp, and assign_res takes dx and dy as +0.0 instead of reading them (float4
// path; the scalar path reads and writes everything).
int launch_layernorm_backward_partials(float *dinp, float *partial, float *dx, float *dy, const float *dout,
                                       const float *inp, const float *weight, const float *mean,
                                       const float *rstd, int rows, int C, int max_blocks, int *nblk,
                                       int dinp_mode = kDinpRw, bool assign_res = false);
int launch_layernorm_reduce(const LnReduceJob *jobs, int njobs, int C);
// The per-op LayerNorm backward (launch_layernorm_residual_backward_into) on
// the float4 path finishes its column sums in its main launch (1) or in a
// second launch (0, the default); both give the same bits. The step driver always
// batches its column sums in one launch at the end.
void set_layernorm_tail(int on);
int layernorm_tail();
// LayerNorm forward and backward in train_bnn.c's order of every addition (1)
// or the default kernels (0); every LayerNorm entry point and the step driver
// follow it.
void set_layernorm_exact(int on);
int layernorm_exact();
int launch_layernorm_forward_exact(float *out, float *mean, float *rstd, const float *inp, const float *weight,
                                   const float *bias, int rows, int C);
int launch_layernorm_backward_exact(float *dinp, float *dweight, float *dbias, const float *dout, const float *inp,
                                    const float *weight, const float *mean, const float *rstd, int rows, int C);
// Both passes with the partial rows in `partial` (room for max_blocks rows of
// 2C floats; every shape takes at most max_blocks), not in the workspace.
int launch_layernorm_residual_backward_into(float *partial, int max_blocks, float *dinp, float *dweight,
                                            float *dbias, float *dx, float *dy, const float *dout,
                                            const float *inp, const float *weight, const float *mean,
                                            const float *rstd, int rows, int C);
// Partial rows one call writes with at most max_blocks of them.
int layernorm_backward_blocks(int rows, int C, bool res, int max_blocks);
// An upper bound on the partial rows of every call with at most `rows` rows
// and C channels (any path, plain or fused), which sizes the workspace.
int layernorm_backward_blocks_bound(int rows, int C);
constexpr int kMaxScalarBlocks = 512;
constexpr int kMaxPartialRows = 1024;  // partial rows the column-sum kernel takes per call
// The allocation-free LayerNorm backward's partial rows live in a file-scope
// device array of this size (one per GPU); noalloc_scratch() is its device
// address on the current device (nullptr with the error set if the lookup
// failed), noalloc_max_blocks(C) the partial rows of C channels it holds.
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
float *noalloc_scratch();
int noalloc_max_blocks(int C);
int launch_softmax_crossentropy(float *losses, float *probs, const float *logits, const int *targets, int rows,
                                int V);
int launch_crossentropy_softmax_backward(float *dlogits, const float *probs, const int *targets, int rows, int V,
                                         float dloss,
                                         bool zeroed = false);
int launch_encoder_forward(float *out, const int *inp, const float *wte,
                           const float *wpe, int B, int T, int C);
int launch_encoder_backward(float *dwte, float *dwpe, const float *dout,
                            const int *inp, int B, int T, int C);
// Buckets of more than 32 rows: 0 (default) blocked adds (64-row blocks, each
// in row order, the block sums in block order), 1 one add per row in row
// order (bit-identical to train_bnn.c).
void set_encoder_exact(int exact);
int encoder_exact();
// Clears the encoder backward's bucket state at mem (encoder_backward_scratch()
// bytes) on the library stream: new memory must be cleared once before the
// first call uses it.
int launch_encoder_state_init(void *mem);
// ids[i] outside [0, bound) are replaced by fill, and `code` is stored in the
// per-device id error word (ids_error_word()).
int launch_ids_guard(int *ids, int n, int bound, int fill, int code);
// Device address of the current device's id error word (nullptr with the
// error set if its lookup failed).
int *ids_error_word();

// Workspace sizes.
size_t layernorm_backward_scratch(int rows, int C);  // bytes of one call's partial rows
size_t encoder_backward_scratch();                   // the bucket state (fixed)
size_t kl_forward_scratch();                         // partial sums (fixed)
size_t softmax_scratch(int rows, int V);             // row statistics: long rows, and the exact mode
// softmax's row sum: 0 (default) a fixed tree, 1 train_bnn.c's serial order
void set_softmax_exact(int exact);
int softmax_exact();

}  // namespace ugk
