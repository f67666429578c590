// ugk_softmax.hip - the row ops at the head of the network: softmax +
// cross-entropy forward (train_bnn.c:279-304) and its backward
// (train_bnn.c:358-378).
//
// Forward: one workgroup per (b,t) row of V logits. Each thread keeps its
// kPer logits (v = tid, tid + kThreads, ...) in registers, so the row is read
// from HBM once and the probabilities written once (8 bytes per logit):
//   max   thread-local `x > m ? x : m` from -1e30 (the CPU loop's rule), then
//         a wavefront butterfly and the block's wavefronts through LDS;
//   exp   e = expf(x - max) with the glibc-exact expf (the CPU's values);
//   sum   thread-local in v order, wavefront butterfly, wavefronts in order
//         (a fixed tree: deterministic, within float rounding of the CPU's
//         sequential sum);
//   prob  e / sum with IEEE division, stored non-temporally;
//   loss  -log(prob[target]) by the owning thread, from the same register.
// Rows are V floats long and V is odd for GPT-2, so rows are not 16-byte
// aligned: loads and stores are dwords, coalesced across the wavefront.
// Rows longer than kThreads * kMaxPer take a three-pass kernel that re-reads
// the logits from memory.
//
// Backward: dlogits[v] += (probs[v] - (v == target)) * (1 / (B*T)), a map
// over a (row, column block) grid; bit-identical to the CPU loop.
#include "ugk_internal.h"
#include "ugk_libm_dev.h"

namespace ugk {
namespace {

constexpr float kNegInit = -1e30f;  // train_bnn.c:287

__device__ __forceinline__ float max_rule(float m, float x) { return x > m ? x : m; }

template <int kThreads>
__device__ __forceinline__ float block_max(float v, float *lds) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = max_rule(v, __shfl_xor(v, off));
  constexpr int kW = kThreads / kWave;
  if (kW == 1) return v;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  float m = lds[0];
#pragma unroll
  for (int w = 1; w < kW; w++) m = max_rule(m, lds[w]);
  __syncthreads();
  return m;
}

template <int kThreads>
__device__ __forceinline__ float block_sum(float v, float *lds) {
  v = wave_sum(v);
  constexpr int kW = kThreads / kWave;
  if (kW == 1) return v;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  float s = lds[0];
#pragma unroll
  for (int w = 1; w < kW; w++) s += lds[w];
  __syncthreads();
  return s;
}

// -logf(p), from the double logarithm rounded to float (the correctly rounded
// logf but for astronomically rare ties; glibc's logf agrees with it on
// 99.8% of inputs).
__device__ __forceinline__ float neg_logf(float p) { return -(float)log((double)p); }

template <int kThreads, int kPer>
__global__ __launch_bounds__(kThreads) void k_softmax_xent(float *__restrict__ losses, float *__restrict__ probs,
                                                           const float *__restrict__ logits,
                                                           const int *__restrict__ targets, int V) {
  __shared__ uint64_t tab[32];
  __shared__ float lds[kThreads / kWave];
  ugk_exp2_stage(tab);
  const size_t row = blockIdx.x;
  const float *lg = logits + row * (size_t)V;
  float *pr = probs + row * (size_t)V;
  const int tid = threadIdx.x;
  float x[kPer];
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    const int v = tid + k * kThreads;
    x[k] = v < V ? ld_nt(lg + v) : kNegInit;
  }
  float m = kNegInit;
#pragma unroll
  for (int k = 0; k < kPer; k++) m = max_rule(m, x[k]);
  __syncthreads();  // tab staged
  m = block_max<kThreads>(m, lds);
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    const int v = tid + k * kThreads;
    x[k] = ugk_expf_t<UGK_EXPF_CONTRACT>(x[k] - m, UgkExp2Lds{tab});
    if (v < V) s += x[k];
  }
  s = block_sum<kThreads>(s, lds);
  const int tgt = targets[row];
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    const int v = tid + k * kThreads;
    if (v < V) {
      const float p = x[k] / s;
      st_nt(pr + v, p);
      if (v == tgt) losses[row] = neg_logf(p);
    }
  }
}

// Any V: three passes over the row in memory (max; exp and sum, e stored;
// divide), one workgroup per row.
constexpr int kLongThreads = 1024;
__global__ __launch_bounds__(kLongThreads) void k_softmax_xent_long(float *losses, float *probs,
                                                                    const float *logits, const int *targets,
                                                                    int V) {
  __shared__ uint64_t tab[32];
  __shared__ float lds[kLongThreads / kWave];
  ugk_exp2_stage(tab);
  const size_t row = blockIdx.x;
  const float *lg = logits + row * (size_t)V;
  float *pr = probs + row * (size_t)V;
  float m = kNegInit;
  for (int v = threadIdx.x; v < V; v += kLongThreads) m = max_rule(m, lg[v]);
  __syncthreads();
  m = block_max<kLongThreads>(m, lds);
  float s = 0.0f;
  for (int v = threadIdx.x; v < V; v += kLongThreads) {
    const float e = ugk_expf_t<UGK_EXPF_CONTRACT>(lg[v] - m, UgkExp2Lds{tab});
    pr[v] = e;
    s += e;
  }
  s = block_sum<kLongThreads>(s, lds);
  const int tgt = targets[row];
  for (int v = threadIdx.x; v < V; v += kLongThreads) {
    const float p = pr[v] / s;
    pr[v] = p;
    if (v == tgt) losses[row] = neg_logf(p);
  }
}

constexpr int kBwdThreads = 256, kBwdPer = 4;
__global__ __launch_bounds__(kBwdThreads) void k_xent_softmax_bwd(float *__restrict__ dlogits,
                                                                  const float *__restrict__ probs,
                                                                  const int *__restrict__ targets, int V,
                                                                  float dloss) {
  const size_t row = blockIdx.x;
  const int tgt = targets[row];
  const size_t base = row * (size_t)V;
  const int v0 = blockIdx.y * (kBwdThreads * kBwdPer) + threadIdx.x;
  float p[kBwdPer], d[kBwdPer];
#pragma unroll
  for (int k = 0; k < kBwdPer; k++) {
    const int v = v0 + k * kBwdThreads;
    if (v < V) {
      p[k] = ld_nt(probs + base + v);
      d[k] = ld_nt(dlogits + base + v);
    }
  }
#pragma unroll
  for (int k = 0; k < kBwdPer; k++) {
    const int v = v0 + k * kBwdThreads;
    if (v < V) {
      const float indicator = (v == tgt) ? 1.0f : 0.0f;
      st_nt(dlogits + base + v, d[k] + (p[k] - indicator) * dloss);
    }
  }
}

template <int kThreads, int kPer>
void launch_rows(float *losses, float *probs, const float *logits, const int *targets, int rows, int V) {
  hipLaunchKernelGGL((k_softmax_xent<kThreads, kPer>), dim3(rows), dim3(kThreads), 0, stream(), losses, probs,
                     logits, targets, V);
}

}  // namespace

int launch_softmax_crossentropy(float *losses, float *probs, const float *logits, const int *targets, int rows,
                                int V) {
  if (rows == 0 || V == 0) return 0;
  if (V <= 64) launch_rows<64, 1>(losses, probs, logits, targets, rows, V);
  else if (V <= 256) launch_rows<64, 4>(losses, probs, logits, targets, rows, V);
  else if (V <= 1024) launch_rows<256, 4>(losses, probs, logits, targets, rows, V);
  else if (V <= 4096) launch_rows<1024, 4>(losses, probs, logits, targets, rows, V);
  else if (V <= 16384) launch_rows<1024, 16>(losses, probs, logits, targets, rows, V);
  else if (V <= 32768) launch_rows<1024, 32>(losses, probs, logits, targets, rows, V);
  else if (V <= 51200) launch_rows<1024, 50>(losses, probs, logits, targets, rows, V);
  else
    hipLaunchKernelGGL(k_softmax_xent_long, dim3(rows), dim3(kLongThreads), 0, stream(), losses, probs, logits,
                       targets, V);
  return check_launch("softmax_crossentropy");
}

int launch_crossentropy_softmax_backward(float *dlogits, const float *probs, const int *targets, int rows, int V,
                                         float dloss) {
  if (rows == 0 || V == 0) return 0;
  const dim3 grid(rows, grid_for((size_t)V, (size_t)kBwdThreads * kBwdPer));
  hipLaunchKernelGGL(k_xent_softmax_bwd, grid, dim3(kBwdThreads), 0, stream(), dlogits, probs, targets, V, dloss);
  return check_launch("crossentropy_softmax_backward");
}

}  // namespace ugk
