// ugk_softmax.hip - the row ops at the head of the network: softmax +
// cross-entropy forward (train_bnn.c:279-304) and its backward
// (train_bnn.c:358-378).
//
// Forward: one workgroup per (b,t) row of V logits. Each thread keeps its
// kPer logits (v = tid, tid + kThreads, ...) in registers, so the row is read
// from HBM once and the probabilities written once (8 bytes per logit):
//   max   thread-local `x > m ? x : m` from -1e30 (the CPU loop's rule), then
//         a wavefront butterfly and the block's wavefronts through LDS;
//   exp   e = expf(x - max) with the glibc-exact expf (the CPU's values),
//         in its branch-free form for arguments <= 0;
//   sum   thread-local in v order, a wavefront sum (DPP), wavefronts in order
//         (a fixed tree: deterministic, within float rounding of the CPU's
//         sequential sum);
//   prob  e / sum correctly rounded, from the reciprocal of the sum and one
//         fma correction (ugk_div_recip; a wavefront holding an e below
//         2^-86 divides instead), stored non-temporally;
//   loss  -logf(prob[target]) (glibc's logf, restated) by the thread holding
//         the target, which recomputes that probability from the logit.
// Rows are V floats long and V is odd for GPT-2, so rows are not 16-byte
// aligned: loads and stores are dwords, coalesced across the wavefront.
// A row's elements are laid on the threads from a 256-byte boundary of probs
// so that stores fill whole lines. Rows of up to 32,705 logits fit in the
// registers of one workgroup; rows of up to 51,393 (GPT-2's 50257) keep 42
// slots per thread in registers and 25 in LDS (768 threads), two rows resident
// per CU so that one row's loads overlap the other's arithmetic and stores
// (k_softmax_xent_split). Longer rows take two passes
// instead: one wavefront per row streams the logits once for the exact max
// and the sum (kept per lane in double and rescaled as the max grows), then a
// flat map over all rows forms expf(x - max) / sum, 12 bytes per logit.
//
// Exact mode (ugk_set_softmax_exact): the row sum in train_bnn.c's order, one
// element after another, so that every probability and loss is the CPU's bit
// for bit (the kernels after the backward's).
//
// Backward: dlogits[v] += (probs[v] - (v == target)) * (1 / (B*T)), one
// workgroup per row streaming float4 (dwords for misaligned arrays);
// bit-identical to the CPU loop.
#include <atomic>
#include <type_traits>

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

// -logf(p) with glibc's logf (train_bnn.c:301), restated in ugk_libm.h.
__device__ __forceinline__ float neg_logf(float p) { return -ugk_logf(p); }

// The loss of a row held in slots (element v in slot v + skew, slot u on
// thread u % threads): the thread holding the target recomputes its
// probability from the logit, with the same expf and the correctly rounded
// quotient the stores hold, and writes -log of it.
__device__ __forceinline__ void store_loss(float *losses, size_t row, const float *lg, int tgt, int skew, float m,
                                           float s, const uint64_t *tab, int threads) {
  if ((int)threadIdx.x == (tgt + skew) % threads)
    losses[row] = neg_logf(ugk_dev_expf_nooverflow(lg[tgt] - m, UgkExp2Lds{tab}, UgkExpfAddends{}) / s);
}

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
  // Slot u of the row holds element v = u - skew, where skew places u = 0 on a
  // 256-byte boundary of probs: every wavefront then stores whole 256-byte
  // spans (a misaligned row's stores would write partial cache lines).
  const int skew = (int)(((uintptr_t)pr >> 2) & 63);
  const int tid = threadIdx.x;
  float x[kPer];
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    const int v = tid + k * kThreads - skew;
    x[k] = (v >= 0 && v < V) ? ld_nt(lg + v) : kNegInit;
  }
  float m = kNegInit;
#pragma unroll
  for (int k = 0; k < kPer; k++) m = max_rule(m, x[k]);
  __syncthreads();  // tab staged
  m = block_max<kThreads>(m, lds);
  float s = 0.0f;
  uint32_t lo = 0xffffffffu;
  const UgkExpfAddends add = ugk_expf_addends_vgpr();
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    const int v = tid + k * kThreads - skew;
    x[k] = ugk_dev_expf_nooverflow(x[k] - m, UgkExp2Lds{tab}, add);
    lo = min(lo, ugk_div_recip_key(x[k]));
    if (v >= 0 && v < V) s += x[k];
  }
  s = block_sum<kThreads>(s, lds);
  const float y = 1.0f / s;
  auto store = [&](auto recip) {
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const int v = tid + k * kThreads - skew;
      if (v >= 0 && v < V) st_nt(pr + v, decltype(recip)::value ? ugk_div_recip(x[k], s, y) : x[k] / s);
    }
  };
  if (__all(lo >= kUgkDivRecipKeyMin)) store(std::true_type{});
  else store(std::false_type{});
  store_loss(losses, row, lg, targets[row], skew, m, s, tab, kThreads);
}

// The same row computation for rows of up to 51,393 logits, with two rows
// resident per CU: each thread keeps kReg slots in registers (the bound of 8
// wavefronts per SIMD caps it at 64 VGPRs, so two 1024-thread workgroups fit a
// CU) and kLds slots in LDS, which
// global_load_lds fills straight from memory without passing through
// registers. Slots are visited in the same order (registers, then LDS), so
// every value, the sums included, is bit-identical to k_softmax_xent's with
// the same thread count.
template <int kThreads, int kReg, int kLds>
__global__ __launch_bounds__(kThreads, 2 * kThreads / kWave / 4) void k_softmax_xent_split(
    float *__restrict__ losses, float *__restrict__ probs, const float *__restrict__ logits,
    const int *__restrict__ targets, int V) {
  // one LDS block with the expf table first, so that its address fits the
  // offset field of the table reads
  __shared__ struct {
    uint64_t tab[32];
    float lds[kThreads / kWave];
    float part[kLds * kThreads];
  } sh;
  uint64_t *tab = sh.tab;
  float *lds = sh.lds, *part = sh.part;
  ugk_exp2_stage(tab);
  const size_t row = blockIdx.x;
  const float *lg = logits + row * (size_t)V;
  float *pr = probs + row * (size_t)V;
  const int skew = (int)(((uintptr_t)pr >> 2) & 63);  // as in k_softmax_xent
  const int tid = threadIdx.x, wave = tid / kWave;
  const int v0 = tid - skew;  // element of slot tid; slot tid + k * kThreads holds v0 + k * kThreads
  // Slots outside the row hold -inf: the max rule skips it and expf gives +0,
  // which leaves the sum's bits unchanged, so only the loads and stores test
  // for the row's bounds (registers stay within the 2-rows-per-CU budget).
  const float kNegInf = -__builtin_huge_valf();
#pragma unroll 1
  for (int k = 0; k < kLds; k++) {
    const int v = v0 + (kReg + k) * kThreads;
    if ((unsigned)v < (unsigned)V)  // lane i of the wavefront lands at part[base + i]; nt as the other loads
      __builtin_amdgcn_global_load_lds(lg + v, part + k * kThreads + wave * kWave, 4, 0, 2);
    else
      part[k * kThreads + tid] = kNegInf;
  }
  // Rows are longer than the register slots (V >= kReg * kThreads, checked at
  // launch), so only slot 0 can fall outside the row, below its start. Its
  // load reads element 0 there instead and the value is replaced afterwards:
  // a load under a branch would make the wait for it, at the branch's end,
  // wait for every load issued before it as well, and the other register
  // slots would then be loaded only after the LDS slots had arrived.
  float x[kReg];
#pragma unroll
  for (int k = 0; k < kReg; k++) {
    const int v = v0 + k * kThreads;
    x[k] = ld_nt(lg + (k > 0 ? v : max(v, 0)));
  }
  if (v0 < 0) x[0] = kNegInf;
  float m = kNegInit;
#pragma unroll
  for (int k = 0; k < kReg; k++) m = max_rule(m, x[k]);
  __syncthreads();  // tab staged, LDS slots filled
#pragma unroll 1
  for (int k = 0; k < kLds; k++) m = max_rule(m, part[k * kThreads + tid]);
  m = block_max<kThreads>(m, lds);
  float s = 0.0f;
  uint32_t lo = 0xffffffffu;
  const UgkExpfAddends add = ugk_expf_addends_vgpr();
#pragma unroll
  for (int k = 0; k < kReg; k++) {
    x[k] = ugk_dev_expf_nooverflow(x[k] - m, UgkExp2Lds{tab}, add);
    s += x[k];
    lo = min(lo, ugk_div_recip_key(x[k]));
  }
#pragma unroll 1
  for (int k = 0; k < kLds; k++) {
    const float e = ugk_dev_expf_nooverflow(part[k * kThreads + tid] - m, UgkExp2Lds{tab}, add);
    part[k * kThreads + tid] = e;
    s += e;
    lo = min(lo, ugk_div_recip_key(e));
  }
  s = block_sum<kThreads>(s, lds);
  const float y = 1.0f / s;
  // a fresh copy of v0: the compiler would otherwise keep every slot's index
  // (and bounds test) alive from the loads to the stores, past the budget
  int vs = v0;
  asm volatile("" : "+v"(vs));
  auto store = [&](auto recip) {
    auto div = [&](float e) { return decltype(recip)::value ? ugk_div_recip(e, s, y) : e / s; };
#pragma unroll
    for (int k = 0; k < kReg; k++) {
      const int v = vs + k * kThreads;
      if (k > 0 || v >= 0) st_nt(pr + v, div(x[k]));
    }
#pragma unroll 1
    for (int k = 0; k < kLds; k++) {
      const int v = vs + (kReg + k) * kThreads;
      if ((unsigned)v < (unsigned)V) st_nt(pr + v, div(part[k * kThreads + tid]));
    }
  };
  if (__all(lo >= kUgkDivRecipKeyMin)) store(std::true_type{});
  else store(std::false_type{});
  store_loss(losses, row, lg, targets[row], skew, m, s, tab, kThreads);
}

// Row of flat element i (rows of V elements): a double-precision quotient,
// then exact integer correction (the estimate is off by at most one).
__device__ __forceinline__ size_t row_of(size_t i, size_t V, double inv_v) {
  size_t r = (size_t)((double)i * inv_v);
  if (r * V > i) r--;
  else if ((r + 1) * V <= i) r++;
  return r;
}

// Long rows, pass 1: one wavefront per row streams its logits once and keeps,
// per lane, the running max (the CPU's rule, from -1e30) and the sum of
// exp(x - running max) in double, rescaled when the max grows; the lanes are
// then combined onto the row max. stats[row] = {max, sum}. The max is exact;
// the sum is within float rounding of the exact sum of expf(x - max).
constexpr int kStatsWaves = 4, kStatsUnroll = 8;
__global__ __launch_bounds__(kStatsWaves * kWave) void k_softmax_stats(float2 *__restrict__ stats,
                                                                       const float *__restrict__ logits, int rows,
                                                                       int V) {
  __shared__ uint64_t tab[32];
  ugk_exp2_stage(tab);
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * kStatsWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float *lg = logits + (size_t)row * V;
  float m = kNegInit;
  double s = 0.0;
  for (int v0 = lane; v0 < V; v0 += kWave * kStatsUnroll) {
    float x[kStatsUnroll];
#pragma unroll
    for (int k = 0; k < kStatsUnroll; k++) {
      const int v = v0 + k * kWave;
      x[k] = v < V ? ld_nt(lg + v) : kNegInit;
    }
    float mb = m;
#pragma unroll
    for (int k = 0; k < kStatsUnroll; k++) mb = max_rule(mb, x[k]);
    if (mb != m) {  // rescale the running sum to the new max
      s *= (double)ugk_expf_t<UGK_EXPF_CONTRACT>(m - mb, UgkExp2Lds{tab});
      m = mb;
    }
#pragma unroll
    for (int k = 0; k < kStatsUnroll; k++)
      if (v0 + k * kWave < V) s += (double)ugk_expf_t<UGK_EXPF_CONTRACT>(x[k] - m, UgkExp2Lds{tab});
  }
  float M = m;
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) M = max_rule(M, __shfl_xor(M, off));
  s *= (double)ugk_expf_t<UGK_EXPF_CONTRACT>(m - M, UgkExp2Lds{tab});
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (lane == 0) stats[row] = make_float2(M, (float)s);
}

// Long rows, pass 2: a flat map over all rows x V: p = expf(x - max) / sum,
// and the thread holding a row's target writes its loss.
constexpr int kNormUnroll = 4;
__global__ __launch_bounds__(kBlock) void k_softmax_norm(float *__restrict__ losses, float *__restrict__ probs,
                                                         const float *__restrict__ logits,
                                                         const int *__restrict__ targets,
                                                         const float2 *__restrict__ stats, size_t n, int V,
                                                         double inv_v) {
  __shared__ uint64_t tab[32];
  ugk_exp2_stage(tab);
  __syncthreads();
  const size_t i0 = (size_t)blockIdx.x * (kBlock * kNormUnroll) + threadIdx.x;
  float x[kNormUnroll];
#pragma unroll
  for (int k = 0; k < kNormUnroll; k++) {
    const size_t i = i0 + (size_t)k * kBlock;
    x[k] = i < n ? ld_nt(logits + i) : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < kNormUnroll; k++) {
    const size_t i = i0 + (size_t)k * kBlock;
    if (i < n) {
      const size_t row = row_of(i, (size_t)V, inv_v);
      const float2 st = stats[row];
      const float p = ugk_expf_t<UGK_EXPF_CONTRACT>(x[k] - st.x, UgkExp2Lds{tab}) / st.y;
      st_nt(probs + i, p);
      if ((int)(i - row * (size_t)V) == targets[row]) losses[row] = neg_logf(p);
    }
  }
}

// Backward over the flat rows x V array, float4 at a time when both arrays
// start 16-byte aligned (their element offsets agree): each float4 spans at
// most two rows (V >= 4), so it looks up two targets.
// kZero: dlogits is taken as +0.0 instead of read (callers that zero it before
// the call); +0.0 + x gives the bits the read of a zero would give.
constexpr int kBwdThreads = 256, kBwdUnroll = 1;  // measured best: 764 against 846 us with 2 at 8,192 x 50,257
template <bool kZero>
__global__ __launch_bounds__(kBwdThreads) void k_xent_softmax_bwd_flat4(float *__restrict__ dlogits,
                                                                        const float *__restrict__ probs,
                                                                        const int *__restrict__ targets, int rows,
                                                                        int V, float dloss, size_t n4,
                                                                        double inv_v) {
  const float4 *p4 = reinterpret_cast<const float4 *>(probs);
  float4 *d4 = reinterpret_cast<float4 *>(dlogits);
  const size_t q0 = (size_t)blockIdx.x * (kBwdThreads * kBwdUnroll) + threadIdx.x;
  float4 p[kBwdUnroll], d[kBwdUnroll];
#pragma unroll
  for (int k = 0; k < kBwdUnroll; k++) {
    const size_t q = q0 + (size_t)k * kBwdThreads;
    if (q < n4) {
      p[k] = ld_nt(p4 + q);
      d[k] = kZero ? make_float4(0.0f, 0.0f, 0.0f, 0.0f) : ld_nt(d4 + q);
    }
  }
#pragma unroll
  for (int k = 0; k < kBwdUnroll; k++) {
    const size_t q = q0 + (size_t)k * kBwdThreads;
    if (q < n4) {
      const size_t i = 4 * q;
      const size_t r0 = row_of(i, (size_t)V, inv_v);
      const size_t t0 = r0 * (size_t)V + (size_t)targets[r0];
      const size_t t1 = (r0 + 1 < (size_t)rows) ? (r0 + 1) * (size_t)V + (size_t)targets[r0 + 1] : ~(size_t)0;
      float4 o;
      o.x = d[k].x + (p[k].x - ((i == t0 || i == t1) ? 1.0f : 0.0f)) * dloss;
      o.y = d[k].y + (p[k].y - ((i + 1 == t0 || i + 1 == t1) ? 1.0f : 0.0f)) * dloss;
      o.z = d[k].z + (p[k].z - ((i + 2 == t0 || i + 2 == t1) ? 1.0f : 0.0f)) * dloss;
      o.w = d[k].w + (p[k].w - ((i + 3 == t0 || i + 3 == t1) ? 1.0f : 0.0f)) * dloss;
      st_nt(d4 + q, o);
    }
  }
}

// Any alignment: dwords, a (row, column block) grid.
constexpr int kBwdPer = 4;
template <bool kZero>
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
      d[k] = kZero ? 0.0f : ld_nt(dlogits + base + v);
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

// ---- exact mode: train_bnn.c's order of the row sum ---------------------------
// train_bnn.c:286-297 takes the row max (any order gives the same value: the
// rule x > m from -1e30 skips NaN, and the sign of a zero max does not change
// x - max), adds expf(x - max) for v = 0, 1, ..., V-1 one at a time, divides
// each exponential by that sum and takes -logf of the target's quotient. The
// exact form keeps that order in three launches:
//   k_softmax_rowmax: one wavefront per row, the max by the CPU's rule;
//   k_softmax_sum_exact: a workgroup per 32 rows, one serial chain per row in
//     wavefront 0 (lanes 0-31) fed from LDS, four terms per read, by fifteen
//     loader wavefronts that stage 240-column tiles of expf(x - max) (the
//     glibc-exact expf) three tiles ahead in registers; the columns past V are
//     staged as +0, which leaves a sum of terms >= +0 (or NaN, inf) unchanged;
//   k_softmax_norm_rows: expf(x - max) / sum (IEEE division) and the loss.
// Its HBM bytes: the logits three times and the probabilities once (16 per
// logit, against 8 for the default kernels); the chains' latency bounds the
// sums.
constexpr int kSxLoaders = 15, kSxThreads = (kSxLoaders + 1) * kWave, kSxLoadLanes = kSxLoaders * kWave;
constexpr int kSxRows = 32, kSxTile = 240, kSxPitch = kSxTile + 4;
constexpr int kSxSlots = kSxRows * kSxTile / kSxLoadLanes;
constexpr int kSxDepth = 3, kSxBatch = 6;
constexpr int kSxMaxWaves = 4, kSxMaxUnroll = 8;
constexpr int kSxNormPer = 16;
static_assert(kSxRows * kSxTile == kSxSlots * kSxLoadLanes && kSxLoadLanes % kSxTile == 0,
              "a tile is whole loader slots, and a loader lane keeps its column in every slot");
static_assert((kSxTile / 4) % (2 * kSxBatch) == 0 && kSxRows <= kWave, "whole batch pairs per tile; chains in one wave");

__global__ __launch_bounds__(kSxMaxWaves * kWave) void k_softmax_rowmax(float2 *__restrict__ stats,
                                                                        const float *__restrict__ logits, int rows,
                                                                        int V) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * kSxMaxWaves + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float *lg = logits + (size_t)row * V;
  float m = kNegInit;
  for (int v0 = lane; v0 < V; v0 += kWave * kSxMaxUnroll) {
    float x[kSxMaxUnroll];
#pragma unroll
    for (int k = 0; k < kSxMaxUnroll; k++) {
      const int v = v0 + k * kWave;
      x[k] = v < V ? lg[v] : kNegInit;
    }
#pragma unroll
    for (int k = 0; k < kSxMaxUnroll; k++) m = max_rule(m, x[k]);
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) m = max_rule(m, __shfl_xor(m, off));
  if (lane == 0) stats[row] = make_float2(m, 0.0f);
}

__global__ __launch_bounds__(kSxThreads) void k_softmax_sum_exact(float2 *__restrict__ stats,
                                                                  const float *__restrict__ logits, int rows, int V) {
  __shared__ __align__(16) float tile[2][kSxRows * kSxPitch];
  __shared__ uint64_t tab[32];
  __shared__ float smax[kSxRows];
  ugk_exp2_stage(tab);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
  const int r0 = blockIdx.x * kSxRows;
  if ((int)threadIdx.x < kSxRows) smax[threadIdx.x] = stats[min(r0 + (int)threadIdx.x, rows - 1)].x;
  __syncthreads();
  const int nt = (V + kSxTile - 1) / kSxTile;
  // loader lane L holds, in slot sl, tile row L / 240 + 4 sl, column L % 240
  const int L = (wave - 1) * kWave + lane;
  const int rb = L / kSxTile, c = L - rb * kSxTile;
  constexpr int kRowStep = kSxLoadLanes / kSxTile;
  const UgkExpfAddends add = ugk_expf_addends_vgpr();
  float reg[kSxDepth][kSxSlots];
  auto load_tile = [&](int t, int k) {
    const int col = min(t * kSxTile + c, V - 1);
#pragma unroll
    for (int sl = 0; sl < kSxSlots; sl++) {
      const int row = min(r0 + rb + kRowStep * sl, rows - 1);
      reg[k][sl] = logits[(size_t)row * V + col];
    }
  };
  auto store_tile = [&](int t, int k) {
    float *const T = tile[t & 1];
    const bool in = t * kSxTile + c < V;
#pragma unroll
    for (int sl = 0; sl < kSxSlots; sl++) {
      const int r = rb + kRowStep * sl;
      T[r * kSxPitch + c] = in ? ugk_dev_expf_nooverflow(reg[k][sl] - smax[r], UgkExp2Lds{tab}, add) : 0.0f;
    }
  };
  float acc[1] = {0.0f};
  if (wave > 0) {
#pragma unroll
    for (int k = 0; k < kSxDepth; k++)
      if (k < nt) load_tile(k, k);
  }
  for (int t0 = 0; t0 < nt; t0 += kSxDepth) {
#pragma unroll
    for (int k = 0; k < kSxDepth; k++) {
      const int t = t0 + k;
      if (t >= nt) break;  // the same in every thread
      if (wave > 0) {
        store_tile(t, k);
        if (t + kSxDepth < nt) load_tile(t + kSxDepth, k);
      }
      // tile t is staged in buffer t & 1; the buffer written next round was
      // last read before this barrier
      __syncthreads();
      if (wave == 0) {
        const float4 *t4[1] = {reinterpret_cast<const float4 *>(tile[t & 1] + (lane & (kSxRows - 1)) * kSxPitch)};
        chain_add4<1, kSxBatch>(acc, t4, kSxTile / 4);
      }
    }
  }
  if (wave == 0 && lane < kSxRows && r0 + lane < rows) stats[r0 + lane] = make_float2(smax[lane], acc[0]);
}

// grid: rows x chunks of kBlock * kSxNormPer logits, the chunks of a row
// adjacent and laid from the 256-byte boundary of probs at or before the
// row's start, so that each wavefront's store covers whole lines
__global__ __launch_bounds__(kBlock) void k_softmax_norm_rows(float *__restrict__ losses, float *__restrict__ probs,
                                                              const float *__restrict__ logits,
                                                              const int *__restrict__ targets,
                                                              const float2 *__restrict__ stats, int V, int chunks) {
  __shared__ uint64_t tab[32];
  ugk_exp2_stage(tab);
  __syncthreads();
  const int row = (int)(blockIdx.x / (unsigned)chunks);
  const size_t base = (size_t)row * V;
  const int skew = (int)((reinterpret_cast<uintptr_t>(probs + base) >> 2) & 63);
  const int v0 = (int)(blockIdx.x - (unsigned)row * chunks) * (kBlock * kSxNormPer) + (int)threadIdx.x - skew;
  const float2 st = stats[row];
  const int tgt = targets[row];
  float x[kSxNormPer];
#pragma unroll
  for (int k = 0; k < kSxNormPer; k++) {
    const int v = v0 + k * kBlock;
    x[k] = (unsigned)v < (unsigned)V ? ld_nt(logits + base + v) : 0.0f;
  }
  const UgkExpfAddends add = ugk_expf_addends_vgpr();
  uint32_t lo = 0xffffffffu;
#pragma unroll
  for (int k = 0; k < kSxNormPer; k++) {
    x[k] = (unsigned)(v0 + k * kBlock) < (unsigned)V ? ugk_dev_expf_nooverflow(x[k] - st.x, UgkExp2Lds{tab}, add)
                                                      : 0.0f;
    lo = min(lo, ugk_div_recip_key(x[k]));
  }
  // e / sum: the reciprocal form where it is the IEEE quotient (a sum in
  // [1, 2^16], every e of the thread +0, NaN or in [2^-86, 1]), else division
  const float y = 1.0f / st.y;
  auto store = [&](auto recip) {
#pragma unroll
    for (int k = 0; k < kSxNormPer; k++) {
      const int v = v0 + k * kBlock;
      if ((unsigned)v < (unsigned)V) {
        const float p = decltype(recip)::value ? ugk_div_recip(x[k], st.y, y) : x[k] / st.y;
        st_nt(probs + base + v, p);
        if (v == tgt) losses[row] = neg_logf(p);
      }
    }
  };
  if (st.y >= 1.0f && st.y <= 0x1p16f && lo >= kUgkDivRecipKeyMin)
    store(std::true_type{});
  else
    store(std::false_type{});
}

std::atomic<int> g_softmax_exact{0};

template <int kThreads, int kPer>
void launch_rows(float *losses, float *probs, const float *logits, const int *targets, int rows, int V) {
  hipLaunchKernelGGL((k_softmax_xent<kThreads, kPer>), dim3(rows), dim3(kThreads), 0, stream(), losses, probs,
                     logits, targets, V);
}

}  // namespace

// Rows of more than kSplitMaxV logits take the two-pass form, whose row
// statistics live in the workspace.
constexpr int kSplitSlots = 768 * (42 + 25);
constexpr int kSplitMaxV = kSplitSlots - 63;

// The row statistics of the two-pass form and of the exact mode (whichever
// form the calls take, so that a workspace sized once serves both).
size_t softmax_scratch(int rows, int V) { return V > 0 ? (size_t)rows * sizeof(float2) : 0; }

void set_softmax_exact(int on) { g_softmax_exact.store(on ? 1 : 0); }
int softmax_exact() { return g_softmax_exact.load(); }

int launch_softmax_crossentropy(float *losses, float *probs, const float *logits, const int *targets, int rows,
                                int V) {
  if (rows == 0 || V == 0) return 0;
  if (softmax_exact()) {
    float2 *stats = static_cast<float2 *>(workspace(kRegSoftmax, softmax_scratch(rows, V)));
    if (!stats) return UGK_ENOMEM;
    hipLaunchKernelGGL(k_softmax_rowmax, dim3(grid_for((size_t)rows, kSxMaxWaves)), dim3(kSxMaxWaves * kWave), 0,
                       stream(), stats, logits, rows, V);
    hipLaunchKernelGGL(k_softmax_sum_exact, dim3(grid_for((size_t)rows, kSxRows)), dim3(kSxThreads), 0, stream(),
                       stats, logits, rows, V);
    const int chunks = (int)grid_for((size_t)V + 63, (size_t)kBlock * kSxNormPer);  // the skew: up to 63
    hipLaunchKernelGGL(k_softmax_norm_rows, dim3((unsigned)((size_t)rows * chunks)), dim3(kBlock), 0, stream(),
                       losses, probs, logits, targets, stats, V, chunks);
    return check_launch("softmax_crossentropy (exact)");
  }
  // a row takes V + 63 slots at most (the alignment skew)
  const int W = V + 63;
  if (W <= 64 * 2) launch_rows<64, 2>(losses, probs, logits, targets, rows, V);
  else if (W <= 256) launch_rows<64, 4>(losses, probs, logits, targets, rows, V);
  else if (W <= 1024) launch_rows<256, 4>(losses, probs, logits, targets, rows, V);
  else if (W <= 4096) launch_rows<256, 16>(losses, probs, logits, targets, rows, V);
  else if (W <= 16384) launch_rows<1024, 16>(losses, probs, logits, targets, rows, V);
  else if (W <= 32768) launch_rows<1024, 32>(losses, probs, logits, targets, rows, V);
  else if (V <= kSplitMaxV) {  // 42 slots per thread in registers, 25 in LDS: two rows per CU
    static_assert(32768 - 63 >= 768 * 42, "the split kernel's register slots must lie inside every row it takes");
    hipLaunchKernelGGL((k_softmax_xent_split<768, 42, 25>), dim3(rows), dim3(768), 0, stream(), losses, probs,
                       logits, targets, V);
  } else {
    // Rows too long for the registers of one workgroup: a statistics pass
    // and a flat normalising pass (12 bytes per logit rather than 8).
    float2 *stats = static_cast<float2 *>(workspace(kRegSoftmax, softmax_scratch(rows, V)));
    if (!stats) return UGK_ENOMEM;
    hipLaunchKernelGGL(k_softmax_stats, dim3(grid_for((size_t)rows, kStatsWaves)), dim3(kStatsWaves * kWave), 0,
                       stream(), stats, logits, rows, V);
    const size_t n = (size_t)rows * V;
    hipLaunchKernelGGL(k_softmax_norm, dim3(grid_for(n, (size_t)kBlock * kNormUnroll)), dim3(kBlock), 0, stream(),
                       losses, probs, logits, targets, stats, n, V, 1.0 / (double)V);
  }
  return check_launch("softmax_crossentropy");
}

int launch_crossentropy_softmax_backward(float *dlogits, const float *probs, const int *targets, int rows, int V,
                                         float dloss, bool zeroed) {
  if (rows == 0 || V == 0) return 0;
  const size_t n = (size_t)rows * V;
  if (V >= 4 && (n & 3) == 0 && aligned16(dlogits) && aligned16(probs)) {
    const size_t n4 = n / 4;
    const dim3 grid(grid_for(n4, (size_t)kBwdThreads * kBwdUnroll));
    if (zeroed)
      hipLaunchKernelGGL(k_xent_softmax_bwd_flat4<true>, grid, dim3(kBwdThreads), 0, stream(), dlogits, probs, targets,
                         rows, V, dloss, n4, 1.0 / (double)V);
    else
      hipLaunchKernelGGL(k_xent_softmax_bwd_flat4<false>, grid, dim3(kBwdThreads), 0, stream(), dlogits, probs,
                         targets, rows, V, dloss, n4, 1.0 / (double)V);
  } else {
    const dim3 grid(rows, grid_for((size_t)V, (size_t)kBwdThreads * kBwdPer));
    if (zeroed)
      hipLaunchKernelGGL(k_xent_softmax_bwd<true>, grid, dim3(kBwdThreads), 0, stream(), dlogits, probs, targets, V,
                         dloss);
    else
      hipLaunchKernelGGL(k_xent_softmax_bwd<false>, grid, dim3(kBwdThreads), 0, stream(), dlogits, probs, targets, V,
                         dloss);
  }
  return check_launch("crossentropy_softmax_backward");
}

}  // namespace ugk
