// ugk_layernorm.hip - LayerNorm forward and backward (train_bnn.c:81-115,
// :439-477), and the residual -> LayerNorm / LayerNorm -> residual pairs of
// the reference launch sequence fused into one pass each.
//
// Layout: rows of C fp32 values, row-major; mean/rstd one float per row;
// weight/bias/dweight/dbias C floats.
//
// Forward: one wavefront per row. Each lane holds V float4 of the row in
// registers (V = ceil(C/256); C = 768 -> 3), so the row is read from HBM once
// and written once (8 bytes per element). Mean and variance are two-pass over
// the registers with wavefront sums (DPP within rows of 16 lanes, the four
// row sums added in scalar registers), rstd = 1/sqrtf(var/C + 1e-5) with IEEE
// division and square root, exactly the CPU formula.
//
// Backward: one wavefront per row for dinp (two wavefront sums). Each
// wavefront adds the dweight/dbias terms of its rows, in row order, in
// registers; after one barrier the workgroup's W per-wavefront sums are added
// column by column in wavefront order into one partial row per workgroup, and
// a second, small kernel adds the partial rows in index order into
// dweight/dbias. No atomics, so the result is identical run to run.
//
// Every load of the float4 paths is unconditional: a lane's columns past the
// row are clamped onto the row's last float4, and rows past a wavefront's
// range repeat its last row; the values so loaded are masked out of the sums
// (added as -0.0f, the identity of IEEE addition) or skipped by a branch that
// is uniform across the wavefront, and never stored. Per-lane
// conditions around loads made the compiler wait for one row's loads before
// it issued the next row's.
// Streamed rows (x, dout, dinp, out) use non-temporal loads and stores.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "ugk_internal.h"

namespace ugk {
namespace {

constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kMaxV = 8;  // float4 per lane held in registers: C <= 2048

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// Clamped float4 column of each of a lane's V slots, and whether it is in the row.
template <int V>
struct Cols {
  int col[V];
  bool in[V];
  __device__ __forceinline__ Cols(int lane, int C4) {
#pragma unroll
    for (int v = 0; v < V; v++) {
      const int c4 = lane + v * kWave;
      in[v] = c4 < C4;
      col[v] = in[v] ? c4 : C4 - 1;
    }
  }
};

// Normalise one row held in registers (V float4 per lane) and store out, mean
// and rstd: two-pass mean and variance with wavefront sums, IEEE 1/sqrtf.
// Shared by every forward kernel, so that they give the same bits.
template <int V>
__device__ __forceinline__ void ln_row_out(const float4 (&xv)[V], const Cols<V> &cl, int C, int row, int lane,
                                           const float4 *__restrict__ w4, const float4 *__restrict__ b4,
                                           float4 *__restrict__ o4, float *__restrict__ mean,
                                           float *__restrict__ rstd) {
  const size_t off = (size_t)row * (C >> 2);
  float s = 0.0f;
#pragma unroll
  for (int v = 0; v < V; v++) {
    const bool c = cl.in[v];
    s += c ? xv[v].x : -0.0f; s += c ? xv[v].y : -0.0f; s += c ? xv[v].z : -0.0f; s += c ? xv[v].w : -0.0f;
  }
  s = wave_sum(s);
  const float m = s / (float)C;
  float vs = 0.0f;
#pragma unroll
  for (int v = 0; v < V; v++) {
    const bool c = cl.in[v];
    float d;
    d = xv[v].x - m; vs += c ? d * d : -0.0f;
    d = xv[v].y - m; vs += c ? d * d : -0.0f;
    d = xv[v].z - m; vs += c ? d * d : -0.0f;
    d = xv[v].w - m; vs += c ? d * d : -0.0f;
  }
  vs = wave_sum(vs);
  const float r = 1.0f / sqrtf(vs / (float)C + 1e-5f);
#pragma unroll
  for (int v = 0; v < V; v++) {
    if (cl.in[v]) {
      const float4 w = w4[cl.col[v]], b = b4[cl.col[v]];
      float4 o;
      o.x = (xv[v].x - m) * r * w.x + b.x;
      o.y = (xv[v].y - m) * r * w.y + b.y;
      o.z = (xv[v].z - m) * r * w.z + b.z;
      o.w = (xv[v].w - m) * r * w.w + b.w;
      st_nt(o4 + off + cl.col[v], o);
    }
  }
  if (lane == 0) {
    mean[row] = m;
    rstd[row] = r;
  }
}

// Forward, RPW rows per wavefront (consecutive). The loads of row k+1 are
// issued before row k is normalised and stored, so a wavefront has a row in
// flight while it writes one.
// kRes: the row is first formed as res = inp + inp2 (residual_forward,
// train_bnn.c:182-186), stored to res, and normalised from the registers, the
// pair gpt2_kernels.cuh:793-797 launches back to back.
template <int V, bool kRes, int RPW>
__global__ __launch_bounds__(kBlock) void k_ln_fwd_vec(float *__restrict__ out, float *__restrict__ mean,
                                                       float *__restrict__ rstd, const float *__restrict__ inp,
                                                       const float *__restrict__ weight,
                                                       const float *__restrict__ bias, int rows, int C,
                                                       float *__restrict__ res, const float *__restrict__ inp2) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row0 = (blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6)) * RPW;
  if (row0 >= rows) return;
  const int C4 = C >> 2;
  const Cols<V> cl(lane, C4);
  const float4 *x4 = reinterpret_cast<const float4 *>(inp);
  const float4 *y4 = reinterpret_cast<const float4 *>(inp2);
  float4 *r4 = reinterpret_cast<float4 *>(res);
  float4 *o4 = reinterpret_cast<float4 *>(out);
  const float4 *w4 = reinterpret_cast<const float4 *>(weight);
  const float4 *b4 = reinterpret_cast<const float4 *>(bias);
  float4 xa[V], ya[kRes ? V : 1];
  {
    const size_t off = (size_t)row0 * C4;
#pragma unroll
    for (int v = 0; v < V; v++) {
      xa[v] = ld_nt(x4 + off + cl.col[v]);
      if (kRes) ya[kRes ? v : 0] = ld_nt(y4 + off + cl.col[v]);
    }
  }
#pragma unroll
  for (int k = 0; k < RPW; k++) {
    const int row = row0 + k;
    if (row >= rows) break;
    float4 xb[V], yb[kRes ? V : 1];
    if (k + 1 < RPW) {
      const size_t off = (size_t)min(row + 1, rows - 1) * C4;
#pragma unroll
      for (int v = 0; v < V; v++) {
        xb[v] = ld_nt(x4 + off + cl.col[v]);
        if (kRes) yb[kRes ? v : 0] = ld_nt(y4 + off + cl.col[v]);
      }
    }
    const size_t off = (size_t)row * C4;
    float4 xv[V];
#pragma unroll
    for (int v = 0; v < V; v++) {
      xv[v] = xa[v];
      if (kRes) {
        xv[v] = add4(xv[v], ya[kRes ? v : 0]);
        if (cl.in[v]) st_nt(r4 + off + cl.col[v], xv[v]);
      }
    }
    ln_row_out<V>(xv, cl, C, row, lane, w4, b4, o4, mean, rstd);
    if (k + 1 < RPW) {
#pragma unroll
      for (int v = 0; v < V; v++) {
        xa[v] = xb[v];
        if (kRes) ya[kRes ? v : 0] = yb[kRes ? v : 0];
      }
    }
  }
}

// Encoder forward then LayerNorm forward of its output, RPW rows per
// wavefront: row (b, t) is formed as wte[inp[b,t]] + wpe[t] in registers (the
// single add of train_bnn.c:41-65, the encoder's own order), stored to enc,
// and normalised from the registers as k_ln_fwd_vec does: the pair
// gpt2_kernels.cuh:775 -> :784 (or :813 when L = 0) launches back to back.
// The rows of wte and wpe are read through the cache: tokens repeat, and the
// B rows of a position share its wpe row.
template <int V, int RPW>
__global__ __launch_bounds__(kBlock) void k_enc_ln_fwd_vec(float *__restrict__ enc, float *__restrict__ out,
                                                           float *__restrict__ mean, float *__restrict__ rstd,
                                                           const int *__restrict__ inp,
                                                           const float *__restrict__ wte,
                                                           const float *__restrict__ wpe,
                                                           const float *__restrict__ weight,
                                                           const float *__restrict__ bias, int rows, int T, int C) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row0 = (blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6)) * RPW;
  if (row0 >= rows) return;
  const int C4 = C >> 2;
  const Cols<V> cl(lane, C4);
  const float4 *te4 = reinterpret_cast<const float4 *>(wte);
  const float4 *pe4 = reinterpret_cast<const float4 *>(wpe);
  float4 *e4 = reinterpret_cast<float4 *>(enc);
  float4 *o4 = reinterpret_cast<float4 *>(out);
  const float4 *w4 = reinterpret_cast<const float4 *>(weight);
  const float4 *b4 = reinterpret_cast<const float4 *>(bias);
  float4 xa[V], ya[V];
  {
    const size_t ot = (size_t)inp[row0] * C4, op = (size_t)(row0 % T) * C4;
#pragma unroll
    for (int v = 0; v < V; v++) {
      xa[v] = te4[ot + cl.col[v]];
      ya[v] = pe4[op + cl.col[v]];
    }
  }
#pragma unroll
  for (int k = 0; k < RPW; k++) {
    const int row = row0 + k;
    if (row >= rows) break;
    float4 xb[V], yb[V];
    if (k + 1 < RPW) {
      const int nx = min(row + 1, rows - 1);
      const size_t ot = (size_t)inp[nx] * C4, op = (size_t)(nx % T) * C4;
#pragma unroll
      for (int v = 0; v < V; v++) {
        xb[v] = te4[ot + cl.col[v]];
        yb[v] = pe4[op + cl.col[v]];
      }
    }
    const size_t off = (size_t)row * C4;
    float4 xv[V];
#pragma unroll
    for (int v = 0; v < V; v++) {
      xv[v] = add4(xa[v], ya[v]);
      if (cl.in[v]) st_nt(e4 + off + cl.col[v], xv[v]);
    }
    ln_row_out<V>(xv, cl, C, row, lane, w4, b4, o4, mean, rstd);
    if (k + 1 < RPW) {
#pragma unroll
      for (int v = 0; v < V; v++) {
        xa[v] = xb[v];
        ya[v] = yb[v];
      }
    }
  }
}

// Any C and alignment: one wavefront per row, three passes over the row.
__global__ __launch_bounds__(kBlock) void k_ln_fwd_scalar(float *out, float *mean, float *rstd,
                                                          const float *inp, const float *weight,
                                                          const float *bias, int rows, int C) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float *x = inp + (size_t)row * C;
  float *o = out + (size_t)row * C;
  float s = 0.0f;
  for (int c = lane; c < C; c += kWave) s += x[c];
  s = wave_sum(s);
  const float m = s / (float)C;
  float vs = 0.0f;
  for (int c = lane; c < C; c += kWave) {
    const float d = x[c] - m;
    vs += d * d;
  }
  vs = wave_sum(vs);
  const float r = 1.0f / sqrtf(vs / (float)C + 1e-5f);
  for (int c = lane; c < C; c += kWave) o[c] = (x[c] - m) * r * weight[c] + bias[c];
  if (lane == 0) {
    mean[row] = m;
    rstd[row] = r;
  }
}

__device__ __forceinline__ float4 zero4() { return make_float4(0.0f, 0.0f, 0.0f, 0.0f); }

// ---- column sums in the main launch (the per-op entry points) ----------------
// Instead of a second launch over the partial rows, the workgroups finish the
// column sums themselves, in the order the column-sum kernel uses (so with the
// same bits): the partial rows form kTailGroups groups of J = ceil(nblk / 16)
// consecutive rows; the last workgroup of a group to finish adds the group's
// rows in index order, starting from +0.0f, and writes the sum over the
// group's first row; the last group to finish adds the group sums in group
// order (an empty group adds +0.0f) into dweight/dbias.
//
// Publishing without a cache write-back: the rows and group sums are written
// with device-scope stores (sc1: written through to the point where all of the
// device's L2 caches are coherent) and read with device-scope loads. Each
// thread waits for its own stores to complete (s_waitcnt vmcnt(0)) before the
// workgroup barrier after which one thread increments the group's counter (a
// device-scope atomic), so when a counter shows a workgroup that it is the
// last, every row it is about to read is already at the coherence point. This
// is the release/acquire pair that an agent-scope fence would implement with
// an L2 write-back (buffer_wbl2 sc1) and invalidation on gfx950, confined to
// the bytes that need it; the fence itself, once per workgroup, took the call
// from 23 to 180 us at 8,192 x 768. Without it the call still takes longer
// than with the second launch (32.7 against 23.3 us at 8,192 x 768, 108
// against 38 us at 4,096 x 2,048): the last workgroup's chain of dependent
// device-scope round trips (its stores' completion, the counter, the group's
// rows, the group sum's completion, the counter, the group sums), about
// 0.85 us each, outlasts a launch that needs two. So it is not the default
// (ugk_diag_layernorm_tail selects it).
//
// The counters are per device and zero when the code object is loaded; the
// last arriver of each level resets its counter, so every call finds them at
// zero. Calls that overlap on one device (other streams) would share them,
// as they would share the workspace.
constexpr int kTailGroups = 16;
}  // namespace
}  // namespace ugk

static __device__ int ln_tail_count[ugk::kTailGroups + 1];

namespace ugk {
namespace {

__device__ __forceinline__ void st_dev(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Called by every thread of a workgroup (NT threads) after it has written its
// partial row with st_dev.
template <int NT>
__device__ __forceinline__ void ln_bwd_tail(float *partial, int nblk, int C, float *dweight, float *dbias) {
  __shared__ int last;
  constexpr int kBatch = 16;
  const int C2 = 2 * C;
  const int J = (nblk + kTailGroups - 1) / kTailGroups;
  const int g = blockIdx.x / J;
  const int j0 = g * J, j1 = min(j0 + J, nblk);
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(&ln_tail_count[g], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == j1 - j0 - 1;
    if (last) __hip_atomic_store(&ln_tail_count[g], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  for (int c = threadIdx.x; c < C2; c += NT) {
    float acc = 0.0f;
    for (int b = j0; b < j1; b += kBatch) {
      float v[kBatch];
#pragma unroll
      for (int q = 0; q < kBatch; q++) v[q] = ld_dev(partial + (size_t)min(b + q, j1 - 1) * C2 + c);
#pragma unroll
      for (int q = 0; q < kBatch; q++) acc += b + q < j1 ? v[q] : -0.0f;
    }
    st_dev(partial + (size_t)j0 * C2 + c, acc);
  }
  wait_stores();
  __syncthreads();
  const int G = (nblk + J - 1) / J;  // groups with rows
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(&ln_tail_count[kTailGroups], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == G - 1;
    if (last) __hip_atomic_store(&ln_tail_count[kTailGroups], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  for (int c = threadIdx.x; c < C2; c += NT) {
    float v[kTailGroups];
#pragma unroll
    for (int k = 0; k < kTailGroups; k++) v[k] = ld_dev(partial + (size_t)min(k, G - 1) * J * C2 + c);
    float t = v[0];
#pragma unroll
    for (int k = 1; k < kTailGroups; k++) t += k < G ? v[k] : 0.0f;
    if (c < C)
      dweight[c] += t;
    else
      dbias[c - C] += t;
  }
}

// Backward, register-resident rows. A workgroup is W wavefronts; wavefront w
// of workgroup g takes the rpw consecutive rows starting at (W g + w) * rpw,
// R at a time: the loads of R rows (x and dout first, which the row sums
// need, then dinp and the residual rows) are all issued before the first
// arithmetic instruction. It writes dinp and adds its rows' dweight/dbias
// terms, in row order, into its registers. After one barrier, thread t of the
// workgroup adds float4 column t of the W wavefronts' sums in wavefront order
// and writes the workgroup's partial row:
// partial[g] = [dweight part (C floats) | dbias part (C floats)].
// The weight row is read from global memory (it stays in L2), so the first
// rows' loads go out without waiting for anything.
//
// kRes: the new dinp row is also added to rdx and rdy (residual_backward with
// dout = dinp, train_bnn.c:491-496; twice into rdx when same), the pair
// gpt2_kernels.cuh:870-876 launches back to back.
// kDinp: kDinpRw reads and writes dinp. kDinpRead (kRes only) reads it but
// does not write it back: the step driver's pairs, whose dinp nothing reads
// after the residual split. kDinpNone (kRes only) neither reads nor writes
// it, taking it as +0.0: the first pair of the zeroed-gradient driver.
// kAssign (kRes only): rdx and rdy are not read but taken as +0.0 (the
// zeroed-gradient driver, whose residual targets are first written there).
// +0.0 + x is x with -0.0 turned to +0.0, so both give the bits the reads
// would give on a zero buffer.
// MINW: wavefronts per SIMD the register allocation must allow.
// kNt: dinp is written with non-temporal stores (always with kRes). Without
// kRes, large calls write it with ordinary stores, which measured faster
// (8,192 x 768: 17.5 against 19.0 us in the step, 22.7 against 23.9 us with
// the column sums); below 2^21 elements, where the written rows fit the
// caches and are written back at the end of the launch, non-temporal stores
// are kept. The fused pair keeps non-temporal stores for all three rows:
// an ordinary dinp store made it faster alone (35.7 against 37.2 us cold at
// 8,192 x 768) but the step slower (3.02 against 2.93 ms), the dirty lines
// of its 24 launches being written back during the kernels that follow.
template <int V, int W, int R, bool kRes, int MINW, bool kNt, int kDinp, bool kAssign, bool kTail>
__global__ __launch_bounds__(W * kWave, MINW) void k_ln_bwd_vec(
    float *__restrict__ dinp, float *__restrict__ partial, const float *__restrict__ dout,
    const float *__restrict__ inp, const float *__restrict__ weight, const float *__restrict__ mean,
    const float *__restrict__ rstd, int rows, int C, int rpw, float *__restrict__ rdx,
    float *__restrict__ rdy, int same, float *dweight, float *dbias) {
  __shared__ float4 red[W][2][V * kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int C4 = C >> 2;
  const float Cf = (float)C;
  const Cols<V> cl(lane, C4);
  const float4 *x4 = reinterpret_cast<const float4 *>(inp);
  const float4 *dy4 = reinterpret_cast<const float4 *>(dout);
  float4 *dx4 = reinterpret_cast<float4 *>(dinp);
  float4 *a4 = reinterpret_cast<float4 *>(rdx);
  float4 *b4 = reinterpret_cast<float4 *>(rdy);
  const float4 *w4 = reinterpret_cast<const float4 *>(weight);
  float4 ag[V], ab[V];
#pragma unroll
  for (int v = 0; v < V; v++) ag[v] = ab[v] = make_float4(0.f, 0.f, 0.f, 0.f);
  const int row0 = (blockIdx.x * W + wave) * rpw;
  const int row1 = min(row0 + rpw, rows);
  for (int row = row0; row < row1; row += R) {
    const int nr = min(R, row1 - row);
    int rq[R];
    size_t off[R];
#pragma unroll
    for (int q = 0; q < R; q++) {
      rq[q] = row + min(q, nr - 1);
      off[q] = (size_t)rq[q] * C4;
    }
    float4 x[R][V], dy[R][V], dx[R][V], wv[V];
    float4 ra[kRes ? R : 1][kRes ? V : 1], rb[kRes ? R : 1][kRes ? V : 1];
    float m[R], r[R];
#pragma unroll
    for (int q = 0; q < R; q++)
#pragma unroll
      for (int v = 0; v < V; v++) x[q][v] = ld_nt(x4 + off[q] + cl.col[v]);
#pragma unroll
    for (int q = 0; q < R; q++)
#pragma unroll
      for (int v = 0; v < V; v++) dy[q][v] = ld_nt(dy4 + off[q] + cl.col[v]);
#pragma unroll
    for (int v = 0; v < V; v++) wv[v] = w4[cl.col[v]];
#pragma unroll
    for (int q = 0; q < R; q++) {
      m[q] = mean[rq[q]];
      r[q] = rstd[rq[q]];
    }
#pragma unroll
    for (int q = 0; q < R; q++)
#pragma unroll
      for (int v = 0; v < V; v++) dx[q][v] = kDinp == kDinpNone ? zero4() : ld_nt(dx4 + off[q] + cl.col[v]);
    if (kRes) {
      // rdy is loaded even when it is rdx (same): a valid address, never used
#pragma unroll
      for (int q = 0; q < R; q++)
#pragma unroll
        for (int v = 0; v < V; v++) {
          ra[kRes ? q : 0][kRes ? v : 0] = kAssign ? zero4() : ld_nt(a4 + off[q] + cl.col[v]);
          rb[kRes ? q : 0][kRes ? v : 0] = kAssign ? zero4() : ld_nt(b4 + off[q] + cl.col[v]);
        }
    }
    // keep every load above the arithmetic (the scheduler would otherwise
    // sink the dinp and residual loads past the row sums)
    __builtin_amdgcn_sched_barrier(0);
    float s1[R], s2[R];
#pragma unroll
    for (int q = 0; q < R; q++) {
      s1[q] = 0.0f;
      s2[q] = 0.0f;
#pragma unroll
      for (int v = 0; v < V; v++) {
        const float4 w = wv[v];
        float4 xh, dn;
        xh.x = (x[q][v].x - m[q]) * r[q]; dn.x = dy[q][v].x * w.x;
        xh.y = (x[q][v].y - m[q]) * r[q]; dn.y = dy[q][v].y * w.y;
        xh.z = (x[q][v].z - m[q]) * r[q]; dn.z = dy[q][v].z * w.z;
        xh.w = (x[q][v].w - m[q]) * r[q]; dn.w = dy[q][v].w * w.w;
        const bool c = cl.in[v];
        s1[q] += c ? dn.x : -0.0f; s2[q] += c ? dn.x * xh.x : -0.0f;
        s1[q] += c ? dn.y : -0.0f; s2[q] += c ? dn.y * xh.y : -0.0f;
        s1[q] += c ? dn.z : -0.0f; s2[q] += c ? dn.z * xh.z : -0.0f;
        s1[q] += c ? dn.w : -0.0f; s2[q] += c ? dn.w * xh.w : -0.0f;
      }
    }
#pragma unroll
    for (int q = 0; q < R; q++) {
      s1[q] = wave_sum(s1[q]);
      s2[q] = wave_sum(s2[q]);
    }
#pragma unroll
    for (int q = 0; q < R; q++) {
      const bool live = q < nr;  // rows past nr repeat row nr-1: computed, neither stored nor summed
      const float dnm = s1[q] / Cf, dnxm = s2[q] / Cf;
#pragma unroll
      for (int v = 0; v < V; v++) {
        const float4 w = wv[v];
        float4 xh, dn;
        xh.x = (x[q][v].x - m[q]) * r[q]; dn.x = dy[q][v].x * w.x;
        xh.y = (x[q][v].y - m[q]) * r[q]; dn.y = dy[q][v].y * w.y;
        xh.z = (x[q][v].z - m[q]) * r[q]; dn.z = dy[q][v].z * w.z;
        xh.w = (x[q][v].w - m[q]) * r[q]; dn.w = dy[q][v].w * w.w;
        float4 o;
        o.x = dx[q][v].x + r[q] * (dn.x - dnm - xh.x * dnxm);
        o.y = dx[q][v].y + r[q] * (dn.y - dnm - xh.y * dnxm);
        o.z = dx[q][v].z + r[q] * (dn.z - dnm - xh.z * dnxm);
        o.w = dx[q][v].w + r[q] * (dn.w - dnm - xh.w * dnxm);
        if (cl.in[v] && live) {
          const size_t e = off[q] + cl.col[v];
          if (kDinp == kDinpRw) {
            if (kNt)
              st_nt(dx4 + e, o);
            else
              dx4[e] = o;
          }
          if (kRes) {
            float4 a = add4(ra[kRes ? q : 0][kRes ? v : 0], o);
            if (same) {
              a = add4(a, o);
            } else {
              st_nt(b4 + e, add4(rb[kRes ? q : 0][kRes ? v : 0], o));
            }
            st_nt(a4 + e, a);
          }
        }
        if (q > 0 && !live) continue;  // uniform across the wavefront: a branch, not a mask per lane
        const bool c = cl.in[v];
        ab[v].x += c ? dy[q][v].x : -0.0f; ag[v].x += c ? dy[q][v].x * xh.x : -0.0f;
        ab[v].y += c ? dy[q][v].y : -0.0f; ag[v].y += c ? dy[q][v].y * xh.y : -0.0f;
        ab[v].z += c ? dy[q][v].z : -0.0f; ag[v].z += c ? dy[q][v].z * xh.z : -0.0f;
        ab[v].w += c ? dy[q][v].w : -0.0f; ag[v].w += c ? dy[q][v].w * xh.w : -0.0f;
      }
    }
  }
#pragma unroll
  for (int v = 0; v < V; v++) {
    red[wave][0][v * kWave + lane] = ag[v];
    red[wave][1][v * kWave + lane] = ab[v];
  }
  __syncthreads();
  float4 *prow = reinterpret_cast<float4 *>(partial + (size_t)blockIdx.x * 2 * C);
  for (int e = threadIdx.x; e < 2 * V * kWave; e += W * kWave) {
    const int which = e >= V * kWave ? 1 : 0;
    const int c4 = e - which * V * kWave;
    if (c4 < C4) {
      float4 t = red[0][which][c4];
#pragma unroll
      for (int k = 1; k < W; k++) t = add4(t, red[k][which][c4]);
      if (kTail) {
        float *q = reinterpret_cast<float *>(prow + which * C4 + c4);
        st_dev(q, t.x); st_dev(q + 1, t.y); st_dev(q + 2, t.z); st_dev(q + 3, t.w);
      } else {
        prow[which * C4 + c4] = t;
      }
    }
  }
  if (kTail) ln_bwd_tail<W * kWave>(partial, (int)gridDim.x, C, dweight, dbias);
}

// Backward with each row split over a team of P wavefronts, one float4 per
// lane (C/4 <= 64 P). T teams form a workgroup; team t of workgroup g takes the
// rpt consecutive rows starting at (T g + t) * rpt, R at a time, all their
// loads issued before the first arithmetic instruction. Each wavefront adds
// its part of a row's two sums (the four components in order, then a
// wavefront sum) and writes it to LDS; after a barrier every wavefront of the
// team adds the P parts in part order, so all of them hold the same row sums.
// The dweight/dbias terms of a wavefront's columns are added in registers in
// row order; at the end the T teams' sums are added column by column in team
// order into the workgroup's partial row, as in k_ln_bwd_vec. With four rows
// in flight the fused pair needs 155 registers, so a 12-wavefront workgroup
// (P = 3, T = 4) runs alone on a CU: 35.7 against 37.2 us for the
// two-rows-per-wavefront kernel at 8,192 x 768, cold, with the same 512
// partial rows. rpt and T fix the order of every addition; R does not, so the
// plain backward (R = 2) and the fused pair (R = 4) give the same bits.
template <int P, int T, int R, bool kRes, int MINW, bool kNt, int kDinp, bool kAssign, bool kTail>
__global__ __launch_bounds__(P * T * kWave, MINW) void k_ln_bwd_team(
    float *__restrict__ dinp, float *__restrict__ partial, const float *__restrict__ dout,
    const float *__restrict__ inp, const float *__restrict__ weight, const float *__restrict__ mean,
    const float *__restrict__ rstd, int rows, int C, int rpt, float *__restrict__ rdx,
    float *__restrict__ rdy, int same, float *dweight, float *dbias) {
  __shared__ float parts[2][T][R][P][2];  // a row's two sums by part, double-buffered by pass
  __shared__ float4 red[T][2][P * kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int team = wave / P, part = wave - team * P;
  const int C4 = C >> 2;
  const float Cf = (float)C;
  const int c4 = part * kWave + lane;
  const bool in = c4 < C4;
  const int col = in ? c4 : C4 - 1;  // past the row: a valid column, masked out of the sums, never stored
  const float4 *x4 = reinterpret_cast<const float4 *>(inp);
  const float4 *dy4 = reinterpret_cast<const float4 *>(dout);
  float4 *dx4 = reinterpret_cast<float4 *>(dinp);
  float4 *a4 = reinterpret_cast<float4 *>(rdx);
  float4 *b4 = reinterpret_cast<float4 *>(rdy);
  const float4 w = reinterpret_cast<const float4 *>(weight)[col];
  float4 ag = make_float4(0.f, 0.f, 0.f, 0.f), ab = ag;
  const int t0 = (blockIdx.x * T + team) * rpt;
  const int t1 = min(t0 + rpt, rows);
  const int last = t1 > t0 ? t1 - 1 : rows - 1;  // a team past the last row loads that row, uses nothing
  const int passes = (rpt + R - 1) / R;  // the same for every team: all reach every barrier
  for (int ps = 0; ps < passes; ps++) {
    const int row = t0 + ps * R;
    bool live[R];
    int rq[R];
    size_t off[R];
#pragma unroll
    for (int q = 0; q < R; q++) {
      live[q] = row + q < t1;
      rq[q] = live[q] ? row + q : last;
      off[q] = (size_t)rq[q] * C4 + col;
    }
    float4 x[R], dy[R], dx[R], ra[kRes ? R : 1], rb[kRes ? R : 1];
    float m[R], r[R];
#pragma unroll
    for (int q = 0; q < R; q++) {
      x[q] = ld_nt(x4 + off[q]);
      dy[q] = ld_nt(dy4 + off[q]);
    }
#pragma unroll
    for (int q = 0; q < R; q++) {
      m[q] = mean[rq[q]];
      r[q] = rstd[rq[q]];
    }
#pragma unroll
    for (int q = 0; q < R; q++) dx[q] = kDinp == kDinpNone ? zero4() : ld_nt(dx4 + off[q]);
    if (kRes) {
      // rdy is loaded even when it is rdx (same): a valid address, never used
#pragma unroll
      for (int q = 0; q < R; q++) {
        ra[kRes ? q : 0] = kAssign ? zero4() : ld_nt(a4 + off[q]);
        rb[kRes ? q : 0] = kAssign ? zero4() : ld_nt(b4 + off[q]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    float4 xh[R], dn[R];
#pragma unroll
    for (int q = 0; q < R; q++) {
      xh[q].x = (x[q].x - m[q]) * r[q]; dn[q].x = dy[q].x * w.x;
      xh[q].y = (x[q].y - m[q]) * r[q]; dn[q].y = dy[q].y * w.y;
      xh[q].z = (x[q].z - m[q]) * r[q]; dn[q].z = dy[q].z * w.z;
      xh[q].w = (x[q].w - m[q]) * r[q]; dn[q].w = dy[q].w * w.w;
      float s1 = in ? ((dn[q].x + dn[q].y) + dn[q].z) + dn[q].w : -0.0f;
      float s2 = in ? ((dn[q].x * xh[q].x + dn[q].y * xh[q].y) + dn[q].z * xh[q].z) + dn[q].w * xh[q].w : -0.0f;
      s1 = wave_sum(s1);
      s2 = wave_sum(s2);
      if (lane == 0) {
        parts[ps & 1][team][q][part][0] = s1;
        parts[ps & 1][team][q][part][1] = s2;
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < R; q++) {
      if (!live[q]) break;  // the same for the team's wavefronts; dead rows are all at the end
      float s1 = parts[ps & 1][team][q][0][0], s2 = parts[ps & 1][team][q][0][1];
#pragma unroll
      for (int k = 1; k < P; k++) {
        s1 += parts[ps & 1][team][q][k][0];
        s2 += parts[ps & 1][team][q][k][1];
      }
      const float dnm = s1 / Cf, dnxm = s2 / Cf;
      float4 o;
      o.x = dx[q].x + r[q] * (dn[q].x - dnm - xh[q].x * dnxm);
      o.y = dx[q].y + r[q] * (dn[q].y - dnm - xh[q].y * dnxm);
      o.z = dx[q].z + r[q] * (dn[q].z - dnm - xh[q].z * dnxm);
      o.w = dx[q].w + r[q] * (dn[q].w - dnm - xh[q].w * dnxm);
      if (in) {
        if (kDinp == kDinpRw) {
          if (kNt)
            st_nt(dx4 + off[q], o);
          else
            dx4[off[q]] = o;
        }
        if (kRes) {
          float4 a = add4(ra[kRes ? q : 0], o);
          if (same) {
            a = add4(a, o);
          } else {
            st_nt(b4 + off[q], add4(rb[kRes ? q : 0], o));
          }
          st_nt(a4 + off[q], a);
        }
      }
      ab.x += dy[q].x; ag.x += dy[q].x * xh[q].x;
      ab.y += dy[q].y; ag.y += dy[q].y * xh[q].y;
      ab.z += dy[q].z; ag.z += dy[q].z * xh[q].z;
      ab.w += dy[q].w; ag.w += dy[q].w * xh[q].w;
    }
  }
  red[team][0][c4] = ag;
  red[team][1][c4] = ab;
  __syncthreads();
  float4 *prow = reinterpret_cast<float4 *>(partial + (size_t)blockIdx.x * 2 * C);
  for (int e = threadIdx.x; e < 2 * C4; e += P * T * kWave) {
    const int which = e >= C4 ? 1 : 0;
    const int cc = e - which * C4;
    float4 t = red[0][which][cc];
#pragma unroll
    for (int k = 1; k < T; k++) t = add4(t, red[k][which][cc]);
    if (kTail) {
      float *q = reinterpret_cast<float *>(prow + which * C4 + cc);
      st_dev(q, t.x); st_dev(q + 1, t.y); st_dev(q + 2, t.z); st_dev(q + 3, t.w);
    } else {
      prow[which * C4 + cc] = t;
    }
  }
  if (kTail) ln_bwd_tail<P * T * kWave>(partial, (int)gridDim.x, C, dweight, dbias);
}

// Backward for any C and alignment. Phase 1: one wavefront per row writes
// dinp. Phase 2: thread-per-channel column sums over the workgroup's rows.
__global__ __launch_bounds__(kBlock) void k_ln_bwd_scalar(float *dinp, float *partial, const float *dout,
                                                          const float *inp, const float *weight,
                                                          const float *mean, const float *rstd, int rows,
                                                          int C, int rpb) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const float Cf = (float)C;
  const int row0 = blockIdx.x * rpb;
  const int row1 = min(row0 + rpb, rows);
  for (int row = row0 + wave; row < row1; row += kWavesPerBlock) {
    const float *x = inp + (size_t)row * C;
    const float *dy = dout + (size_t)row * C;
    float *dx = dinp + (size_t)row * C;
    const float m = mean[row], r = rstd[row];
    float s1 = 0.0f, s2 = 0.0f;
    for (int c = lane; c < C; c += kWave) {
      const float xhat = (x[c] - m) * r;
      const float dnorm = dy[c] * weight[c];
      s1 += dnorm;
      s2 += dnorm * xhat;
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float dnm = s1 / Cf, dnxm = s2 / Cf;
    for (int c = lane; c < C; c += kWave) {
      const float xhat = (x[c] - m) * r;
      const float dnorm = dy[c] * weight[c];
      dx[c] += r * (dnorm - dnm - xhat * dnxm);
    }
  }
  float *prow = partial + (size_t)blockIdx.x * 2 * C;
  for (int c = threadIdx.x; c < C; c += kBlock) {
    float g = 0.0f, b = 0.0f;
    for (int row = row0; row < row1; row++) {
      const float dy = dout[(size_t)row * C + c];
      const float xhat = (inp[(size_t)row * C + c] - mean[row]) * rstd[row];
      b += dy;
      g += dy * xhat;
    }
    prow[c] = g;
    prow[C + c] = b;
  }
}

// Column totals of the partial rows, added to dweight (columns [0,C)) and
// dbias (columns [C,2C)). Workgroup: 32 columns x 16 groups; group k sums the
// partial rows [k*J, (k+1)*J), J = ceil(nblk/16) <= 64, in index order, 32
// loads in flight per batch; the 16 group sums are then added in group order.
// 32 columns rather than 64 spread one LayerNorm's totals over twice the
// workgroups (48 at C = 768): the per-op backward at 8,192 x 768 took 22.3-22.6
// against 23.3 us cold, and the step's batched launch 12.7 against 13.1-13.3 us
// (16 columns: 22.6 us). The order of the additions does not depend on it.
constexpr int kRedGroups = 16;
constexpr int kRedCols = 32;
static_assert(kRedGroups == kTailGroups, "the in-launch column sums follow the column-sum kernel's order");
constexpr int kRedBatch = 32;
static_assert(kMaxPartialRows <= kRedGroups * 2 * kRedBatch, "two load batches per group at most");
__device__ __forceinline__ void ln_bwd_reduce_tile(float *dweight, float *dbias, const float *partial, int nblk,
                                                   int C, float (*red)[kRedCols]) {
  const int cl = threadIdx.x % kRedCols;
  const int g = threadIdx.x / kRedCols;
  const int col = blockIdx.x * kRedCols + cl;
  const int C2 = 2 * C;
  const int J = (nblk + kRedGroups - 1) / kRedGroups;
  const int j0 = g * J, j1 = min(j0 + J, nblk);
  const int cc = col < C2 ? col : C2 - 1;
  // the value the total is added to, loaded with the partial rows rather than
  // after them (one memory round trip fewer at the end)
  float* const dst = col < C ? dweight + col : dbias + (cc - C);
  const float prev = g == 0 && col < C2 ? *dst : 0.0f;
  float acc = 0.0f;
  for (int b = j0; b < j1; b += kRedBatch) {
    float v[kRedBatch];
#pragma unroll
    for (int q = 0; q < kRedBatch; q++) v[q] = partial[(size_t)min(b + q, j1 - 1) * C2 + cc];
#pragma unroll
    for (int q = 0; q < kRedBatch; q++) acc += b + q < j1 ? v[q] : -0.0f;
  }
  red[g][cl] = acc;
  __syncthreads();
  if (g == 0 && col < C2) {
    float t = red[0][cl];
#pragma unroll
    for (int k = 1; k < kRedGroups; k++) t += red[k][cl];
    *dst = prev + t;
  }
}

// Several LayerNorm backwards' column totals in one launch (blockIdx.y picks
// the job).
constexpr int kMaxReduceJobs = 32;
struct LnReduceBatch {
  LnReduceJob job[kMaxReduceJobs];
};
__global__ __launch_bounds__(kRedCols * kRedGroups) void k_ln_bwd_reduce_batch(LnReduceBatch b, int C) {
  __shared__ float red[kRedGroups][kRedCols];
  const LnReduceJob &j = b.job[blockIdx.y];
  ln_bwd_reduce_tile(j.dweight, j.dbias, j.partial, j.nblk, C, red);
}

bool vec_ok(int C, std::initializer_list<const void *> ptrs) {
  if ((C & 3) != 0 || C > kMaxV * kWave * 4) return false;
  for (const void *p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

// Scalar path: workgroups of 4 wavefronts, at most max_blocks of them.
void bwd_shape(int rows, int max_blocks, int *nblk, int *rpb) {
  int nb = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
  if (nb > max_blocks) nb = max_blocks;
  if (nb < 1) nb = 1;
  int per = (rows + nb - 1) / nb;
  per = (per + kWavesPerBlock - 1) / kWavesPerBlock * kWavesPerBlock;
  *rpb = per;
  *nblk = (rows + per - 1) / per;
}

// Vector path shapes: 8 wavefronts per workgroup, 4 when a lane holds more
// than 4 float4 of a row. Each wavefront takes S consecutive rows (S = 2 while
// C <= 768, else 1) while that leaves at most max_blocks workgroups, else
// more: at 16,384 x 768 one pass over 1,024 workgroups took 72 us for the
// fused pair against 81 us with two passes over 512. The plain backward and
// the fused pair share this shape (the rows of each wavefront and workgroup),
// hence the order in which dweight/dbias are summed, so that the pair is
// bit-identical to the plain backward followed by residual_backward.
// Rows in flight differ: the fused pair loads both of its rows at once (214
// registers, two wavefronts per SIMD); the plain backward takes one row at a
// time within 128 registers, four wavefronts per SIMD, which measured 18.9
// against 20.1 us at 8,192 x 768 (35.9 against 39.5 us at 16,384) with the
// same sums.
struct BwdCfg {
  int W, S, R, MINW;
};
constexpr BwdCfg bwd_cfg(int V, bool res) {
  return BwdCfg{V <= 4 ? 8 : 4, V <= 3 ? 2 : 1, (V <= 3 && res) ? 2 : 1, (V <= 3 && !res) ? 4 : 1};
}
void bwd_shape_vec(int rows, BwdCfg k, int max_blocks, int *nblk, int *rpw) {
  const int per_wave = (rows + max_blocks * k.W - 1) / (max_blocks * k.W);
  *rpw = per_wave < k.S ? k.S : per_wave;
  *nblk = (rows + k.W * *rpw - 1) / (k.W * *rpw);
}

// Compute units of the current device (cached per device; 256 if unknown).
int cu_count() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();  // leave no error for the next launch check to report
    return 256;
  }
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      n = 256;
    }
    cus[dev] = n;
  }
  return cus[dev];
}

// Team path, V = 3 (C/4 in 129..192), while the rows fill the GPU at most
// once at 32 rows per CU (8,192 on MI355X): teams of 3 wavefronts, 4 teams
// per workgroup, at least 4 rows per team (16 per workgroup, 512 workgroups
// at 8,192 rows), more while that would leave more than max_blocks
// workgroups. The plain backward keeps 2 rows in flight (70 registers), the
// fused pair 4 (156). Beyond that the two-rows-per-wavefront kernels are
// used: at 16,384 x 768 they measured as fast for the fused pair and faster
// for the plain backward (41.7 against 45.0 us with the column sums).
constexpr int kTeamParts = 3, kTeams = 4, kTeamRows = 4;
bool team_path(int rows, int C) {
  return ((C >> 2) + kWave - 1) / kWave == kTeamParts && rows <= cu_count() * 32;
}
void team_shape(int rows, int max_blocks, int *nblk, int *rpt) {
  const int per_team = (rows + max_blocks * kTeams - 1) / (max_blocks * kTeams);
  *rpt = per_team < kTeamRows ? kTeamRows : per_team;
  *nblk = (rows + kTeams * *rpt - 1) / (kTeams * *rpt);
}

// Workgroups (partial rows) of a vector-path call, for sizing its workspace:
// at V = 3 the larger of the two kernels' counts, so that the size does not
// depend on the device the call later runs on.
int vec_blocks(int rows, int C, bool res, int max_blocks) {
  int nblk, rpw;
  const int V = ((C >> 2) + kWave - 1) / kWave;
  bwd_shape_vec(rows, bwd_cfg(V, res), max_blocks, &nblk, &rpw);
  if (V == kTeamParts) {
    int nt, rpt;
    team_shape(rows, max_blocks, &nt, &rpt);
    if (nt > nblk) nblk = nt;
  }
  return nblk;
}

// Rows per wavefront of the fused forward: two while one wavefront per row
// would fill the GPU only once (the reads and writes of a single round of
// wavefronts cannot overlap; measured 17.7 against 18.8 us at 8,192 x 768),
// else one (35.0 against 37.1 us at 16,384 x 768). The plain forward keeps
// one (9.3 against 9.6 us with two at 8,192 x 768).
int fwd_rpw(int rows, bool res) {
  if (!res) return 1;
  return rows <= cu_count() * 32 ? 2 : 1;
}

}  // namespace

int layernorm_backward_blocks(int rows, int C, bool res, int max_blocks) {
  if (rows <= 0) return 0;
  if ((C & 3) == 0 && C <= kMaxV * kWave * 4) return vec_blocks(rows, C, res, max_blocks);
  int nblk, rpb;
  bwd_shape(rows, max_blocks < kMaxScalarBlocks ? max_blocks : kMaxScalarBlocks, &nblk, &rpb);
  return nblk;
}

// An upper bound on the partial rows of every call with at most `rows` rows
// and at most C channels, on any path. A path's count is not monotone in the
// rows (once a call would exceed the cap, each workgroup takes more rows and
// the count drops below the cap), but it never exceeds
// min(cap, ceil(rows / floor)), where floor is the fewest rows a workgroup of
// that path takes: 4 on the scalar path (cap 512) and on the wave-per-row path
// above 1,024 channels (one row per wavefront, four wavefronts), 8 from 772
// channels (eight wavefronts, one row each), 16 below (eight wavefronts of two
// rows, or four teams of four rows; cap 1,024). Sizing a workspace by this
// bound at a config's rows therefore covers every smaller call.
int layernorm_backward_blocks_bound(int rows, int C) {
  const auto cap_div = [rows](int cap, int floor) {
    const long long q = ((long long)rows + floor - 1) / floor;
    return (int)(q < cap ? q : cap);
  };
  int nb = cap_div(kMaxScalarBlocks, 4);
  if (C > kWave * 4 * 4) nb = std::max(nb, cap_div(kMaxPartialRows, 4));
  if (C > kWave * 4 * 3) nb = std::max(nb, cap_div(kMaxPartialRows, 8));
  nb = std::max(nb, cap_div(kMaxPartialRows, 16));
  return rows > 0 ? nb : 0;
}

size_t layernorm_backward_scratch(int rows, int C) {
  return (size_t)layernorm_backward_blocks_bound(rows, C) * 2 * (size_t)C * sizeof(float);
}

namespace {
template <bool kRes>
void launch_ln_fwd_vec(float *out, float *mean, float *rstd, const float *inp, const float *weight,
                       const float *bias, int rows, int C, float *res, const float *inp2) {
  const int V = ((C >> 2) + kWave - 1) / kWave;
  const int rpw = fwd_rpw(rows, kRes);
  const dim3 grid(grid_for((size_t)rows, (size_t)kWavesPerBlock * rpw)), block(kBlock);
  switch (V * 2 + (rpw - 1)) {
#define UGK_LN_FWD(v)                                                                                           \
  case 2 * v:                                                                                                   \
    launch((k_ln_fwd_vec<v, kRes, 1>), grid, block, 0, out, mean, rstd, inp, weight, bias, \
                       rows, C, res, inp2);                                                                     \
    break;                                                                                                      \
  case 2 * v + 1:                                                                                               \
    launch((k_ln_fwd_vec<v, kRes, 2>), grid, block, 0, out, mean, rstd, inp, weight, bias, \
                       rows, C, res, inp2);                                                                     \
    break;
    UGK_LN_FWD(1) UGK_LN_FWD(2) UGK_LN_FWD(3) UGK_LN_FWD(4)
    UGK_LN_FWD(5) UGK_LN_FWD(6) UGK_LN_FWD(7) UGK_LN_FWD(8)
#undef UGK_LN_FWD
  }
}
}  // namespace

int launch_residual_layernorm_forward(float *res, float *out, float *mean, float *rstd, const float *x,
                                      const float *y, const float *weight, const float *bias, int rows,
                                      int C) {
  if (rows == 0) return 0;
  if (layernorm_exact() || !vec_ok(C, {res, out, x, y, weight, bias})) {
    if (int e = launch_residual_forward(res, x, y, (size_t)rows * C)) return e;
    return launch_layernorm_forward(out, mean, rstd, res, weight, bias, rows, C);
  }
  launch_ln_fwd_vec<true>(out, mean, rstd, x, weight, bias, rows, C, res, y);
  return check_launch("residual_layernorm_forward");
}

int launch_encoder_layernorm_forward(float *enc, float *out, float *mean, float *rstd, const int *inp,
                                     const float *wte, const float *wpe, const float *weight, const float *bias,
                                     int B, int T, int C) {
  const int rows = B * T;
  if (rows == 0) return 0;
  if (layernorm_exact() || !vec_ok(C, {enc, out, wte, wpe, weight, bias})) {
    if (int e = launch_encoder_forward(enc, inp, wte, wpe, B, T, C)) return e;
    return launch_layernorm_forward(out, mean, rstd, enc, weight, bias, rows, C);
  }
  const int V = ((C >> 2) + kWave - 1) / kWave;
  const int rpw = fwd_rpw(rows, true);
  const dim3 grid(grid_for((size_t)rows, (size_t)kWavesPerBlock * rpw)), block(kBlock);
  switch (V * 2 + (rpw - 1)) {
#define UGK_ENC_LN(v)                                                                                          \
  case 2 * v:                                                                                                  \
    launch((k_enc_ln_fwd_vec<v, 1>), grid, block, 0, enc, out, mean, rstd, inp, wte, wpe, weight, bias, rows, \
           T, C);                                                                                              \
    break;                                                                                                     \
  case 2 * v + 1:                                                                                              \
    launch((k_enc_ln_fwd_vec<v, 2>), grid, block, 0, enc, out, mean, rstd, inp, wte, wpe, weight, bias, rows, \
           T, C);                                                                                              \
    break;
    UGK_ENC_LN(1) UGK_ENC_LN(2) UGK_ENC_LN(3) UGK_ENC_LN(4)
    UGK_ENC_LN(5) UGK_ENC_LN(6) UGK_ENC_LN(7) UGK_ENC_LN(8)
#undef UGK_ENC_LN
  }
  return check_launch("encoder_layernorm_forward");
}

namespace {
// ---- exact mode: train_bnn.c's order of every addition ------------------------
// train_bnn.c:81-115 and :439-477 add each row's terms one column at a time
// (c = 0, 1, ..., C-1), and dweight/dbias one row at a time. The exact kernels
// keep those orders, each sum a serial chain in one lane of wavefront 0, which
// does nothing but the chains' additions; fifteen loader wavefronts keep it fed:
//   rows: a workgroup per 60 rows. The loaders stream 64-column tiles of the
//     rows, three tiles ahead in registers, and stage each row's terms in LDS
//     (the forward: x, then (x - mean)^2; the backward: dout * w and
//     dout * w * xhat), row-major at a pitch of 68 floats, so that the chains
//     read four terms at a time without bank conflicts. One chain per row
//     (lane = row; lanes 60-63 follow copies and store nothing; 60 rows make a
//     tile whole loader slots, scalar and float4). Then every wavefront writes out (or adds to dinp) whole
//     rows with the row statistics.
//   columns: a workgroup per 16 columns. The loaders stage 240-row tiles of
//     the dweight terms dout * xhat and the dbias terms dout, transposed (a
//     column's terms contiguous, pitch 244 floats); lanes 0-15 chain dweight,
//     lanes 16-31 dbias, one row after another, from the values the arrays hold.
// Every term is rounded as the CPU rounds it (no product is contracted into an
// fma; the square root and quotients are IEEE's), so every result is
// train_bnn.c's bit for bit. The backward's row and column workgroups are
// independent and share one launch. kVec: C a multiple of 4 and the row
// arrays 16-byte aligned, every global access of the rows a float4 (a quarter
// of the memory instructions, which bound these kernels); otherwise scalar
// accesses, any C, any alignment.
constexpr int kExLoaders = 15;
constexpr int kExThreads = (kExLoaders + 1) * kWave;
constexpr int kExLoadLanes = kExLoaders * kWave;
constexpr int kExDepth = 3;  // tiles in registers ahead of the chains
constexpr int kExRows = 60;  // rows per row workgroup (one chain per lane of wavefront 0)
constexpr int kExTile = 64;  // columns per tile of a row workgroup
constexpr int kExPitch = kExTile + 4;
constexpr int kExSlots = (kExRows * kExTile + kExLoadLanes - 1) / kExLoadLanes;
constexpr int kExVecSlots = (kExRows * kExTile / 4 + kExLoadLanes - 1) / kExLoadLanes;
constexpr int kExApply = 8;       // scalar elements per lane in flight when the rows are written
constexpr int kExApplyVec = 4;    // float4 per lane in flight when the rows are written
constexpr int kExCols = 16;       // columns per column workgroup (two chains each)
constexpr int kExChains = 2 * kExCols;
constexpr int kExColRows = 240;   // rows per tile of a column workgroup
constexpr int kExColPitch = kExColRows + 4;
constexpr int kExColSlots = kExColRows * kExCols / kExLoadLanes;
// float4 reads per chain and batch (two batches in flight): 32 additions a
// batch in the row chains; 24 in the column chains, whose loaders hold more
// registers
constexpr int kExBatch = 8;
constexpr int kExColBatch = 6;
static_assert(kExRows <= kWave && kWave % kExCols == 0 && kExChains <= kWave, "chains in wavefront 0");
static_assert(kExRows * kExTile == kExSlots * kExLoadLanes && kExRows * kExTile / 4 == kExVecSlots * kExLoadLanes,
              "a row tile is whole loader slots, scalar and float4");
static_assert(kExColRows * kExCols == kExColSlots * kExLoadLanes && kExColRows * kExCols / 4 == kExLoadLanes,
              "a column tile is whole loader slots, scalar and float4");
static_assert(kExTile % (8 * kExBatch) == 0 && kExColRows % (8 * kExColBatch) == 0, "whole batch pairs per tile");
static_assert(kExLoadLanes % (kExTile / 4) == 0, "a loader lane keeps its float4 column in every slot");
// LDS of a row workgroup (floats): term tiles (a row per lane of wavefront 0),
// per-row statistics and sums
constexpr int ex_row_lds(int arrays) { return 2 * arrays * kWave * kExPitch + 4 * kWave; }
constexpr int kExColLds = 2 * kExChains * kExColPitch;
constexpr int kExBwdLds = ex_row_lds(2) > kExColLds ? ex_row_lds(2) : kExColLds;

__device__ __forceinline__ float f4_get(const float4 &v, int j) {
  return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

template <bool kBwd, bool kVec>
__device__ __forceinline__ void ln_rows_exact(float *lds, int blk, float *__restrict__ outp, float *__restrict__ mean,
                                              float *__restrict__ rstd, const float *__restrict__ inp,
                                              const float *__restrict__ dout, const float *__restrict__ weight,
                                              const float *__restrict__ bias, int rows, int C) {
  constexpr int kArr = kBwd ? 2 : 1;  // staged term arrays
  constexpr int kTileF = kWave * kExPitch;
  constexpr int kSlots = kVec ? kExVecSlots : kExSlots;
  constexpr int kW = kVec ? 4 : 1;  // floats per lane and slot
  float *const tile = lds;  // [2][kArr][kTileF]
  float2 *const stat = reinterpret_cast<float2 *>(lds + 2 * kArr * kTileF);  // [kWave]: mean, rstd
  float2 *const rsum = stat + kWave;  // [kWave]: the backward's row sums / C
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
  const int r0 = blk * kExRows;
  const int nt = (C + kExTile - 1) / kExTile;
  const int nu = (kBwd ? 1 : 2) * nt;  // tiles streamed: the forward reads every tile twice
  const float Cf = (float)C;
  float s[kArr];  // the chains of wavefront 0's lane: row r0 + lane
#pragma unroll
  for (int a = 0; a < kArr; a++) s[a] = 0.0f;
  if (kBwd) {
    // the rows' statistics, for the loaders' terms and the writes
    if (wave == 0) {
      const int crow = min(r0 + lane, rows - 1);
      stat[lane] = make_float2(mean[crow], rstd[crow]);
    }
    __syncthreads();
  }
  // Loader lane L = 64 lw + lane. Scalar: slot sl holds tile row lw + 15 sl,
  // column lane. float4: slot sl holds float4 f = L + 960 sl of the tile (row
  // f / 16, columns 4 (f % 16) + 0..3), the column the same in every slot.
  const int lw = wave - 1;
  const int L = lw * kWave + lane;
  float reg[kExDepth][kArr][kSlots][kW];
  float wreg[kExDepth][kW];
  auto slot_row = [&](int sl) { return kVec ? (L + kExLoadLanes * sl) / (kExTile / 4) : lw + kExLoaders * sl; };
  const int lcol = kVec ? 4 * (L % (kExTile / 4)) : lane;
  auto load_tile = [&](int u, int k) {
    const int col = min((u % nt) * kExTile + lcol, C - kW);
#pragma unroll
    for (int sl = 0; sl < kSlots; sl++) {
      const int ri = min(slot_row(sl), kExRows - 1);
      const size_t off = (size_t)min(r0 + ri, rows - 1) * C + col;
      if constexpr (kVec) {
        const float4 x = *reinterpret_cast<const float4 *>(inp + off);
        reg[k][0][sl][0] = x.x, reg[k][0][sl][1] = x.y, reg[k][0][sl][2] = x.z, reg[k][0][sl][3] = x.w;
        if (kBwd) {
          const float4 y = *reinterpret_cast<const float4 *>(dout + off);
          reg[k][kArr - 1][sl][0] = y.x, reg[k][kArr - 1][sl][1] = y.y;
          reg[k][kArr - 1][sl][2] = y.z, reg[k][kArr - 1][sl][3] = y.w;
        }
      } else {
        reg[k][0][sl][0] = inp[off];
        if (kBwd) reg[k][kArr - 1][sl][0] = dout[off];
      }
    }
    if constexpr (kBwd) {
      if constexpr (kVec) {
        const float4 w = *reinterpret_cast<const float4 *>(weight + col);
        wreg[k][0] = w.x, wreg[k][1] = w.y, wreg[k][2] = w.z, wreg[k][3] = w.w;
      } else {
        wreg[k][0] = weight[col];
      }
    }
  };
  auto store_tile = [&](int u, int k) {
    float *const T = tile + (u & 1) * kArr * kTileF;
#pragma unroll
    for (int sl = 0; sl < kSlots; sl++) {
      const int ri = slot_row(sl);
      if (ri < kExRows) {
        float t0[kW], t1[kW];
        if (kBwd) {
          const float2 st = stat[ri];
#pragma unroll
          for (int j = 0; j < kW; j++) {
            const float xh = (reg[k][0][sl][j] - st.x) * st.y;
            t0[j] = reg[k][kArr - 1][sl][j] * wreg[k][j];
            t1[j] = t0[j] * xh;
          }
        } else if (u < nt) {
#pragma unroll
          for (int j = 0; j < kW; j++) t0[j] = reg[k][0][sl][j];
        } else {
          const float m = stat[ri].x;
#pragma unroll
          for (int j = 0; j < kW; j++) {
            const float d = reg[k][0][sl][j] - m;
            t0[j] = d * d;
          }
        }
        float *const p = T + ri * kExPitch + lcol;
        if constexpr (kVec) {
          *reinterpret_cast<float4 *>(p) = make_float4(t0[0], t0[1], t0[2], t0[3]);
          if (kBwd) *reinterpret_cast<float4 *>(p + kTileF) = make_float4(t1[0], t1[1], t1[2], t1[3]);
        } else {
          p[0] = t0[0];
          if (kBwd) p[kTileF] = t1[0];
        }
      }
    }
  };
  if (wave > 0) {
#pragma unroll
    for (int k = 0; k < kExDepth; k++)
      if (k < nu) load_tile(k, k);
  }
  for (int u0 = 0; u0 < nu; u0 += kExDepth) {
#pragma unroll
    for (int k = 0; k < kExDepth; k++) {
      const int u = u0 + k;
      if (u >= nu) break;  // the same in every thread
      if (!kBwd && u == nt) {
        // the second pass's terms need the means: wavefront 0 has written them
        // after its last first-pass tile
        __syncthreads();
      }
      if (wave > 0) {
        store_tile(u, k);
        if (u + kExDepth < nu) load_tile(u + kExDepth, k);
      }
      // tile u is staged in buffer u & 1; the buffer written next round was
      // last read before this barrier
      __syncthreads();
      if (wave == 0) {
        const int cmax = min(kExTile, C - (u % nt) * kExTile);
        const float *X = tile + (u & 1) * kArr * kTileF + lane * kExPitch;
        if (cmax == kExTile) {
          const float4 *t[kArr];
#pragma unroll
          for (int a = 0; a < kArr; a++) t[a] = reinterpret_cast<const float4 *>(X + a * kTileF);
          chain_add4<kArr, kExBatch / kArr>(s, t, kExTile / 4);
        } else {
          for (int c = 0; c < cmax; c++) {
#pragma unroll
            for (int a = 0; a < kArr; a++) s[a] = s[a] + X[a * kTileF + c];
          }
        }
        if (!kBwd && u == nt - 1) {
          stat[lane].x = s[0] / Cf;
          s[0] = 0.0f;
        }
      }
    }
  }
  if (wave == 0) {
    if (kBwd) {
      rsum[lane] = make_float2(s[0] / Cf, s[kArr - 1] / Cf);
    } else {
      const float m = stat[lane].x;
      const float r = 1.0f / sqrtf(s[0] / Cf + 1e-5f);
      if (lane < kExRows && r0 + lane < rows) {
        mean[r0 + lane] = m;
        rstd[r0 + lane] = r;
      }
      stat[lane].y = r;
    }
  }
  __syncthreads();
  // the rows' elements, every wavefront on whole rows (inp and dout again,
  // from the cache), all the loads of a batch issued together
  for (int ri = wave; ri < kExRows; ri += kExLoaders + 1) {
    const int row = r0 + ri;
    if (row >= rows) break;
    const float m = stat[ri].x, r = stat[ri].y;
    const float2 rs = kBwd ? rsum[ri] : make_float2(0.0f, 0.0f);
    const size_t base = (size_t)row * C;
    if constexpr (kVec) {
      const int C4 = C >> 2;
      const float4 *x4 = reinterpret_cast<const float4 *>(inp + base);
      const float4 *y4 = reinterpret_cast<const float4 *>(kBwd ? dout + base : bias);
      const float4 *w4 = reinterpret_cast<const float4 *>(weight);
      float4 *o4 = reinterpret_cast<float4 *>(outp + base);
      for (int q0 = 0; q0 < C4; q0 += kExApplyVec * kWave) {
        float4 xv[kExApplyVec], wv[kExApplyVec], yv[kExApplyVec], dv[kExApplyVec];
#pragma unroll
        for (int k = 0; k < kExApplyVec; k++) {
          const int q = min(q0 + k * kWave + lane, C4 - 1);
          xv[k] = x4[q];
          wv[k] = w4[q];
          yv[k] = y4[q];
          if (kBwd) dv[k] = o4[q];
        }
#pragma unroll
        for (int k = 0; k < kExApplyVec; k++) {
          const int q = q0 + k * kWave + lane;
          if (q < C4) {
            float o[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
              const float xj = f4_get(xv[k], j), wj = f4_get(wv[k], j), yj = f4_get(yv[k], j);
              if (kBwd) {
                const float xh = (xj - m) * r;
                const float dn = yj * wj;
                o[j] = f4_get(dv[k], j) + r * (dn - rs.x - xh * rs.y);
              } else {
                o[j] = (xj - m) * r * wj + yj;
              }
            }
            o4[q] = make_float4(o[0], o[1], o[2], o[3]);
          }
        }
      }
    } else {
      for (int c0 = 0; c0 < C; c0 += kExApply * kWave) {
        float xv[kExApply], wv[kExApply], yv[kExApply], dv[kExApply];
#pragma unroll
        for (int k = 0; k < kExApply; k++) {
          const int c = min(c0 + k * kWave + lane, C - 1);
          xv[k] = inp[base + c];
          wv[k] = weight[c];
          yv[k] = kBwd ? dout[base + c] : bias[c];
          dv[k] = kBwd ? outp[base + c] : 0.0f;
        }
#pragma unroll
        for (int k = 0; k < kExApply; k++) {
          const int c = c0 + k * kWave + lane;
          if (c < C) {
            if (kBwd) {
              const float xh = (xv[k] - m) * r;
              const float dn = yv[k] * wv[k];
              outp[base + c] = dv[k] + r * (dn - rs.x - xh * rs.y);
            } else {
              outp[base + c] = (xv[k] - m) * r * wv[k] + yv[k];
            }
          }
        }
      }
    }
  }
}

template <bool kVec>
__device__ __forceinline__ void ln_cols_exact(float *lds, int blk, float *__restrict__ dweight,
                                              float *__restrict__ dbias, const float *__restrict__ dout,
                                              const float *__restrict__ inp, const float *__restrict__ mean,
                                              const float *__restrict__ rstd, int rows, int C) {
  constexpr int kTileF = kExChains * kExColPitch;
  constexpr int kSlots = kVec ? 1 : kExColSlots;
  constexpr int kW = kVec ? 4 : 1;  // floats per lane and slot
  float *const tile = lds;  // [2][kExChains][kExColPitch]: chain j's terms of the tile's rows
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
  const int c0 = blk * kExCols;
  const int nt = (rows + kExColRows - 1) / kExColRows;
  // Loader lane L = 64 lw + lane. Scalar: slot sl holds tile row
  // 4 lw + 60 sl + lane / 16, column lane % 16. float4: tile row L / 4,
  // columns 4 (L % 4) + 0..3.
  const int lw = wave - 1;
  const int L = lw * kWave + lane;
  const int lc = kVec ? 4 * (L & 3) : (lane & (kExCols - 1));
  const int lcol = min(c0 + lc, C - kW);
  float rx[kExDepth][kSlots][kW], ry[kExDepth][kSlots][kW], rm[kExDepth][kSlots], rr[kExDepth][kSlots];
  auto tile_row = [&](int sl) {
    return kVec ? L >> 2 : (kWave / kExCols) * (lw + kExLoaders * sl) + lane / kExCols;
  };
  auto load_tile = [&](int t, int k) {
#pragma unroll
    for (int sl = 0; sl < kSlots; sl++) {
      const int row = min(t * kExColRows + tile_row(sl), rows - 1);
      const size_t off = (size_t)row * C + lcol;
      if constexpr (kVec) {
        const float4 x = *reinterpret_cast<const float4 *>(inp + off);
        const float4 y = *reinterpret_cast<const float4 *>(dout + off);
        rx[k][sl][0] = x.x, rx[k][sl][1] = x.y, rx[k][sl][2] = x.z, rx[k][sl][3] = x.w;
        ry[k][sl][0] = y.x, ry[k][sl][1] = y.y, ry[k][sl][2] = y.z, ry[k][sl][3] = y.w;
      } else {
        rx[k][sl][0] = inp[off];
        ry[k][sl][0] = dout[off];
      }
      rm[k][sl] = mean[row];
      rr[k][sl] = rstd[row];
    }
  };
  auto store_tile = [&](int t, int k) {
    float *const T = tile + (t & 1) * kTileF;
#pragma unroll
    for (int sl = 0; sl < kSlots; sl++) {
      const int ri = tile_row(sl);
#pragma unroll
      for (int j = 0; j < kW; j++) {
        const float xh = (rx[k][sl][j] - rm[k][sl]) * rr[k][sl];
        T[(lc + j) * kExColPitch + ri] = ry[k][sl][j] * xh;
        T[(kExCols + lc + j) * kExColPitch + ri] = ry[k][sl][j];
      }
    }
  };
  // the chain of wavefront 0's lane: dweight (lanes 0-15) or dbias (16-31) of
  // column c0 + lane % 16; lanes 32-63 follow a copy and store nothing
  const bool chain = wave == 0 && lane < kExChains;
  const int cc = c0 + (lane & (kExCols - 1));
  float *const dst = (lane < kExCols ? dweight : dbias) + min(cc, C - 1);
  float acc[1] = {chain ? *dst : 0.0f};
  if (wave > 0) {
#pragma unroll
    for (int k = 0; k < kExDepth; k++)
      if (k < nt) load_tile(k, k);
  }
  for (int t0 = 0; t0 < nt; t0 += kExDepth) {
#pragma unroll
    for (int k = 0; k < kExDepth; k++) {
      const int t = t0 + k;
      if (t >= nt) break;  // the same in every thread
      if (wave > 0) {
        store_tile(t, k);
        if (t + kExDepth < nt) load_tile(t + kExDepth, k);
      }
      __syncthreads();
      if (wave == 0) {
        const float *T = tile + (t & 1) * kTileF + (lane & (kExChains - 1)) * kExColPitch;
        const int rmax = min(kExColRows, rows - t * kExColRows);
        if (rmax == kExColRows) {
          const float4 *t4[1] = {reinterpret_cast<const float4 *>(T)};
          chain_add4<1, kExColBatch>(acc, t4, kExColRows / 4);
        } else {
          for (int i = 0; i < rmax; i++) acc[0] = acc[0] + T[i];
        }
      }
    }
  }
  if (chain && cc < C) *dst = acc[0];
}

template <bool kVec>
__global__ __launch_bounds__(kExThreads) void k_ln_fwd_exact(float *__restrict__ out, float *__restrict__ mean,
                                                             float *__restrict__ rstd, const float *__restrict__ inp,
                                                             const float *__restrict__ weight,
                                                             const float *__restrict__ bias, int rows, int C) {
  __shared__ __align__(16) float lds[ex_row_lds(1)];
  ln_rows_exact<false, kVec>(lds, blockIdx.x, out, mean, rstd, inp, nullptr, weight, bias, rows, C);
}

// workgroups [0, nrow) the rows (dinp), the others the columns (dweight, dbias)
template <bool kVec>
__global__ __launch_bounds__(kExThreads) void k_ln_bwd_exact(float *__restrict__ dinp, float *__restrict__ dweight,
                                                             float *__restrict__ dbias, const float *__restrict__ dout,
                                                             const float *__restrict__ inp,
                                                             const float *__restrict__ weight,
                                                             const float *__restrict__ mean,
                                                             const float *__restrict__ rstd, int rows, int C,
                                                             int nrow) {
  __shared__ __align__(16) float lds[kExBwdLds];
  if ((int)blockIdx.x < nrow)
    ln_rows_exact<true, kVec>(lds, blockIdx.x, dinp, const_cast<float *>(mean), const_cast<float *>(rstd), inp, dout,
                              weight, nullptr, rows, C);
  else
    ln_cols_exact<kVec>(lds, (int)blockIdx.x - nrow, dweight, dbias, dout, inp, mean, rstd, rows, C);
}

}  // namespace

namespace {
std::atomic<int> g_ln_exact{0};
}  // namespace

void set_layernorm_exact(int on) { g_ln_exact.store(on ? 1 : 0); }
int layernorm_exact() { return g_ln_exact.load(); }

int launch_layernorm_forward_exact(float *out, float *mean, float *rstd, const float *inp, const float *weight,
                                   const float *bias, int rows, int C) {
  if (rows == 0 || C == 0) return 0;
  const bool vec = C % 4 == 0 && aligned16(out) && aligned16(inp) && aligned16(weight) && aligned16(bias);
  const dim3 grid(grid_for((size_t)rows, kExRows)), block(kExThreads);
  if (vec)
    launch(k_ln_fwd_exact<true>, grid, block, 0, out, mean, rstd, inp, weight, bias, rows, C);
  else
    launch(k_ln_fwd_exact<false>, grid, block, 0, out, mean, rstd, inp, weight, bias, rows, C);
  return check_launch("layernorm_forward (exact)");
}

int launch_layernorm_backward_exact(float *dinp, float *dweight, float *dbias, const float *dout, const float *inp,
                                    const float *weight, const float *mean, const float *rstd, int rows, int C) {
  if (rows == 0 || C == 0) return 0;
  const bool vec = C % 4 == 0 && aligned16(dinp) && aligned16(dout) && aligned16(inp) && aligned16(weight);
  const int nrow = (int)grid_for((size_t)rows, kExRows), ncol = (int)grid_for((size_t)C, kExCols);
  const dim3 grid(nrow + ncol), block(kExThreads);
  if (vec)
    launch(k_ln_bwd_exact<true>, grid, block, 0, dinp, dweight, dbias, dout, inp, weight, mean, rstd, rows, C, nrow);
  else
    launch(k_ln_bwd_exact<false>, grid, block, 0, dinp, dweight, dbias, dout, inp, weight, mean, rstd, rows, C, nrow);
  return check_launch("layernorm_backward (exact)");
}

int launch_layernorm_forward(float *out, float *mean, float *rstd, const float *inp,
                             const float *weight, const float *bias, int rows, int C) {
  if (rows == 0) return 0;
  if (layernorm_exact()) return launch_layernorm_forward_exact(out, mean, rstd, inp, weight, bias, rows, C);
  if (vec_ok(C, {out, inp, weight, bias})) {
    launch_ln_fwd_vec<false>(out, mean, rstd, inp, weight, bias, rows, C, nullptr, nullptr);
  } else {
    const dim3 grid(grid_for((size_t)rows, kWavesPerBlock)), block(kBlock);
    launch(k_ln_fwd_scalar, grid, block, 0, out, mean, rstd, inp, weight, bias,
                       rows, C);
  }
  return check_launch("layernorm_forward");
}

namespace {
// tail: the workgroups finish the column sums into dweight/dbias themselves
// (ln_bwd_tail); only for the per-op modes (dinp read and written, residual
// targets read).
template <bool kRes, int kDinp, bool kAssign>
int launch_ln_bwd_vec(float *dinp, float *partial, const float *dout, const float *inp,
                      const float *weight, const float *mean, const float *rstd, int rows, int C,
                      float *rdx, float *rdy, int max_blocks, bool tail = false, float *dweight = nullptr,
                      float *dbias = nullptr) {
  static_assert(kRes || (kDinp == kDinpRw && !kAssign), "the plain backward reads and writes dinp");
  constexpr bool kTailOk = kDinp == kDinpRw && !kAssign;
  int nblk, rpw;
  const int V = ((C >> 2) + kWave - 1) / kWave;
  const int same = rdx == rdy ? 1 : 0;
  const bool nt = (size_t)rows * (size_t)C < ((size_t)1 << 21);
  // the kernel with and without the in-launch column sums
  const auto both = [&](auto k_plain, auto k_tail, dim3 grid, dim3 block, int rp) {
    if (kTailOk && tail)
      launch(k_tail, grid, block, 0, dinp, partial, dout, inp, weight, mean, rstd, rows, C, rp, rdx, rdy, same,
             dweight, dbias);
    else
      launch(k_plain, grid, block, 0, dinp, partial, dout, inp, weight, mean, rstd, rows, C, rp, rdx, rdy, same,
             nullptr, nullptr);
  };
  if (team_path(rows, C)) {
    int rpt;
    team_shape(rows, max_blocks, &nblk, &rpt);
    const dim3 grid(nblk), block(kTeamParts * kTeams * kWave);
    if constexpr (kRes)
      both(k_ln_bwd_team<kTeamParts, kTeams, 4, true, 3, true, kDinp, kAssign, false>,
           k_ln_bwd_team<kTeamParts, kTeams, 4, true, 3, true, kDinp, kAssign, kTailOk>, grid, block, rpt);
    else if (nt)
      both(k_ln_bwd_team<kTeamParts, kTeams, 2, false, 1, true, kDinpRw, false, false>,
           k_ln_bwd_team<kTeamParts, kTeams, 2, false, 1, true, kDinpRw, false, true>, grid, block, rpt);
    else
      both(k_ln_bwd_team<kTeamParts, kTeams, 2, false, 1, false, kDinpRw, false, false>,
           k_ln_bwd_team<kTeamParts, kTeams, 2, false, 1, false, kDinpRw, false, true>, grid, block, rpt);
    return nblk;
  }
  const BwdCfg k = bwd_cfg(V, kRes);
  bwd_shape_vec(rows, k, max_blocks, &nblk, &rpw);
  const dim3 grid(nblk), block(k.W * kWave);
  switch (V) {
#define UGK_LN_BWD_K(v, ntv, tl)                                                                                    \
  k_ln_bwd_vec<v, bwd_cfg(v, kRes).W, bwd_cfg(v, kRes).R, kRes, bwd_cfg(v, kRes).MINW, ntv, kDinp, kAssign, tl>
#define UGK_LN_BWD(v)                                                                                               \
  case v:                                                                                                           \
    if (kRes || nt)                                                                                                 \
      both(UGK_LN_BWD_K(v, true, false), UGK_LN_BWD_K(v, true, kTailOk), grid, block, rpw);                         \
    else                                                                                                            \
      both(UGK_LN_BWD_K(v, kRes, false), UGK_LN_BWD_K(v, kRes, kTailOk), grid, block, rpw);                         \
    break;
    UGK_LN_BWD(1) UGK_LN_BWD(2) UGK_LN_BWD(3) UGK_LN_BWD(4)
    UGK_LN_BWD(5) UGK_LN_BWD(6) UGK_LN_BWD(7) UGK_LN_BWD(8)
#undef UGK_LN_BWD
#undef UGK_LN_BWD_K
  }
  return nblk;
}

// Whether the per-op backward finishes its column sums in the main launch (1)
// or in a second one (0, the default: faster, see ln_bwd_tail); both give the
// same bits.
std::atomic<int> g_ln_tail{0};
}  // namespace

void set_layernorm_tail(int on) { g_ln_tail.store(on ? 1 : 0); }
int layernorm_tail() { return g_ln_tail.load(); }

int launch_layernorm_backward_partials(float *dinp, float *partial, float *dx, float *dy, const float *dout,
                                       const float *inp, const float *weight, const float *mean,
                                       const float *rstd, int rows, int C, int max_blocks, int *nblk,
                                       int dinp_mode, bool assign_res) {
  *nblk = 0;
  if (rows == 0) return 0;
  const bool res = dx != nullptr;
  if (vec_ok(C, {dinp, dout, inp, weight}) && (!res || vec_ok(C, {dx, dy}))) {
#define UGK_LN_BWD_MODE(d, a) \
  launch_ln_bwd_vec<true, d, a>(dinp, partial, dout, inp, weight, mean, rstd, rows, C, dx, dy, max_blocks)
    if (!res)
      *nblk = launch_ln_bwd_vec<false, kDinpRw, false>(dinp, partial, dout, inp, weight, mean, rstd, rows, C,
                                                       nullptr, nullptr, max_blocks);
    else if (dinp_mode == kDinpRw && !assign_res)
      *nblk = UGK_LN_BWD_MODE(kDinpRw, false);
    else if (dinp_mode == kDinpRead && !assign_res)
      *nblk = UGK_LN_BWD_MODE(kDinpRead, false);
    else if (dinp_mode == kDinpRead)
      *nblk = UGK_LN_BWD_MODE(kDinpRead, true);
    else if (dinp_mode == kDinpNone && assign_res)
      *nblk = UGK_LN_BWD_MODE(kDinpNone, true);
    else
      return set_error(UGK_EINVAL, "layernorm_backward: unsupported dinp mode %d with assign %d", dinp_mode,
                       (int)assign_res);
#undef UGK_LN_BWD_MODE
    return check_launch("layernorm_backward");
  }
  int rpb;
  bwd_shape(rows, max_blocks < kMaxScalarBlocks ? max_blocks : kMaxScalarBlocks, nblk, &rpb);
  launch(k_ln_bwd_scalar, dim3(*nblk), dim3(kBlock), 0, dinp, partial, dout, inp, weight,
                     mean, rstd, rows, C, rpb);
  if (int e = check_launch("layernorm_backward")) return e;
  return res ? launch_residual_backward(dx, dy, dinp, (size_t)rows * C) : 0;
}

int launch_layernorm_reduce(const LnReduceJob *jobs, int njobs, int C) {
  for (int j0 = 0; j0 < njobs; j0 += kMaxReduceJobs) {
    LnReduceBatch b{};
    const int n = njobs - j0 < kMaxReduceJobs ? njobs - j0 : kMaxReduceJobs;
    for (int k = 0; k < n; k++) b.job[k] = jobs[j0 + k];
    launch(k_ln_bwd_reduce_batch, dim3(grid_for((size_t)2 * C, kRedCols), n), dim3(kRedCols * kRedGroups), 0, b,
           C);
  }
  return check_launch("layernorm_backward (column sums)");
}

int launch_layernorm_residual_backward_into(float *partial, int max_blocks, float *dinp, float *dweight,
                                            float *dbias, float *dx, float *dy, const float *dout,
                                            const float *inp, const float *weight, const float *mean,
                                            const float *rstd, int rows, int C) {
  if (rows == 0) return 0;
  const bool res = dx != nullptr;
  if (layernorm_exact()) {  // no partial rows: the exact kernels keep their chains in LDS and registers
    if (int e = launch_layernorm_backward_exact(dinp, dweight, dbias, dout, inp, weight, mean, rstd, rows, C))
      return e;
    return res ? launch_residual_backward(dx, dy, dinp, (size_t)rows * C) : 0;
  }
  if (layernorm_tail() && vec_ok(C, {dinp, dout, inp, weight}) && (!res || vec_ok(C, {dx, dy}))) {
    if (res)
      launch_ln_bwd_vec<true, kDinpRw, false>(dinp, partial, dout, inp, weight, mean, rstd, rows, C, dx, dy,
                                              max_blocks, true, dweight, dbias);
    else
      launch_ln_bwd_vec<false, kDinpRw, false>(dinp, partial, dout, inp, weight, mean, rstd, rows, C, nullptr,
                                               nullptr, max_blocks, true, dweight, dbias);
    return check_launch("layernorm_backward");
  }
  int nblk;
  if (int e = launch_layernorm_backward_partials(dinp, partial, dx, dy, dout, inp, weight, mean, rstd, rows, C,
                                                 max_blocks, &nblk))
    return e;
  const LnReduceJob job{partial, dweight, dbias, nblk};
  return launch_layernorm_reduce(&job, 1, C);
}

int launch_layernorm_residual_backward(float *dinp, float *dweight, float *dbias, float *dx, float *dy,
                                       const float *dout, const float *inp, const float *weight,
                                       const float *mean, const float *rstd, int rows, int C) {
  if (rows == 0) return 0;
  float *partial = static_cast<float *>(workspace(kRegLn, layernorm_backward_scratch(rows, C)));
  if (!partial) return UGK_ENOMEM;
  // the workspace holds the bound's number of partial rows, and no shape takes
  // more workgroups than the cap it is given
  return launch_layernorm_residual_backward_into(partial, layernorm_backward_blocks_bound(rows, C), dinp, dweight,
                                                 dbias, dx, dy, dout, inp, weight, mean, rstd, rows, C);
}

// ---- allocation-free variant ------------------------------------------------
// The partial rows in a file-scope device array (one copy per GPU, held until
// the process ends) instead of the workspace. Host code never passes the
// array's name to a kernel (on the host it stands for a host-side shadow):
// it looks up the array's device address once per device with
// hipGetSymbolAddress and passes that.
}  // namespace ugk

static __device__ __align__(256) float scratch[ugk::kNoAllocScratchBytes / sizeof(float)];

namespace ugk {
namespace {
struct NoAllocAddr {
  float *ptr = nullptr;
  hipError_t err = hipSuccess;
  bool looked_up = false;
};
NoAllocAddr g_noalloc[64];
std::mutex g_noalloc_mu;
}  // namespace

float *noalloc_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    set_error(UGK_EHIP, "no-alloc scratch: hipGetDevice failed");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  NoAllocAddr &a = g_noalloc[dev];
  if (!a.looked_up) {  // once per device, with that device current
    void *p = nullptr;
    a.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (a.err != hipSuccess) (void)hipGetLastError();
    a.ptr = a.err == hipSuccess ? static_cast<float *>(p) : nullptr;
    a.looked_up = true;
  }
  if (!a.ptr) set_error(UGK_EHIP, "no-alloc scratch: hipGetSymbolAddress failed: %s", hipGetErrorString(a.err));
  return a.ptr;
}

int noalloc_max_blocks(int C) {
  const size_t per_row = 2 * (size_t)C * sizeof(float);
  const size_t fit = kNoAllocScratchBytes / per_row;
  return fit < (size_t)kMaxPartialRows ? (int)fit : kMaxPartialRows;
}

int launch_layernorm_backward(float *dinp, float *dweight, float *dbias, const float *dout,
                              const float *inp, const float *weight, const float *mean,
                              const float *rstd, int rows, int C) {
  return launch_layernorm_residual_backward(dinp, dweight, dbias, nullptr, nullptr, dout, inp, weight, mean,
                                            rstd, rows, C);
}

}  // namespace ugk
