// ugk_layernorm.hip - LayerNorm forward and backward (train_bnn.c:81-115,
// :439-477).
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
// Backward: one wavefront per row for dinp (two wavefront sums), and the
// dweight/dbias column sums are accumulated per wavefront (in LDS) across the
// rows it visits, then combined in a fixed order: the wavefronts of a
// workgroup through an LDS tree into one partial row per workgroup (at most
// 512 workgroups), then the partial rows in index order by a small second
// kernel that adds the totals into dweight/dbias. No atomics, so the result
// is identical run to run.
// Streamed rows (x, dout, dinp, out) use non-temporal loads and stores.
#include "ugk_internal.h"

namespace ugk {
namespace {

constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kMaxV = 8;  // float4 per lane held in registers: C <= 2048
constexpr int kMaxBwdBlocks = 512;

// kRes: the row is first formed as res = inp + inp2 (residual_forward,
// train_bnn.c:182-186), stored to res, and normalised from the registers, the
// pair gpt2_kernels.cuh:793-797 launches back to back.
template <int V, bool kRes>
__global__ __launch_bounds__(kBlock) void k_ln_fwd_vec(float *__restrict__ out, float *__restrict__ mean,
                                                       float *__restrict__ rstd,
                                                       const float *__restrict__ inp,
                                                       const float *__restrict__ weight,
                                                       const float *__restrict__ bias, int rows, int C,
                                                       float *__restrict__ res, const float *__restrict__ inp2) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int C4 = C >> 2;
  const float4 *x4 = reinterpret_cast<const float4 *>(inp + (size_t)row * C);
  float4 xv[V];
#pragma unroll
  for (int v = 0; v < V; v++) {
    const int c4 = lane + v * kWave;
    xv[v] = (c4 < C4) ? ld_nt(x4 + c4) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (kRes) {
    const float4 *y4 = reinterpret_cast<const float4 *>(inp2 + (size_t)row * C);
    float4 *r4 = reinterpret_cast<float4 *>(res + (size_t)row * C);
    float4 yv[V];
#pragma unroll
    for (int v = 0; v < V; v++) {
      const int c4 = lane + v * kWave;
      yv[v] = (c4 < C4) ? ld_nt(y4 + c4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int v = 0; v < V; v++) {
      xv[v] = make_float4(xv[v].x + yv[v].x, xv[v].y + yv[v].y, xv[v].z + yv[v].z, xv[v].w + yv[v].w);
      if (lane + v * kWave < C4) st_nt(r4 + lane + v * kWave, xv[v]);
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int v = 0; v < V; v++) {
    s += xv[v].x; s += xv[v].y; s += xv[v].z; s += xv[v].w;
  }
  s = wave_sum(s);
  const float m = s / (float)C;
  float vs = 0.0f;
#pragma unroll
  for (int v = 0; v < V; v++) {
    if (lane + v * kWave < C4) {
      float d;
      d = xv[v].x - m; vs += d * d;
      d = xv[v].y - m; vs += d * d;
      d = xv[v].z - m; vs += d * d;
      d = xv[v].w - m; vs += d * d;
    }
  }
  vs = wave_sum(vs);
  const float r = 1.0f / sqrtf(vs / (float)C + 1e-5f);
  const float4 *w4 = reinterpret_cast<const float4 *>(weight);
  const float4 *b4 = reinterpret_cast<const float4 *>(bias);
  float4 *o4 = reinterpret_cast<float4 *>(out + (size_t)row * C);
#pragma unroll
  for (int v = 0; v < V; v++) {
    const int c4 = lane + v * kWave;
    if (c4 < C4) {
      const float4 w = w4[c4], b = b4[c4];
      float4 o;
      o.x = (xv[v].x - m) * r * w.x + b.x;
      o.y = (xv[v].y - m) * r * w.y + b.y;
      o.z = (xv[v].z - m) * r * w.z + b.z;
      o.w = (xv[v].w - m) * r * w.w + b.w;
      st_nt(o4 + c4, o);
    }
  }
  if (lane == 0) {
    mean[row] = m;
    rstd[row] = r;
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

// Backward, register-resident rows. A workgroup is W wavefronts; wavefront w
// of workgroup g takes the rpw consecutive rows starting at (W g + w) * rpw,
// R at a time (the loads of R rows are in flight together), writes dinp and
// adds the dweight/dbias terms of its rows, in row order, into its own column
// sums in LDS. The W wavefronts' sums are then folded pairwise (upper half
// into lower half, a fixed tree) and wavefront 0 writes the workgroup's
// partial row: partial[g] = [dweight part (C floats) | dbias part (C floats)].
//
// kRes: the new dinp row is also added to rdx and rdy (residual_backward with
// dout = dinp, train_bnn.c:491-496; twice into rdx when same), the pair
// gpt2_kernels.cuh:870-876 launches back to back. The rdx/rdy rows are loaded
// with the others, before any arithmetic.
template <int V, int W, int R, bool kRes>
__global__ __launch_bounds__(W * kWave) void k_ln_bwd_vec(
    float *__restrict__ dinp, float *__restrict__ partial, const float *__restrict__ dout,
    const float *__restrict__ inp, const float *__restrict__ weight, const float *__restrict__ mean,
    const float *__restrict__ rstd, int rows, int C, int rpw, float *__restrict__ rdx,
    float *__restrict__ rdy, int same) {
  // the weight row, and each wavefront's dweight/dbias column sums, live in
  // LDS rather than registers, which leaves the registers to the rows in
  // flight and lets two workgroups share a CU
  __shared__ float4 w4s[V * kWave];
  __shared__ float4 acc[W][2][V * kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int C4 = C >> 2;
  const float Cf = (float)C;
  const float4 *w4 = reinterpret_cast<const float4 *>(weight);
  for (int e = threadIdx.x; e < V * kWave; e += W * kWave) w4s[e] = e < C4 ? w4[e] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int v = 0; v < V; v++) {
    acc[wave][0][v * kWave + lane] = make_float4(0.f, 0.f, 0.f, 0.f);
    acc[wave][1][v * kWave + lane] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  __syncthreads();
  const int row0 = (blockIdx.x * W + wave) * rpw;
  const int row1 = min(row0 + rpw, rows);
  for (int row = row0; row < row1; row += R) {
    const int nr = min(R, row1 - row);
    float4 x[R][V], dy[R][V], dx[R][V];
    float4 ra[kRes ? R : 1][kRes ? V : 1], rb[kRes ? R : 1][kRes ? V : 1];
    float m[R], r[R];
#pragma unroll
    for (int q = 0; q < R; q++) {
      const int rq = q < nr ? row + q : row;
      const float4 *x4 = reinterpret_cast<const float4 *>(inp + (size_t)rq * C);
      const float4 *dy4 = reinterpret_cast<const float4 *>(dout + (size_t)rq * C);
      const float4 *dx4 = reinterpret_cast<const float4 *>(dinp + (size_t)rq * C);
#pragma unroll
      for (int v = 0; v < V; v++) {
        const int c4 = lane + v * kWave;
        if (c4 < C4 && q < nr) {
          x[q][v] = ld_nt(x4 + c4);
          dy[q][v] = ld_nt(dy4 + c4);
          dx[q][v] = ld_nt(dx4 + c4);
        } else {
          x[q][v] = dy[q][v] = dx[q][v] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      if (kRes) {
        const float4 *a4 = reinterpret_cast<const float4 *>(rdx + (size_t)rq * C);
        const float4 *b4 = reinterpret_cast<const float4 *>(rdy + (size_t)rq * C);
#pragma unroll
        for (int v = 0; v < V; v++) {
          const int c4 = lane + v * kWave;
          const bool in = c4 < C4 && q < nr;
          ra[q][v] = in ? ld_nt(a4 + c4) : make_float4(0.f, 0.f, 0.f, 0.f);
          rb[q][v] = (in && !same) ? ld_nt(b4 + c4) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
      m[q] = mean[rq];
      r[q] = rstd[rq];
    }
    float s1[R], s2[R];
#pragma unroll
    for (int q = 0; q < R; q++) {
      s1[q] = 0.0f;
      s2[q] = 0.0f;
#pragma unroll
      for (int v = 0; v < V; v++) {
        const float4 w = w4s[v * kWave + lane];
        float4 xh, dn;
        xh.x = (x[q][v].x - m[q]) * r[q]; dn.x = dy[q][v].x * w.x;
        xh.y = (x[q][v].y - m[q]) * r[q]; dn.y = dy[q][v].y * w.y;
        xh.z = (x[q][v].z - m[q]) * r[q]; dn.z = dy[q][v].z * w.z;
        xh.w = (x[q][v].w - m[q]) * r[q]; dn.w = dy[q][v].w * w.w;
        if (lane + v * kWave < C4) {
          s1[q] += dn.x; s2[q] += dn.x * xh.x;
          s1[q] += dn.y; s2[q] += dn.y * xh.y;
          s1[q] += dn.z; s2[q] += dn.z * xh.z;
          s1[q] += dn.w; s2[q] += dn.w * xh.w;
        }
      }
    }
#pragma unroll
    for (int q = 0; q < R; q++) {
      s1[q] = wave_sum(s1[q]);
      s2[q] = wave_sum(s2[q]);
    }
#pragma unroll
    for (int q = 0; q < R; q++) {
      if (q >= nr) break;
      const float dnm = s1[q] / Cf, dnxm = s2[q] / Cf;
      float4 *dx4 = reinterpret_cast<float4 *>(dinp + (size_t)(row + q) * C);
#pragma unroll
      for (int v = 0; v < V; v++) {
        const int c4 = lane + v * kWave;
        if (c4 < C4) {
          const float4 w = w4s[c4];
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
          st_nt(dx4 + c4, o);
          if (kRes) {
            float4 *a4 = reinterpret_cast<float4 *>(rdx + (size_t)(row + q) * C);
            float4 *b4 = reinterpret_cast<float4 *>(rdy + (size_t)(row + q) * C);
            float4 a = ra[q][v];
            a = make_float4(a.x + o.x, a.y + o.y, a.z + o.z, a.w + o.w);
            if (same) {
              a = make_float4(a.x + o.x, a.y + o.y, a.z + o.z, a.w + o.w);
            } else {
              const float4 b = rb[q][v];
              st_nt(b4 + c4, make_float4(b.x + o.x, b.y + o.y, b.z + o.z, b.w + o.w));
            }
            st_nt(a4 + c4, a);
          }
          float4 g = acc[wave][0][c4], bb = acc[wave][1][c4];
          bb.x += dy[q][v].x; g.x += dy[q][v].x * xh.x;
          bb.y += dy[q][v].y; g.y += dy[q][v].y * xh.y;
          bb.z += dy[q][v].z; g.z += dy[q][v].z * xh.z;
          bb.w += dy[q][v].w; g.w += dy[q][v].w * xh.w;
          acc[wave][0][c4] = g;
          acc[wave][1][c4] = bb;
        }
      }
    }
  }
  // fold the W wavefronts' column sums: upper half adds into lower half
#pragma unroll
  for (int half = W / 2; half >= 1; half >>= 1) {
    __syncthreads();
    if (wave < half) {
#pragma unroll
      for (int v = 0; v < V; v++) {
        const int e = v * kWave + lane;
        const float4 g = acc[wave + half][0][e], b = acc[wave + half][1][e];
        float4 dg = acc[wave][0][e], db = acc[wave][1][e];
        dg.x += g.x; dg.y += g.y; dg.z += g.z; dg.w += g.w;
        db.x += b.x; db.y += b.y; db.z += b.z; db.w += b.w;
        acc[wave][0][e] = dg;
        acc[wave][1][e] = db;
      }
    }
  }
  if (wave == 0) {
    float4 *pg = reinterpret_cast<float4 *>(partial + (size_t)blockIdx.x * 2 * C);
    float4 *pb = reinterpret_cast<float4 *>(partial + (size_t)blockIdx.x * 2 * C + C);
#pragma unroll
    for (int v = 0; v < V; v++) {
      const int c4 = lane + v * kWave;
      if (c4 < C4) {
        pg[c4] = acc[0][0][c4];
        pb[c4] = acc[0][1][c4];
      }
    }
  }
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

// Column totals of the partial rows in workgroup order, added to dweight
// (columns [0,C)) and dbias (columns [C,2C)). Block: 64 columns x 16 groups;
// group k sums the partial rows [k*J, (k+1)*J), J = ceil(nblk/16) <= 32, with
// all its loads issued before the first add; the 16 group sums are then added
// in group order.
constexpr int kRedGroups = 16;
constexpr int kRedMaxPer = 32;
__device__ __forceinline__ void ln_bwd_reduce_tile(float *dweight, float *dbias, const float *partial, int nblk,
                                                   int C, float (*red)[kWave]) {
  const int cl = threadIdx.x & (kWave - 1);
  const int g = threadIdx.x >> 6;
  const int col = blockIdx.x * kWave + cl;
  const int C2 = 2 * C;
  const int J = (nblk + kRedGroups - 1) / kRedGroups;
  const int j0 = g * J, j1 = min(j0 + J, nblk);
  float v[kRedMaxPer];
#pragma unroll
  for (int q = 0; q < kRedMaxPer; q++)
    v[q] = (col < C2 && j0 + q < j1) ? partial[(size_t)(j0 + q) * C2 + col] : 0.0f;
  float acc = 0.0f;
#pragma unroll
  for (int q = 0; q < kRedMaxPer; q++) acc += v[q];
  red[g][cl] = acc;
  __syncthreads();
  if (g == 0 && col < C2) {
    float t = red[0][cl];
#pragma unroll
    for (int k = 1; k < kRedGroups; k++) t += red[k][cl];
    if (col < C)
      dweight[col] += t;
    else
      dbias[col - C] += t;
  }
}

__global__ __launch_bounds__(kWave * kRedGroups) void k_ln_bwd_reduce(float *dweight, float *dbias,
                                                                      const float *partial, int nblk,
                                                                      int C) {
  __shared__ float red[kRedGroups][kWave];
  ln_bwd_reduce_tile(dweight, dbias, partial, nblk, C, red);
}

// Several LayerNorm backwards' column totals in one launch (blockIdx.y picks
// the job); each job is reduced exactly as k_ln_bwd_reduce would.
constexpr int kMaxReduceJobs = 32;
struct LnReduceBatch {
  LnReduceJob job[kMaxReduceJobs];
};
__global__ __launch_bounds__(kWave * kRedGroups) void k_ln_bwd_reduce_batch(LnReduceBatch b, int C) {
  __shared__ float red[kRedGroups][kWave];
  const LnReduceJob &j = b.job[blockIdx.y];
  ln_bwd_reduce_tile(j.dweight, j.dbias, j.partial, j.nblk, C, red);
}

bool vec_ok(int C, std::initializer_list<const void *> ptrs) {
  if ((C & 3) != 0 || C > kMaxV * kWave * 4) return false;
  for (const void *p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

// Scalar path: workgroups of 4 wavefronts, at most 512 of them.
void bwd_shape(int rows, int *nblk, int *rpb) {
  int nb = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
  if (nb > kMaxBwdBlocks) nb = kMaxBwdBlocks;
  if (nb < 1) nb = 1;
  int per = (rows + nb - 1) / nb;
  per = (per + kWavesPerBlock - 1) / kWavesPerBlock * kWavesPerBlock;
  *rpb = per;
  *nblk = (rows + per - 1) / per;
}

// Rows whose loads a wavefront issues together: two while that fits the
// registers (C <= 768; measured 43.9 -> 41.7 us for the fused pair at config
// 5, where each wavefront then takes its two rows in one pass), else one.
constexpr int bwd_rows(int V) { return V <= 3 ? 2 : 1; }
// Vector path: W wavefronts per workgroup (8, or 4 when a lane holds more
// than 4 float4 of a row, so that the registers fit without spilling), rpw
// rows each, at most kBwdMaxBlocks workgroups, so the reduce reads at most 32
// partial rows per group.
constexpr int kBwdMaxBlocks = 512;
inline int bwd_waves(int V) { return V <= 4 ? 8 : 4; }
void bwd_shape_vec(int rows, int W, int *nblk, int *rpw) {
  const int per_wave = (rows + kBwdMaxBlocks * W - 1) / (kBwdMaxBlocks * W);
  *rpw = per_wave < 1 ? 1 : per_wave;
  *nblk = (rows + W * *rpw - 1) / (W * *rpw);
}

}  // namespace

size_t layernorm_backward_scratch(int rows, int C) {
  int nblk, rpb, nv, rpw;
  bwd_shape(rows, &nblk, &rpb);
  for (int W = 4; W <= 8; W *= 2) {
    bwd_shape_vec(rows, W, &nv, &rpw);
    if (nv > nblk) nblk = nv;
  }
  return (size_t)nblk * 2 * (size_t)C * sizeof(float);
}

namespace {
template <bool kRes>
void launch_ln_fwd_vec(float *out, float *mean, float *rstd, const float *inp, const float *weight,
                       const float *bias, int rows, int C, float *res, const float *inp2) {
  const dim3 grid(grid_for((size_t)rows, kWavesPerBlock)), block(kBlock);
  const int V = ((C >> 2) + kWave - 1) / kWave;
  switch (V) {
#define UGK_LN_FWD(v) \
  case v: hipLaunchKernelGGL((k_ln_fwd_vec<v, kRes>), grid, block, 0, stream(), out, mean, rstd, inp, weight, bias, rows, C, res, inp2); break;
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
  if (!vec_ok(C, {res, out, x, y, weight, bias})) {
    if (int e = launch_residual_forward(res, x, y, (size_t)rows * C)) return e;
    return launch_layernorm_forward(out, mean, rstd, res, weight, bias, rows, C);
  }
  launch_ln_fwd_vec<true>(out, mean, rstd, x, weight, bias, rows, C, res, y);
  return check_launch("residual_layernorm_forward");
}

int launch_layernorm_forward(float *out, float *mean, float *rstd, const float *inp,
                             const float *weight, const float *bias, int rows, int C) {
  if (rows == 0) return 0;
  const dim3 grid(grid_for((size_t)rows, kWavesPerBlock)), block(kBlock);
  if (vec_ok(C, {out, inp, weight, bias})) {
    launch_ln_fwd_vec<false>(out, mean, rstd, inp, weight, bias, rows, C, nullptr, nullptr);
  } else {
    hipLaunchKernelGGL(k_ln_fwd_scalar, grid, block, 0, stream(), out, mean, rstd, inp, weight, bias,
                       rows, C);
  }
  return check_launch("layernorm_forward");
}

namespace {
template <bool kRes>
int launch_ln_bwd_vec(float *dinp, float *partial, const float *dout, const float *inp,
                      const float *weight, const float *mean, const float *rstd, int rows, int C,
                      float *rdx, float *rdy) {
  int nblk, rpw;
  const int V = ((C >> 2) + kWave - 1) / kWave;
  const int W = bwd_waves(V);
  bwd_shape_vec(rows, W, &nblk, &rpw);
  const dim3 grid(nblk), block(W * kWave);
  const int same = rdx == rdy ? 1 : 0;
  switch (V) {
#define UGK_LN_BWD(v) \
  case v: hipLaunchKernelGGL((k_ln_bwd_vec<v, (v <= 4 ? 8 : 4), bwd_rows(v), kRes>), grid, block, 0, stream(), dinp, partial, dout, inp, weight, mean, rstd, rows, C, rpw, rdx, rdy, same); break;
    UGK_LN_BWD(1) UGK_LN_BWD(2) UGK_LN_BWD(3) UGK_LN_BWD(4)
    UGK_LN_BWD(5) UGK_LN_BWD(6) UGK_LN_BWD(7) UGK_LN_BWD(8)
#undef UGK_LN_BWD
  }
  return nblk;
}
}  // namespace

int launch_layernorm_backward_partials(float *dinp, float *partial, float *dx, float *dy, const float *dout,
                                       const float *inp, const float *weight, const float *mean,
                                       const float *rstd, int rows, int C, int *nblk) {
  *nblk = 0;
  if (rows == 0) return 0;
  const bool res = dx != nullptr;
  if (vec_ok(C, {dinp, dout, inp, weight}) && (!res || vec_ok(C, {dx, dy}))) {
    if (res)
      *nblk = launch_ln_bwd_vec<true>(dinp, partial, dout, inp, weight, mean, rstd, rows, C, dx, dy);
    else
      *nblk = launch_ln_bwd_vec<false>(dinp, partial, dout, inp, weight, mean, rstd, rows, C, nullptr, nullptr);
    return check_launch("layernorm_backward");
  }
  int rpb;
  bwd_shape(rows, nblk, &rpb);
  hipLaunchKernelGGL(k_ln_bwd_scalar, dim3(*nblk), dim3(kBlock), 0, stream(), dinp, partial, dout, inp, weight,
                     mean, rstd, rows, C, rpb);
  if (int e = check_launch("layernorm_backward")) return e;
  return res ? launch_residual_backward(dx, dy, dinp, (size_t)rows * C) : 0;
}

int launch_layernorm_reduce(const LnReduceJob *jobs, int njobs, int C) {
  for (int j0 = 0; j0 < njobs; j0 += kMaxReduceJobs) {
    LnReduceBatch b{};
    const int n = njobs - j0 < kMaxReduceJobs ? njobs - j0 : kMaxReduceJobs;
    for (int k = 0; k < n; k++) b.job[k] = jobs[j0 + k];
    hipLaunchKernelGGL(k_ln_bwd_reduce_batch, dim3(grid_for((size_t)2 * C, kWave), n), dim3(kWave * kRedGroups), 0,
                       stream(), b, C);
  }
  return check_launch("layernorm_backward (column sums)");
}

int launch_layernorm_residual_backward(float *dinp, float *dweight, float *dbias, float *dx, float *dy,
                                       const float *dout, const float *inp, const float *weight,
                                       const float *mean, const float *rstd, int rows, int C) {
  if (rows == 0) return 0;
  float *partial = static_cast<float *>(scratch(layernorm_backward_scratch(rows, C)));
  if (!partial) return UGK_ENOMEM;
  int nblk;
  if (int e = launch_layernorm_backward_partials(dinp, partial, dx, dy, dout, inp, weight, mean, rstd, rows, C,
                                                 &nblk))
    return e;
  hipLaunchKernelGGL(k_ln_bwd_reduce, dim3(grid_for((size_t)2 * C, kWave)), dim3(kWave * kRedGroups), 0,
                     stream(), dweight, dbias, partial, nblk, C);
  return check_launch("layernorm_residual_backward");
}

int launch_layernorm_backward(float *dinp, float *dweight, float *dbias, const float *dout,
                              const float *inp, const float *weight, const float *mean,
                              const float *rstd, int rows, int C) {
  return launch_layernorm_residual_backward(dinp, dweight, dbias, nullptr, nullptr, dout, inp, weight, mean,
                                            rstd, rows, C);
}

}  // namespace ugk
