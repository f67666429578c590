// ugk_layernorm.hip - LayerNorm forward and backward (train_bnn.c:81-115,
// :439-477).
//
// Layout: rows of C fp32 values, row-major; mean/rstd one float per row;
// weight/bias/dweight/dbias C floats.
//
// Forward: one wavefront per row. Each lane holds V float4 of the row in
// registers (V = ceil(C/256); C = 768 -> 3), so the row is read from HBM once
// and written once (8 bytes per element). Mean and variance are two-pass over
// the registers with 64-lane butterfly sums, rstd = 1/sqrtf(var/C + 1e-5)
// with IEEE division and square root, exactly the CPU formula.
//
// Backward: one wavefront per row for dinp (two butterfly sums), and the
// dweight/dbias column sums are carried in registers across the rows a
// wavefront visits, then combined in a fixed order: 4 wavefronts through LDS
// into one partial row per workgroup, then workgroups in index order by a
// small second kernel that adds the totals into dweight/dbias. No atomics, so
// the result is identical run to run.
#include "ugk_internal.h"

namespace ugk {
namespace {

constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kMaxV = 8;  // float4 per lane held in registers: C <= 2048
constexpr int kMaxBwdBlocks = 512;

template <int V>
__global__ __launch_bounds__(kBlock) void k_ln_fwd_vec(float *__restrict__ out, float *__restrict__ mean,
                                                       float *__restrict__ rstd,
                                                       const float *__restrict__ inp,
                                                       const float *__restrict__ weight,
                                                       const float *__restrict__ bias, int rows, int C) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int C4 = C >> 2;
  const float4 *x4 = reinterpret_cast<const float4 *>(inp + (size_t)row * C);
  float4 xv[V];
#pragma unroll
  for (int v = 0; v < V; v++) {
    const int c4 = lane + v * kWave;
    xv[v] = (c4 < C4) ? x4[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
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
      o4[c4] = o;
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

// Backward, register-resident rows. Workgroup g handles rows
// [g*rpb, min((g+1)*rpb, rows)); its wavefront w takes rows g*rpb + w + 4k.
// partial: one row of 2*C floats per workgroup, dweight part then dbias part.
template <int V>
__global__ __launch_bounds__(kBlock) void k_ln_bwd_vec(float *__restrict__ dinp, float *__restrict__ partial,
                                                       const float *__restrict__ dout,
                                                       const float *__restrict__ inp,
                                                       const float *__restrict__ weight,
                                                       const float *__restrict__ mean,
                                                       const float *__restrict__ rstd, int rows, int C,
                                                       int rpb) {
  __shared__ float red[kWavesPerBlock][2][V * kWave * 4];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x >> 6;
  const int C4 = C >> 2;
  const float Cf = (float)C;
  const float4 *w4 = reinterpret_cast<const float4 *>(weight);
  float4 w[V], dg[V], db[V];
#pragma unroll
  for (int v = 0; v < V; v++) {
    const int c4 = lane + v * kWave;
    w[v] = (c4 < C4) ? w4[c4] : make_float4(0.f, 0.f, 0.f, 0.f);
    dg[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    db[v] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const int row0 = blockIdx.x * rpb;
  const int row1 = min(row0 + rpb, rows);
  for (int row = row0 + wave; row < row1; row += kWavesPerBlock) {
    const float4 *x4 = reinterpret_cast<const float4 *>(inp + (size_t)row * C);
    const float4 *dy4 = reinterpret_cast<const float4 *>(dout + (size_t)row * C);
    float4 *dx4 = reinterpret_cast<float4 *>(dinp + (size_t)row * C);
    float4 x[V], dy[V], dx[V];
#pragma unroll
    for (int v = 0; v < V; v++) {
      const int c4 = lane + v * kWave;
      if (c4 < C4) {
        x[v] = x4[c4];
        dy[v] = dy4[c4];
        dx[v] = dx4[c4];
      } else {
        x[v] = dy[v] = dx[v] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    const float m = mean[row], r = rstd[row];
    float s1 = 0.0f, s2 = 0.0f;
    float4 xh[V], dn[V];
#pragma unroll
    for (int v = 0; v < V; v++) {
      xh[v].x = (x[v].x - m) * r; dn[v].x = dy[v].x * w[v].x;
      xh[v].y = (x[v].y - m) * r; dn[v].y = dy[v].y * w[v].y;
      xh[v].z = (x[v].z - m) * r; dn[v].z = dy[v].z * w[v].z;
      xh[v].w = (x[v].w - m) * r; dn[v].w = dy[v].w * w[v].w;
      if (lane + v * kWave < C4) {
        s1 += dn[v].x; s2 += dn[v].x * xh[v].x;
        s1 += dn[v].y; s2 += dn[v].y * xh[v].y;
        s1 += dn[v].z; s2 += dn[v].z * xh[v].z;
        s1 += dn[v].w; s2 += dn[v].w * xh[v].w;
      }
    }
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    const float dnm = s1 / Cf, dnxm = s2 / Cf;
#pragma unroll
    for (int v = 0; v < V; v++) {
      const int c4 = lane + v * kWave;
      if (c4 < C4) {
        float4 o;
        o.x = dx[v].x + r * (dn[v].x - dnm - xh[v].x * dnxm);
        o.y = dx[v].y + r * (dn[v].y - dnm - xh[v].y * dnxm);
        o.z = dx[v].z + r * (dn[v].z - dnm - xh[v].z * dnxm);
        o.w = dx[v].w + r * (dn[v].w - dnm - xh[v].w * dnxm);
        dx4[c4] = o;
        db[v].x += dy[v].x; dg[v].x += dy[v].x * xh[v].x;
        db[v].y += dy[v].y; dg[v].y += dy[v].y * xh[v].y;
        db[v].z += dy[v].z; dg[v].z += dy[v].z * xh[v].z;
        db[v].w += dy[v].w; dg[v].w += dy[v].w * xh[v].w;
      }
    }
  }
#pragma unroll
  for (int v = 0; v < V; v++) {
    const int c = (lane + v * kWave) * 4;
    red[wave][0][c + 0] = dg[v].x; red[wave][0][c + 1] = dg[v].y;
    red[wave][0][c + 2] = dg[v].z; red[wave][0][c + 3] = dg[v].w;
    red[wave][1][c + 0] = db[v].x; red[wave][1][c + 1] = db[v].y;
    red[wave][1][c + 2] = db[v].z; red[wave][1][c + 3] = db[v].w;
  }
  __syncthreads();
  float *prow = partial + (size_t)blockIdx.x * 2 * C;
  for (int c = threadIdx.x; c < C; c += kBlock) {
    float g = red[0][0][c], b = red[0][1][c];
#pragma unroll
    for (int k = 1; k < kWavesPerBlock; k++) {
      g += red[k][0][c];
      b += red[k][1][c];
    }
    prow[c] = g;
    prow[C + c] = b;
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
// group k sums partial rows k, k+16, ...; the 16 group sums are then added in
// group order.
constexpr int kRedGroups = 16;
__global__ __launch_bounds__(kWave * kRedGroups) void k_ln_bwd_reduce(float *dweight, float *dbias,
                                                                      const float *partial, int nblk,
                                                                      int C) {
  __shared__ float red[kRedGroups][kWave];
  const int cl = threadIdx.x & (kWave - 1);
  const int g = threadIdx.x >> 6;
  const int col = blockIdx.x * kWave + cl;
  const int C2 = 2 * C;
  float acc = 0.0f;
  if (col < C2)
    for (int j = g; j < nblk; j += kRedGroups) acc += partial[(size_t)j * C2 + col];
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

bool vec_ok(int C, std::initializer_list<const void *> ptrs) {
  if ((C & 3) != 0 || C > kMaxV * kWave * 4) return false;
  for (const void *p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

void bwd_shape(int rows, int *nblk, int *rpb) {
  int nb = (rows + kWavesPerBlock - 1) / kWavesPerBlock;
  if (nb > kMaxBwdBlocks) nb = kMaxBwdBlocks;
  if (nb < 1) nb = 1;
  int per = (rows + nb - 1) / nb;
  per = (per + kWavesPerBlock - 1) / kWavesPerBlock * kWavesPerBlock;
  *rpb = per;
  *nblk = (rows + per - 1) / per;
}

}  // namespace

size_t layernorm_backward_scratch(int rows, int C) {
  int nblk, rpb;
  bwd_shape(rows, &nblk, &rpb);
  return (size_t)nblk * 2 * (size_t)C * sizeof(float);
}

int launch_layernorm_forward(float *out, float *mean, float *rstd, const float *inp,
                             const float *weight, const float *bias, int rows, int C) {
  if (rows == 0) return 0;
  const dim3 grid(grid_for((size_t)rows, kWavesPerBlock)), block(kBlock);
  if (vec_ok(C, {out, inp, weight, bias})) {
    const int V = ((C >> 2) + kWave - 1) / kWave;
    switch (V) {
#define UGK_LN_FWD(v) \
  case v: hipLaunchKernelGGL(k_ln_fwd_vec<v>, grid, block, 0, stream(), out, mean, rstd, inp, weight, bias, rows, C); break;
      UGK_LN_FWD(1) UGK_LN_FWD(2) UGK_LN_FWD(3) UGK_LN_FWD(4)
      UGK_LN_FWD(5) UGK_LN_FWD(6) UGK_LN_FWD(7) UGK_LN_FWD(8)
#undef UGK_LN_FWD
    }
  } else {
    hipLaunchKernelGGL(k_ln_fwd_scalar, grid, block, 0, stream(), out, mean, rstd, inp, weight, bias,
                       rows, C);
  }
  return check_launch("layernorm_forward");
}

int launch_layernorm_backward(float *dinp, float *dweight, float *dbias, const float *dout,
                              const float *inp, const float *weight, const float *mean,
                              const float *rstd, int rows, int C) {
  if (rows == 0) return 0;
  int nblk, rpb;
  bwd_shape(rows, &nblk, &rpb);
  float *partial = static_cast<float *>(scratch(layernorm_backward_scratch(rows, C)));
  if (!partial) return 3;
  const dim3 grid(nblk), block(kBlock);
  if (vec_ok(C, {dinp, dout, inp, weight})) {
    const int V = ((C >> 2) + kWave - 1) / kWave;
    switch (V) {
#define UGK_LN_BWD(v) \
  case v: hipLaunchKernelGGL(k_ln_bwd_vec<v>, grid, block, 0, stream(), dinp, partial, dout, inp, weight, mean, rstd, rows, C, rpb); break;
      UGK_LN_BWD(1) UGK_LN_BWD(2) UGK_LN_BWD(3) UGK_LN_BWD(4)
      UGK_LN_BWD(5) UGK_LN_BWD(6) UGK_LN_BWD(7) UGK_LN_BWD(8)
#undef UGK_LN_BWD
    }
  } else {
    hipLaunchKernelGGL(k_ln_bwd_scalar, grid, block, 0, stream(), dinp, partial, dout, inp, weight,
                       mean, rstd, rows, C, rpb);
  }
  hipLaunchKernelGGL(k_ln_bwd_reduce, dim3(grid_for((size_t)2 * C, kWave)), dim3(kWave * kRedGroups), 0,
                     stream(), dweight, dbias, partial, nblk, C);
  return check_launch("layernorm_backward");
}

}  // namespace ugk
