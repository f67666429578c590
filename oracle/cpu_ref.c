/*
 * cpu_ref.c - CPU oracle for the uncertain-gpt layer-kernel set.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libugk.so or the ugk
 * Python package) links, loads or calls this file. Only tests/, the smoke()
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py use it, and
 * only as the checker or the timed CPU baseline.
 *
 * It restates the single-threaded fp32 ops of the reference oracle
 * train_bnn.c (kthaisociety/uncertain-gpt) with the same loop order and the
 * same evaluation order of every floating-point expression, so that, built
 * with gcc -O2 -ffp-contract=off for baseline x86-64 and linked to the same
 * glibc, it returns bit-identical results. Each function cites the lines it
 * restates. Pointers are host pointers; backward outputs accumulate (+=)
 * exactly like the reference.
 *
 * How it is pinned (tests/test_oracle.py):
 *   - against the reference itself, compiled from /root/reference/train_bnn.c
 *     by oracle/Makefile into oracle/_ref/ (bit-identical, every op, several
 *     shapes and seeds), when that build exists;
 *   - against committed fixtures in tests/golden/ produced from that build;
 *   - against mathematics that fixes each op independently of the loop code:
 *     encoder fwd is one IEEE add per element, encoder bwd equals a float64
 *     brute-force scatter within the fp32 rounding bound and reproduces
 *     encoder_backward_check's repeated-token case, LN satisfies its mean /
 *     variance / sum(dinp) invariants and matches a float64 recomputation,
 *     GELU matches float64 tanh within a few ulp and hits gelu(0)=0 and
 *     gelu'(0)=0.5 exactly, materialize hits eps=0 -> w=mu, rho>20 -> mu+rho*eps
 *     and rho<=-104 -> softplus=0.
 */
#include "cpu_ref.h"

#include <math.h>
#include <string.h>

/* train_bnn.c:41-65 */
void oracle_encoder_forward(float *out, const int *inp, const float *wte,
                            const float *wpe, int B, int T, int C) {
  for (int b = 0; b < B; b++) {
    for (int t = 0; t < T; t++) {
      int ix = inp[b * T + t];
      float *out_bt = out + (size_t)b * T * C + (size_t)t * C;
      const float *wte_ix = wte + (size_t)ix * C;
      const float *wpe_t = wpe + (size_t)t * C;
      for (int c = 0; c < C; c++) out_bt[c] = wte_ix[c] + wpe_t[c];
    }
  }
}

/* train_bnn.c:81-115 */
void oracle_layernorm_forward(float *out, float *mean, float *rstd,
                              const float *inp, const float *weight,
                              const float *bias, int B, int T, int C) {
  const float eps = 1e-5f;
  for (int b = 0; b < B; b++) {
    for (int t = 0; t < T; t++) {
      const float *x = inp + (size_t)b * T * C + (size_t)t * C;
      float *o = out + (size_t)b * T * C + (size_t)t * C;
      float sum = 0.0f;
      for (int c = 0; c < C; c++) sum += x[c];
      float m = sum / C;
      float varsum = 0.0f;
      for (int c = 0; c < C; c++) {
        float d = x[c] - m;
        varsum += d * d;
      }
      float r = 1.0f / sqrtf(varsum / C + eps);
      mean[b * T + t] = m;
      rstd[b * T + t] = r;
      for (int c = 0; c < C; c++) o[c] = (x[c] - m) * r * weight[c] + bias[c];
    }
  }
}

/* train_bnn.c:163-170 */
void oracle_gelu_forward(float *out, const float *inp, int N) {
  const float k = 0.7978845608f;
  for (int i = 0; i < N; i++) {
    float x = inp[i];
    float inner = k * (x + 0.044715f * x * x * x);
    out[i] = 0.5f * x * (1.0f + tanhf(inner));
  }
}

/* train_bnn.c:182-186 */
void oracle_residual_forward(float *out, const float *x, const float *y, int N) {
  for (int i = 0; i < N; i++) out[i] = x[i] + y[i];
}

/* train_bnn.c:439-477 */
void oracle_layernorm_backward(float *dinp, float *dweight, float *dbias,
                               const float *dout, const float *inp,
                               const float *weight, const float *mean,
                               const float *rstd, int B, int T, int C) {
  for (int b = 0; b < B; b++) {
    for (int t = 0; t < T; t++) {
      const float *x = inp + (size_t)b * T * C + (size_t)t * C;
      const float *dy = dout + (size_t)b * T * C + (size_t)t * C;
      float *dx = dinp + (size_t)b * T * C + (size_t)t * C;
      float m = mean[b * T + t];
      float r = rstd[b * T + t];
      float dnorm_mean = 0.0f;
      float dnorm_xhat_mean = 0.0f;
      for (int c = 0; c < C; c++) {
        float xhat = (x[c] - m) * r;
        float dnorm = dy[c] * weight[c];
        dnorm_mean += dnorm;
        dnorm_xhat_mean += dnorm * xhat;
      }
      dnorm_mean /= C;
      dnorm_xhat_mean /= C;
      for (int c = 0; c < C; c++) {
        float xhat = (x[c] - m) * r;
        float dnorm = dy[c] * weight[c];
        dbias[c] += dy[c];
        dweight[c] += dy[c] * xhat;
        dx[c] += r * (dnorm - dnorm_mean - xhat * dnorm_xhat_mean);
      }
    }
  }
}

/* train_bnn.c:491-496 */
void oracle_residual_backward(float *dx, float *dy, const float *dout, int N) {
  for (int i = 0; i < N; i++) {
    dx[i] += dout[i];
    dy[i] += dout[i];
  }
}

/* train_bnn.c:520-533 */
void oracle_gelu_backward(float *dinp, const float *inp, const float *dout,
                          int N) {
  const float k = 0.7978845608f;
  for (int i = 0; i < N; i++) {
    float x = inp[i];
    float u = k * (x + 0.044715f * x * x * x);
    float tanh_u = tanhf(u);
    float sech2 = 1.0f - tanh_u * tanh_u;
    float du_dx = k * (1.0f + 3.0f * 0.044715f * x * x);
    float local_grad = 0.5f * (1.0f + tanh_u) + 0.5f * x * sech2 * du_dx;
    dinp[i] += local_grad * dout[i];
  }
}

/* train_bnn.c:647-662 */
void oracle_encoder_backward(float *dwte, float *dwpe, const float *dout,
                             const int *inp, int B, int T, int C) {
  for (int b = 0; b < B; b++) {
    for (int t = 0; t < T; t++) {
      const float *dy = dout + (size_t)b * T * C + (size_t)t * C;
      int ix = inp[b * T + t];
      float *dwte_row = dwte + (size_t)ix * C;
      float *dwpe_row = dwpe + (size_t)t * C;
      for (int c = 0; c < C; c++) {
        dwte_row[c] += dy[c];
        dwpe_row[c] += dy[c];
      }
    }
  }
}

/* train_bnn.c:814-816 */
float oracle_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

/* train_bnn.c:831-835 */
void oracle_bayes_materialize(float *w, const float *mu, const float *rho,
                              const float *eps, size_t n) {
  for (size_t i = 0; i < n; i++) w[i] = mu[i] + oracle_softplus(rho[i]) * eps[i];
}

/* Elementwise host libm entry points, so tests can compare device math with
 * the very functions the oracle calls. */
void oracle_expf_n(float *y, const float *x, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = expf(x[i]);
}
void oracle_log1pf_n(float *y, const float *x, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = log1pf(x[i]);
}
void oracle_tanhf_n(float *y, const float *x, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = tanhf(x[i]);
}
void oracle_softplus_n(float *y, const float *x, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = oracle_softplus(x[i]);
}

/* Bit patterns [lo, lo+n) as floats, the input of an exhaustive sweep. */
void oracle_float_range(float *x, unsigned lo, size_t n) {
  for (size_t i = 0; i < n; i++) {
    unsigned u = lo + (unsigned)i;
    memcpy(&x[i], &u, 4);
  }
}

/* Count positions whose bit patterns differ (NaN == NaN). */
size_t oracle_count_bit_mismatch(const float *a, const float *b, size_t n,
                                 size_t *first) {
  size_t bad = 0;
  for (size_t i = 0; i < n; i++) {
    unsigned ua, ub;
    memcpy(&ua, &a[i], 4);
    memcpy(&ub, &b[i], 4);
    if (ua != ub && !(a[i] != a[i] && b[i] != b[i])) {
      if (bad == 0 && first) *first = i;
      bad++;
    }
  }
  return bad;
}
