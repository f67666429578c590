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
 *   - the posterior update (bayes_backward, kl_forward/backward, adamw) against
 *     the compiled reference, which exports all four; Philox4x32-10 against
 *     the published Random123 known-answer vectors; philox_normal against a
 *     float64 Box-Muller of the same words; the fused step against the
 *     composition of the unfused ops.
 */
#include "cpu_ref.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
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

/* train_bnn.c:279-304 */
void oracle_softmax_crossentropy(float *losses, float *probs, const float *logits,
                                 const int *targets, int B, int T, int V) {
  for (int b = 0; b < B; b++) {
    for (int t = 0; t < T; t++) {
      const float *logit_bt = logits + (size_t)b * T * V + (size_t)t * V;
      float *prob_bt = probs + (size_t)b * T * V + (size_t)t * V;
      float max = -1e30f;
      for (int v = 0; v < V; v++)
        if (logit_bt[v] > max) max = logit_bt[v];
      float sum = 0.0f;
      for (int v = 0; v < V; v++) {
        prob_bt[v] = expf(logit_bt[v] - max);
        sum += prob_bt[v];
      }
      for (int v = 0; v < V; v++) prob_bt[v] /= sum;
      int target_token = targets[b * T + t];
      losses[b * T + t] = -logf(prob_bt[target_token]);
    }
  }
}

/* train_bnn.c:358-378 */
void oracle_crossentropy_softmax_backward(float *dlogits, const float *probs,
                                          const int *targets, int B, int T, int V) {
  float dloss = 1.0f / (B * T);
  for (int b = 0; b < B; b++) {
    for (int t = 0; t < T; t++) {
      float *dlogit_bt = dlogits + (size_t)b * T * V + (size_t)t * V;
      const float *prob_bt = probs + (size_t)b * T * V + (size_t)t * V;
      int target_token = targets[b * T + t];
      for (int v = 0; v < V; v++) {
        float indicator = (v == target_token) ? 1.0f : 0.0f;
        dlogit_bt[v] += (prob_bt[v] - indicator) * dloss;
      }
    }
  }
}

/* ---- the posterior update ------------------------------------------------ */

/* train_bnn.c:820-822 */
static float oracle_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* train_bnn.c:855-861 */
void oracle_bayes_backward(float *dmu, float *drho, const float *dw,
                           const float *eps, const float *rho, size_t n) {
  for (size_t i = 0; i < n; i++) {
    dmu[i] += dw[i];
    drho[i] += dw[i] * eps[i] * oracle_sigmoid(rho[i]);
  }
}

/* train_bnn.c:941-957 */
double oracle_kl_forward(const float *mu, const float *rho, size_t n,
                         float sigma_prior) {
  float sp2 = sigma_prior * sigma_prior;
  double kl = 0.0;
  for (size_t i = 0; i < n; i++) {
    double sigma = (double)oracle_softplus(rho[i]);
    double m = (double)mu[i];
    kl += log((double)sigma_prior / sigma) + (sigma * sigma + m * m) / (2.0 * (double)sp2) - 0.5;
  }
  return kl;
}

/* train_bnn.c:966-979 */
void oracle_kl_backward(float *dmu, float *drho, const float *mu, const float *rho,
                        size_t n, float sigma_prior, float weight) {
  float sp2 = sigma_prior * sigma_prior;
  for (size_t i = 0; i < n; i++) {
    float sigma = oracle_softplus(rho[i]);
    dmu[i] += weight * (mu[i] / sp2);
    float dsigma = sigma / sp2 - 1.0f / sigma;
    drho[i] += weight * dsigma * oracle_sigmoid(rho[i]);
  }
}

/* train_bnn.c:699-717 */
void oracle_adamw_update(float *params, const float *grads, float *m, float *v,
                         size_t n, int t, float lr, float beta1, float beta2,
                         float eps, float wd) {
  float bc1 = 1.0f - powf(beta1, (float)t);
  float bc2 = 1.0f - powf(beta2, (float)t);
  for (size_t i = 0; i < n; i++) {
    float g = grads[i];
    m[i] = beta1 * m[i] + (1.0f - beta1) * g;
    v[i] = beta2 * v[i] + (1.0f - beta2) * g * g;
    float m_hat = m[i] / bc1;
    float v_hat = v[i] / bc2;
    params[i] -= lr * (m_hat / (sqrtf(v_hat) + eps) + wd * params[i]);
  }
}

/* gpt2_kernels.cuh:148-175: Philox4x32-10, ten rounds, the key bumped after
 * every round. */
void oracle_philox4x32_10(const unsigned *ctr, const unsigned *key, unsigned *out) {
  const unsigned M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
  const unsigned W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
  unsigned c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  unsigned k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; r++) {
    unsigned long long p0 = (unsigned long long)M0 * c0;
    unsigned long long p1 = (unsigned long long)M1 * c2;
    unsigned n0 = (unsigned)(p1 >> 32) ^ c1 ^ k0, n1 = (unsigned)p1;
    unsigned n2 = (unsigned)(p0 >> 32) ^ c3 ^ k1, n3 = (unsigned)p0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += W0; k1 += W1;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* gpt2_kernels.cuh:177-179 */
float oracle_u01(unsigned x) { return ((float)x + 0.5f) * 2.3283064365386963e-10f; }

/* gpt2_kernels.cuh:181-192, as the host compiler builds it (glibc logf, cosf,
 * sqrtf). */
float oracle_philox_normal(unsigned long long seed, int step, size_t index) {
  unsigned ctr[4], key[2], out[4];
  ctr[0] = (unsigned)(index & 0xffffffffu);
  ctr[1] = (unsigned)((unsigned long long)index >> 32);
  ctr[2] = (unsigned)step;
  ctr[3] = 0u;
  key[0] = (unsigned)(seed & 0xffffffffu);
  key[1] = (unsigned)(seed >> 32);
  oracle_philox4x32_10(ctr, key, out);
  float u1 = oracle_u01(out[0]), u2 = oracle_u01(out[1]);
  return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958647692f * u2);
}

/* eps[i] = philox_normal(seed, step, first + i). */
void oracle_philox_normal_n(float *eps, size_t n, unsigned long long seed, int step,
                            size_t first) {
  for (size_t i = 0; i < n; i++) eps[i] = oracle_philox_normal(seed, step, first + i);
}

/* train_bnn_gpu.cu:93-97 (k_bayes_sample); eps also stored when non-NULL, as
 * train_bnn.c:841-845 keeps it. */
void oracle_bayes_sample_philox(float *w, float *eps, const float *mu, const float *rho,
                                size_t n, unsigned long long seed, int step) {
  for (size_t i = 0; i < n; i++) {
    float e = oracle_philox_normal(seed, step, i);
    w[i] = mu[i] + oracle_softplus(rho[i]) * e;
    if (eps) eps[i] = e;
  }
}

/* train_bnn_gpu.cu:99-109 (k_bayes_backward) */
void oracle_bayes_backward_philox(float *dmu, float *drho, const float *dw, const float *rho,
                                  size_t n, unsigned long long seed, int step) {
  for (size_t i = 0; i < n; i++) {
    float g = dw[i];
    float eps = oracle_philox_normal(seed, step, i);
    dmu[i] += g;
    drho[i] += g * eps * oracle_sigmoid(rho[i]);
  }
}

/* train_bnn_gpu.cu:173-217 (k_bbb_step_fused), statement by statement. */
void oracle_bbb_step_fused(float *mu, float *rho, float *m_mu, float *v_mu, float *m_rho,
                           float *v_rho, float *w, float *dw, size_t n,
                           unsigned long long seed, int step, float sp, float klw,
                           float bc1, float bc2, float lr, float beta1, float beta2,
                           float aeps, float wd) {
  for (size_t i = 0; i < n; i++) {
    float g = dw[i], r = rho[i], mm = mu[i];
    dw[i] = 0.0f;
    float sg = oracle_sigmoid(r);
    float gmu = g;
    float grho = g * oracle_philox_normal(seed, step, i) * sg;
    if (klw > 0.0f) {
      float sp2 = sp * sp, sigma = oracle_softplus(r);
      gmu += klw * (mm / sp2);
      grho += klw * (sigma / sp2 - 1.0f / sigma) * sg;
    }
    float m1 = beta1 * m_mu[i] + (1.0f - beta1) * gmu;
    float v1 = beta2 * v_mu[i] + (1.0f - beta2) * gmu * gmu;
    m_mu[i] = m1; v_mu[i] = v1;
    float mu_new = mm - lr * ((m1 / bc1) / (sqrtf(v1 / bc2) + aeps) + wd * mm);
    mu[i] = mu_new;
    float m2 = beta1 * m_rho[i] + (1.0f - beta1) * grho;
    float v2 = beta2 * v_rho[i] + (1.0f - beta2) * grho * grho;
    m_rho[i] = m2; v_rho[i] = v2;
    float rho_new = r - lr * ((m2 / bc1) / (sqrtf(v2 / bc2) + aeps) + wd * r);
    rho[i] = rho_new;
    w[i] = mu_new + oracle_softplus(rho_new) * oracle_philox_normal(seed, step + 1, i);
  }
}

/* ---- file formats ----------------------------------------------------------
 * gpt2_kernels.cuh:898-930 (Loader), :1318-1331 (loader_count), :944-964
 * (ckpt_save) and :1281-1316 (ckpt_load), with host buffers in place of the
 * device copies and a status return in place of the abort. */

/* OracleLoader (cpu_ref.h) mirrors Loader, gpt2_kernels.cuh:903. */

/* gpt2_kernels.cuh:904-921; returns 0, or -1 (missing, bad header, bad magic,
 * short read) */
int oracle_loader_init(OracleLoader *ld, const char *path) {
  FILE *f = fopen(path, "rb");
  if (!f) return -1;
  int header[256];
  if (fread(header, sizeof(int), 256, f) != 256) { fclose(f); return -1; }
  if (header[0] != 20240520) { fclose(f); return -1; }
  long ntok = header[2];
  unsigned short *raw = (unsigned short *)malloc((ntok > 0 ? ntok : 1) * sizeof(unsigned short));
  if (fread(raw, sizeof(unsigned short), ntok, f) != (size_t)ntok) { free(raw); fclose(f); return -1; }
  fclose(f);
  ld->tokens = (int *)malloc((ntok > 0 ? ntok : 1) * sizeof(int));
  for (long i = 0; i < ntok; i++) ld->tokens[i] = (int)raw[i];
  free(raw);
  ld->n = ntok;
  ld->pos = 0;
  return 0;
}

/* gpt2_kernels.cuh:924-929 */
void oracle_loader_next(OracleLoader *ld, int *h_inp, int *h_tgt, int BT) {
  if (ld->pos + BT + 1 > ld->n) ld->pos = 0;
  memcpy(h_inp, ld->tokens + ld->pos, BT * sizeof(int));
  memcpy(h_tgt, ld->tokens + ld->pos + 1, BT * sizeof(int));
  ld->pos += BT;
}

void oracle_loader_free(OracleLoader *ld) { free(ld->tokens); }

/* gpt2_kernels.cuh:1318-1331; -1 on error */
long oracle_loader_count(const char *path) {
  FILE *f = fopen(path, "rb");
  if (!f) return -1;
  int header[256];
  if (fread(header, sizeof(int), 256, f) != 256) { fclose(f); return -1; }
  fclose(f);
  if (header[0] != 20240520) return -1;
  return header[2];
}

/* gpt2_kernels.cuh:950-951 */
void oracle_ckpt_path(char *buf, size_t size, const char *arm, const char *what,
                      int C, int L, int steps) {
  snprintf(buf, size, "runs/%s_C%d_L%d_%dk_%s.bin", arm, C, L, steps / 1000, what);
}

/* gpt2_kernels.cuh:958-959: the 8-int header */
void oracle_ckpt_header(int *hdr, size_t n, int C, int L, int V, int NH, int steps) {
  int h[8] = {20240520, (int)(n & 0xffffffffu), C, L, V, NH, steps, (int)(n >> 32)};
  memcpy(hdr, h, sizeof h);
}

/* gpt2_kernels.cuh:944-964 with a host buffer; 0 or -1 */
int oracle_ckpt_save(const char *path, const float *h, size_t n, int C, int L, int V,
                     int NH, int steps) {
  FILE *f = fopen(path, "wb");
  if (!f) return -1;
  int hdr[8];
  oracle_ckpt_header(hdr, n, C, L, V, NH, steps);
  fwrite(hdr, sizeof(int), 8, f);
  fwrite(h, sizeof(float), n, f);
  fclose(f);
  return 0;
}

/* gpt2_kernels.cuh:1281-1316 with a host buffer: the header's steps, or -1 */
int oracle_ckpt_load(const char *path, float *h, size_t n, int C, int L, int V, int NH) {
  FILE *f = fopen(path, "rb");
  if (!f) return -1;
  int hdr[8];
  if (fread(hdr, sizeof(int), 8, f) != 8) { fclose(f); return -1; }
  if (hdr[0] != 20240520) { fclose(f); return -1; }
  size_t got = (size_t)(unsigned int)hdr[1] | ((size_t)(unsigned int)hdr[7] << 32);
  if (got != n || hdr[2] != C || hdr[3] != L || hdr[4] != V || hdr[5] != NH) { fclose(f); return -1; }
  if (fread(h, sizeof(float), n, f) != n) { fclose(f); return -1; }
  fclose(f);
  return hdr[6];
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
void oracle_logf_n(float *y, const float *x, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = logf(x[i]);
}
void oracle_cosf_n(float *y, const float *x, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = cosf(x[i]);
}
void oracle_sqrtf_n(float *y, const float *x, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = sqrtf(x[i]);
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
