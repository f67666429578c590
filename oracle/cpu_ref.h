/* cpu_ref.h - CPU oracle (test infrastructure only; see cpu_ref.c). */
#ifndef UGK_ORACLE_CPU_REF_H
#define UGK_ORACLE_CPU_REF_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

void oracle_encoder_forward(float *out, const int *inp, const float *wte,
                            const float *wpe, int B, int T, int C);
void oracle_encoder_backward(float *dwte, float *dwpe, const float *dout,
                             const int *inp, int B, int T, int C);
void oracle_layernorm_forward(float *out, float *mean, float *rstd,
                              const float *inp, const float *weight,
                              const float *bias, int B, int T, int C);
void oracle_layernorm_backward(float *dinp, float *dweight, float *dbias,
                               const float *dout, const float *inp,
                               const float *weight, const float *mean,
                               const float *rstd, int B, int T, int C);
void oracle_gelu_forward(float *out, const float *inp, int N);
void oracle_gelu_backward(float *dinp, const float *inp, const float *dout, int N);
void oracle_residual_forward(float *out, const float *x, const float *y, int N);
void oracle_residual_backward(float *dx, float *dy, const float *dout, int N);
float oracle_softplus(float x);
void oracle_bayes_materialize(float *w, const float *mu, const float *rho,
                              const float *eps, size_t n);

void oracle_softmax_crossentropy(float *losses, float *probs, const float *logits,
                                 const int *targets, int B, int T, int V);
void oracle_crossentropy_softmax_backward(float *dlogits, const float *probs,
                                          const int *targets, int B, int T, int V);
void oracle_bayes_backward(float *dmu, float *drho, const float *dw,
                           const float *eps, const float *rho, size_t n);
double oracle_kl_forward(const float *mu, const float *rho, size_t n,
                         float sigma_prior);
void oracle_kl_backward(float *dmu, float *drho, const float *mu, const float *rho,
                        size_t n, float sigma_prior, float weight);
void oracle_adamw_update(float *params, const float *grads, float *m, float *v,
                         size_t n, int t, float lr, float beta1, float beta2,
                         float eps, float wd);
void oracle_philox4x32_10(const unsigned *ctr, const unsigned *key, unsigned *out);
float oracle_u01(unsigned x);
float oracle_philox_normal(unsigned long long seed, int step, size_t index);
void oracle_philox_normal_n(float *eps, size_t n, unsigned long long seed, int step,
                            size_t first);
void oracle_bayes_sample_philox(float *w, float *eps, const float *mu, const float *rho,
                                size_t n, unsigned long long seed, int step);
void oracle_bayes_backward_philox(float *dmu, float *drho, const float *dw, const float *rho,
                                  size_t n, unsigned long long seed, int step);
void oracle_bbb_step_fused(float *mu, float *rho, float *m_mu, float *v_mu, float *m_rho,
                           float *v_rho, float *w, float *dw, size_t n,
                           unsigned long long seed, int step, float sp, float klw,
                           float bc1, float bc2, float lr, float beta1, float beta2,
                           float aeps, float wd);

typedef struct {
  int *tokens;
  long n;
  long pos;
} OracleLoader;
int oracle_loader_init(OracleLoader *ld, const char *path);
void oracle_loader_next(OracleLoader *ld, int *h_inp, int *h_tgt, int BT);
void oracle_loader_free(OracleLoader *ld);
long oracle_loader_count(const char *path);
void oracle_ckpt_path(char *buf, size_t size, const char *arm, const char *what,
                      int C, int L, int steps);
void oracle_ckpt_header(int *hdr, size_t n, int C, int L, int V, int NH, int steps);
int oracle_ckpt_save(const char *path, const float *h, size_t n, int C, int L, int V,
                     int NH, int steps);
int oracle_ckpt_load(const char *path, float *h, size_t n, int C, int L, int V, int NH);

void oracle_expf_n(float *y, const float *x, size_t n);
void oracle_log1pf_n(float *y, const float *x, size_t n);
void oracle_tanhf_n(float *y, const float *x, size_t n);
void oracle_softplus_n(float *y, const float *x, size_t n);
void oracle_logf_n(float *y, const float *x, size_t n);
void oracle_cosf_n(float *y, const float *x, size_t n);
void oracle_sqrtf_n(float *y, const float *x, size_t n);
void oracle_float_range(float *x, unsigned lo, size_t n);
size_t oracle_count_bit_mismatch(const float *a, const float *b, size_t n,
                                 size_t *first);

#ifdef __cplusplus
}
#endif
#endif
