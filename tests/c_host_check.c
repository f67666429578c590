/* c_host_check.c - the drop-in boundary exercised from C, the way the
 * reference's C callers reach the layer ops: a C99 program built by gcc
 * against include/ugk.h (and the HIP runtime's C API for device buffers),
 * linked with libugk.so, calls each op with train_bnn.c's argument lists and
 * compares the result with the CPU oracle (oracle/liboracle.so, test
 * infrastructure) on the same seeded inputs, at config 1's shapes (B=4, T=64,
 * C=384, V=27) and a materialize over 100,003 parameters.
 *
 * Bars: bit-exact for the encoder, residual, materialize and GELU in its
 * glibc-exact mode; 1e-5 relative + 1e-6 absolute for LayerNorm (2e-5
 * absolute for its column sums) and the default GELU (1e-5 absolute for its
 * accumulated backward, whose upstream gradients are of order 1). Also checks the error channel: a NULL pointer returns UGK_EINVAL with
 * a message, and zero-size work returns UGK_OK.
 *
 * Prints one line per check and "c host check: <n> failures"; the exit status
 * is the number of failures (capped at 100). */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cpu_ref.h"
#include "ugk.h"

static int failures = 0;

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static double uniform(void) { /* splitmix64 -> (0, 1) */
  uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return ((double)(z >> 11) + 0.5) / 9007199254740992.0;
}
static float normal(float mean, float sd) {
  return mean + sd * (float)(sqrt(-2.0 * log(uniform())) * cos(6.283185307179586 * uniform()));
}
static float *host_normal(size_t n, float mean, float sd) {
  float *p = malloc(n * sizeof(float));
  for (size_t i = 0; i < n; i++) p[i] = normal(mean, sd);
  return p;
}

static void *to_device(const void *h, size_t bytes) {
  void *d = NULL;
  if (hipMalloc(&d, bytes) != hipSuccess || hipMemcpy(d, h, bytes, hipMemcpyHostToDevice) != hipSuccess) {
    fprintf(stderr, "device copy of %zu bytes failed\n", bytes);
    exit(100);
  }
  return d;
}
static float *from_device(const float *d, size_t n) {
  float *h = malloc(n * sizeof(float));
  if (hipMemcpy(h, d, n * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) {
    fprintf(stderr, "device read of %zu floats failed\n", n);
    exit(100);
  }
  return h;
}

static void call_ok(int rc, const char *what) {
  if (rc != UGK_OK) {
    printf("%-32s FAIL: status %d (%s)\n", what, rc, ugk_last_error());
    failures++;
  }
}

/* the device result d (n floats) against the oracle's h: bit-exact when
 * rtol == 0, else |g - c| <= atol + rtol |c| */
static void check(const char *what, const float *d, const float *h, size_t n, double rtol, double atol) {
  float *g = from_device(d, n);
  size_t bad = 0, first = 0;
  double worst = 0.0;
  for (size_t i = 0; i < n; i++) {
    int ok;
    if (rtol == 0.0 && atol == 0.0) {
      uint32_t a, b;
      memcpy(&a, &g[i], 4);
      memcpy(&b, &h[i], 4);
      ok = a == b || (g[i] != g[i] && h[i] != h[i]);
    } else {
      const double e = fabs((double)g[i] - (double)h[i]);
      ok = e <= atol + rtol * fabs((double)h[i]);
      if (e > worst) worst = e;
    }
    if (!ok && bad++ == 0) first = i;
  }
  if (bad) {
    printf("%-32s FAIL: %zu of %zu differ (first at %zu: %.9g vs %.9g)\n", what, bad, n, first, g[first], h[first]);
    failures++;
  } else if (rtol == 0.0 && atol == 0.0) {
    printf("%-32s ok: %zu values bit-exact\n", what, n);
  } else {
    printf("%-32s ok: %zu values, max abs error %.3g\n", what, n, worst);
  }
  free(g);
}

int main(void) {
  const int B = 4, T = 64, C = 384, V = 27;
  const size_t BT = (size_t)B * T, NB = BT * C, N4 = 4 * NB;

  /* encoder */
  int *tok = malloc(BT * sizeof(int));
  for (size_t i = 0; i < BT; i++) tok[i] = (int)(uniform() * V);
  float *wte = host_normal((size_t)V * C, 0.0f, 0.02f), *wpe = host_normal((size_t)T * C, 0.0f, 0.01f);
  float *out = calloc(NB, sizeof(float));
  int *d_tok = to_device(tok, BT * sizeof(int));
  float *d_wte = to_device(wte, (size_t)V * C * 4), *d_wpe = to_device(wpe, (size_t)T * C * 4);
  float *d_out = to_device(out, NB * 4);
  call_ok(ugk_encoder_forward(d_out, d_tok, d_wte, d_wpe, B, T, C), "ugk_encoder_forward");
  oracle_encoder_forward(out, tok, wte, wpe, B, T, C);
  check("encoder_forward out", d_out, out, NB, 0, 0);

  float *dout = host_normal(NB, 0.0f, 1.0f);
  float *dwte = host_normal((size_t)V * C, 0.0f, 1.0f), *dwpe = host_normal((size_t)T * C, 0.0f, 1.0f);
  float *d_dout = to_device(dout, NB * 4), *d_dwte = to_device(dwte, (size_t)V * C * 4);
  float *d_dwpe = to_device(dwpe, (size_t)T * C * 4);
  call_ok(ugk_encoder_backward(d_dwte, d_dwpe, d_dout, d_tok, B, T, C), "ugk_encoder_backward");
  oracle_encoder_backward(dwte, dwpe, dout, tok, B, T, C);
  check("encoder_backward dwte", d_dwte, dwte, (size_t)V * C, 0, 0);
  check("encoder_backward dwpe", d_dwpe, dwpe, (size_t)T * C, 0, 0);

  /* LayerNorm */
  float *x = host_normal(NB, 0.0f, 1.0f), *w = host_normal(C, 1.0f, 0.1f), *b = host_normal(C, 0.0f, 0.1f);
  float *mean = calloc(BT, 4), *rstd = calloc(BT, 4);
  float *d_x = to_device(x, NB * 4), *d_w = to_device(w, C * 4), *d_b = to_device(b, C * 4);
  float *d_mean = to_device(mean, BT * 4), *d_rstd = to_device(rstd, BT * 4);
  call_ok(ugk_layernorm_forward(d_out, d_mean, d_rstd, d_x, d_w, d_b, B, T, C), "ugk_layernorm_forward");
  oracle_layernorm_forward(out, mean, rstd, x, w, b, B, T, C);
  check("layernorm_forward out", d_out, out, NB, 1e-5, 1e-6);
  check("layernorm_forward mean", d_mean, mean, BT, 1e-5, 1e-6);
  check("layernorm_forward rstd", d_rstd, rstd, BT, 1e-5, 1e-6);

  /* the encoder and the LayerNorm of its rows in one call: the rows bit-exact,
     their normalisation within the LayerNorm tolerance */
  float *enc = calloc(NB, 4), *lno = calloc(NB, 4), *lnm = calloc(BT, 4), *lnr = calloc(BT, 4);
  float *d_enc = to_device(enc, NB * 4), *d_lno = to_device(lno, NB * 4);
  float *d_lnm = to_device(lnm, BT * 4), *d_lnr = to_device(lnr, BT * 4);
  call_ok(ugk_encoder_layernorm_forward(d_enc, d_lno, d_lnm, d_lnr, d_tok, d_wte, d_wpe, d_w, d_b, B, T, C),
          "ugk_encoder_layernorm_forward");
  oracle_encoder_forward(enc, tok, wte, wpe, B, T, C);
  oracle_layernorm_forward(lno, lnm, lnr, enc, w, b, B, T, C);
  check("encoder_layernorm_forward enc", d_enc, enc, NB, 0, 0);
  check("encoder_layernorm_forward out", d_lno, lno, NB, 1e-5, 1e-6);
  check("encoder_layernorm_forward mean", d_lnm, lnm, BT, 1e-5, 1e-6);
  check("encoder_layernorm_forward rstd", d_lnr, lnr, BT, 1e-5, 1e-6);

  float *dinp = host_normal(NB, 0.0f, 1.0f), *dw = host_normal(C, 0.0f, 1.0f), *db = host_normal(C, 0.0f, 1.0f);
  float *d_dinp = to_device(dinp, NB * 4), *d_dw = to_device(dw, C * 4), *d_db = to_device(db, C * 4);
  call_ok(ugk_layernorm_backward(d_dinp, d_dw, d_db, d_dout, d_x, d_w, d_mean, d_rstd, B, T, C),
          "ugk_layernorm_backward");
  oracle_layernorm_backward(dinp, dw, db, dout, x, w, mean, rstd, B, T, C);
  check("layernorm_backward dinp", d_dinp, dinp, NB, 1e-5, 1e-6);
  check("layernorm_backward dweight", d_dw, dw, C, 1e-5, 2e-5);
  check("layernorm_backward dbias", d_db, db, C, 1e-5, 2e-5);

  /* GELU over the MLP hidden tensor (4C wide) */
  float *h = host_normal(N4, 0.0f, 1.0f), *hout = calloc(N4, 4);
  float *d_h = to_device(h, N4 * 4), *d_hout = to_device(hout, N4 * 4);
  call_ok(ugk_gelu_forward(d_hout, d_h, (int)N4), "ugk_gelu_forward");
  oracle_gelu_forward(hout, h, (int)N4);
  check("gelu_forward out", d_hout, hout, N4, 1e-5, 1e-6);
  float *hd = host_normal(N4, 0.0f, 1.0f), *hdin = host_normal(N4, 0.0f, 1.0f);
  float *hdin0 = malloc(N4 * 4);
  memcpy(hdin0, hdin, N4 * 4);
  float *d_hd = to_device(hd, N4 * 4), *d_hdin = to_device(hdin, N4 * 4);
  call_ok(ugk_gelu_backward(d_hdin, d_h, d_hd, (int)N4), "ugk_gelu_backward");
  oracle_gelu_backward(hdin, h, hd, (int)N4);
  check("gelu_backward dinp", d_hdin, hdin, N4, 1e-5, 1e-5);
  /* the glibc-exact mode: bit for bit */
  call_ok(ugk_set_gelu_exact(1), "ugk_set_gelu_exact");
  call_ok(ugk_gelu_forward(d_hout, d_h, (int)N4), "ugk_gelu_forward (exact)");
  check("gelu_forward out (exact)", d_hout, hout, N4, 0, 0);
  float *d_hdin0 = to_device(hdin0, N4 * 4);
  call_ok(ugk_gelu_backward(d_hdin0, d_h, d_hd, (int)N4), "ugk_gelu_backward (exact)");
  check("gelu_backward dinp (exact)", d_hdin0, hdin, N4, 0, 0);
  call_ok(ugk_set_gelu_exact(0), "ugk_set_gelu_exact");

  /* residual */
  float *y = host_normal(NB, 0.0f, 1.0f);
  float *d_y = to_device(y, NB * 4);
  call_ok(ugk_residual_forward(d_out, d_x, d_y, (int)NB), "ugk_residual_forward");
  oracle_residual_forward(out, x, y, (int)NB);
  check("residual_forward out", d_out, out, NB, 0, 0);
  float *rx = host_normal(NB, 0.0f, 1.0f), *ry = host_normal(NB, 0.0f, 1.0f);
  float *d_rx = to_device(rx, NB * 4), *d_ry = to_device(ry, NB * 4);
  call_ok(ugk_residual_backward(d_rx, d_ry, d_dout, (int)NB), "ugk_residual_backward");
  oracle_residual_backward(rx, ry, dout, (int)NB);
  check("residual_backward dx", d_rx, rx, NB, 0, 0);
  check("residual_backward dy", d_ry, ry, NB, 0, 0);

  /* materialize: w = mu + softplus(rho) * eps */
  const size_t np = 100003;
  float *mu = host_normal(np, 0.0f, 0.02f), *rho = host_normal(np, -5.0f, 0.1f), *eps = host_normal(np, 0.0f, 1.0f);
  float *wm = calloc(np, 4);
  float *d_mu = to_device(mu, np * 4), *d_rho = to_device(rho, np * 4), *d_eps = to_device(eps, np * 4);
  float *d_wm = to_device(wm, np * 4);
  call_ok(ugk_bayes_materialize(d_wm, d_mu, d_rho, d_eps, np), "ugk_bayes_materialize");
  oracle_bayes_materialize(wm, mu, rho, eps, np);
  check("bayes_materialize w", d_wm, wm, np, 0, 0);

  /* the error channel */
  {
    const int rc = ugk_gelu_forward(NULL, d_h, 16);
    const char *msg = ugk_last_error();
    if (rc == UGK_EINVAL && msg && msg[0]) {
      printf("%-32s ok: status %d, \"%s\"\n", "NULL pointer rejected", rc, msg);
    } else {
      printf("%-32s FAIL: status %d\n", "NULL pointer rejected", rc);
      failures++;
    }
    if (ugk_residual_forward(d_out, d_x, d_y, 0) != UGK_OK) {
      printf("%-32s FAIL\n", "zero-size call");
      failures++;
    } else {
      printf("%-32s ok\n", "zero-size call");
    }
  }
  call_ok(ugk_synchronize(), "ugk_synchronize");

  printf("c host check: %d failures\n", failures);
  return failures > 100 ? 100 : failures;
}
