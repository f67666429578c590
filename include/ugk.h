/*
 * ugk.h - C-ABI of libugk.so, the MI355X (gfx950) layer-kernel set of
 * uncertain-gpt: LayerNorm, GELU, residual, encoder and bayes_materialize.
 *
 * Every entry point keeps the parameter list and parameter order of the CPU
 * op it replaces in the reference oracle train_bnn.c, so a caller swaps
 *     layernorm_forward(out, mean, rstd, inp, w, b, B, T, C);
 * for
 *     UGK_CHECK(ugk_layernorm_forward(out, mean, rstd, inp, w, b, B, T, C));
 * The differences are:
 *   - all pointers are DEVICE pointers (hipMalloc / torch device memory);
 *   - each call returns an int status (UGK_OK = 0) instead of void; the text
 *     of the last failure on the calling thread is ugk_last_error();
 *   - work is queued on the library's stream (ugk_set_stream, default the
 *     null stream, which is also what the reference's <<<>>> launches use),
 *     and a call returns before the GPU has finished.
 * Semantics are the reference's: backward outputs ACCUMULATE (+=) into the
 * caller's buffers, and the caller zeroes them when it wants plain gradients.
 * Results: encoder fwd/bwd, residual fwd/bwd and bayes_materialize are
 * bit-identical to train_bnn.c on a host with glibc 2.35 and FMA; GELU fwd/bwd
 * are within 1e-5 relative / 1e-6 absolute of it on every input, and
 * bit-identical after ugk_set_gelu_exact(1); LayerNorm row statistics and dinp
 * are within fp32 rounding of it, and LayerNorm dweight/dbias are reduced in a
 * fixed, run-to-run deterministic order (bit-identical to it after
 * ugk_set_layernorm_exact(1)).
 *
 * The library never allocates inside a kernel. A few entry points need device
 * workspace beyond their arguments: the LayerNorm backward's partial column
 * sums (one slot per call, 2L+1 for the step driver), the encoder backward's
 * bucket state, the KL total's partial sums and the softmax's row
 * statistics (rows too long for one workgroup, and the exact mode's), each in
 * a region of its own. By default the library allocates
 * a region on the first call that needs it and grows it, after waiting for
 * the device, when a larger shape arrives; ugk_reserve / ugk_reserve_config
 * allocate everything up front, after which calls at those shapes neither
 * allocate nor wait. A call under HIP graph capture that would have to
 * allocate fails with UGK_ENOMEM before launching anything (reserve first, or
 * make one call at that shape outside the capture). A caller that owns all device memory (as the reference's
 * arms do) sizes a workspace with ugk_workspace_bytes and hands it over with
 * ugk_set_workspace; the library then never allocates. The workspace is used
 * in stream order: ugk_set_stream waits for the work already queued on the
 * previous stream, so calls on two streams never share it at once. The
 * library's state is per device and meant for one host thread per device at a
 * time, as the reference's one host thread and one stream.
 */
#ifndef UGK_H
#define UGK_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UGK_OK 0
#define UGK_EINVAL 1  /* invalid argument: NULL pointer, negative size, ... */
#define UGK_EHIP 2    /* the HIP runtime reported an error */
#define UGK_ENOMEM 3  /* scratch allocation failed */

/* train_bnn.c:41-65 / gpt2_kernels.cuh:245-252 (k_encoder_forward).
 * out[b,t,:] = wte[inp[b,t],:] + wpe[t,:].  0 <= inp[i] < V is the caller's
 * contract, as in the reference. */
int ugk_encoder_forward(float *out, const int *inp, const float *wte,
                        const float *wpe, int B, int T, int C);

/* train_bnn.c:647-662 / gpt2_kernels.cuh:254-263 (k_encoder_backward).
 * dwte[inp[b,t],:] += dout[b,t,:];  dwpe[t,:] += dout[b,t,:].
 * dwpe, and every wte row that at most 32 rows of a 65,536-row chunk add
 * into, take their rows in ascending (b,t) order, the order of the CPU loop,
 * bit-identical to it. A token with more rows in a chunk is added in blocks
 * (the default; see ugk_set_encoder_exact): its rows, ascending, in blocks of
 * 64, each block added in row order (the first onto dwte's value, the others
 * from zero), then the block sums in block order. That is deterministic (the
 * same bits on every run) and, up to 64 rows, the CPU's order too. Rows with
 * a negative token are skipped. Its bucket table lives in the workspace
 * and every call leaves it cleared, on the device, so the calls may be
 * captured in a HIP graph and replayed any number of times. New workspace
 * memory is cleared by ugk_set_workspace and ugk_reserve_config, or else by
 * the first call; that first call, if made under graph capture, is refused
 * (UGK_EINVAL) rather than leave the clearing inside the graph alone. */
int ugk_encoder_backward(float *dwte, float *dwpe, const float *dout,
                         const int *inp, int B, int T, int C);

/* The order of the encoder backward's adds for a token with more than 32 rows
 * in a chunk, for later calls from any thread: 0 (the default) in 64-row
 * blocks as above, the blocks of a token spread over a workgroup's 16
 * wavefronts; nonzero one add per row in ascending order, bit-identical to
 * train_bnn.c, a serial chain as long as the token's rows. No counterpart in
 * the reference, whose GPU kernel adds with atomicAdd in no fixed order. */
int ugk_set_encoder_exact(int exact);
int ugk_get_encoder_exact(void);

/* train_bnn.c:81-115 / gpt2_kernels.cuh:265-288 (k_layernorm_forward).
 * eps = 1e-5; writes out (B,T,C), mean (B,T), rstd (B,T). */
int ugk_layernorm_forward(float *out, float *mean, float *rstd,
                          const float *inp, const float *weight,
                          const float *bias, int B, int T, int C);

/* train_bnn.c:439-477 / gpt2_kernels.cuh:290-316 (k_layernorm_backward).
 * dinp += ..., dweight += sum_rows dout*xhat, dbias += sum_rows dout. */
int ugk_layernorm_backward(float *dinp, float *dweight, float *dbias,
                           const float *dout, const float *inp,
                           const float *weight, const float *mean,
                           const float *rstd, int B, int T, int C);

/* LayerNorm order of additions for later calls from any thread: 0 (the
 * default) the kernels above, whose row sums are trees (within fp32 rounding
 * of train_bnn.c) and whose dweight/dbias are summed over per-workgroup
 * partial rows (deterministic, within the scale-aware bar of the CPU's serial
 * sums); nonzero train_bnn.c's own order, each row's sums one column at a
 * time and dweight/dbias one row at a time, so that every LayerNorm output
 * (out, mean, rstd, dinp, dweight, dbias) is bit-identical to it. Every
 * LayerNorm entry point follows it, the fused pairs (as the two ops in
 * sequence), the allocation-free backward and the step driver included. The
 * exact form takes about twice the time of the default or more. No
 * counterpart in the reference, whose CPU and GPU builds each sum in their
 * own order. */
int ugk_set_layernorm_exact(int exact);
int ugk_get_layernorm_exact(void);

/* No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). ugk_layernorm_backward with its partial column sums in a fixed
 * device array of 8 MiB per GPU, held until the process ends, instead of the
 * workspace: the call allocates nothing and never waits. The array holds up to
 * 1,024 partial rows of 2C floats, so C up to 1,048,576 (larger C is refused
 * with UGK_EINVAL); rows are unlimited. It keeps the last call's contents and
 * needs no clearing (every call writes the rows it reads). Calls that overlap
 * on one GPU (other streams, other threads) race on the array. Results equal
 * ugk_layernorm_backward's bit for bit for C <= 1,024 (the same partial rows;
 * above that, once a call needs more partial rows than the array holds, its
 * column sums take fewer, longer partial rows). */
int ugk_layernorm_backward_noalloc(float *dinp, float *dweight, float *dbias,
                                   const float *dout, const float *inp,
                                   const float *weight, const float *mean,
                                   const float *rstd, int B, int T, int C);

/* train_bnn.c:41-65 then :81-115 on its output, in one pass: the pair
 * gpt2_kernels.cuh:775-776 -> :784 (block 0's first LayerNorm; -> :813 when
 * L = 0) launches back to back. enc = the encoder output (bit-identical to
 * encoder_forward); out, mean, rstd = layernorm_forward(enc) (identical to
 * calling it on enc). No single counterpart in the reference;
 * ugk_gpt2_layers_forward uses it. */
int ugk_encoder_layernorm_forward(float *enc, float *out, float *mean,
                                  float *rstd, const int *inp,
                                  const float *wte, const float *wpe,
                                  const float *weight, const float *bias,
                                  int B, int T, int C);

/* train_bnn.c:182-186 then :81-115 on its output, in one pass: the pair
 * gpt2_kernels.cuh:793-797 (and :806 -> the next block's :784, :806 -> :813)
 * launches back to back. res = x + y (bit-identical to residual_forward);
 * out, mean, rstd = layernorm_forward(res) (identical to calling it on res).
 * No single counterpart in the reference; ugk_gpt2_layers_forward uses it. */
int ugk_residual_layernorm_forward(float *res, float *out, float *mean,
                                   float *rstd, const float *x, const float *y,
                                   const float *weight, const float *bias,
                                   int B, int T, int C);

/* train_bnn.c:439-477 then :491-496 with dout = the new dinp, in one pass: the
 * pairs gpt2_kernels.cuh:870-876 and :888 -> :855 (the next block down), and
 * :846 -> :855. Identical to ugk_layernorm_backward followed by
 * ugk_residual_backward(dx, dy, dinp). dinp must differ from dx and dy;
 * dx == dy adds twice, as residual_backward does. No single counterpart in the
 * reference; ugk_gpt2_layers_backward uses it. */
int ugk_layernorm_residual_backward(float *dinp, float *dweight, float *dbias,
                                    float *dx, float *dy, const float *dout,
                                    const float *inp, const float *weight,
                                    const float *mean, const float *rstd,
                                    int B, int T, int C);

/* train_bnn.c:163-170 / gpt2_kernels.cuh:318-325 (k_gelu_forward).
 * By default GELU is evaluated as x / (1 + e^{-2u}), the same function
 * through the hardware exponential and reciprocal: within 1e-5 relative /
 * 1e-6 absolute of train_bnn.c on every float input, not bit-identical to it.
 * After ugk_set_gelu_exact(1) both GELU entry points (and the step driver)
 * use a restatement of glibc's tanhf and equal train_bnn.c bit for bit. */
int ugk_gelu_forward(float *out, const float *inp, int N);

/* train_bnn.c:520-533 / gpt2_kernels.cuh:327-338 (k_gelu_backward).
 * dinp += gelu'(inp) * dout; the form follows ugk_set_gelu_exact. */
int ugk_gelu_backward(float *dinp, const float *inp, const float *dout, int N);

/* GELU form for later calls from any thread: 0 (the default) the logistic
 * form above, nonzero the glibc-exact tanhf. No counterpart in the reference,
 * whose CPU and GPU builds each use their own tanhf. */
int ugk_set_gelu_exact(int exact);
int ugk_get_gelu_exact(void);

/* train_bnn.c:182-186 / gpt2_kernels.cuh:340-344 (k_residual_forward). */
int ugk_residual_forward(float *out, const float *x, const float *y, int N);

/* train_bnn.c:491-496 / gpt2_kernels.cuh:346-350 (k_residual_backward).
 * dx += dout; dy += dout. */
int ugk_residual_backward(float *dx, float *dy, const float *dout, int N);

/* train_bnn.c:831-835 with softplus :814-816 / dev/bayes_materialize.cu:64-75.
 * w = mu + softplus(rho) * eps, eps given. */
int ugk_bayes_materialize(float *w, const float *mu, const float *rho,
                          const float *eps, size_t n);

/* train_bnn.c:279-304 / gpt2_kernels.cuh:352-374 (k_softmax_crossentropy).
 * Per (b,t) row of V logits: probs = softmax (max-shifted, glibc-exact expf,
 * each e divided by the row sum), losses[b,t] = -logf(probs[target]) with
 * glibc's logf. The exps are the CPU's bit for bit; by default the row sum is
 * added in a fixed tree order (deterministic, within float rounding of the
 * CPU's sequential sum), so probs and losses agree to a few ulp; with
 * ugk_set_softmax_exact(1) in the CPU's order, and both are the CPU's bit for
 * bit. 0 <= targets[i] < V is the caller's contract, as in the reference. */
int ugk_softmax_crossentropy(float *losses, float *probs, const float *logits,
                             const int *targets, int B, int T, int V);

/* Order of ugk_softmax_crossentropy's row sums for later calls from any
 * thread: 0 (the default) a fixed tree, nonzero train_bnn.c's serial order
 * (v = 0, 1, ..., V-1; one chain per row, about twice the default's time).
 * No counterpart in the reference, whose GPU kernel sums in its own tree. */
int ugk_set_softmax_exact(int exact);
int ugk_get_softmax_exact(void);

/* train_bnn.c:358-378 / gpt2_kernels.cuh:376-384
 * (k_crossentropy_softmax_backward). dlogits += (probs - onehot(target)) *
 * (1 / (B*T)); bit-identical to the CPU loop. */
int ugk_crossentropy_softmax_backward(float *dlogits, const float *probs,
                                      const int *targets, int B, int T, int V);

/* ugk_crossentropy_softmax_backward for callers whose dlogits is zero before
 * the call, as in every reference arm (its memset of d_gacts, which holds the
 * logits gradient, before the step: train_bnn_gpu.cu:475). No counterpart in
 * the reference. dlogits = 0 + (probs - onehot(target)) * (1 / (B*T)),
 * without reading dlogits: the same bits as ugk_crossentropy_softmax_backward
 * on a zero buffer, whatever it holds. */
int ugk_crossentropy_softmax_backward_zeroed(float *dlogits, const float *probs,
                                             const int *targets, int B, int T,
                                             int V);

/* Form of the softplus and sigmoid inside the ops that draw eps on the device
 * (ugk_bayes_sample, ugk_bayes_backward_philox, ugk_bbb_step_fused), for
 * later calls from any thread: 0 (the default) the hardware-transcendental
 * forms (2^x, log2 and reciprocal instructions; within a few ulp of glibc's
 * and within 1e-6 absolute / 1e-5 relative of train_bnn.c:814-822 on every
 * float input), nonzero the glibc-exact forms of the eps-taking ops, with which
 * each Philox op equals its eps-taking twin fed the same eps bit for bit. The
 * eps draw follows the same setting: by default its radius from the hardware
 * log2 and square root and its cosine from the device library's sequence
 * (within a few ulp of the host's eps); otherwise glibc's logf and cosf
 * (restated) and the correctly rounded square root, so that eps, and every
 * output of every Philox op, equals the host's bit for bit. No counterpart in
 * the reference, whose GPU arms build these ops with --use_fast_math
 * (Makefile:13). */
int ugk_set_philox_exact(int exact);
int ugk_get_philox_exact(void);

/* ---- the posterior update around the layer kernels ----------------------
 * Flat parameter vectors of n floats. The ops that take eps are
 * bit-identical to train_bnn.c. The *_philox ops draw
 *     eps_i = philox_normal(seed, step, i)
 * on the fly (gpt2_kernels.cuh:148-192: Philox4x32-10 with counter
 * {i low, i high, step, 0} and key {seed low, seed high}, Box-Muller cosine
 * branch); the integer stream is exact, and the transform is the host's bit
 * for bit in the glibc-exact form (ugk_set_philox_exact), within a few ulp of
 * it by default. Buffers written by one call must not overlap each other. */

/* train_bnn.c:841-845 with the draw of train_bnn_gpu.cu:93-97 (k_bayes_sample):
 * w = mu + softplus(rho) * eps_i. eps may be NULL (the GPU arms regenerate
 * it); otherwise eps_i is stored there too. */
int ugk_bayes_sample(float *w, float *eps, const float *mu, const float *rho,
                     size_t n, unsigned long long seed, int step);

/* train_bnn.c:855-861. dmu += dw; drho += dw * eps * sigmoid(rho). */
int ugk_bayes_backward(float *dmu, float *drho, const float *dw,
                       const float *eps, const float *rho, size_t n);

/* train_bnn_gpu.cu:99-109 (k_bayes_backward): as ugk_bayes_backward with
 * eps_i regenerated from (seed, step). */
int ugk_bayes_backward_philox(float *dmu, float *drho, const float *dw,
                              const float *rho, size_t n,
                              unsigned long long seed, int step);

/* train_bnn.c:941-957. *kl (a HOST pointer) = sum over i of
 * log(sp/sigma_i) + (sigma_i^2 + mu_i^2)/(2 sp^2) - 1/2 in double, with
 * sigma_i = softplus(rho_i) and sp = sigma_prior. Summed in a fixed tree
 * order (deterministic). The float sigma_i follows ugk_set_kl_exact: by
 * default the hardware-transcendental softplus while rho_i >= -80 (within
 * 8 ulp of train_bnn.c's sigma_i, so each term within
 * 8 * 2^-23 * (1 + sigma_i^2/sp^2) of the CPU's), otherwise train_bnn.c's
 * own sigma_i (the total then within double rounding of the CPU's sequential
 * sum). Waits for the library stream. */
int ugk_kl_forward(double *kl, const float *mu, const float *rho, size_t n,
                   float sigma_prior);

/* Form of ugk_kl_forward's softplus for later calls from any thread: 0 (the
 * default) the hardware-transcendental form where sigma is a normal float,
 * nonzero the glibc-exact form throughout. No counterpart in the reference,
 * whose GPU KL (k_kl_stats, train_bnn_gpu.cu:225-250) is built with
 * --use_fast_math (Makefile:13) and takes each term in float. */
int ugk_set_kl_exact(int exact);
int ugk_get_kl_exact(void);

/* train_bnn.c:966-979 / train_bnn_gpu.cu:111-119 (k_kl_backward).
 * dmu += weight * mu / sp^2; drho += weight * (sigma/sp^2 - 1/sigma) *
 * sigmoid(rho). */
int ugk_kl_backward(float *dmu, float *drho, const float *mu, const float *rho,
                    size_t n, float sigma_prior, float weight);

/* train_bnn.c:699-717 / gpt2_kernels.cuh:973-984 (k_adamw). t >= 1; the bias
 * corrections 1 - beta^t are computed on the host with powf, as in the
 * reference. Updates params, m and v in place. */
int ugk_adamw_update(float *params, const float *grads, float *m, float *v,
                     size_t n, int t, float lr, float beta1, float beta2,
                     float eps, float wd);

/* train_bnn_gpu.cu:173-217 (k_bbb_step_fused): one Bayes-by-Backprop update
 * in one pass. gmu = dw, grho = dw * eps_i(step) * sigmoid(rho), plus the KL
 * gradient when klw > 0; AdamW on (mu, m_mu, v_mu) and (rho, m_rho, v_rho)
 * with the caller's bias corrections bc1, bc2; dw cleared to 0; and
 * w = mu' + softplus(rho') * eps_i(step + 1) for the next step. */
int ugk_bbb_step_fused(float *mu, float *rho, float *m_mu, float *v_mu,
                       float *m_rho, float *v_rho, float *w, float *dw,
                       size_t n, unsigned long long seed, int step, float sp,
                       float klw, float bc1, float bc2, float lr, float beta1,
                       float beta2, float aeps, float wd);

/* ---- library control (no counterpart in the reference: its kernels run on
 * the CUDA legacy default stream and abort on error, gpt2_kernels.cuh:88-101) */

/* Text of the last failure on this thread ("" if none). */
const char *ugk_last_error(void);
/* Stream for subsequent calls from any thread (a hipStream_t; NULL = the
 * null stream). When the stream changes, first waits for the work queued on
 * the previous one (it may still use the library's scratch). */
int ugk_set_stream(void *stream);
void *ugk_get_stream(void);
/* Allocate the current device's workspace for the per-op entry points at
 * shapes up to (rows = B*T, C) now instead of on first use. */
int ugk_reserve(int rows, int C);
/* Bytes of workspace held on the current device (the caller's, if set). */
size_t ugk_scratch_bytes(void);
/* Wait for all work queued on the library's stream. Then reports, as
 * UGK_EINVAL naming the op, an id that ugk_ids_guard found out of range since
 * the last report (and clears that record). */
int ugk_synchronize(void);
/* The device-side id check of bindings that cannot trust their callers' ids
 * (no counterpart in the reference, where 0 <= id < V is the caller's
 * contract and is not checked). Each of the n ids outside [0, bound) is
 * replaced IN PLACE by fill (ids in range are not written), and `code` (> 0,
 * one of UGK_IDS_*) is recorded in a per-device word that the next
 * ugk_synchronize reports. Asynchronous and allocation-free (it may be
 * captured in a graph); the op called next with the same ids can then no
 * longer index outside its table. */
#define UGK_IDS_ENCODER_FORWARD 1
#define UGK_IDS_ENCODER_BACKWARD 2
#define UGK_IDS_ENCODER_LAYERNORM_FORWARD 3
#define UGK_IDS_SOFTMAX_CROSSENTROPY 4
#define UGK_IDS_CROSSENTROPY_BACKWARD 5
int ugk_ids_guard(int *ids, int n, int bound, int fill, int code);
/* Library version, major*10000 + minor*100 + patch. */
int ugk_version(void);

/* ---- diagnostics of the kernels' float math (no counterpart in the
 * reference; used by the parity tests). fn: 0 expf, 1 log1pf, 2 expm1f,
 * 3 tanhf, 4 softplus as train_bnn.c:814-816 writes it, 8 GELU
 * (train_bnn.c:163-170) and 9 its derivative (train_bnn.c:520-533) as the
 * GELU kernels evaluate them; 10+s, 20+s, 30+s: tanhf, log1pf, expm1f with
 * the candidate division sequence s = 0..3; 40+j: x / b for eight fixed
 * divisors b (1, 3, 50257, 2 - 2^-23, 65536 - 2^-8, 1 + 2^-23, 12345.678,
 * 21504) by the softmax's reciprocal-and-correction quotient, against the
 * IEEE quotient; 48 the square root of the Box-Muller transform (inputs
 * >= 2^-96) against the correctly rounded one; 49+s: 1 / x for x >= 1 by the
 * division sequence s = 0..3 against the IEEE quotient; 53 the sigmoid's
 * 1 / x for x >= 1 against the IEEE quotient; 54+j: x / b for eight
 * launch-wide divisors b (0.01, 0.1, 1e-3, 0.19, 2^-24, 1e-7, 0.999, 2^24) as
 * AdamW and the KL gradient divide, against the IEEE quotient; 62 the square
 * root AdamW takes, against the correctly rounded one; 63 the branch-free
 * expf of the softmax and softplus, for x <= 88.72 (finite results) and NaN,
 * against expf; 64 and 65 the default GELU and its derivative (logistic
 * form) against fn 8 and 9's glibc-exact expressions, counting results
 * outside |a - b| <= 1e-6 + 1e-5 |b|; 66 and 67 the hardware-transcendental
 * softplus and sigmoid of the Philox ops (their default form) against the
 * glibc-exact softplus and train_bnn.c:820-822's sigmoid, likewise; 69 the
 * default form's Box-Muller cosf (0 <= x < 2^17) against the device library's
 * cosf (the library's own function outside that domain); 70 and 71 the Box-Muller radius sqrt(-2 ln u1) for
 * u1 in [2^-33, 1] as the Philox ops' default form (hardware log2 and square
 * root) and their glibc-exact form compute it, against the double radius
 * rounded to float (ugk_diag_math_ulp only). */

/* Over the inputs whose bit patterns are lo, lo+1, ..., lo+count-1, count
 * those where the kernels' SIMD-shaped math differs from its line-by-line
 * restatement of the host C library; *first gets the smallest such pattern
 * (0xffffffff if none). Synchronous. */
int ugk_diag_math_mismatch(int fn, unsigned lo, unsigned long long count,
                           unsigned long long *mismatches, unsigned *first);
/* out[i] = f(in[i]) on the device; variant 0 = the kernels' math, 1 = the
 * line-by-line restatement. fn: 0 expf, 1 log1pf, 2 expm1f, 3 tanhf,
 * 4 softplus, 5 logf and 6 cosf (variant 0 glibc's, as the loss and the
 * glibc-exact Box-Muller transform take them: logf on every input, cosf on
 * |x| < 120 and the device library's elsewhere; variant 1 the device
 * library's), 7 sqrtf, 8 GELU, 9 GELU derivative; 10+s, 20+s, 30+s tanhf,
 * log1pf, expm1f with division sequence s. */
int ugk_diag_math_eval(int fn, int variant, float *out, const float *in, size_t n);
/* For fn 63-67: the largest distance in ulp between the kernels' form and
 * its reference over the same inputs (NaN against NaN 0, NaN against a
 * number 2^32 - 1), and the input pattern where it occurs. Synchronous. */
int ugk_diag_math_ulp(int fn, unsigned lo, unsigned long long count, unsigned *max_ulp,
                      unsigned *at);
/* Philox4x32-10 on the device: in holds n tuples of 6 words (counter c0..c3,
 * key k0, k1), out receives n x 4 output words. */
int ugk_diag_philox(unsigned *out, const unsigned *in, size_t n);
/* The practical HBM ceiling of a load/store mix: a pure stream over nr input
 * and nw output tensors of n floats each, consecutive in buf (16-byte
 * aligned, n a multiple of 4, 1 <= nr <= 5, 1 <= nw <= 3). out_w[i] =
 * sum_r in_r[i] + w, non-temporal, per_thread (1-3) float4 per thread in
 * workgroups of block (256 or 512) threads. The benchmark times it at each
 * kernel's size, takes the best shape, and reports how close the kernel comes
 * to what its access pattern allows. Asynchronous. */
int ugk_diag_stream(float *buf, size_t n, int nr, int nw, int per_thread, int block);
/* The partial rows (workgroups) a LayerNorm backward of rows x C writes
 * (fused: the LayerNorm -> residual pair), and the bound the workspace's
 * LayerNorm slots are sized by, which covers every call with at most `rows`
 * rows. Host arithmetic only; no HIP call. */
int ugk_diag_layernorm_partial_rows(int rows, int C, int fused, int *actual, int *bound);
/* How the per-op LayerNorm backward entry points (ugk_layernorm_backward,
 * ugk_layernorm_residual_backward, ugk_layernorm_backward_noalloc) finish
 * their dweight/dbias column sums on the float4 path: on 0 (the default) a
 * second launch adds the partial rows; on 1 the main launch's workgroups add
 * them themselves, the last of each group of rows and then the last group,
 * through device-scope stores and loads and a counter, without an L2
 * write-back. Both add in the same order and give the same bits; the second
 * launch is the faster on MI355X (the in-launch form's chain of dependent
 * device-scope round trips costs more than the launch). on < 0 only
 * queries. Returns the previous setting. */
int ugk_diag_layernorm_tail(int on);

/* ---- GPT-2 layer-kernel step driver ------------------------------------
 * gpt2_kernels.cuh:634-719 (Config, param_offsets, act_offsets) and the
 * launch sequence of gpt2_forward / gpt2_backward (:756-896), restricted to
 * this library's kernels. The dense ops between them (QKV / proj / fc / fc2
 * GEMMs and attention) are the caller's: pass them as callbacks in
 * ugk_dense_ops, or pass NULL to run the layer kernels alone over whatever
 * those ops' output buffers already hold (what the benchmark does). Buffers
 * use the reference's flat layout, so the same params/acts/grads pointers
 * the reference allocates work unchanged. */
typedef struct {
  int B, T, C, V, NH, maxT, L;
} ugk_config;

typedef struct {
  void *ctx;
  /* out (M,OC) = inp (M,C) @ weight (C,OC) + bias */
  int (*matmul_forward)(void *ctx, float *out, const float *inp,
                        const float *weight, const float *bias, int M, int C,
                        int OC);
  /* dinp += dout @ weight^T; dweight += inp^T @ dout; dbias += colsum(dout) */
  int (*matmul_backward)(void *ctx, float *dinp, float *dweight, float *dbias,
                         const float *inp, const float *weight,
                         const float *dout, int M, int C, int OC);
  int (*attention_forward)(void *ctx, float *out, const float *qkv, int B,
                           int T, int C, int NH);
  int (*attention_backward)(void *ctx, float *dqkv, const float *dout,
                            const float *qkv, int B, int T, int C, int NH);
} ugk_dense_ops;

/* Float counts of the reference's parameter and activation buffers. */
size_t ugk_param_count(ugk_config cfg);
size_t ugk_act_count(ugk_config cfg);

/* ---- workspace (no counterpart in the reference: its kernels need none
 * beyond their arguments, and the caller owns every buffer, _C.cu:239-244) */

/* Bytes of device workspace every entry point needs at shapes up to cfg:
 * rows B*T of C channels, the step driver's L blocks, V logits per row. */
size_t ugk_workspace_bytes(ugk_config cfg);
/* Allocate the current device's workspace for shapes up to cfg now (library
 * owned, like ugk_reserve, but also covering the step driver). */
int ugk_reserve_config(ugk_config cfg);
/* Hand the current device a caller-owned workspace of `bytes` device bytes
 * (256-byte aligned, at least ugk_workspace_bytes(cfg)) for shapes up to cfg.
 * The library frees its own regions (after waiting for the device) and from
 * then on allocates nothing on this device; a call whose shape needs more
 * than cfg provides fails with UGK_ENOMEM. The memory must stay valid and be
 * left to the library until the next ugk_set_workspace on this device; NULL
 * returns to library-owned regions. Waits for the library stream. */
int ugk_set_workspace(void *ptr, size_t bytes, ugk_config cfg);

/* ---- per-op timing of the step driver (no counterpart in the reference,
 * which times single launches with cudaEvents in its dev/ harnesses). While
 * started, ugk_gpt2_layers_forward/backward time each library op they issue
 * (at most `capacity`) with a pair of HIP events recorded by the op's own
 * dispatches (hipExtLaunchKernelGGL): the start with its first kernel, the
 * stop with its last, so they measure the kernels themselves; the encoder
 * backward (three kernels) is bracketed by two event records on the library
 * stream instead. ugk_op_timer_read waits for the last
 * event, writes each op's duration in milliseconds and its kind (UGK_OP_*)
 * in issue order, sets *count, and stops the timer. The events are created by
 * ugk_op_timer_start. */
#define UGK_OP_ENCODER_FORWARD 1
#define UGK_OP_LAYERNORM_FORWARD 2
#define UGK_OP_RESIDUAL_LAYERNORM_FORWARD 3
#define UGK_OP_GELU_FORWARD 4
#define UGK_OP_LAYERNORM_BACKWARD_MAIN 5          /* dinp + partial column sums */
#define UGK_OP_LAYERNORM_RESIDUAL_BACKWARD_MAIN 6 /* the same, fused with residual_backward */
#define UGK_OP_GELU_BACKWARD 7
#define UGK_OP_LAYERNORM_COLUMN_SUMS 8            /* all LayerNorms' dweight/dbias, batched */
#define UGK_OP_ENCODER_BACKWARD 9
#define UGK_OP_ENCODER_LAYERNORM_FORWARD 10       /* encoder_forward + the first layernorm_forward */
int ugk_op_timer_start(int capacity);
int ugk_op_timer_read(float *ms, int *ops, int capacity, int *count);

/* Forward from the encoder to the final LayerNorm (gpt2_kernels.cuh:775-813).
 * The head GEMM and softmax/cross-entropy are not part of it. */
int ugk_gpt2_layers_forward(float *acts, const float *params, const int *inputs,
                            ugk_config cfg, const ugk_dense_ops *ops);

/* Backward from the final LayerNorm down to the encoder
 * (gpt2_kernels.cuh:846-894). On entry grads_acts holds d(final LN output)
 * at the reference's flo offset; accumulates into grads and grads_acts,
 * except that each LayerNorm backward fused with the residual_backward after
 * it adds into its dinp (res1 of every block, each block's resa) without
 * writing the sum back: the reference reads those gradients only in that
 * residual_backward (:855,874), so their contents after the call are
 * unspecified. Every other buffer equals the op-by-op sequence's. The
 * LayerNorm dweight/dbias column sums are completed by one launch at the end,
 * and their partial rows live in the workspace's LayerNorm region meanwhile,
 * so the dense callbacks must not call ugk_layernorm_backward or
 * ugk_layernorm_residual_backward (the other entry points use other regions). */
int ugk_gpt2_layers_backward(float *grads, float *grads_acts, const float *acts,
                             const float *params, const int *inputs,
                             ugk_config cfg, const ugk_dense_ops *ops);

/* ugk_gpt2_layers_backward for callers that zero grads_acts outside the flo
 * region before every backward, as every reference arm does (cudaMemset of
 * d_gacts before gpt2_backward: train_bnn_gpu.cu:475, train_bnn_vadam.cu:422,
 * train_bnn_lowrank.cu:919, train_ensemble.cu:281, uncertain/_C.cu:482,625,777,975).
 * No counterpart in the reference. Under that precondition every buffer
 * equals ugk_gpt2_layers_backward's; the zeros are not read: GELU backward
 * writes its dinp (fch), the fused residual splits write their dx and dy
 * (resa, mlpo, apr and res1 of every block), and the final LayerNorm takes
 * its dinp as zero. With C a multiple of 4 and at most 2,048, 16-byte
 * aligned buffers and L >= 1 the layer kernels therefore read none of those
 * buffers, and the result does not depend on what they hold on entry; the
 * dense callbacks still accumulate into theirs. */
int ugk_gpt2_layers_backward_zeroed(float *grads, float *grads_acts, const float *acts,
                                    const float *params, const int *inputs,
                                    ugk_config cfg, const ugk_dense_ops *ops);

/* ---- file formats of an end-to-end run ----------------------------------
 * Token files (llm.c's .bin: 256 int32 header with magic 20240520 and the
 * token count in header[2], then uint16 token ids) and checkpoints (8 int32
 * header {20240520, n low word, C, L, V, NH, steps, n high word}, then n
 * floats), as the reference reads and writes them. */

typedef struct ugk_loader ugk_loader;

/* gpt2_kernels.cuh:904-921 (loader_init): read the whole token file into host
 * memory. *ld is NULL on failure (missing file, short header, bad magic,
 * short read). */
int ugk_loader_open(ugk_loader **ld, const char *path);

/* gpt2_kernels.cuh:1318-1331 (loader_count): the token count from the header
 * alone. */
int ugk_loader_count(const char *path, long *ntok);

/* gpt2_kernels.cuh:924-929 (loader_next): inputs = tokens[pos, pos+BT),
 * targets = tokens[pos+1, pos+BT+1) into HOST buffers, pos += BT, restarting
 * at 0 when the window would pass the end. */
int ugk_loader_next(ugk_loader *ld, int *h_inp, int *h_tgt, int BT);

/* The same window into DEVICE buffers, widened on the GPU from a uint16 copy
 * of the tokens kept in device memory (made on the first call; 2 bytes per
 * token), so no tokens cross PCIe per step. No counterpart in the reference,
 * which copies each window from the host (train_bnn_gpu.cu:439-441). */
int ugk_loader_next_device(ugk_loader *ld, int *d_inp, int *d_tgt, int BT);

long ugk_loader_tokens(const ugk_loader *ld);    /* token count, -1 if NULL */
long ugk_loader_position(const ugk_loader *ld);  /* next window start */
int ugk_loader_close(ugk_loader *ld);

/* gpt2_kernels.cuh:950-951: "runs/<arm>_C<C>_L<L>_<steps/1000>k_<what>.bin". */
int ugk_ckpt_path(char *buf, size_t size, const char *arm, const char *what,
                  ugk_config cfg, int steps);

/* gpt2_kernels.cuh:944-964 (ckpt_save) at an explicit path: the n floats of
 * the DEVICE buffer d_buf, behind the 8-int header. Waits for the stream. */
int ugk_ckpt_save(const char *path, const float *d_buf, size_t n,
                  ugk_config cfg, int steps);

/* gpt2_kernels.cuh:1281-1316 (ckpt_load) at an explicit path: checks the
 * magic and the header's n, C, L, V, NH against the run's (an error, not a
 * load, on any mismatch), fills the DEVICE buffer d_buf and returns the
 * header's step count in *steps (may be NULL). Waits for the stream. */
int ugk_ckpt_load(const char *path, float *d_buf, size_t n, ugk_config cfg,
                  int *steps);

#ifdef __cplusplus
}
#endif

/* Abort-on-error wrapper with the reference's UNCERTAIN_ABORT behaviour
 * (gpt2_kernels.cuh:88-101): print file:line and the message, then exit. */
#define UGK_CHECK(call)                                                      \
  do {                                                                       \
    int ugk_status_ = (call);                                                \
    if (ugk_status_ != UGK_OK) {                                             \
      fprintf(stderr, "[UGK ERROR] at %s:%d\n%s\n", __FILE__, __LINE__,      \
              ugk_last_error());                                             \
      exit(EXIT_FAILURE);                                                    \
    }                                                                        \
  } while (0)

#endif /* UGK_H */
