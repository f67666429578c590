// ugk_diag.hip - diagnostics of the kernels' float math (no reference
// counterpart): exhaustive comparison of the SIMD-shaped math in
// ugk_libm_dev.h with its IEEE restatement in ugk_libm.h, and elementwise
// evaluation of either for comparison with the host C library.
#include "../../include/ugk.h"
#include "ugk_internal.h"
#include "ugk_libm_dev.h"
#include "ugk_philox.h"

namespace ugk {
namespace {

// fn codes: 0 expf, 1 log1pf, 2 expm1f, 3 tanhf, 4 softplus (the kernels'
// math); 5 logf, 6 cosf (evaluation only: the glibc restatements, ugk_logf
// on every input and ugk_cosf_small on |x| < 120, the device library's cosf
// elsewhere; variant 1 the device library's everywhere), 7 sqrtf (its reference: the double square
// root rounded to float, which is the correctly rounded result); 8 GELU and
// 9 its derivative as the GELU kernels evaluate them (reference: the same
// expressions over ugk_tanhf);
// 10+s, 20+s, 30+s: tanhf, log1pf, expm1f with division sequence s
// (ugk_div_t<s>), to compare the candidate sequences; 40+j: x / b for the
// divisor kDivisors[j] by ugk_div_recip on its domain (IEEE division outside
// it; reference: x / b); 48: ugk_dev_sqrtf_large on its domain (sqrtf
// outside; reference as fn 7); 49+s: 1 / x by ugk_div_t<s> for x >= 1, +inf
// and NaN (1.0f / x elsewhere; reference 1.0f / x), the candidate sequences
// for the sigmoid's quotient; 53: ugk_dev_recip_ge1, the one it uses, on the
// same domain; 54+j: x / b for the launch-wide divisor kSharedDivisors[j] by
// ugk_div_shared (reference x / b); 62: ugk_dev_sqrtf (reference as fn 7);
// 63: ugk_dev_expf_nooverflow on its domain, x <= 0x1.62e42ep6 or NaN
// (ugk_expf_t elsewhere; reference ugk_expf); 64 and 65: the default GELU
// and its derivative (the logistic form, ugk_fast_gelu*) against the
// glibc-exact expressions of fn 8 and 9, where a "mismatch" is a result
// outside |a - b| <= 1e-6 + 1e-5 |b| (equal bits and NaN against NaN pass);
// 66 and 67 the hardware-transcendental softplus and sigmoid of the Philox
// ops (ugk_fast_softplus, ugk_fast_sigmoid) against the glibc-exact
// softplus of fn 4 and train_bnn.c:820-822's 1 / (1 + expf(-x)), likewise
// counting results outside that bar; 69: ugk_dev_cosf_small on
// 0 <= x < 2^17, the default form's Box-Muller cosf (the library's cosf
// elsewhere; reference: the library's cosf); 70 and 71 the Box-Muller radius
// sqrt(-2 ln u1) on u1 in [2^-33, 1] (the reference elsewhere), 70 as the
// Philox ops' default form computes it (hardware log2 and square root), 71 as
// the glibc-exact form does (glibc's logf, the correctly rounded root),
// against the double radius rounded to float.
__constant__ float kDivisors[8] = {1.0f, 3.0f, 50257.0f, 0x1.fffffep0f, 0x1.fffffep15f, 0x1.000002p0f, 12345.678f,
                                   0x1.5p14f};

__constant__ float kSharedDivisors[8] = {0.01f, 0.1f, 1e-3f, 0.19f, 0x1p-24f, 1e-7f, 0.999f, 0x1p24f};

__device__ __forceinline__ float div_shared_by(float x, int j) {
  const float b = kSharedDivisors[j];
  return ugk_div_shared(x, b, 1.0f / b, ugk_div_shared_ok(b));
}

__device__ __forceinline__ float div_by(float x, int j) {
  const float b = kDivisors[j], y = 1.0f / b;
  const float ax = fabsf(x);
  const bool dom = ugk_f2u(x) == 0u || x != x || (ax >= 0x1p-86f && ax <= 0x1p100f);
  return dom ? ugk_div_recip(x, b, y) : x / b;
}

template <int FN>
__device__ __forceinline__ float kernel_math(float x, const uint64_t *tab) {
  if (FN == 0) return ugk_expf_t<UGK_EXPF_CONTRACT>(x, UgkExp2Lds{tab});
  if (FN == 1) return ugk_dev_log1pf(x);
  if (FN == 2) return ugk_dev_expm1f(x);
  if (FN == 3) return ugk_dev_tanhf(x);
  if (FN == 4) return ugk_dev_softplusf_lds(x, tab);
  if (FN == 5) return ugk_logf(x);
  if (FN == 6) return fabsf(x) < 120.0f ? ugk_cosf_small(x) : cosf(x);
  if (FN == 7) return sqrtf(x);
  if (FN == 8) return ugk_dev_gelu(x);
  if (FN == 9) return ugk_dev_gelu_grad(x);
  if (FN >= 10 && FN < 14) return ugk_dev_tanhf_t<FN - 10>(x);
  if (FN >= 20 && FN < 24) return ugk_dev_log1pf_t<FN - 20>(x);
  if (FN >= 40 && FN < 48) return div_by(x, FN - 40);
  if (FN == 48) return (fabsf(x) >= 0x1p-96f || x == 0.0f || x != x) ? ugk_dev_sqrtf_large(x) : sqrtf(x);
  if (FN >= 49 && FN < 53) return (x >= 1.0f || x != x) ? ugk_div_t<FN - 49>(1.0f, x) : 1.0f / x;
  if (FN == 53) return (x >= 1.0f || x != x) ? ugk_dev_recip_ge1(x) : 1.0f / x;
  if (FN >= 54 && FN < 62) return div_shared_by(x, FN - 54);
  if (FN == 62) return ugk_dev_sqrtf(x);
  if (FN == 63)
    return (x <= 0x1.62e42ep6f || x != x) ? ugk_dev_expf_nooverflow(x, UgkExp2Lds{tab}, UgkExpfAddends{})
                                          : ugk_expf_t<UGK_EXPF_CONTRACT>(x, UgkExp2Lds{tab});
  if (FN == 64) return ugk_fast_gelu(x);
  if (FN == 65) return ugk_fast_gelu_grad(x);
  if (FN == 66) return ugk_fast_softplus(x);
  if (FN == 67) return ugk_fast_sigmoid(x);
  if (FN == 69) return (x >= 0.0f && x < 0x1p17f) ? ugk_dev_cosf_small(x) : cosf(x);
  if (FN == 70 || FN == 71) {
    if (!(x >= 0x1p-33f && x <= 1.0f)) return (float)sqrt(-2.0 * log((double)x));
    return FN == 70 ? ugk_dev_bm_radius_fast(x) : ugk_dev_sqrtf_large(-2.0f * ugk_logf_normal(x));
  }
  return ugk_dev_expm1f_t<(FN >= 30 ? FN - 30 : 0)>(x);
}

template <int FN>
__device__ __forceinline__ float reference_math(float x) {
  if (FN == 0 || FN == 63) return ugk_expf(x);
  if (FN == 1 || (FN >= 20 && FN < 24)) return ugk_log1pf(x);
  if (FN == 3 || (FN >= 10 && FN < 14)) return ugk_tanhf(x);
  if (FN == 4 || FN == 66) return ugk_softplusf(x);
  if (FN == 67) return 1.0f / (1.0f + ugk_expf(-x));
  if (FN == 70 || FN == 71) return (float)sqrt(-2.0 * log((double)x));
  if (FN == 5) return logf(x);
  if (FN == 6 || FN == 69) return cosf(x);
  if (FN == 7) return (float)sqrt((double)x);
  if (FN == 8 || FN == 64) return ugk_gelu_with(x, [](float u) { return ugk_tanhf(u); });
  if (FN == 9 || FN == 65) return ugk_gelu_grad_with(x, [](float u) { return ugk_tanhf(u); });
  if (FN >= 40 && FN < 48) return x / kDivisors[FN - 40];
  if (FN == 48) return (float)sqrt((double)x);
  if (FN >= 49 && FN < 54) return 1.0f / x;
  if (FN >= 54 && FN < 62) return x / kSharedDivisors[FN - 54];
  if (FN == 62) return (float)sqrt((double)x);
  return ugk_expm1f(x);
}

template <int FN>
__global__ __launch_bounds__(kBlock) void k_math_mismatch(unsigned long long lo, unsigned long long count,
                                                          unsigned long long *nbad, unsigned *first) {
  __shared__ uint64_t tab[32];
  ugk_exp2_stage(tab);
  __syncthreads();
  unsigned long long local = 0;
  unsigned lfirst = 0xffffffffu;
  for (unsigned long long i = (unsigned long long)blockIdx.x * kBlock + threadIdx.x; i < count;
       i += (unsigned long long)gridDim.x * kBlock) {
    const unsigned u = (unsigned)(lo + i);
    const float x = ugk_u2f(u);
    const float a = kernel_math<FN>(x, tab), b = reference_math<FN>(x);
    // fn 64/65: the literal bar; the others: the same bits
    const bool within = FN >= 64 && fabsf(a - b) <= 1e-6f + 1e-5f * fabsf(b);
    if (ugk_f2u(a) != ugk_f2u(b) && !(a != a && b != b) && !within) {
      local++;
      lfirst = min(lfirst, u);
    }
  }
  if (local) {
    atomicAdd(nbad, local);
    atomicMin(first, lfirst);
  }
}

template <int FN>
__global__ __launch_bounds__(kBlock) void k_math_eval(int variant, float *out, const float *in, size_t n) {
  __shared__ uint64_t tab[32];
  ugk_exp2_stage(tab);
  __syncthreads();
  for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (size_t)gridDim.x * kBlock)
    out[i] = variant == 0 ? kernel_math<FN>(in[i], tab) : reference_math<FN>(in[i]);
}

// Philox4x32-10 of arbitrary (counter, key) tuples: in holds 6 words per
// tuple (c0..c3, k0, k1), out receives the 4 output words.
__global__ __launch_bounds__(kBlock) void k_philox(unsigned *out, const unsigned *in, size_t n) {
  for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (size_t)gridDim.x * kBlock) {
    const unsigned *c = in + 6 * i;
    const UgkPhilox4 o = ugk_philox4x32_10(c[0], c[1], c[2], c[3], c[4], c[5]);
    for (int j = 0; j < 4; j++) out[4 * i + j] = o.w[j];
  }
}

// A pure stream with the load/store mix of a kernel: element group i reads
// float4 i of each of NR input tensors and writes float4 i of NW output
// tensors (their sum, plus w for output w), non-temporal, U float4 per thread
// in BS-thread workgroups. Tensors are consecutive in buf, n floats each.
template <int NR, int NW, int U, int BS>
__global__ __launch_bounds__(BS) void k_stream(float4 *buf, size_t n4) {
  const size_t base = (size_t)blockIdx.x * (BS * U) + threadIdx.x;
  float4 a[U][NR];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const size_t i = base + (size_t)u * BS;
#pragma unroll
    for (int r = 0; r < NR; r++) a[u][r] = i < n4 ? ld_nt(buf + (size_t)r * n4 + i) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int u = 0; u < U; u++) {
    const size_t i = base + (size_t)u * BS;
    if (i >= n4) continue;
    float4 s = a[u][0];
#pragma unroll
    for (int r = 1; r < NR; r++) s = make_float4(s.x + a[u][r].x, s.y + a[u][r].y, s.z + a[u][r].z, s.w + a[u][r].w);
#pragma unroll
    for (int w = 0; w < NW; w++)
      st_nt(buf + (size_t)(NR + w) * n4 + i, make_float4(s.x + w, s.y + w, s.z + w, s.w + w));
  }
}

template <int NR, int NW>
int launch_stream(float4 *b, size_t n4, int per_thread, int block) {
  const int key = per_thread * 10000 + block;
  switch (key) {
#define UGK_SH(u, bs) \
  case u * 10000 + bs: hipLaunchKernelGGL((k_stream<NR, NW, u, bs>), dim3(grid_for(n4, (size_t)u * bs)), dim3(bs), 0, stream(), b, n4); break;
    UGK_SH(1, 256) UGK_SH(2, 256) UGK_SH(3, 256) UGK_SH(1, 512) UGK_SH(2, 512) UGK_SH(3, 512)
#undef UGK_SH
    default: return set_error(UGK_EINVAL, "ugk_diag_stream: per_thread must be 1-3 and block 256 or 512");
  }
  return UGK_OK;
}

bool fn_ok(int fn) {
  return (fn >= 0 && fn <= 9) || (fn >= 10 && fn < 14) || (fn >= 20 && fn < 24) || (fn >= 30 && fn < 34) ||
         (fn >= 40 && fn < 72 && fn != 68);
}

// The largest distance in ulp (as ordered integers) between the kernels' math
// and its reference over bit patterns, packed with the input that gives it:
// (distance << 32) | pattern, the largest pattern among ties. NaN against NaN
// counts 0, NaN against a number 2^32 - 1.
__device__ __forceinline__ long long ordered_bits(float v) {
  const int i = (int)ugk_f2u(v);
  return i < 0 ? -(long long)(i & 0x7fffffff) : (long long)i;
}

template <int FN>
__global__ __launch_bounds__(kBlock) void k_math_ulp(unsigned long long lo, unsigned long long count,
                                                     unsigned long long *best) {
  __shared__ uint64_t tab[32];
  ugk_exp2_stage(tab);
  __syncthreads();
  unsigned long long local = 0;
  for (unsigned long long i = (unsigned long long)blockIdx.x * kBlock + threadIdx.x; i < count;
       i += (unsigned long long)gridDim.x * kBlock) {
    const unsigned u = (unsigned)(lo + i);
    const float x = ugk_u2f(u);
    const float a = kernel_math<FN>(x, tab), b = reference_math<FN>(x);
    unsigned long long d;
    if (a != a || b != b) {
      d = (a != a && b != b) ? 0ull : 0xffffffffull;
    } else {
      const long long diff = ordered_bits(a) - ordered_bits(b);
      const unsigned long long ad = (unsigned long long)(diff < 0 ? -diff : diff);
      d = ad > 0xffffffffull ? 0xffffffffull : ad;
    }
    const unsigned long long key = (d << 32) | u;
    local = key > local ? key : local;
  }
  if (local) atomicMax(best, local);
}
int bad_fn(const char *fn) { return set_error(UGK_EINVAL, "%s: unknown fn code", fn); }

}  // namespace
}  // namespace ugk

using namespace ugk;

extern "C" int ugk_diag_math_mismatch(int fn, unsigned lo, unsigned long long count,
                                      unsigned long long *mismatches, unsigned *first) {
  if (!fn_ok(fn)) return bad_fn("ugk_diag_math_mismatch");
  if (!mismatches || !first) return set_error(UGK_EINVAL, "ugk_diag_math_mismatch: NULL result pointer");
  if (count > (1ull << 32) - lo) return set_error(UGK_EINVAL, "ugk_diag_math_mismatch: range beyond 2^32");
  struct Res {
    unsigned long long n;
    unsigned first;
  } h{0, 0xffffffffu};
  Res *d = nullptr;
  if (hipMalloc(&d, sizeof(Res)) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(UGK_ENOMEM, "ugk_diag_math_mismatch: hipMalloc failed");
  }
  int rc = UGK_OK;
  if (hipMemcpyAsync(d, &h, sizeof h, hipMemcpyHostToDevice, stream()) != hipSuccess) rc = UGK_EHIP;
  const dim3 grid(8192), block(kBlock);
  if (rc == UGK_OK && count) {
    switch (fn) {
#define UGK_MM(f) \
  case f: hipLaunchKernelGGL(k_math_mismatch<f>, grid, block, 0, stream(), (unsigned long long)lo, count, &d->n, &d->first); break;
      UGK_MM(0) UGK_MM(1) UGK_MM(2) UGK_MM(3) UGK_MM(4) UGK_MM(5) UGK_MM(6) UGK_MM(7) UGK_MM(8) UGK_MM(9)
      UGK_MM(10) UGK_MM(11) UGK_MM(12) UGK_MM(13) UGK_MM(20) UGK_MM(21) UGK_MM(22) UGK_MM(23)
      UGK_MM(30) UGK_MM(31) UGK_MM(32) UGK_MM(33)
      UGK_MM(40) UGK_MM(41) UGK_MM(42) UGK_MM(43) UGK_MM(44) UGK_MM(45) UGK_MM(46) UGK_MM(47)
      UGK_MM(48) UGK_MM(49) UGK_MM(50) UGK_MM(51) UGK_MM(52) UGK_MM(53)
      UGK_MM(54) UGK_MM(55) UGK_MM(56) UGK_MM(57) UGK_MM(58) UGK_MM(59) UGK_MM(60) UGK_MM(61) UGK_MM(62) UGK_MM(63)
      UGK_MM(64) UGK_MM(65) UGK_MM(66) UGK_MM(67) UGK_MM(69) UGK_MM(70) UGK_MM(71)
#undef UGK_MM
    }
    rc = check_launch("ugk_diag_math_mismatch");
  }
  if (rc == UGK_OK && hipMemcpyAsync(&h, d, sizeof h, hipMemcpyDeviceToHost, stream()) != hipSuccess) rc = UGK_EHIP;
  if (rc == UGK_OK && hipStreamSynchronize(stream()) != hipSuccess) rc = UGK_EHIP;
  (void)hipFree(d);
  if (rc != UGK_OK) return rc == UGK_EHIP ? set_error(rc, "ugk_diag_math_mismatch: HIP error") : rc;
  *mismatches = h.n;
  *first = h.first;
  return UGK_OK;
}

extern "C" int ugk_diag_math_eval(int fn, int variant, float *out, const float *in, size_t n) {
  if (!fn_ok(fn)) return bad_fn("ugk_diag_math_eval");
  if (n == 0) return UGK_OK;
  if (!out || !in) return set_error(UGK_EINVAL, "ugk_diag_math_eval: NULL pointer");
  unsigned g = grid_for(n, kBlock);
  if (g > 65536u) g = 65536u;
  switch (fn) {
#define UGK_EV(f) \
  case f: hipLaunchKernelGGL(k_math_eval<f>, dim3(g), dim3(kBlock), 0, stream(), variant, out, in, n); break;
    UGK_EV(0) UGK_EV(1) UGK_EV(2) UGK_EV(3) UGK_EV(4) UGK_EV(5) UGK_EV(6) UGK_EV(7) UGK_EV(8) UGK_EV(9)
    UGK_EV(10) UGK_EV(11) UGK_EV(12) UGK_EV(13) UGK_EV(20) UGK_EV(21) UGK_EV(22) UGK_EV(23)
    UGK_EV(30) UGK_EV(31) UGK_EV(32) UGK_EV(33)
    UGK_EV(40) UGK_EV(41) UGK_EV(42) UGK_EV(43) UGK_EV(44) UGK_EV(45) UGK_EV(46) UGK_EV(47)
    UGK_EV(48) UGK_EV(49) UGK_EV(50) UGK_EV(51) UGK_EV(52) UGK_EV(53)
    UGK_EV(54) UGK_EV(55) UGK_EV(56) UGK_EV(57) UGK_EV(58) UGK_EV(59) UGK_EV(60) UGK_EV(61) UGK_EV(62) UGK_EV(63)
    UGK_EV(64) UGK_EV(65) UGK_EV(66) UGK_EV(67) UGK_EV(69) UGK_EV(70) UGK_EV(71)
#undef UGK_EV
  }
  return check_launch("ugk_diag_math_eval");
}

extern "C" int ugk_diag_stream(float *buf, size_t n, int nr, int nw, int per_thread, int block) {
  if (nr < 1 || nr > 5 || nw < 1 || nw > 3) return set_error(UGK_EINVAL, "ugk_diag_stream: need 1 <= nr <= 5, 1 <= nw <= 3");
  if (n == 0) return UGK_OK;
  if (!buf || (n & 3) || !aligned16(buf)) return set_error(UGK_EINVAL, "ugk_diag_stream: buf must be 16-byte aligned and n a multiple of 4");
  const size_t n4 = n / 4;
  float4 *b = reinterpret_cast<float4 *>(buf);
  int rc = UGK_OK;
  switch (nr * 10 + nw) {
#define UGK_ST(r, w) \
  case r * 10 + w: rc = launch_stream<r, w>(b, n4, per_thread, block); break;
    UGK_ST(1, 1) UGK_ST(1, 2) UGK_ST(1, 3) UGK_ST(2, 1) UGK_ST(2, 2) UGK_ST(2, 3) UGK_ST(3, 1) UGK_ST(3, 2)
    UGK_ST(3, 3) UGK_ST(4, 1) UGK_ST(4, 2) UGK_ST(4, 3) UGK_ST(5, 1) UGK_ST(5, 2) UGK_ST(5, 3)
#undef UGK_ST
  }
  return rc != UGK_OK ? rc : check_launch("ugk_diag_stream");
}

extern "C" int ugk_diag_philox(unsigned *out, const unsigned *in, size_t n) {
  if (n == 0) return UGK_OK;
  if (!out || !in) return set_error(UGK_EINVAL, "ugk_diag_philox: NULL pointer");
  unsigned g = grid_for(n, kBlock);
  if (g > 65536u) g = 65536u;
  hipLaunchKernelGGL(k_philox, dim3(g), dim3(kBlock), 0, stream(), out, in, n);
  return check_launch("ugk_diag_philox");
}

extern "C" int ugk_diag_layernorm_partial_rows(int rows, int C, int fused, int *actual, int *bound) {
  if (rows < 0 || C <= 0) return set_error(UGK_EINVAL, "ugk_diag_layernorm_partial_rows: need rows >= 0, C > 0");
  if (!actual || !bound) return set_error(UGK_EINVAL, "ugk_diag_layernorm_partial_rows: NULL result pointer");
  *actual = layernorm_backward_blocks(rows, C, fused != 0, kMaxPartialRows);
  *bound = layernorm_backward_blocks_bound(rows, C);
  return UGK_OK;
}

extern "C" int ugk_diag_layernorm_tail(int on) {
  const int prev = layernorm_tail();
  if (on >= 0) set_layernorm_tail(on);
  return prev;
}

extern "C" int ugk_diag_math_ulp(int fn, unsigned lo, unsigned long long count, unsigned *max_ulp,
                                 unsigned *at) {
  if (fn < 63 || fn > 71 || fn == 68 || fn == 69)
    return set_error(UGK_EINVAL, "ugk_diag_math_ulp: fn must be 63-67, 70 or 71");
  if (!max_ulp || !at) return set_error(UGK_EINVAL, "ugk_diag_math_ulp: NULL result pointer");
  if (count > (1ull << 32) - lo) return set_error(UGK_EINVAL, "ugk_diag_math_ulp: range beyond 2^32");
  unsigned long long h = 0, *d = nullptr;
  if (hipMalloc(&d, sizeof h) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(UGK_ENOMEM, "ugk_diag_math_ulp: hipMalloc failed");
  }
  int rc = UGK_OK;
  if (hipMemcpyAsync(d, &h, sizeof h, hipMemcpyHostToDevice, stream()) != hipSuccess) rc = UGK_EHIP;
  if (rc == UGK_OK && count) {
    const dim3 grid(8192), block(kBlock);
    switch (fn) {
#define UGK_UL(f) \
  case f: hipLaunchKernelGGL(k_math_ulp<f>, grid, block, 0, stream(), (unsigned long long)lo, count, d); break;
      UGK_UL(63) UGK_UL(64) UGK_UL(65) UGK_UL(66) UGK_UL(67) UGK_UL(70) UGK_UL(71)
#undef UGK_UL
    }
    rc = check_launch("ugk_diag_math_ulp");
  }
  if (rc == UGK_OK && hipMemcpyAsync(&h, d, sizeof h, hipMemcpyDeviceToHost, stream()) != hipSuccess) rc = UGK_EHIP;
  if (rc == UGK_OK && hipStreamSynchronize(stream()) != hipSuccess) rc = UGK_EHIP;
  (void)hipFree(d);
  if (rc != UGK_OK) return rc == UGK_EHIP ? set_error(rc, "ugk_diag_math_ulp: HIP error") : rc;
  *max_ulp = (unsigned)(h >> 32);
  *at = (unsigned)h;
  return UGK_OK;
}
