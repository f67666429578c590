// ugk_libm_dev.h - the float math of the kernels, shaped for a 64-lane SIMD.
//
// Same operations as ugk_libm.h (the line-by-line restatement of glibc's
// expm1f/tanhf/log1pf), in the same order and with the same rounding, but
// arranged for wavefronts:
//   * tanhf evaluates one expm1f instead of two inlined copies, and that
//     expm1f is specialised to the arguments tanhf gives it (2|x| for
//     |x| >= 1, -2|x| below), with the fdlibm cases computed side by side and
//     selected rather than branched on, since neighbouring lanes of a GELU
//     input routinely fall in different cases;
//   * log1pf keeps branches, because the inputs softplus feeds it (expf of a
//     weight's rho) are coherent across a wavefront and the common case then
//     runs alone;
//   * divisions are a reciprocal seed plus Newton-Raphson corrections
//     (ugk_div) rather than the compiler's general IEEE sequence.
//
// That each function here equals its ugk_libm.h counterpart on every one of
// the 2^32 inputs is checked on the GPU by ugk_diag_math_mismatch
// (tests/test_parity_gpu.py); ugk_libm.h itself equals the host glibc on
// every input (oracle/libm_exhaustive.cpp).
//
// The fdlibm algorithms and coefficients used here carry fdlibm's notice:
//   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//   Developed at SunPro, a Sun Microsystems, Inc. business.
//   Permission to use, copy, modify, and distribute this
//   software is freely granted, provided that this notice
//   is preserved.
// expf follows ARM optimized-routines (Copyright (c) 2017-2018 Arm Limited;
// MIT OR Apache-2.0 WITH LLVM-exception); see the LICENSE file.
#pragma once

#include "ugk_libm.h"

// a / b rounded to nearest-even, for the operand ranges these functions
// produce (b normal, quotient normal or zero). kSteps selects the sequence:
//   0 the compiler's IEEE division;
//   1 v_rcp_f32 seed, q = a*r, one residual correction;
//   2 as 1 with the reciprocal refined by one Newton step first;
//   3 as 2 with a second residual correction.
template <int kSteps>
__device__ __forceinline__ float ugk_div_t(float a, float b) {
  if (kSteps == 0) return a / b;
  float r = __builtin_amdgcn_rcpf(b);
  if (kSteps >= 2) {
    const float t = __builtin_fmaf(-b, r, 1.0f);
    r = __builtin_fmaf(t, r, r);
  }
  float q = a * r;
  float e = __builtin_fmaf(-b, q, a);
  q = __builtin_fmaf(e, r, q);
  if (kSteps >= 3) {
    e = __builtin_fmaf(-b, q, a);
    q = __builtin_fmaf(e, r, q);
  }
  return q;
}

#ifndef UGK_DIV_STEPS
#define UGK_DIV_STEPS 1
#endif

// a / b, correctly rounded, from y = 1.0f / b (itself correctly rounded), for
// a divisor shared by many quotients: q = a*y is within one ulp of a/b, so the
// remainder a - b*q is exact in one fma, and q + r*y rounds to the correctly
// rounded quotient (Markstein, "Computation of elementary functions on the
// IBM RISC System/6000 processor", IBM J. Res. Develop. 34(1), 1990). Three
// operations instead of the dozen of a general division. Domain:
// 1 <= b <= 2^16, and a == +0, NaN, or 2^-86 <= |a| <= 2^100 (-0 would come
// out +0). There the quotient is at least 2^-102, so the exact remainder is a
// multiple of 2^-149 and stays representable where it is subnormal, and
// nothing overflows.
// Checked against a / b on every a for a set of b (ugk_diag.hip fn 40-47)
// and on the CPU (tests/div_recip_check.c).
__device__ __forceinline__ float ugk_div_recip(float a, float b, float y) {
  const float q = a * y;
  const float r = __builtin_fmaf(-b, q, a);
  return __builtin_fmaf(r, y, q);
}

// a / b for a divisor shared by a whole launch (a per-launch scalar), given
// y = 1.0f / b: ugk_div_recip where it is exact, IEEE division elsewhere (a
// rare branch). Exact for b in [2^-24, 2^24] (b_ok, decided by the caller)
// and a == +0 or 2^-102 <= |a| <= 2^100: then a/b >= 2^-126 is normal, and
// the exponents of b and of the quotient sum to at least -103, so the exact
// remainder is a multiple of 2^-149 (ugk_diag.hip fn 54-61 check eight
// divisors on every a).
__device__ __forceinline__ float ugk_div_shared(float a, float b, float y, bool b_ok) {
  float q = ugk_div_recip(a, b, y);
  const float aa = fabsf(a);
  const bool ok = b_ok && ((aa >= 0x1p-102f && aa <= 0x1p100f) || ugk_f2u(a) == 0u);
  if (__builtin_expect(!ok, 0)) q = a / b;
  return q;
}

// Whether b may take ugk_div_shared's reciprocal form.
__host__ __device__ inline bool ugk_div_shared_ok(float b) { return b >= 0x1p-24f && b <= 0x1p24f; }

// The domain test of ugk_div_recip for a in [0, 1] or NaN, folded over many
// a with a running unsigned minimum: lo = min(lo, ugk_div_recip_key(a)) stays
// >= kUgkDivRecipKeyMin exactly when every a was +0, NaN or in [2^-86, 1].
__device__ __forceinline__ uint32_t ugk_div_recip_key(float a) { return ugk_f2u(a) - 1u; }
constexpr uint32_t kUgkDivRecipKeyMin = 0x14800000u - 1u;  // bits of 2^-86, minus 1

__device__ __forceinline__ float ugk_div(float a, float b) { return ugk_div_t<UGK_DIV_STEPS>(a, b); }

// 1 / b for b >= 1 or NaN, correctly rounded (the sigmoid's quotient): the
// reciprocal seed with one correction (ugk_div_t<1>) is the IEEE quotient for
// every b in [1, 2^126] (ugk_diag.hip fn 50 finds it wrong only above, where
// the quotient is subnormal or 0), and the rare larger b divide.
__device__ __forceinline__ float ugk_dev_recip_ge1(float b) {
  float q = ugk_div_t<1>(1.0f, b);
  if (__builtin_expect(b > 0x1p126f, 0)) q = 1.0f / b;
  return q;
}

// sqrtf, correctly rounded, for x >= 2^-96 and for +-0, +inf and NaN: the
// hardware square root s is within one ulp, and its neighbour below (above)
// replaces it when the remainder x - neighbour * s shows that neighbour to be
// the nearer one. This is the device library's sequence without the rescaling
// it applies first to inputs below 2^-96 and its +-0/inf/NaN selects, which the
// sequence already gets right. Checked on every input of the domain
// (ugk_diag.hip fn 48).
__device__ __forceinline__ float ugk_dev_sqrtf_large(float x) {
  const float s = __builtin_amdgcn_sqrtf(x);
  const float dn = ugk_u2f(ugk_f2u(s) - 1u), up = ugk_u2f(ugk_f2u(s) + 1u);
  float t = __builtin_fmaf(-dn, s, x) <= 0.0f ? dn : s;
  t = __builtin_fmaf(-up, s, x) > 0.0f ? up : t;
  return t;
}

// The device library's cosf (ocml, as hipcc builds it for gfx950) on its
// small-argument path, 0 <= x < 2^17: k = rint(x 2/pi), the remainder
// x - k pi/2 by three fused multiply-adds (Cody-Waite, pi/2 in three
// parts), the sine and cosine polynomials of the remainder, and the quadrant
// k mod 4 choosing cos, -sin, -cos or sin. Larger x take the library's
// Payne-Hanek reduction and infinities its NaN case, neither of which the
// Box-Muller angle 2 pi u2 in (0, 2 pi] reaches. Bit-identical to cosf on
// 0 <= x < 2^17 (ugk_diag.hip fn 69). The default (fast-math) form of the
// Philox ops' Box-Muller transform; the glibc-exact form takes glibc's cosf
// (ugk_cosf_small in ugk_libm.h).
__device__ __forceinline__ float ugk_dev_cosf_small(float x) {
  const float kf = __builtin_rintf(x * 0x1.45f306p-1f);
  const int q = (int)kf;
  float r = __builtin_fmaf(kf, -0x1.921fb4p0f, x);
  r = __builtin_fmaf(kf, -0x1.4442d0p-24f, r);
  r = __builtin_fmaf(kf, -0x1.846988p-48f, r);
  const float s = r * r;
  float p = __builtin_fmaf(s, -0x1.983304p-13f, 0x1.110388p-7f);
  p = __builtin_fmaf(s, p, -0x1.55553ap-3f);
  const float sn = __builtin_fmaf(r, s * p, r);
  float c = __builtin_fmaf(s, 0x1.aea668p-16f, -0x1.6c9e76p-10f);
  c = __builtin_fmaf(s, c, 0x1.5557eep-5f);
  c = __builtin_fmaf(s, c, -0x1.000008p-1f);
  const float cs = __builtin_fmaf(s, c, 1.0f);
  const float v = (q & 1) ? -sn : cs;
  return __uint_as_float(__float_as_uint(v) ^ (((uint32_t)q << 30) & 0x80000000u));
}

// sqrtf for any input: ugk_dev_sqrtf_large on its domain, the library's
// sqrtf (which rescales) for the rare tiny or negative inputs (fn 62).
__device__ __forceinline__ float ugk_dev_sqrtf(float x) {
  float r = ugk_dev_sqrtf_large(x);
  if (__builtin_expect(x < 0x1p-96f && x != 0.0f, 0)) r = sqrtf(x);
  return r;
}

// expm1f for any input, branch-free (used by the exhaustive diagnostic and as
// the general form of the specialised copy inside tanhf).
template <int kDiv>
__device__ __forceinline__ float ugk_dev_expm1f_t(float x) {
  const float o_threshold = 8.8721679688e+01f;
  const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
  const float invln2 = 1.4426950216e+00f;
  const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f,
              Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f,
              Q5 = -2.0109921195e-07f;
  const uint32_t ux = ugk_f2u(x);
  const uint32_t hx = ux & 0x7fffffffu;
  const bool neg = (ux >> 31) != 0;
  // argument reduction: k = 0 (|x| <= ln2/2), +-1 (|x| < 1.5 ln2) or round(x/ln2)
  const bool red = hx > 0x3eb17218u;
  const bool near = hx < 0x3F851592u;
  const float kf = invln2 * x + (neg ? -0.5f : 0.5f);
  const int kg = (hx < 0x4e000000u) ? (int)kf : 0;  // |x| < 2^29 keeps kf in int range; larger x are masked below
  const int k = red ? (near ? (neg ? -1 : 1) : kg) : 0;
  const float t = (float)k;
  const float hi = x - t * ln2_hi;
  const float lo = t * ln2_lo;
  const float xr = hi - lo;
  const float c = (hi - xr) - lo;
  // x in the primary range
  const float hfx = 0.5f * xr;
  const float hxs = xr * hfx;
  const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  const float tt = 3.0f - r1 * hfx;
  const float e = hxs * ugk_div_t<kDiv>(r1 - tt, 6.0f - xr * tt);
  float e2 = (xr * (e - c) - c);
  e2 -= hxs;
  // k == 0: fdlibm's xr - (xr*e - hxs); there t = 0 gives c = +0, so e2 rounds
  // exactly as xr*e - hxs
  const float y0 = xr - e2;
  const float ym1 = 0.5f * (xr - e2) - 0.5f;  // k == -1
  const float yp1 = (xr < -0.25f) ? -2.0f * (e2 - (xr + 0.5f)) : 1.0f + 2.0f * (xr - e2);  // k == 1
  const uint32_t kbits = (uint32_t)k << 23;
  float ys = 1.0f - (e2 - xr);  // k <= -2 or k > 56
  ys = (k == 128) ? ys * 2.0f * 0x1p127f : ugk_u2f(ugk_f2u(ys) + kbits);
  ys = ys - 1.0f;
  const int ks = (k >= 0 && k < 32) ? k : 0;
  const float tlo = ugk_u2f(0x3f800000u - (0x1000000u >> ks));  // 1 - 2^-k
  float ylo = tlo - (e2 - xr);  // 2 <= k < 23
  ylo = ugk_u2f(ugk_f2u(ylo) + kbits);
  const float thi = ugk_u2f((uint32_t)(0x7f - k) << 23);  // 2^-k
  float yhi = xr - (e2 + thi);  // 23 <= k <= 56
  yhi += 1.0f;
  yhi = ugk_u2f(ugk_f2u(yhi) + kbits);
  float y = (k <= -2 || k > 56) ? ys : (k < 23 ? ylo : yhi);
  y = (k == 1) ? yp1 : y;
  y = (k == -1) ? ym1 : y;
  y = (k == 0) ? y0 : y;
  // the reference's early returns
  y = (!red && hx < 0x33000000u) ? x : y;             // |x| < 2^-25
  if (hx >= 0x4195b844u) {                            // |x| >= 27 ln2
    if (neg) y = -1.0f;
    if (hx >= 0x42b17218u) {
      if (!neg && x > o_threshold) y = ugk_u2f(0x7f800000u);
      if (hx == 0x7f800000u) y = neg ? -1.0f : x;
      if (hx > 0x7f800000u) y = x + x;
    }
  }
  return y;
}

// expm1f(a) for the arguments tanhf passes: a = 2|x| in [2, 44] (so k >= 3)
// when big, a = -2|x| in (-2, 0] otherwise (so k is 0, -1, -2 or -3).
// tanhf clamps 2|x| to 44: every |x| >= 22 then gives t near 2^63, for which
// 1 - 2/(t+2) rounds to 1 as the reference's |x| >= 22 case returns.
template <int kDiv>
__device__ __forceinline__ float ugk_dev_expm1f_tanh(float a, bool big) {
  const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
  const float invln2 = 1.4426950216e+00f;
  const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f,
              Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f,
              Q5 = -2.0109921195e-07f;
  // fdlibm takes k = 0 for |a| <= ln2/2 and k = -1 for |a| < 1.5 ln2 (a < 0
  // there); the rounding formula it uses beyond gives the same k over those
  // ranges too, up to the bit patterns at the two thresholds, where the
  // exhaustive comparison finds the same tanhf either way.
  const float kf = invln2 * a + (big ? 0.5f : -0.5f);
  const int k = (int)kf;
  const float t = (float)k;
  // ln2_hi has 17 significant bits and |k| <= 64, so t * ln2_hi is exact and
  // one fused multiply-add rounds a - t * ln2_hi exactly as the product and
  // the subtraction do
  const float hi = __builtin_fmaf(-t, ln2_hi, a);
  const float lo = t * ln2_lo;
  const float xr = hi - lo;
  const float c = (hi - xr) - lo;
  const float hfx = 0.5f * xr;
  const float hxs = xr * hfx;
  const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  const float tt = 3.0f - r1 * hfx;
  const float e = hxs * ugk_div_t<kDiv>(r1 - tt, 6.0f - xr * tt);
  float e2 = (xr * (e - c) - c);
  e2 -= hxs;
  const float d = e2 - xr;
  // Scaled cases, "base - d, then add k to the exponent": base is 1 - 2^-k
  // for k < 25 and 1 above (the shift amount min(k, 31) as unsigned also
  // maps k = -2, -3 to 1), then 1 is subtracted when !big (k = -2, -3).
  // expm1f itself uses (xr - (e2 + 2^-k)) + 1 for 23 <= k <= 56; for tanhf
  // the two forms give the same result on every input, checked exhaustively.
  const uint32_t ks = min((uint32_t)k, 31u);
  const float base = ugk_u2f(0x3f800000u - (0x1000000u >> ks));
  float y = ugk_u2f(ugk_f2u(base - d) + ((uint32_t)k << 23));
  y = big ? y : y - 1.0f;
  y = (k == -1) ? 0.5f * (xr - e2) - 0.5f : y;
  // k == 0: fdlibm's xr - (xr*e - hxs). There t = 0 makes hi = xr = a and
  // lo = c = +0, so e2 = xr*(e - c) - c - hxs rounds exactly as xr*e - hxs
  // and xr - e2 is that result. fdlibm returns a itself for |a| < 2^-25; the
  // general formula gives a there too (a*a/2 is below half an ulp of a, and
  // underflows to 0 for subnormal a), so that case needs no select of its own.
  y = (k == 0) ? xr - e2 : y;
  return y;
}

// kNan = false drops the NaN case (tanhf(NaN) then gives +-1), for callers
// whose result is NaN anyway when x is (GELU multiplies by x).
template <int kDiv, bool kNan = true>
__device__ __forceinline__ float ugk_dev_tanhf_t(float x) {
  const uint32_t jx = ugk_f2u(x);
  const uint32_t ix = jx & 0x7fffffffu;
  const float a2 = fminf(2.0f * ugk_u2f(ix), 44.0f);  // also maps NaN (quieted by the product) to 44
  const bool big = a2 >= 2.0f;                        // |x| >= 1
  const float a = big ? a2 : -a2;
  const float t = ugk_dev_expm1f_tanh<kDiv>(a, big);
  const float q = ugk_div_t<kDiv>(big ? 2.0f : -t, t + 2.0f);
  const float z = big ? 1.0f - q : q;
  float r = ugk_u2f(ugk_f2u(z) ^ (jx & 0x80000000u));
  // fdlibm's |x| < 2^-55 case, x*(1+x) = x, needs no select either: there
  // expm1f gives t = -2|x| exactly, 2 - 2|x| rounds to 2, and -t/(t+2) = |x|,
  // so r = x (also for +-0 and subnormals).
  if (kNan) r = (ix > 0x7f800000u) ? x + x : r;
  return r;
}

template <int kDiv>
__device__ __forceinline__ float ugk_dev_log1pf_t(float x) {
  const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
  const float Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f,
              Lp3 = 2.8571429849e-01f, Lp4 = 2.2222198546e-01f,
              Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f,
              Lp7 = 1.4798198640e-01f;
  const int32_t hx = (int32_t)ugk_f2u(x);
  const int32_t ax = hx & 0x7fffffff;
  int k = 0, hu = 1;
  float f = x, c = 0.0f;
  if (!(hx < 0x3ed413d7 && (hx > 0 || hx <= (int32_t)0xbe95f61fu))) {  // 1 + x = 2^k (1 + f)
    float u;
    if (hx < 0x5a000000) {
      u = 1.0f + x;
      hu = (int32_t)ugk_f2u(u);
      k = (hu >> 23) - 127;
      c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);
      c = ugk_div_t<kDiv>(c, u);
    } else {
      u = x;
      hu = (int32_t)ugk_f2u(u);
      k = (hu >> 23) - 127;
      c = 0.0f;
    }
    hu &= 0x007fffff;
    if (hu < 0x3504f7) {
      u = ugk_u2f((uint32_t)(hu | 0x3f800000));
    } else {
      k += 1;
      u = ugk_u2f((uint32_t)(hu | 0x3f000000));
      hu = (0x00800000 - hu) >> 2;
    }
    f = u - 1.0f;
  }
  const float fk = (float)k;
  const float hfsq = 0.5f * f * f;
  float r;
  if (hu == 0) {  // |f| < 2^-20
    const float R0 = hfsq * (1.0f - 0.66666666666666666f * f);
    const float rz = (k == 0) ? 0.0f : fk * ln2_hi + (c + fk * ln2_lo);
    const float rs = (k == 0) ? f - R0 : fk * ln2_hi - ((R0 - (c + fk * ln2_lo)) - f);
    r = (f == 0.0f) ? rz : rs;
  } else {
    const float s = ugk_div_t<kDiv>(f, 2.0f + f);
    const float z = s * s;
    const float R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
    r = (k == 0) ? f - (hfsq - s * (hfsq + R))
                 : fk * ln2_hi - ((hfsq - (s * (hfsq + R) + (c + fk * ln2_lo))) - f);
  }
  if (hx < 0x3ed413d7) {
    if (ax < 0x31000000) r = (ax < 0x24800000) ? x : x - x * x * 0.5f;  // |x| < 2^-29
    if (ax >= 0x3f800000) r = (x == -1.0f) ? ugk_u2f(0xff800000u) : ugk_u2f(0x7fc00000u);
  } else if (hx >= 0x7f800000) {
    r = x + x;
  }
  return r;
}

__device__ __forceinline__ float ugk_dev_expm1f(float x) { return ugk_dev_expm1f_t<UGK_DIV_STEPS>(x); }
__device__ __forceinline__ float ugk_dev_tanhf(float x) { return ugk_dev_tanhf_t<UGK_DIV_STEPS>(x); }
__device__ __forceinline__ float ugk_dev_log1pf(float x) { return ugk_dev_log1pf_t<UGK_DIV_STEPS>(x); }

// GELU (tanh form) and its derivative, train_bnn.c:163-170 and :520-533, with
// the reference's tanhf. A NaN x gives NaN through the factor x (0.5 x sech2
// in the derivative), whatever tanhf returns, so the NaN case of tanhf is
// dropped. Exhaustively equal to the same expressions over ugk_tanhf
// (ugk_diag.hip, fn 8 and 9).
template <class Tanh>
__device__ __host__ __forceinline__ float ugk_gelu_with(float x, Tanh tanh_fn) {
  const float k = 0.7978845608f;
  const float inner = k * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanh_fn(inner));
}

template <class Tanh>
__device__ __host__ __forceinline__ float ugk_gelu_grad_with(float x, Tanh tanh_fn) {
  const float k = 0.7978845608f;
  const float u = k * (x + 0.044715f * x * x * x);
  const float tanh_u = tanh_fn(u);
  const float sech2 = 1.0f - tanh_u * tanh_u;
  const float du_dx = k * (1.0f + 3.0f * 0.044715f * x * x);
  return 0.5f * (1.0f + tanh_u) + 0.5f * x * sech2 * du_dx;
}

struct UgkDevTanhNoNan {
  __device__ float operator()(float u) const { return ugk_dev_tanhf_t<UGK_DIV_STEPS, false>(u); }
};

__device__ __forceinline__ float ugk_dev_gelu(float x) { return ugk_gelu_with(x, UgkDevTanhNoNan{}); }
__device__ __forceinline__ float ugk_dev_gelu_grad(float x) { return ugk_gelu_grad_with(x, UgkDevTanhNoNan{}); }

// GELU and its derivative through the logistic form of the same function:
// with u = k (x + 0.044715 x^3) (computed as train_bnn.c:166 computes it),
// e = e^{-2u} and s = 1 / (1 + e),
//   0.5 (1 + tanh u) = s,   1 - tanh^2 u = 4 s (1 - s) = 4 e s^2,
// so gelu = x s and gelu' = s + 2 x s (e s) du/dx = s (1 + 2 x (e s) du/dx),
// with e s = 1 - s formed first. The hardware 2^t (v_exp_f32)
// and reciprocal (v_rcp_f32) replace fdlibm's tanhf: about 10 instructions per
// element instead of 74, no cancellation in 1 + tanh or 1 - tanh^2, and the
// result is within 1e-5 relative / 1e-6 absolute of the CPU's on every input
// (checked over all 2^32 floats by ugk_diag_math_mismatch, fn 64 and 65),
// though not bit-identical to it. For |x| > 10 glibc's tanhf(u) is exactly
// +-1, and the derivative is the CPU's own expression with that value (1 or
// 0, NaN where it overflows), which also keeps e^{-2u} = inf away from 0 * inf.
constexpr float kNeg2Log2e = -2.0f * 1.4426950408889634f;

__device__ __forceinline__ float ugk_fast_gelu(float x) {
  const float k = 0.7978845608f;
  const float u = k * (x + 0.044715f * x * x * x);
  const float e = __builtin_amdgcn_exp2f(u * kNeg2Log2e);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float ugk_fast_gelu_grad(float x) {
  const float k = 0.7978845608f;
  const float u = k * (x + 0.044715f * x * x * x);
  const float du_dx = k * (1.0f + 3.0f * 0.044715f * x * x);
  const float e = __builtin_amdgcn_exp2f(u * kNeg2Log2e);
  const float s = __builtin_amdgcn_rcpf(1.0f + e);
  const float es = e * s;  // 1 - s, at most 1: formed first, as e alone can near FLT_MAX at |x| = 10
  const float near = s * (1.0f + 2.0f * x * es * du_dx);
  const float t = x > 0.0f ? 1.0f : -1.0f;  // tanhf(u) for |x| > 10
  const float far = 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * du_dx;
  return fabsf(x) <= 10.0f ? near : far;
}

// ---- hardware-transcendental softplus and sigmoid (the Philox ops' default) ----
// e^x as 2^t with t = x log2(e) carried to about 2^-48 relative (the product's
// rounding error and the constant's tail, by fma), then one correction
// e (1 + dt ln 2) after the hardware 2^t (v_exp_f32). x is first clamped
// from below to -104, where e^x is below every float (NaN passes through).
// The hardware 2^t flushes results below 2^-126 to zero; with kSubnormal,
// below t = -64 it takes 2^(t + 64) 2^-64 instead, whose multiply rounds into
// the subnormals (a branch, which wavefronts of ordinary arguments skip).
// Where 2^t overflows, the correction (inf + inf * c) would be NaN for c < 0:
// with kKeepOverflow the overflow is kept, as is a NaN x.
constexpr float kUgkLog2e = 1.44269502162933349609f;       // log2(e) rounded to float
constexpr float kUgkLog2eLo = 1.92596299112661746887e-8f;  // log2(e) - kUgkLog2e
constexpr float kUgkLn2 = 0.693147180559945309417f;

template <bool kSubnormal, bool kKeepOverflow>
__device__ __forceinline__ float ugk_fast_exp_t(float x) {
  const float xc = x < -104.0f ? -104.0f : x;
  const float t = xc * kUgkLog2e;
  const float dt = __builtin_fmaf(xc, kUgkLog2e, -t) + xc * kUgkLog2eLo;
  float e = __builtin_amdgcn_exp2f(t);
  if (kSubnormal && t < -64.0f) {
    asm volatile("");  // keeps the rare case a branch rather than a second 2^t and a select
    e = __builtin_amdgcn_exp2f(t + 64.0f) * 0x1p-64f;
  }
  const float r = __builtin_fmaf(e, dt * kUgkLn2, e);
  return (kKeepOverflow && r != r) ? e : r;
}

// softplus(x) = log1p(e^x) (train_bnn.c:814-816's formula; x for x > 20 as
// there). log1p(e): below e = 1/16 its series to e^6 (the remainder is below
// e^7/7, a tenth of an ulp); above, Goldberg's form log(u) e / (u - 1)
// with u = 1 + e rounded, whose quotient cancels the rounding of u, and the
// hardware log2 (v_log_f32) times ln 2. The two forms are branches: the
// arguments of a wavefront (a run of rho) mostly lie on one side of
// x = ln(1/16). e^x's overflow need not be kept: above x = 20 the result is x.
// Within a few ulp of glibc's log1pf(expf(x)) and within 1e-6 absolute /
// 1e-5 relative of it on every float input (ugk_diag.hip fn 66); about 20
// VALU instructions on one branch, with two hardware transcendentals, against
// some 70 for the glibc-exact form.
__device__ __forceinline__ float ugk_fast_softplus(float x) {
  const float e = ugk_fast_exp_t<true, false>(x);
  float r;
  if (e < 0.0625f) {
    float p = __builtin_fmaf(e, -1.0f / 6.0f, 0.2f);
    p = __builtin_fmaf(e, p, -0.25f);
    p = __builtin_fmaf(e, p, 1.0f / 3.0f);
    p = __builtin_fmaf(e, p, -0.5f);
    r = e * __builtin_fmaf(e, p, 1.0f);
  } else {
    const float u = 1.0f + e;
    r = __builtin_amdgcn_logf(u) * kUgkLn2 * (e * __builtin_amdgcn_rcpf(u - 1.0f));
  }
  return x > 20.0f ? x : r;
}

// sigmoid(x) = 1 / (1 + e^-x) (train_bnn.c:820-822) with the hardware
// reciprocal (v_rcp_f32); x is clamped to [-104, 104] first (NaN passes), so
// that e^-x is 0 or inf at the ends, as there. Below 2^-64, e^-x leaves
// 1 + e^-x at 1 whether or not it is flushed, so the exponential skips the
// subnormal case. The hardware reciprocal flushes results below 2^-126 to
// zero, so a divisor above 2^64 (x below -44) is scaled by 2^-64 first and
// the quotient by 2^-64 after (a branch, rarely taken). Within a few ulp of
// the glibc-exact form and within the literal bar of it everywhere (fn 67).
__device__ __forceinline__ float ugk_fast_sigmoid(float x) {
  const float xc = x > 104.0f ? 104.0f : (x < -104.0f ? -104.0f : x);
  const float d = 1.0f + ugk_fast_exp_t<false, true>(-xc);
  float q = __builtin_amdgcn_rcpf(d);
  if (d > 0x1p64f) {
    asm volatile("");  // a branch, not a second reciprocal and a select
    q = __builtin_amdgcn_rcpf(d * 0x1p-64f) * 0x1p-64f;
  }
  return q;
}

// The expf table of ugk_libm.h, read from a copy in LDS: a per-lane lookup in
// local memory instead of a dependent global load on every element's path.
struct UgkExp2Lds {
  const uint64_t *p;
  __device__ uint64_t operator()(uint32_t i) const { return p[i]; }
};

// expf's addend constants in vector registers, for a loop of expf calls: the
// empty asm statement hides their values, so the compiler keeps the one copy
// rather than rebuilding both for every call.
__device__ __forceinline__ UgkExpfAddends ugk_expf_addends_vgpr() {
  UgkExpfAddends a;
  asm volatile("" : "+v"(a.shift), "+v"(a.c1));
  return a;
}

// expf(x) without branches for x <= 0x1.62e42ep6 (the largest x whose expf
// is finite; -inf included) or NaN: the softmax's x - max and softplus's
// arguments up to 20. expf's formula for every x, then its underflow case.
// Where that case does not apply (x >= -0x1.9fe368p6) the routine itself
// takes the formula; for -inf it returns +0 as the underflow case does; for
// NaN the formula gives a NaN. Outside the domain the value is meaningless
// (the table index stays in range). Checked against ugk_expf on every input
// of the domain (ugk_diag.hip fn 63).
template <class Tab>
__device__ __forceinline__ float ugk_dev_expf_nooverflow(float x, Tab tab, UgkExpfAddends add) {
  const float y = ugk_expf_core<UGK_EXPF_CONTRACT>(x, tab, add);
  return x < -0x1.9fe368p6f ? 0.0f : y;
}

// Fill a 32-entry LDS table; the caller synchronises the workgroup after.
__device__ __forceinline__ void ugk_exp2_stage(uint64_t *lds_tab) {
  if (threadIdx.x < 32) lds_tab[threadIdx.x] = ugk_exp2_bits(threadIdx.x);
}

__device__ __forceinline__ float ugk_dev_softplusf_lds(float x, const uint64_t *lds_tab) {
  // expf is taken only for x <= 20, inside the branch-free form's domain
  const float e = ugk_dev_expf_nooverflow(x, UgkExp2Lds{lds_tab}, UgkExpfAddends{});
  return x > 20.0f ? x : ugk_dev_log1pf(e);
}
