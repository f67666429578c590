// ugk_libm_dev.h - the float math of the kernels, shaped for a 64-lane SIMD.
//
// Same operations as ugk_libm.h (the line-by-line restatement of glibc's
// expm1f/tanhf/log1pf), in the same order and with the same rounding, but
// without data-dependent branches: every case of the reference is computed
// and the right one selected, so a wavefront whose lanes fall in different
// cases runs each piece of arithmetic once instead of once per case, and
// tanhf evaluates one expm1f instead of two inlined copies. Divisions use
// ugk_div, a reciprocal with Newton-Raphson correction.
//
// That this equals ugk_libm.h on every one of the 2^32 inputs is checked on
// the GPU by ugk_diag_math_mismatch (tests/test_parity_gpu.py); ugk_libm.h
// itself equals the host glibc on every input (oracle/libm_exhaustive.cpp).
#pragma once

#include "ugk_libm.h"

// a / b rounded to nearest-even, for the operand ranges these functions
// produce (b normal, quotient normal or zero): v_rcp_f32 seed, one Newton step
// on the reciprocal, then two residual corrections of the quotient.
__device__ __forceinline__ float ugk_div(float a, float b) {
  float r = __builtin_amdgcn_rcpf(b);
  const float t = __builtin_fmaf(-b, r, 1.0f);
  r = __builtin_fmaf(t, r, r);
  float q = a * r;
  float e = __builtin_fmaf(-b, q, a);
  q = __builtin_fmaf(e, r, q);
  e = __builtin_fmaf(-b, q, a);
  return __builtin_fmaf(e, r, q);
}

__device__ __forceinline__ float ugk_dev_expm1f(float x) {
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
  const float e = hxs * ugk_div(r1 - tt, 6.0f - xr * tt);
  const float y0 = xr - (xr * e - hxs);  // k == 0
  float e2 = (xr * (e - c) - c);
  e2 -= hxs;
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

__device__ __forceinline__ float ugk_dev_tanhf(float x) {
  const uint32_t jx = ugk_f2u(x);
  const uint32_t ix = jx & 0x7fffffffu;
  const float ax = ugk_u2f(ix);
  const bool big = ix >= 0x3f800000u;  // |x| >= 1
  const float t = ugk_dev_expm1f(big ? 2.0f * ax : -2.0f * ax);
  const float q = ugk_div(big ? 2.0f : -t, t + 2.0f);
  float z = big ? 1.0f - q : q;
  z = (ix >= 0x41b00000u) ? 1.0f : z;  // |x| >= 22 and +-inf
  float r = (jx >> 31) ? -z : z;
  r = (ix < 0x24000000u) ? x * (1.0f + x) : r;  // |x| < 2^-55, and +-0
  r = (ix > 0x7f800000u) ? x + x : r;            // nan
  return r;
}

__device__ __forceinline__ float ugk_dev_log1pf(float x) {
  const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
  const float Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f,
              Lp3 = 2.8571429849e-01f, Lp4 = 2.2222198546e-01f,
              Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f,
              Lp7 = 1.4798198640e-01f;
  const int32_t hx = (int32_t)ugk_f2u(x);
  const int32_t ax = hx & 0x7fffffff;
  const bool low = hx < 0x3ed413d7;                              // x < 0.41422
  const bool k0 = low && (hx > 0 || hx <= (int32_t)0xbe95f61fu);  // f = x, k = 0
  // 1 + x = 2^k (1 + f)
  const bool mid = hx < 0x5a000000;
  const float u1 = 1.0f + x;
  const float u = mid ? u1 : x;
  int32_t hu = (int32_t)ugk_f2u(u);
  int k = (hu >> 23) - 127;
  float c = (k > 0) ? 1.0f - (u1 - x) : x - (u1 - 1.0f);
  c = mid ? ugk_div(c, u1) : 0.0f;
  hu &= 0x007fffff;
  const bool lm = hu < 0x3504f7;
  const float un = ugk_u2f((uint32_t)(hu | (lm ? 0x3f800000 : 0x3f000000)));
  k = lm ? k : k + 1;
  hu = lm ? hu : (0x00800000 - hu) >> 2;
  const float f = k0 ? x : un - 1.0f;
  k = k0 ? 0 : k;
  hu = k0 ? 1 : hu;
  const float fk = (float)k;
  const float hfsq = 0.5f * f * f;
  // |f| < 2^-20
  const float R0 = hfsq * (1.0f - 0.66666666666666666f * f);
  const float rz = (k == 0) ? 0.0f : fk * ln2_hi + (c + fk * ln2_lo);
  const float rs = (k == 0) ? f - R0 : fk * ln2_hi - ((R0 - (c + fk * ln2_lo)) - f);
  const float r_hu0 = (f == 0.0f) ? rz : rs;
  // general
  const float s = ugk_div(f, 2.0f + f);
  const float z = s * s;
  const float R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
  const float rg = (k == 0) ? f - (hfsq - s * (hfsq + R))
                            : fk * ln2_hi - ((hfsq - (s * (hfsq + R) + (c + fk * ln2_lo))) - f);
  float r = (hu == 0) ? r_hu0 : rg;
  if (low) {
    if (ax < 0x31000000) r = (ax < 0x24800000) ? x : x - x * x * 0.5f;  // |x| < 2^-29
    if (ax >= 0x3f800000) r = (x == -1.0f) ? ugk_u2f(0xff800000u) : ugk_u2f(0x7fc00000u);
  } else if (hx >= 0x7f800000) {
    r = x + x;
  }
  return r;
}

__device__ __forceinline__ float ugk_dev_softplusf(float x) {
  return x > 20.0f ? x : ugk_dev_log1pf(ugk_expf(x));
}
