// ugk_libm.h - float math that reproduces the host C library bit for bit.
//
// The CPU oracle of this kernel set (train_bnn.c) calls glibc's expf, log1pf
// and tanhf (train_bnn.c:164-168, :525-529 tanhf; :814-816 expf/log1pf).
// glibc's float versions are not correctly rounded, so a device kernel that
// calls the GPU's own libm (or any more accurate routine) differs from the
// oracle in the last bit on a fraction of inputs. To make bayes_materialize
// and GELU bit-exact, this header restates the published algorithms that
// glibc 2.35 ships for these functions, in plain IEEE arithmetic that gives
// the same result on the x86 host and on gfx950:
//
//   expf    - glibc sysdeps/ieee754/flt-32/e_expf.c (Szabolcs Nagy, from
//             ARM optimized-routines): x*32/ln2 = k + r, 2^(k/32) from a
//             32-entry table, cubic polynomial in r, all in double.
//   log1pf  - glibc sysdeps/ieee754/flt-32/s_log1pf.c (fdlibm, Sun 1993):
//             1+x = 2^k (1+f), log1p = k ln2 + f - hfsq + s (hfsq + R(s*s)).
//   expm1f  - glibc sysdeps/ieee754/flt-32/s_expm1f.c (fdlibm): x = k ln2 + r,
//             rational approximation of expm1 on the reduced argument.
//   tanhf   - glibc sysdeps/ieee754/flt-32/s_tanhf.c (fdlibm) on top of
//             expm1f.
//   logf    - glibc sysdeps/ieee754/flt-32/e_logf.c (ARM optimized-routines),
//             for normal finite x > 0: a 16-entry table of 1/c and log(c),
//             a polynomial in z/c - 1, all in double.
//   cosf    - glibc sysdeps/ieee754/flt-32/s_cosf.c (ARM optimized-routines),
//             for |x| < 120: the reduction by pi/2 in double and the sine and
//             cosine polynomials of sincosf.
// logf and cosf serve the Box-Muller transform (train_bnn.c's
// sqrtf(-2 logf(u1)) cosf(2 pi u2)); the other arguments of those functions
// (zero, subnormal, negative, large, infinite and NaN) are not restated.
//
// Every operation here is a single IEEE-754 binary32/binary64 operation with
// round-to-nearest-even, an explicit fma(), an integer operation on the bit
// pattern, or a comparison. The file must be compiled with
// -ffp-contract=off so that the compiler does not fuse a*b+c on its own, and
// with fp32 denormals enabled on the GPU (the HIP default for gfx950).
//
// Whether each function equals the host glibc on ALL 2^32 inputs is checked
// exhaustively by oracle/libm_exhaustive.cpp (CPU) and on the GPU by
// tests/test_parity_gpu.py.
//
// Attribution. log1pf, expm1f and tanhf restate fdlibm, whose notice reads:
//   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//   Developed at SunPro, a Sun Microsystems, Inc. business.
//   Permission to use, copy, modify, and distribute this
//   software is freely granted, provided that this notice
//   is preserved.
// expf, logf and cosf restate ARM optimized-routines' expf, logf and
// sincosf (Copyright (c) 2017-2018 Arm Limited; MIT OR Apache-2.0 WITH
// LLVM-exception). The LICENSE file at the repository root repeats both
// notices.
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define UGK_HD __host__ __device__ __forceinline__
#define UGK_HD_MEMBER __host__ __device__ __forceinline__
#else
#define UGK_HD static inline
#define UGK_HD_MEMBER inline
#endif

UGK_HD uint32_t ugk_f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
UGK_HD float ugk_u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
UGK_HD uint64_t ugk_d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
UGK_HD double ugk_u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
// The double with high word hi and low word lo (on the GPU, a register pair
// filled without 64-bit integer arithmetic).
UGK_HD double ugk_hilo2d(uint32_t hi, uint32_t lo) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __hiloint2double((int)hi, (int)lo);
#else
  return ugk_u2d(((uint64_t)hi << 32) | lo);
#endif
}

// 2^(i/32) correctly rounded to binary64, minus (i << 47): adding (k << 47) to
// entry k%32 gives the bit pattern of 2^(k/32) for any integer k in range.
// Regenerate with: float(Decimal(2)**(Decimal(i)/32)) at 60 digits.
UGK_HD uint64_t ugk_exp2_bits(uint32_t i) {
  const uint64_t tab[32] = {
      0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
      0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
      0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
      0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
      0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
      0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
      0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
      0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
      0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
      0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
      0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
  return tab[i];
}

// The table read from the array above (callers may pass their own copy of it,
// e.g. one staged in GPU local memory).
struct UgkExp2Table {
  UGK_HD_MEMBER uint64_t operator()(uint32_t i) const { return ugk_exp2_bits(i); }
};

// expf. kContract selects how the multiply-adds are rounded, because the x86
// glibc picks an FMA-compiled copy of this routine at run time on CPUs with
// FMA (the x86_64 multiarch e_expf-fma.c build):
//   0: every product and sum rounded separately (no FMA);
//   1: the three polynomial multiply-adds fused;
//   2: as 1, and also the two uses of InvLn2N*x in the reduction fused.
// The two constants that enter expf only as addends. Callers may pass copies
// held in registers (GPU code, where an instruction takes one scalar operand
// and a constant addend would otherwise be copied into a vector register
// before every call); the values are always these.
struct UgkExpfAddends {
  double shift = 0x1.8p+52;
  double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
};

// expf's formula without its special cases: correct for |x| < 88, and for
// x in [-0x1.9fe368p6, -88] too, where the routine falls through to it.
template <int kContract, class Tab>
UGK_HD float ugk_expf_core(float x, Tab tab, UgkExpfAddends add = UgkExpfAddends{}) {
  const double kInvLn2N = 0x1.71547652b82fep+0 * 32;
  const double kShift = add.shift;
  const double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double kC1 = add.c1;
  const double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double xd = (double)x;
  double kd, r;
  if (kContract == 2) {
    kd = __builtin_fma(kInvLn2N, xd, kShift);
  } else {
    kd = kInvLn2N * xd + kShift;
  }
  const uint64_t ki = ugk_d2u(kd);
  kd -= kShift;
  if (kContract == 2) {
    r = __builtin_fma(kInvLn2N, xd, -kd);
  } else {
    r = kInvLn2N * xd - kd;
  }
  // 2^(k/32) = table entry k % 32 plus (k << 47) as a 64-bit integer; the
  // addend's low word is zero, so only the high words are added.
  const uint64_t tb = tab((uint32_t)(ki % 32));
  const double s = ugk_hilo2d((uint32_t)(tb >> 32) + ((uint32_t)ki << 15), (uint32_t)tb);
  double z, y;
  const double r2 = r * r;
  if (kContract >= 1) {
    z = __builtin_fma(kC0, r, kC1);
    y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
  } else {
    z = kC0 * r + kC1;
    y = kC2 * r + 1.0;
    y = z * r2 + y;
  }
  y = y * s;
  return (float)y;
}

template <int kContract, class Tab>
UGK_HD float ugk_expf_t(float x, Tab tab, UgkExpfAddends add = UgkExpfAddends{}) {
  const uint32_t ux = ugk_f2u(x);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= 0x42b) {                        // |x| >= 88 or nan
    if (ux == 0xff800000u) return 0.0f;         // -inf
    if (abstop >= 0x7f8) return x + x;          // +inf, nan
    if (x > 0x1.62e42ep6f) return ugk_u2f(0x7f800000u);  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;        // underflow
  }
  return ugk_expf_core<kContract>(x, tab, add);
}

template <int kContract>
UGK_HD float ugk_expf_v(float x) {
  return ugk_expf_t<kContract>(x, UgkExp2Table{});
}

// log1pf, fdlibm.
UGK_HD float ugk_log1pf(float x) {
  const float ln2_hi = 6.9313812256e-01f;  // 0x3f317180
  const float ln2_lo = 9.0580006145e-06f;  // 0x3717f7d1
  const float Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f,
              Lp3 = 2.8571429849e-01f, Lp4 = 2.2222198546e-01f,
              Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f,
              Lp7 = 1.4798198640e-01f;
  float hfsq, f = 0.0f, c = 0.0f, s, z, R, u;
  int32_t k, hu = 0;
  const int32_t hx = (int32_t)ugk_f2u(x);
  const int32_t ax = hx & 0x7fffffff;
  k = 1;
  if (hx < 0x3ed413d7) {                      // x < 0.41422
    if (ax >= 0x3f800000) {                   // x <= -1.0
      if (x == -1.0f) return ugk_u2f(0xff800000u);       // -inf
      return ugk_u2f(0x7fc00000u) ;           // nan
    }
    if (ax < 0x31000000) {                    // |x| < 2**-29
      if (ax < 0x24800000) return x;          // |x| < 2**-54
      return x - x * x * 0.5f;
    }
    if (hx > 0 || hx <= (int32_t)0xbe95f61fu) {  // -0.2929 < x < 0.41422
      k = 0; f = x; hu = 1;
    }
  } else if (hx >= 0x7f800000) {
    return x + x;
  }
  if (k != 0) {
    if (hx < 0x5a000000) {
      u = 1.0f + x;
      hu = (int32_t)ugk_f2u(u);
      k = (hu >> 23) - 127;
      c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);  // correction term
      c /= u;
    } else {
      u = x;
      hu = (int32_t)ugk_f2u(u);
      k = (hu >> 23) - 127;
      c = 0;
    }
    hu &= 0x007fffff;
    if (hu < 0x3504f7) {
      u = ugk_u2f((uint32_t)(hu | 0x3f800000));          // normalize u
    } else {
      k += 1;
      u = ugk_u2f((uint32_t)(hu | 0x3f000000));          // normalize u/2
      hu = (0x00800000 - hu) >> 2;
    }
    f = u - 1.0f;
  }
  hfsq = 0.5f * f * f;
  if (hu == 0) {                              // |f| < 2**-20
    if (f == 0.0f) {
      if (k == 0) return 0.0f;
      c += (float)k * ln2_lo;
      return (float)k * ln2_hi + c;
    }
    R = hfsq * (1.0f - 0.66666666666666666f * f);
    if (k == 0) return f - R;
    return (float)k * ln2_hi - ((R - (c + (float)k * ln2_lo)) - f);
  }
  s = f / (2.0f + f);
  z = s * s;
  R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
  if (k == 0) return f - (hfsq - s * (hfsq + R));
  return (float)k * ln2_hi - ((hfsq - (s * (hfsq + R) + (c + (float)k * ln2_lo))) - f);
}

// expm1f, fdlibm.
UGK_HD float ugk_expm1f(float x) {
  const float o_threshold = 8.8721679688e+01f;  // 0x42b17180
  const float ln2_hi = 6.9313812256e-01f;       // 0x3f317180
  const float ln2_lo = 9.0580006145e-06f;       // 0x3717f7d1
  const float invln2 = 1.4426950216e+00f;       // 0x3fb8aa3b
  const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f,
              Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f,
              Q5 = -2.0109921195e-07f;
  float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
  int32_t k;
  uint32_t hx = ugk_f2u(x);
  const int32_t xsb = (int32_t)(hx & 0x80000000u);
  hx &= 0x7fffffffu;
  if (hx >= 0x4195b844u) {                    // |x| >= 27*ln2
    if (hx >= 0x42b17218u) {                  // |x| >= 88.721...
      if (hx > 0x7f800000u) return x + x;     // nan
      if (hx == 0x7f800000u) return (xsb == 0) ? x : -1.0f;
      if (x > o_threshold) return ugk_u2f(0x7f800000u);  // overflow
    }
    if (xsb != 0) return -1.0f;               // x < -27*ln2
  }
  if (hx > 0x3eb17218u) {                     // |x| > 0.5 ln2
    if (hx < 0x3F851592u) {                   // and |x| < 1.5 ln2
      if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
      else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
    } else {
      k = (int32_t)(invln2 * x + ((xsb == 0) ? 0.5f : -0.5f));
      t = (float)k;
      hi = x - t * ln2_hi;                    // t*ln2_hi is exact here
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x33000000u) {              // |x| < 2**-25
    return x;
  } else {
    k = 0;
  }
  hfx = 0.5f * x;
  hxs = x * hfx;
  r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  t = 3.0f - r1 * hfx;
  e = hxs * ((r1 - t) / (6.0f - x * t));
  if (k == 0) return x - (x * e - hxs);
  e = (x * (e - c) - c);
  e -= hxs;
  if (k == -1) return 0.5f * (x - e) - 0.5f;
  if (k == 1) {
    if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
    return 1.0f + 2.0f * (x - e);
  }
  if (k <= -2 || k > 56) {                    // suffice to return exp(x)-1
    y = 1.0f - (e - x);
    if (k == 128) {
      y = y * 2.0f * 0x1p127f;
    } else {
      y = ugk_u2f(ugk_f2u(y) + ((uint32_t)k << 23));
    }
    return y - 1.0f;
  }
  if (k < 23) {
    t = ugk_u2f(0x3f800000u - (0x1000000u >> k));  // t = 1-2^-k
    y = t - (e - x);
    y = ugk_u2f(ugk_f2u(y) + ((uint32_t)k << 23));
  } else {
    t = ugk_u2f((uint32_t)(0x7f - k) << 23);        // 2^-k
    y = x - (e + t);
    y += 1.0f;
    y = ugk_u2f(ugk_f2u(y) + ((uint32_t)k << 23));
  }
  return y;
}

// tanhf, fdlibm.
UGK_HD float ugk_tanhf(float x) {
  float t, z;
  const int32_t jx = (int32_t)ugk_f2u(x);
  const int32_t ix = jx & 0x7fffffff;
  if (ix >= 0x7f800000) {                     // inf or nan
    if (jx >= 0) return 1.0f / x + 1.0f;
    return 1.0f / x - 1.0f;
  }
  if (ix < 0x41b00000) {                      // |x| < 22
    if (ix == 0) return x;
    if (ix < 0x24000000) return x * (1.0f + x);   // |x| < 2**-55
    if (ix >= 0x3f800000) {                   // |x| >= 1
      t = ugk_expm1f(2.0f * ugk_u2f((uint32_t)ix));
      z = 1.0f - 2.0f / (t + 2.0f);
    } else {
      t = ugk_expm1f(-2.0f * ugk_u2f((uint32_t)ix));
      z = -t / (t + 2.0f);
    }
  } else {
    z = 1.0f;                                 // 1 - tiny rounds to 1
  }
  return (jx >= 0) ? z : -z;
}

#ifndef UGK_EXPF_CONTRACT
#define UGK_EXPF_CONTRACT 2
#endif

UGK_HD float ugk_expf(float x) { return ugk_expf_v<UGK_EXPF_CONTRACT>(x); }

// softplus exactly as train_bnn.c:814-816 writes it.
UGK_HD float ugk_softplusf(float x) {
  return x > 20.0f ? x : ugk_log1pf(ugk_expf(x));
}

// logf's table: for each of 16 subintervals of [0x1.6666p-1, 0x1.6666p0)
// (the top 4 fraction bits of x - 0x3f330000) the double 1/c for a c near
// its centre, and log(c). GPU code reads it from constant memory, one load
// per lane (a table in the function's body becomes a branch tree there).
#define UGK_LOGF_TABLE                                                                                      \
  {0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2, 0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2,               \
   0x1.49539f0f010bp+0,  -0x1.01eae7f513a67p-2, 0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3,               \
   0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3, 0x1.25e227b0b8eap+0,  -0x1.1aa2bc79c81p-3,                 \
   0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4, 0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4,               \
   0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5, 0x1p+0,               0x0p+0,                              \
   0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5,  0x1.ca4b31f026aap-1,  0x1.c5e53aa362eb4p-4,                \
   0x1.b2036576afce6p-1, 0x1.526e57720db08p-3,  0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3,                 \
   0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2,  0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2}

struct UgkLogfEntry {
  double invc, logc;
};

#if defined(__HIPCC__)
static __constant__ __align__(16) double ugk_logf_tab_dev[32] = UGK_LOGF_TABLE;  // read as double2
#endif
static const double ugk_logf_tab_host[32] = UGK_LOGF_TABLE;

UGK_HD UgkLogfEntry ugk_logf_entry(uint32_t i) {
#if defined(__HIP_DEVICE_COMPILE__)
  const double2 e = reinterpret_cast<const double2 *>(ugk_logf_tab_dev)[i];
  return UgkLogfEntry{e.x, e.y};
#else
  return UgkLogfEntry{ugk_logf_tab_host[2 * i], ugk_logf_tab_host[2 * i + 1]};
#endif
}

struct UgkLogfTable {
  UGK_HD_MEMBER UgkLogfEntry operator()(uint32_t i) const { return ugk_logf_entry(i); }
};

template <int kContract, class Tab>
UGK_HD float ugk_logf_normal_t(float x, Tab tab) {
  const double kLn2 = 0x1.62e42fefa39efp-1;
  const double kA0 = -0x1.00ea348b88334p-2, kA1 = 0x1.5575b0be00b6ap-2, kA2 = -0x1.ffffef20a4123p-2;
  const uint32_t ix = ugk_f2u(x);
  const uint32_t tmp = ix - 0x3f330000u;
  const uint32_t i = (tmp >> 19) & 15u;
  const int k = (int32_t)tmp >> 23;
  const uint32_t iz = ix - (tmp & 0xff800000u);
  const UgkLogfEntry e = tab(i);
  const double z = (double)ugk_u2f(iz);
  double r, y0, y;
  if (kContract) {
    r = __builtin_fma(z, e.invc, -1.0);
    y0 = __builtin_fma((double)k, kLn2, e.logc);
  } else {
    r = z * e.invc - 1.0;
    y0 = e.logc + (double)k * kLn2;
  }
  const double r2 = r * r;
  if (kContract) {
    y = __builtin_fma(kA1, r, kA2);
    y = __builtin_fma(kA0, r2, y);
    y = __builtin_fma(y, r2, y0 + r);
  } else {
    y = kA1 * r + kA2;
    y = kA0 * r2 + y;
    y = y * r2 + (y0 + r);
  }
  return (float)y;
}

UGK_HD float ugk_logf_normal(float x) { return ugk_logf_normal_t<1>(x, UgkLogfTable{}); }

// logf for every input, glibc's special cases included: -inf at +-0, +inf at
// +inf, NaN for negative x and NaN, and a subnormal x scaled by 2^23 into the
// normal range first (the exponent taken back by 23 in the bit pattern, as
// glibc does); normal x as ugk_logf_normal.
UGK_HD float ugk_logf(float x) {
  uint32_t ix = ugk_f2u(x);
  if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
    if (ix * 2u == 0u) return -ugk_u2f(0x7f800000u);  // +-0: -inf
    if (ix == 0x7f800000u) return x;                   // +inf
    if ((ix & 0x80000000u) || ix * 2u >= 0xff000000u) return ugk_u2f(0x7fc00000u);  // x < 0 or NaN
    ix = ugk_f2u(x * 0x1p23f) - (23u << 23);            // subnormal
  }
  return ugk_logf_normal_t<1>(ugk_u2f(ix), UgkLogfTable{});
}

// cosf for |x| < 120 (sincosf's fast path): x - n pi/2 with n = round(x 2/pi)
// (from the product with 2^24 2/pi and an integer shift), then the sine or
// cosine polynomial of the remainder by n's parity, negated for n mod 4 = 1
// or 2; all in double, rounded to float once. glibc also branches for
// |x| < 0x1p-12 (the result 1) and below about pi/4 (the cosine polynomial of
// x unreduced); the general path gives the same bits there (n = 0, an exact
// remainder, the polynomial rounding to 1 below 0x1p-12), and the sign flips
// glibc takes from its two coefficient tables are exact negations of the
// result, so this form evaluates both polynomials and selects, without
// branches. The multiply-adds are fused as in the x86_64 glibc's FMA build
// (the unfused form differs from it on 22 inputs near |x| = 64;
// oracle/libm_exhaustive.cpp checks both).
template <int kContract>
UGK_HD float ugk_cosf_small_t(float y) {
  const double kC0 = 0x1p0, kC1 = -0x1.ffffffd0c621cp-2, kC2 = 0x1.55553e1068f19p-5;
  const double kC3 = -0x1.6c087e89a359dp-10, kC4 = 0x1.99343027bf8c3p-16;
  const double kS1 = -0x1.555545995a603p-3, kS2 = 0x1.1107605230bc4p-7, kS3 = -0x1.994eb3774cf24p-13;
  const double kHpi = 0x1.921fb54442d18p0;
  const double x0 = (double)y;
  const double r = x0 * 0x1.45f306dc9c883p+23;  // x 2/pi 2^24
  const int n = ((int32_t)r + 0x800000) >> 24;
  const double x = kContract ? __builtin_fma(-(double)n, kHpi, x0) : x0 - n * kHpi;
  const double x2 = x * x;
  const double x3 = x * x2, x4 = x2 * x2;
  const double x6 = x4 * x2, x7 = x3 * x2;
  double sv, cv;
  if (kContract) {
    sv = __builtin_fma(x7, __builtin_fma(x2, kS3, kS2), __builtin_fma(x3, kS1, x));
    const double c2 = __builtin_fma(x2, kC4, kC3);
    const double c = __builtin_fma(x4, kC2, __builtin_fma(x2, kC1, kC0));
    cv = __builtin_fma(x6, c2, c);
  } else {
    sv = (x + x3 * kS1) + x7 * (kS2 + x2 * kS3);
    const double c2 = kC3 + x2 * kC4;
    const double c = (kC0 + x2 * kC1) + x4 * kC2;
    cv = c + x6 * c2;
  }
  const float v = (float)((n & 1) ? sv : cv);
  return ((n + 1) & 2) ? -v : v;
}

UGK_HD float ugk_cosf_small(float x) { return ugk_cosf_small_t<1>(x); }
