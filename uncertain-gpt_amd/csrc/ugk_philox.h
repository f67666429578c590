// ugk_philox.h - counter-based normal draws, eps = f(seed, step, index).
//
// Philox4x32-10 (Salmon et al., "Parallel random numbers: as easy as 1, 2, 3",
// SC'11): four 32-bit counter words, a two-word key, ten rounds of two
// 32x32->64 multiplies (constants 0xD2511F53, 0xCD9E8D57) and a Weyl key
// schedule (0x9E3779B9, 0xBB67AE85). The stream is the one of
// gpt2_kernels.cuh:148-192 (philox4x32_10, u01, philox_normal): counter
// {index low, index high, step, 0}, key {seed low, seed high}, the first two
// output words mapped to (0,1) as ((float)x + 0.5f) * 2^-32, and one
// Box-Muller cosine branch per index.
//
// The integer part is exact on host and device. The float part, in the
// glibc-exact form, takes glibc's logf and cosf as ugk_libm.h restates them
// (equal to the host glibc on every input of their domains) and the correctly
// rounded square root, so that eps equals the host's bit for bit; in the ops'
// default (fast-math) form, the radius from the hardware log2 and square root
// and the device library's cosf sequence (ugk_dev_box_muller_fast).
#pragma once

#include <stdint.h>

#ifdef __HIPCC__
#include <hip/hip_runtime.h>

#include "ugk_libm_dev.h"
#define UGK_PHILOX_HD __host__ __device__ __forceinline__
#else
#define UGK_PHILOX_HD static inline
#endif

struct UgkPhilox4 {
  uint32_t w[4];
};

// Ten rounds; each 32x32 product is one 64-bit multiply (one v_mad_u64_u32).
UGK_PHILOX_HD UgkPhilox4 ugk_philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                           uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; r++) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    c1 = (uint32_t)p1;
    c3 = (uint32_t)p0;
    c0 = n0;
    c2 = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return UgkPhilox4{{c0, c1, c2, c3}};
}

// uint32 -> (0, 1]: the conversion rounds to nearest, the add and the
// multiply by 2^-32 round separately (no contraction).
UGK_PHILOX_HD float ugk_u01(uint32_t x) { return ((float)x + 0.5f) * 2.3283064365386963e-10f; }

UGK_PHILOX_HD UgkPhilox4 ugk_philox_words(unsigned long long seed, int step, uint64_t index) {
  return ugk_philox4x32_10((uint32_t)index, (uint32_t)(index >> 32), (uint32_t)step, 0u,
                           (uint32_t)seed, (uint32_t)(seed >> 32));
}

#ifdef __HIPCC__
// a ^ b ^ k in one v_bitop3_b32 (truth table 0x96), k in a scalar register.
// Only for a k that is the same in every lane of the wavefront.
__device__ __forceinline__ uint32_t ugk_xor3_uniform(uint32_t a, uint32_t b, uint32_t k) {
  uint32_t r;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x96" : "=v"(r) : "v"(a), "v"(b), "s"(k));
  return r;
}

// ugk_philox_words for a (seed, step) shared by the whole wavefront (the
// kernels draw eps(seed, step, i) for their own i): the same rounds, with each
// round's two three-way xors as one instruction each, the round key scalar.
__device__ __forceinline__ UgkPhilox4 ugk_dev_philox_words_uniform(unsigned long long seed, int step,
                                                                  uint64_t index) {
  uint32_t c0 = (uint32_t)index, c1 = (uint32_t)(index >> 32), c2 = (uint32_t)step, c3 = 0u;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; r++) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t n0 = ugk_xor3_uniform((uint32_t)(p1 >> 32), c1, k0);
    const uint32_t n2 = ugk_xor3_uniform((uint32_t)(p0 >> 32), c3, k1);
    c1 = (uint32_t)p1;
    c3 = (uint32_t)p0;
    c0 = n0;
    c2 = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return UgkPhilox4{{c0, c1, c2, c3}};
}

// Box-Muller, cosine branch, as gpt2_kernels.cuh:181-192 writes it and the
// host builds it: sqrtf(-2 logf(u1)) * cosf(2 pi u2), with 2 pi rounded to
// float and the product rounded before the cosine. u1 in [2^-33, 1] is a
// normal float and 2 pi u2 lies in (0, 2 pi], inside the domains of the
// restated logf and cosf (ugk_logf_normal, ugk_cosf_small); -2 ln u1 is -0 or
// in [1.1e-7, 46], inside the domain of the correctly rounded square root
// without rescaling. The same bits as the host's for every u1, u2.
__device__ __forceinline__ float ugk_dev_box_muller(uint32_t a, uint32_t b) {
  const float u1 = ugk_u01(a), u2 = ugk_u01(b);
  const float l = ugk_logf_normal(u1);
  const float x = 6.28318530717958647692f * u2;
  return ugk_dev_sqrtf_large(-2.0f * l) * ugk_cosf_small(x);
}

// The same transform with the radius from the hardware log2 and square root
// (v_log_f32, v_sqrt_f32), as a fast-math build computes it: -2 ln u1 as
// log2(u1) times -2 ln 2, rounded once, and a square root within 1 ulp; the
// cosine the device library's (ugk_dev_cosf_small, float arithmetic). The
// Philox ops' default form.
__device__ __forceinline__ float ugk_dev_bm_radius_fast(float u1) {
  return __builtin_amdgcn_sqrtf((-2.0f * __builtin_amdgcn_logf(u1)) * 0x1.62e43p-1f);
}

__device__ __forceinline__ float ugk_dev_box_muller_fast(uint32_t a, uint32_t b) {
  const float u1 = ugk_u01(a), u2 = ugk_u01(b);
  return ugk_dev_bm_radius_fast(u1) * ugk_dev_cosf_small(6.28318530717958647692f * u2);
}

// eps(seed, step, index); seed and step must be the same across the wavefront.
__device__ __forceinline__ float ugk_dev_philox_normal(unsigned long long seed, int step, uint64_t index) {
  const UgkPhilox4 o = ugk_dev_philox_words_uniform(seed, step, index);
  return ugk_dev_box_muller(o.w[0], o.w[1]);
}

__device__ __forceinline__ float ugk_dev_philox_normal_fast(unsigned long long seed, int step, uint64_t index) {
  const UgkPhilox4 o = ugk_dev_philox_words_uniform(seed, step, index);
  return ugk_dev_box_muller_fast(o.w[0], o.w[1]);
}
#endif
