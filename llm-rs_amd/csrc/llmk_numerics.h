// llmk_numerics.h — the engine's fixed floating-point definitions (gfx950).
//
// Every function here uses only IEEE-exact operations (add, mul, fma, div,
// rint, ldexp, conversions), so a CPU restatement of the same steps gives the
// same bits.  The file is compiled with -ffp-contract=off: an FMA appears
// only where it is written.
//
// Provenance of the numerical methods restated here (exp, expm1, tanh):
//  - expf: the method and the exp2f_data constants (the 2^(i/32) table, the
//    cubic's coefficients) of Szabolcs Nagy's expf in Arm's
//    optimized-routines, which glibc 2.28 and later ship as
//    sysdeps/ieee754/flt-32/e_expf.c:
//      Copyright (c) 2017-2018, Arm Limited.
//      SPDX-License-Identifier: MIT
//  - expm1f, tanhf: fdlibm's method and coefficients, as glibc's
//    s_expm1f.c and s_tanhf.c carry them:
//      Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//      Developed at SunPro, a Sun Microsystems, Inc. business.
//      Permission to use, copy, modify, and distribute this
//      software is freely granted, provided that this notice
//      is preserved.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace llmk {

// e^x for x <= 0, bit for bit as glibc's expf computes it (glibc >= 2.28,
// sysdeps/ieee754/flt-32/e_expf.c; the x86-64 FMA build that Rust's
// f32::exp, sampler.rs:61, reaches): x*32/ln2 = k + r, k the nearest integer
// (ties to even, through the 1.5*2^52 shift), 2^(k/32) = the table word of
// k mod 32 with k >> 5 added to its exponent field, 2^(r/32) by a cubic, all
// in double, one rounding to float.  The two reduction steps are fused
// multiply-adds, as that build contracts them.  kExpTab[i] = bits(2^(i/32))
// - (i << 47) with 2^(i/32) correctly rounded; the cubic is glibc's published
// exp2f_data poly scaled by 32^-3, 32^-2, 32^-1.  The CPU tests scan every
// float in [-104, 0] against the host's expf.  Below -0x1.9fe368p6 (e^x
// rounds to 0) and at -inf the result is +0.
constexpr uint64_t kExpTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull,
    0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
    0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull,
    0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull,
    0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
    0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull,
    0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull,
    0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
    0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// The table in LDS (static, per workgroup): every kernel that evaluates
// exp_ref calls exp_tab_init() before its first barrier.
__shared__ uint64_t g_exptab[32];
__device__ __forceinline__ void exp_tab_init() {
  if (threadIdx.x < 32) g_exptab[threadIdx.x] = kExpTab[threadIdx.x];
}

// REMAT: the polynomial's constant term is written into a register pair at
// each call (two moves the compiler cannot hoist), so that a loop calling
// exp_ref does not hold it in registers across its whole body: under
// register pressure the compiler spilled it, and every reload from scratch
// waited for all the loads in flight.
template <bool REMAT = false>
__device__ __forceinline__ float exp_ref(float x) {
  const bool live = x >= -0x1.9fe368p6f;  // false for -inf
  const double xd = live ? (double)x : 0.0;
  double kd = __builtin_fma(0x1.71547652b82fep+5, xd, 0x1.8p+52);
  const uint32_t ki = (uint32_t)__double_as_longlong(kd);
  kd = kd - 0x1.8p+52;
  const double r = __builtin_fma(0x1.71547652b82fep+5, xd, -kd);
  // (ki << 47) mod 2^64 touches only the high word: (ki << 15) << 32
  const uint64_t t = g_exptab[ki & 31u] + ((uint64_t)(ki << 15) << 32);
  const double s = __longlong_as_double((long long)t);
  double c0 = 0x1.ebfce50fac4f3p-13;
  if (REMAT) {
    uint32_t lo, hi;
    asm volatile("v_mov_b32 %0, 0x50fac4f3" : "=v"(lo));
    asm volatile("v_mov_b32 %0, 0x3f2ebfce" : "=v"(hi));
    c0 = __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
  }
  const double z = __builtin_fma(0x1.c6af84b912394p-20, r, c0);
  const double r2 = r * r;
  double y = __builtin_fma(0x1.62e42ff0c52d6p-6, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return live ? (float)y : 0.0f;
}

// tanh(x) bit for bit as glibc's tanhf computes it (glibc 2.35, sysdeps/
// ieee754/flt-32/s_tanhf.c and s_expm1f.c: Sun's fdlibm method, all in
// float, no fused operations): tanh|x| = 1 - 2/(expm1(2|x|) + 2) for
// |x| >= 1, -t/(t + 2) with t = expm1(-2|x|) below, x(1 + x) below 2^-55,
// 1 from 22 on; the sign restored last.  expm1 reduces x = k ln2 + r with ln2
// split into a head of 16 significant bits and a tail (k = +-1 directly
// between 0.5 ln2 and 1.5 ln2, else k = trunc(x/ln2 +- 1/2) and the
// rounding error of the reduction kept in c), approximates expm1 on
// [-ln2/2, ln2/2] through the rational form of fdlibm with its quintic in
// (x^2/2) (coefficients Q1..Q5), and rebuilds 2^k (expm1(r) + 1) - 1 by the
// case on k.  The CPU tests compare every float against the host's tanhf and
// expm1f.
__device__ __forceinline__ float f_of(uint32_t b) { return __uint_as_float(b); }
__device__ __forceinline__ float expm1_ref(float x) {
  const float ln2_head = f_of(0x3f317180u), ln2_tail = f_of(0x3717f7d1u);
  const float inv_ln2 = f_of(0x3fb8aa3bu);
  const float q1 = f_of(0xbd088889u), q2 = f_of(0x3ad00d01u), q3 = f_of(0xb8a670cdu),
              q4 = f_of(0x36867e54u), q5 = f_of(0xb457edbbu);
  const uint32_t bits = __float_as_uint(x);
  const bool neg = (bits >> 31) != 0;
  const uint32_t mag = bits & 0x7fffffffu;
  if (mag >= 0x4195b844u) {  // |x| >= 27 ln2: the result is -1 or overflows
    if (mag >= 0x42b17218u) {
      if (mag > 0x7f800000u) return x + x;  // NaN
      if (mag == 0x7f800000u) return neg ? -1.0f : x;
      if (x > f_of(0x42b17180u)) return __builtin_huge_valf();
    }
    if (neg) return -1.0f;
  }
  int k = 0;
  float c = 0.0f;
  if (mag > 0x3eb17218u) {  // |x| > ln2/2: reduce
    float head, tail;
    if (mag < 0x3f851592u) {  // |x| < 1.5 ln2
      k = neg ? -1 : 1;
      head = neg ? x + ln2_head : x - ln2_head;
      tail = neg ? -ln2_tail : ln2_tail;
    } else {
      k = (int)(inv_ln2 * x + (neg ? -0.5f : 0.5f));
      const float kf = (float)k;
      head = x - kf * ln2_head;
      tail = kf * ln2_tail;
    }
    x = head - tail;
    c = (head - x) - tail;
  } else if (mag < 0x33000000u) {  // |x| < 2^-25
    return x;
  }
  const float half_x = 0.5f * x;
  const float hx2 = x * half_x;
  const float r1 = 1.0f + hx2 * (q1 + hx2 * (q2 + hx2 * (q3 + hx2 * (q4 + hx2 * q5))));
  float t = 3.0f - r1 * half_x;
  float e = hx2 * ((r1 - t) / (6.0f - x * t));
  if (k == 0) return x - (x * e - hx2);
  e = x * (e - c) - c;
  e = e - hx2;
  if (k == -1) return 0.5f * (x - e) - 0.5f;
  if (k == 1) return x < -0.25f ? -2.0f * (e - (x + 0.5f)) : 1.0f + 2.0f * (x - e);
  float y;
  if (k <= -2 || k > 56) {
    y = 1.0f - (e - x);
    return f_of(__float_as_uint(y) + ((uint32_t)k << 23)) - 1.0f;
  }
  if (k < 23) {
    t = f_of(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
    y = t - (e - x);
  } else {
    t = f_of((uint32_t)(0x7f - k) << 23);  // 2^-k
    y = x - (e + t);
    y = y + 1.0f;
  }
  return f_of(__float_as_uint(y) + ((uint32_t)k << 23));
}
__device__ __forceinline__ float tanh_ref(float x) {
  const uint32_t bits = __float_as_uint(x), mag = bits & 0x7fffffffu;
  const bool neg = (bits >> 31) != 0;
  if (mag >= 0x7f800000u) return neg ? 1.0f / x - 1.0f : 1.0f / x + 1.0f;  // +-1, NaN
  float z;
  if (mag >= 0x41b00000u) {  // |x| >= 22
    z = 1.0f;
  } else if (mag == 0) {
    return x;
  } else if (mag < 0x24000000u) {  // |x| < 2^-55
    return x * (1.0f + x);
  } else if (mag >= 0x3f800000u) {
    const float t = expm1_ref(2.0f * __builtin_fabsf(x));
    z = 1.0f - 2.0f / (t + 2.0f);
  } else {
    const float t = expm1_ref(-2.0f * __builtin_fabsf(x));
    z = -t / (t + 2.0f);
  }
  return neg ? -z : z;
}

// Order-preserving map float -> u32 (NaN excluded by callers).
__device__ __forceinline__ uint32_t fkey(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float funkey(uint32_t k) {
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(b);
}

}  // namespace llmk
