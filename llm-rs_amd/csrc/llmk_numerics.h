// llmk_numerics.h — the engine's fixed floating-point definitions (gfx950).
//
// Every function here uses only IEEE-exact operations (add, mul, fma, div,
// rint, ldexp, conversions), so a CPU restatement of the same steps gives the
// same bits.  The file is compiled with -ffp-contract=off: an FMA appears
// only where it is written.
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
  const double z = __builtin_fma(0x1.c6af84b912394p-20, r, 0x1.ebfce50fac4f3p-13);
  const double r2 = r * r;
  double y = __builtin_fma(0x1.62e42ff0c52d6p-6, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return live ? (float)y : 0.0f;
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
