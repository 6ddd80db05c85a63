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

// e^y for y <= 0, as used on the reference's candidate probabilities
// (sampler.rs:61 `(l - max_logit).exp()`).  Cody–Waite reduction
// y = k ln2 + r with ln2 split in two parts, e^r by its degree-13 Taylor
// polynomial (|r| <= ln2/2, truncation < 5e-18) in double, one final rounding
// to float.  Agrees with glibc expf on all but 1 in ~11500 inputs (1 ulp).
__device__ __forceinline__ float exp_m(float y) {
  const bool ok = y >= -110.0f;  // below: far under the smallest subnormal
  const double yd = ok ? (double)y : 0.0;
  const double kd = __builtin_rint(yd * 0x1.71547652b82fep+0);
  double r = __builtin_fma(-kd, 0x1.62e42fee00000p-1, yd);
  r = __builtin_fma(-kd, 0x1.a39ef35793c76p-33, r);
  double p = 0x1.6124613a86d09p-33;
  p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);
  p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);
  p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);
  p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);
  p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);
  p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);
  p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);
  p = __builtin_fma(p, r, 0x1.1111111111111p-7);
  p = __builtin_fma(p, r, 0x1.5555555555555p-5);
  p = __builtin_fma(p, r, 0x1.5555555555555p-3);
  p = __builtin_fma(p, r, 0x1.0000000000000p-1);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  const float res = (float)__builtin_amdgcn_ldexp(p, (int)kd);
  return ok ? res : 0.0f;
}

// 2^d for d <= 0: the terms of the softmax normaliser.  d is clamped to
// [-125, ...] (NaN and -inf give the clamp), rounded to k = rint(d) by adding
// and subtracting 1.5*2^23, f = d - k in [-1/2, 1/2], 2^f by a degree-5
// minimax polynomial (relative error 1.7e-7), and the scaling by 2^k is an
// integer add of k to the exponent field (exact: the result stays normal).
// Elements at or below the clamp contribute 2^-125 * 2^f.
__device__ __forceinline__ float exp2_f(float d) {
  const float dc = __builtin_fmaxf(d, -125.0f);
  const float t = dc + 12582912.0f;
  const float k = t - 12582912.0f;
  const float f = dc - k;
  float p = __builtin_fmaf(0x1.5bba14p-10f, f, 0x1.3cea88p-7f);
  p = __builtin_fmaf(p, f, 0x1.c6b752p-5f);
  p = __builtin_fmaf(p, f, 0x1.ebf9bcp-3f);
  p = __builtin_fmaf(p, f, 0x1.62e42ap-1f);
  p = __builtin_fmaf(p, f, 1.0f);
  return __uint_as_float(__float_as_uint(p) + (__float_as_uint(t) << 23));
}

constexpr float LOG2E_F = 0x1.715476p+0f;

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
