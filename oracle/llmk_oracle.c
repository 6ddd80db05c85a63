/*
 * llmk_oracle.c — CPU oracle for the llm-rs token-sampling path.
 *
 * TEST INFRASTRUCTURE ONLY (see llmk_oracle.h).  Built with
 * -ffp-contract=off so every multiply and add rounds on its own, as Rust does
 * (Rust never contracts a*b+c into an FMA).
 *
 * Reference being restated: /root/reference/llm-core/src/sampler.rs
 *   sample_logits            :25-125   -> sample_row()
 *   apply_repetition_penalty :128-147  -> apply_repetition()
 *   apply_temperature        :150-157  -> apply_temperature()
 *   apply_top_k              :160-173  -> llmk_oracle_apply_top_k()
 *   apply_top_p              :176-216  -> llmk_oracle_apply_top_p()
 *   sample                   :219-228  -> llmk_oracle_sample_simple()
 * Speculative verification (docs/mlc-contracts.md:83-84) -> llmk_oracle_verify_row().
 * Presence/frequency formula: llm-tests/tests/mlc_parity.rs:1074-1089.
 *
 * Provenance of the numerical methods restated here (exp, expm1, tanh):
 *  - expf: the method and the exp2f_data constants (the 2^(i/32) table, the
 *    cubic's coefficients) of Szabolcs Nagy's expf in Arm's
 *    optimized-routines, which glibc 2.28 and later ship as
 *    sysdeps/ieee754/flt-32/e_expf.c:
 *      Copyright (c) 2017-2018, Arm Limited.
 *      SPDX-License-Identifier: MIT
 *  - expm1f, tanhf: fdlibm's method and coefficients, as glibc's
 *    s_expm1f.c and s_tanhf.c carry them:
 *      Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
 *      Developed at SunPro, a Sun Microsystems, Inc. business.
 *      Permission to use, copy, modify, and distribute this
 *      software is freely granted, provided that this notice
 *      is preserved.
 */
#define _GNU_SOURCE
#include "llmk_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Numerics                                                                  */
/* ------------------------------------------------------------------------ */

/* e^x as glibc's expf computes it (glibc >= 2.28, sysdeps/ieee754/flt-32/
 * e_expf.c, the ARM optimized-routines method by Szabolcs Nagy): x*32/ln2 =
 * k + r with k the nearest integer (ties to even), 2^(k/32) from a table of
 * 2^(i/32) (the exponent of 2^(k>>5) added to its bits), 2^(r/32) by a cubic,
 * all in double, one rounding to float.  The x86-64 build that Rust's
 * f32::exp reaches on this platform (the FMA variant) fuses the two
 * reduction steps kd = x*InvLn2N + SHIFT and r = x*InvLn2N - kd; written out
 * with fma() here.  EXP_TAB[i] = bits(2^(i/32)) - (i << 47), 2^(i/32)
 * correctly rounded (oracle/gen_constants.py recomputes it); the cubic's
 * coefficients are glibc's published exp2f_data poly, scaled by 32^-3,
 * 32^-2, 32^-1.  tests/test_oracle_math.py checks every float in [-104, 0]
 * against the host's expf.  Inputs below -0x1.9fe368p6 (where e^x rounds
 * to 0) and -inf give +0. */
static const uint64_t EXP_TAB[32] = {
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
static const double EXP_C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
static const double EXP_C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
static const double EXP_C2 = 0x1.62e42ff0c52d6p-1 / 32;
static const double EXP_INVLN2N = 0x1.71547652b82fep+0 * 32;
static const double EXP_SHIFT = 0x1.8p+52;

float llmk_oracle_exp_ref(float x) {
  if (!(x >= -0x1.9fe368p6f)) return 0.0f;
  const double xd = (double)x;
  double kd = fma(EXP_INVLN2N, xd, EXP_SHIFT);
  uint64_t ki;
  memcpy(&ki, &kd, 8);
  kd -= EXP_SHIFT;
  const double r = fma(EXP_INVLN2N, xd, -kd);
  const uint64_t t = EXP_TAB[ki % 32] + (ki << 47);
  double s;
  memcpy(&s, &t, 8);
  const double z = fma(EXP_C0, r, EXP_C1);
  const double r2 = r * r;
  double y = fma(EXP_C2, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return (float)y;
}

float llmk_oracle_libm_expf(float y) { return expf(y); }

/* ------------------------------------------------------------------------ */
/* Sorting helpers (in-place introsort on u64 / u32 keys, ascending)         */
/* ------------------------------------------------------------------------ */

#define DEFINE_SORT(NAME, T)                                                  \
  static void NAME##_insertion(T* a, int64_t n) {                             \
    for (int64_t i = 1; i < n; ++i) {                                         \
      T v = a[i];                                                             \
      int64_t j = i - 1;                                                      \
      while (j >= 0 && a[j] > v) {                                            \
        a[j + 1] = a[j];                                                      \
        --j;                                                                  \
      }                                                                       \
      a[j + 1] = v;                                                           \
    }                                                                         \
  }                                                                           \
  static void NAME##_sift(T* a, int64_t start, int64_t n) {                   \
    int64_t r = start;                                                        \
    for (;;) {                                                                \
      int64_t c = 2 * r + 1;                                                  \
      if (c >= n) return;                                                     \
      if (c + 1 < n && a[c + 1] > a[c]) ++c;                                  \
      if (a[r] >= a[c]) return;                                               \
      T t = a[r];                                                             \
      a[r] = a[c];                                                            \
      a[c] = t;                                                               \
      r = c;                                                                  \
    }                                                                         \
  }                                                                           \
  static void NAME##_heap(T* a, int64_t n) {                                  \
    for (int64_t s = n / 2 - 1; s >= 0; --s) NAME##_sift(a, s, n);            \
    for (int64_t e = n - 1; e > 0; --e) {                                     \
      T t = a[0];                                                             \
      a[0] = a[e];                                                            \
      a[e] = t;                                                               \
      NAME##_sift(a, 0, e);                                                   \
    }                                                                         \
  }                                                                           \
  static void NAME##_intro(T* a, int64_t n, int depth) {                      \
    while (n > 24) {                                                          \
      if (depth-- == 0) {                                                     \
        NAME##_heap(a, n);                                                    \
        return;                                                               \
      }                                                                       \
      T x = a[0], y = a[n / 2], z = a[n - 1], piv;                            \
      if (x < y) piv = (y < z) ? y : ((x < z) ? z : x);                       \
      else piv = (x < z) ? x : ((y < z) ? z : y);                             \
      int64_t i = 0, j = n - 1;                                               \
      for (;;) {                                                              \
        while (a[i] < piv) ++i;                                               \
        while (a[j] > piv) --j;                                               \
        if (i >= j) break;                                                    \
        T t = a[i];                                                           \
        a[i] = a[j];                                                          \
        a[j] = t;                                                             \
        ++i;                                                                  \
        --j;                                                                  \
      }                                                                       \
      NAME##_intro(a + j + 1, n - j - 1, depth);                              \
      n = j + 1;                                                              \
    }                                                                         \
    NAME##_insertion(a, n);                                                   \
  }                                                                           \
  static void NAME(T* a, int64_t n) {                                         \
    int depth = 0;                                                            \
    for (int64_t m = n; m > 1; m >>= 1) depth += 2;                           \
    NAME##_intro(a, n, depth);                                                \
  }

DEFINE_SORT(sort_u64, uint64_t)
DEFINE_SORT(sort_u32, uint32_t)

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* (p desc, idx asc) order as one ascending u64 key.  p >= 0 here (NaN rows
 * are outside the parity contract; in ref mode a NaN p lands wherever its bit
 * pattern puts it, deterministically). */
static inline uint64_t pkey(float p, uint32_t idx) {
  return ((uint64_t)(~f2u(p)) << 32) | idx;
}

/* ------------------------------------------------------------------------ */
/* Steps                                                                     */
/* ------------------------------------------------------------------------ */

static uint32_t* sorted_history(const uint32_t* hist, uint32_t H) {
  uint32_t* h = (uint32_t*)malloc(sizeof(uint32_t) * (H ? H : 1));
  if (H) memcpy(h, hist, sizeof(uint32_t) * H);
  sort_u32(h, H);
  return h;
}

/* sampler.rs:128-147 */
static void apply_repetition(float* l, uint32_t V, const uint32_t* hist,
                             uint32_t H, float penalty) {
  if (penalty == 1.0f || H == 0) return;
  uint32_t* h = sorted_history(hist, H);
  for (uint32_t i = 0; i < H; ++i) {
    if (i > 0 && h[i] == h[i - 1]) continue; /* dedup */
    uint32_t t = h[i];
    if (t < V) {
      float v = l[t];
      l[t] = (v > 0.0f) ? v / penalty : v * penalty;
    }
  }
  free(h);
}

/* Extension: l -= presence + count*frequency for tokens seen count > 0 times
 * (formula of llm-tests/tests/mlc_parity.rs:1083, evaluated without FMA). */
static void apply_presence_frequency(float* l, uint32_t V, const uint32_t* hist,
                                     uint32_t H, float presence,
                                     float frequency) {
  if ((presence == 0.0f && frequency == 0.0f) || H == 0) return;
  uint32_t* h = sorted_history(hist, H);
  uint32_t i = 0;
  while (i < H) {
    uint32_t j = i;
    while (j < H && h[j] == h[i]) ++j;
    uint32_t t = h[i], count = j - i;
    if (t < V) {
      float cf = (float)count * frequency;
      l[t] = l[t] - (presence + cf);
    }
    i = j;
  }
  free(h);
}

/* sampler.rs:150-157 */
static void apply_temperature(float* l, uint32_t V, float t) {
  if (t <= 1e-5f || t == 1.0f) return;
  for (uint32_t i = 0; i < V; ++i) l[i] = l[i] / t;
}

typedef struct {
  float* p;
  uint32_t* idx;
  uint32_t n;
} plist;

static void renormalize(plist* L) {
  float s = 0.0f;
  for (uint32_t j = 0; j < L->n; ++j) s += L->p[j];
  if (s > 0.0f)
    for (uint32_t j = 0; j < L->n; ++j) L->p[j] = L->p[j] / s;
}

static int params_invalid(const llmk_oracle_params* p) {
  if (isnan(p->temperature) || isinf(p->temperature)) return 1;
  if (p->top_k < 0) return 1;
  if (!isfinite(p->top_p) || !isfinite(p->min_p) || p->min_p < 0.0f) return 1;
  if (!isfinite(p->repetition_penalty) || !isfinite(p->presence_penalty) ||
      !isfinite(p->frequency_penalty))
    return 1;
  return 0;
}

/* min-p, top-k (sampler.rs:80-89), top-p (:92-110) and the draw (:113-124)
 * on a list sorted by (p desc, idx asc); L is truncated in place. */
static void semantics(plist* Lp, const llmk_oracle_params* prm, float u,
                      uint32_t* out_token, uint32_t* out_ids, float* out_probs,
                      uint32_t out_cap, uint32_t* out_count) {
  plist L = *Lp;
  /* min-p (extension): keep p >= min_p * p_max; renormalise if it cut. */
  if (prm->min_p > 0.0f && L.n > 0) {
    float thr = prm->min_p * L.p[0];
    uint32_t cut = L.n;
    for (uint32_t j = 0; j < L.n; ++j)
      if (L.p[j] < thr) {
        cut = j;
        break;
      }
    if (cut < L.n) {
      L.n = cut;
      renormalize(&L);
    }
  }
  /* top-k, :80-89 */
  if (prm->top_k > 0 && (uint32_t)prm->top_k < L.n) {
    L.n = (uint32_t)prm->top_k;
    renormalize(&L);
  }
  /* top-p, :92-110 */
  if (prm->top_p < 1.0f) {
    float cum = 0.0f;
    uint32_t cut = L.n;
    for (uint32_t j = 0; j < L.n; ++j) {
      cum += L.p[j];
      if (cum >= prm->top_p) {
        cut = j + 1;
        break;
      }
    }
    L.n = cut;
    renormalize(&L);
  }
  /* draw, :113-124 */
  uint32_t tok = (L.n > 0) ? L.idx[L.n - 1] : 0;
  {
    float cum = 0.0f;
    for (uint32_t j = 0; j < L.n; ++j) {
      cum += L.p[j];
      if (u <= cum) {
        tok = L.idx[j];
        break;
      }
    }
  }
  *out_token = tok;
  if (out_count) *out_count = L.n;
  for (uint32_t j = 0; j < L.n && j < out_cap; ++j) {
    if (out_ids) out_ids[j] = L.idx[j];
    if (out_probs) out_probs[j] = L.p[j];
  }
  *Lp = L;
}

/* ------------------------------------------------------------------------ */
/* The rounding band of S = 1 on rows that top-k renormalises                 */
/* ------------------------------------------------------------------------ */

/* On a row that top-k renormalises the reference computes p_i = fl(e_i / S)
 * with S its sequential sum over the whole row (sampler.rs:66-71), then
 * renormalises the kept entries (:83-88, and min-p's cut, which comes
 * first).  S cancels in exact arithmetic, so S = 1 gives the same decisions
 * (min-p cut, top-k set and order, top-p cut, drawn token) unless one of
 * them lies within the rounding of the f32 arithmetic.  band_certain proves,
 * from the e_i of the sorted list alone, that every decision is the same
 * for every S the reference can hold: with p_i known only to relative R
 * (R = 2^-24 for fl(e_i / S)), each sequential sum rounds by at most half an
 * ulp of its running value (bounded by u times the value where the scale is
 * S's, by the binade's half ulp once the values are normalised), each
 * renormalisation divides by a sum known to relative sigma and rounds again
 * (R' = (R + sigma + u)(1 + 2^-10), the factor covering second-order
 * terms), and a decision is certain when its exact value (a sum of the e_i
 * in double) lies outside the band of its bound.  Entries whose order could
 * differ (fl(e_a / S) == fl(e_b / S) ties ordered by index: e_a and e_b
 * within 2^-20 relative with their indices inverted; equal e keep their
 * index order under any S) and entries below 2^-100 (p could be
 * subnormal) are uncertain too.
 *
 * The doubles are summed in the order a 64-lane wave computes them on the
 * device (wave_prefix64: a DPP scan within 64 entries, then the chunk's
 * carry), so both sides see the same bits.
 *
 * e: the list's values (p with S = 1) in (p desc, idx asc) order, E of them
 * exact; every entry past E is <= ptail; full: the row's length. */
#define BAND_U 0x1p-24
#define BAND_F (1.0 + 0x1p-10)
#define BAND_SL 0x1p-36
#define BAND_CLOSE (1.0 + 0x1p-20)

/* half an ulp of a float of magnitude x in (0, 2): 2^(floor(log2 x) - 24) */
static double band_hu(double x) {
  if (!(x > 0.0)) return 0.0;
  int ex;
  (void)frexp(x, &ex);
  return ldexp(1.0, ex - 25);
}

/* inclusive prefix of 64 values as the device's wave computes it: steps of
 * row_shr 1, 2, 4, 8 within rows of 16 lanes, then row 0's total added to
 * row 1 and row 2's to row 3 (row_bcast 15), then row 1's new total to rows
 * 2 and 3 (row_bcast 31) */
static void dpp_scan64(double* y) {
  for (int d = 1; d < 16; d <<= 1) {
    double z[64];
    for (int j = 0; j < 64; ++j) z[j] = (j & 15) >= d ? y[j] + y[j - d] : y[j];
    memcpy(y, z, sizeof z);
  }
  const double t15 = y[15], t47 = y[47];
  for (int j = 16; j < 32; ++j) y[j] = y[j] + t15;
  for (int j = 48; j < 64; ++j) y[j] = y[j] + t47;
  const double t31 = y[31];
  for (int j = 32; j < 64; ++j) y[j] = y[j] + t31;
}

/* inclusive prefix of x[0..n) in place: chunks of 64, each scanned as a
 * wave does, plus the carry of the chunks before it */
static void wave_prefix64(double* x, uint32_t n) {
  double carry = 0.0;
  for (uint32_t c0 = 0; c0 < n; c0 += 64) {
    double y[64];
    for (uint32_t j = 0; j < 64; ++j) y[j] = c0 + j < n ? x[c0 + j] : 0.0;
    dpp_scan64(y);
    for (uint32_t j = 0; j < 64; ++j) y[j] = y[j] + carry;
    carry = y[63];
    for (uint32_t j = 0; j < 64 && c0 + j < n; ++j) x[c0 + j] = y[j];
  }
}

/* sigma of a renormalisation over [0, n): the reference's sequential sum of
 * p_i known to relative R, against the exact sum P[n-1] (P: prefix of e) */
static double band_sigma(const double* P, uint32_t n, double R, double* work) {
  for (uint32_t j = 0; j < n; ++j) work[j] = j >= 1 ? P[j] : 0.0;
  wave_prefix64(work, n);
  return R + BAND_U * (1.0 + R) * BAND_F * (work[n - 1] / P[n - 1]);
}

/* the first j < n whose cumulative may reach thr (C + B >= thr); sets
 * *certain when the reference's cumulative surely reaches it there and
 * surely not before; returns n when none may.  C_j = P[j] (1 / P[n-1]),
 * B_j = R C_j + sum_{1 <= i <= j} hu(C_i (1 + R) F) + SL C_j. */
static uint32_t band_find(const double* P, uint32_t n, double R, double thr,
                          double* B, int* certain) {
  const double rt = 1.0 / P[n - 1];
  for (uint32_t j = 0; j < n; ++j)
    B[j] = j >= 1 ? band_hu((P[j] * rt) * (1.0 + R) * BAND_F) : 0.0;
  wave_prefix64(B, n);
  *certain = 1;
  for (uint32_t j = 0; j < n; ++j) {
    const double C = P[j] * rt;
    const double b = R * C + B[j] + BAND_SL * C;
    B[j] = b;
    if (C + b >= thr) {
      *certain = (C - b >= thr);
      return j;
    }
  }
  return n;
}

static int band_certain(const float* e, const uint32_t* idx, uint32_t E,
                        uint32_t full, float ptail,
                        const llmk_oracle_params* prm, float u) {
  const int32_t K = prm->top_k;
  uint32_t len = full;
  double R = BAND_U;
  int normalised = 0;
  /* entries whose p = e / S could be subnormal */
  const uint32_t lim = (K > 0 && (uint32_t)K + 1u < E) ? (uint32_t)K + 1u : E;
  for (uint32_t j = 0; j < lim; ++j)
    if (e[j] > 0.0f && e[j] < 0x1p-100f) return 0;
  double* P = (double*)malloc(sizeof(double) * (E ? E : 1));
  double* W = (double*)malloc(sizeof(double) * (E ? E : 1));
  int ok = 0;
  /* min-p: kept iff fl(e/S) >= fl(min_p * fl(1/S)) (e_0 = 1, the maximum);
   * certain outside min_p (1 -+ 2^-21) */
  if (prm->min_p > 0.0f) {
    if (prm->min_p < 0x1p-100f || E == 0) goto out;
    const double hi = (double)prm->min_p * (1.0 + 0x1p-21);
    const double lo = (double)prm->min_p * (1.0 - 0x1p-21);
    uint32_t cut = 0xffffffffu;
    const uint32_t n = E < len ? E : len;
    for (uint32_t j = 0; j < n; ++j)
      if ((double)e[j] < hi) {
        cut = j;
        break;
      }
    if (cut != 0xffffffffu) {
      if ((double)e[cut] >= lo) goto out;
    } else if (E < len) {
      if ((double)ptail >= lo) goto out;
      cut = E;
    }
    if (cut != 0xffffffffu && cut < len) {
      len = cut;
      if (len == 0) goto out;
      for (uint32_t j = 0; j < len; ++j) P[j] = (double)e[j];
      wave_prefix64(P, len);
      if (!(P[len - 1] > 0.0)) goto out;
      const double sg = band_sigma(P, len, R, W);
      R = (R + sg + BAND_U) * BAND_F;
      normalised = 1;
    }
  }
  /* top-k: the first K in (p desc, idx asc) order; no pair whose order could
   * change, across the boundary included (an unknown entry K close to the
   * last kept one could be either side of it) */
  if (K > 0 && (uint32_t)K < len) {
    if ((uint32_t)K > E) goto out;
    if ((uint32_t)K == E && (double)e[K - 1] < (double)ptail * BAND_CLOSE) goto out;
    const uint32_t np = (uint32_t)K < E ? (uint32_t)K + 1u : (uint32_t)K;
    for (uint32_t j = 0; j + 1 < np; ++j)
      if ((double)e[j] < (double)e[j + 1] * BAND_CLOSE && idx[j] > idx[j + 1]) goto out;
    len = (uint32_t)K;
    for (uint32_t j = 0; j < len; ++j) P[j] = (double)e[j];
    wave_prefix64(P, len);
    if (!(P[len - 1] > 0.0)) goto out;
    const double sg = band_sigma(P, len, R, W);
    R = (R + sg + BAND_U) * BAND_F;
    normalised = 1;
  } else {
    const uint32_t n = E < len ? E : len;
    for (uint32_t j = 0; j + 1 < n; ++j)
      if ((double)e[j] < (double)e[j + 1] * BAND_CLOSE && idx[j] > idx[j + 1]) goto out;
  }
  if (!normalised || len > E) goto out;
  /* top-p: the first cumulative >= top_p, then the renormalisation by that
   * same cumulative */
  if (prm->top_p < 1.0f) {
    int cert;
    const uint32_t j = band_find(P, len, R, (double)prm->top_p, W, &cert);
    if (!cert) goto out;
    const uint32_t cut = j < len ? j + 1 : len;
    const double sp = W[cut - 1] / (P[cut - 1] * (1.0 / P[len - 1]));
    R = (R + sp + BAND_U) * BAND_F;
    len = cut;
  }
  /* the draw: the first cumulative >= u, else the last */
  {
    int cert;
    (void)band_find(P, len, R, (double)u, W, &cert);
    if (!cert) goto out;
  }
  ok = 1;
out:
  free(P);
  free(W);
  return ok;
}

/* The first n entries of a row's sorted list with S = 1: e = exp_ref(l - m)
 * of the processed logits (mirror), in (e desc, idx asc) order. */
int llmk_oracle_sorted_e(const float* logits, uint32_t V, const llmk_oracle_params* prm,
                         const uint32_t* hist, uint32_t H, const uint32_t* mask,
                         uint32_t n, float* e_out, uint32_t* idx_out) {
  if (V == 0) return -1;
  float* l = (float*)malloc(sizeof(float) * V);
  int rc = llmk_oracle_process_logits(LLMK_ORACLE_MIRROR, logits, V, prm, hist, H, mask, l);
  if (rc != 0) {
    free(l);
    return rc;
  }
  apply_temperature(l, V, prm->temperature);
  float m = -INFINITY;
  for (uint32_t i = 0; i < V; ++i) m = fmaxf(m, l[i]);
  uint64_t* keys = (uint64_t*)malloc(sizeof(uint64_t) * V);
  for (uint32_t i = 0; i < V; ++i)
    keys[i] = pkey(l[i] == -INFINITY ? 0.0f : llmk_oracle_exp_ref(l[i] - m), i);
  sort_u64(keys, V);
  for (uint32_t j = 0; j < n && j < V; ++j) {
    idx_out[j] = (uint32_t)(keys[j] & 0xffffffffu);
    e_out[j] = u2f(~(uint32_t)(keys[j] >> 32));
  }
  free(keys);
  free(l);
  return 0;
}

int llmk_oracle_band_certain(const float* e_sorted, const uint32_t* idx, uint32_t E,
                             uint32_t full, float ptail,
                             const llmk_oracle_params* prm, float u) {
  return band_certain(e_sorted, idx, E, full, ptail, prm, u);
}

/* The penalised, masked logits before the greedy check (sampler.rs:34-37
 * plus the extensions in their order); NaN becomes -inf in mirror mode. */
int llmk_oracle_process_logits(int mode, const float* logits, uint32_t V,
                               const llmk_oracle_params* prm,
                               const uint32_t* hist, uint32_t H,
                               const uint32_t* mask, float* out) {
  if (V == 0) return -1;
  if (params_invalid(prm)) return -2;
  memcpy(out, logits, sizeof(float) * V);
  if (mode == LLMK_ORACLE_MIRROR)
    for (uint32_t i = 0; i < V; ++i)
      if (isnan(out[i])) out[i] = -INFINITY;
  apply_repetition(out, V, hist, H, prm->repetition_penalty);
  apply_presence_frequency(out, V, hist, H, prm->presence_penalty,
                           prm->frequency_penalty);
  if (mask)
    for (uint32_t i = 0; i < V; ++i)
      if (!((mask[i >> 5] >> (i & 31)) & 1u)) out[i] = -INFINITY;
  return 0;
}

int llmk_oracle_sample_row(int mode, const float* logits, uint32_t V,
                           const llmk_oracle_params* prm, const uint32_t* hist,
                           uint32_t H, const uint32_t* mask, float u,
                           uint32_t* out_token, uint32_t* out_ids,
                           float* out_probs, uint32_t out_cap,
                           uint32_t* out_count) {
  if (V == 0) return -1; /* sampler.rs:30-32 */
  if (params_invalid(prm)) return -2;
  float* l = (float*)malloc(sizeof(float) * V);
  memcpy(l, logits, sizeof(float) * V); /* sampler.rs:34 */
  if (mode == LLMK_ORACLE_MIRROR)
    for (uint32_t i = 0; i < V; ++i)
      if (isnan(l[i])) l[i] = -INFINITY;

  apply_repetition(l, V, hist, H, prm->repetition_penalty); /* :37 */
  apply_presence_frequency(l, V, hist, H, prm->presence_penalty,
                           prm->frequency_penalty);
  if (mask)
    for (uint32_t i = 0; i < V; ++i)
      if (!((mask[i >> 5] >> (i & 31)) & 1u)) l[i] = -INFINITY;

  if (prm->temperature <= 1e-5f) { /* greedy, :40-50 */
    uint32_t best = 0;
    float bv = l[0];
    for (uint32_t i = 0; i < V; ++i)
      if (l[i] > bv) {
        bv = l[i];
        best = i;
      }
    *out_token = best;
    if (out_count) *out_count = 1;
    if (out_cap > 0) {
      if (out_ids) out_ids[0] = best;
      if (out_probs) out_probs[0] = 1.0f;
    }
    free(l);
    return 0;
  }

  apply_temperature(l, V, prm->temperature); /* :53 */

  /* Softmax, :56-71.  The exp is glibc's expf in both modes (exp_ref
   * restates it bit for bit).  S is the sequential f32 sum in index order
   * (:66), except in mirror mode on rows where top-k renormalises
   * (0 < top_k < V, :80-89): there every probability is divided by a
   * renormalising sum before any step reads it and S cancels in exact
   * arithmetic, so mirror first takes S = 1 (e itself), as the engine does,
   * and keeps that result when band_certain proves that every decision is
   * the reference's for any S; otherwise it computes S and the reference's
   * arithmetic, as the engine then does too.  Tokens, kept counts and kept
   * ids are the reference's on every row either way. */
  float m = -INFINITY;
  for (uint32_t i = 0; i < V; ++i) m = fmaxf(m, l[i]);
  float* e = (float*)malloc(sizeof(float) * V);
  for (uint32_t i = 0; i < V; ++i) {
    if (l[i] == -INFINITY) e[i] = 0.0f;
    else
      e[i] = (mode == LLMK_ORACLE_MIRROR) ? llmk_oracle_exp_ref(l[i] - m)
                                          : expf(l[i] - m);
  }
  const int topk_on = prm->top_k > 0 && (uint32_t)prm->top_k < V;
  uint64_t* keys = (uint64_t*)malloc(sizeof(uint64_t) * V);
  plist L;
  L.p = (float*)malloc(sizeof(float) * V);
  L.idx = (uint32_t*)malloc(sizeof(uint32_t) * V);
  for (int pass = (mode == LLMK_ORACLE_MIRROR && topk_on) ? 0 : 1; pass < 2; ++pass) {
    float S = 1.0f;
    if (pass == 1) {
      S = 0.0f;
      for (uint32_t i = 0; i < V; ++i) S += e[i];
    }
    /* Sort (p desc, idx asc), :77 */
    for (uint32_t i = 0; i < V; ++i) keys[i] = pkey(S > 0.0f ? e[i] / S : e[i], i);
    sort_u64(keys, V);
    L.n = V;
    for (uint32_t j = 0; j < V; ++j) {
      L.idx[j] = (uint32_t)(keys[j] & 0xffffffffu);
      L.p[j] = u2f(~(uint32_t)(keys[j] >> 32));
    }
    if (pass == 0 && !band_certain(L.p, L.idx, V, V, 0.0f, prm, u)) continue;
    semantics(&L, prm, u, out_token, out_ids, out_probs, out_cap, out_count);
    break;
  }
  free(keys);
  free(L.p);
  free(L.idx);
  free(e);
  free(l);
  return 0;
}

/* The steps after the sort on a caller-supplied sorted list. */
int llmk_oracle_semantics(const float* p_sorted, const uint32_t* idx, uint32_t n,
                          const llmk_oracle_params* prm, float u,
                          uint32_t* out_token, uint32_t* out_ids,
                          float* out_probs, uint32_t out_cap,
                          uint32_t* out_count) {
  if (params_invalid(prm)) return -2;
  plist L;
  L.n = n;
  L.p = (float*)malloc(sizeof(float) * (n ? n : 1));
  L.idx = (uint32_t*)malloc(sizeof(uint32_t) * (n ? n : 1));
  if (n) {
    memcpy(L.p, p_sorted, sizeof(float) * n);
    memcpy(L.idx, idx, sizeof(uint32_t) * n);
  }
  semantics(&L, prm, u, out_token, out_ids, out_probs, out_cap, out_count);
  free(L.p);
  free(L.idx);
  return 0;
}

/* ------------------------------------------------------------------------ */
/* Batch driver                                                              */
/* ------------------------------------------------------------------------ */

typedef struct {
  int mode;
  const float* logits;
  uint32_t B, V;
  uint64_t stride;
  const float *T, *tp, *mp, *rp, *pp, *fp;
  const int32_t* tk;
  const uint32_t *ho, *ht, *mask;
  uint32_t mw;
  const float* u;
  uint32_t *out_tokens, *out_ids, *out_count;
  float* out_probs;
  uint32_t out_cap;
  uint32_t r0, r1;
  int status;
} batch_job;

static void* batch_worker(void* arg) {
  batch_job* j = (batch_job*)arg;
  j->status = 0;
  for (uint32_t r = j->r0; r < j->r1; ++r) {
    llmk_oracle_params p;
    p.temperature = j->T ? j->T[r] : 1.0f;
    p.top_k = j->tk ? j->tk[r] : 0;
    p.top_p = j->tp ? j->tp[r] : 1.0f;
    p.min_p = j->mp ? j->mp[r] : 0.0f;
    p.repetition_penalty = j->rp ? j->rp[r] : 1.0f;
    p.presence_penalty = j->pp ? j->pp[r] : 0.0f;
    p.frequency_penalty = j->fp ? j->fp[r] : 0.0f;
    const uint32_t* h = NULL;
    uint32_t H = 0;
    if (j->ho && j->ht) {
      h = j->ht + j->ho[r];
      H = j->ho[r + 1] - j->ho[r];
    }
    uint32_t cnt = 0;
    int s = llmk_oracle_sample_row(
        j->mode, j->logits + (uint64_t)r * j->stride, j->V, &p, h, H,
        j->mask ? j->mask + (uint64_t)r * j->mw : NULL, j->u ? j->u[r] : 0.0f,
        &j->out_tokens[r],
        j->out_ids ? j->out_ids + (uint64_t)r * j->out_cap : NULL,
        j->out_probs ? j->out_probs + (uint64_t)r * j->out_cap : NULL,
        j->out_cap, &cnt);
    if (j->out_count) j->out_count[r] = cnt;
    if (s != 0) {
      j->out_tokens[r] = 0xffffffffu;
      if (j->status == 0) j->status = s;
    }
  }
  return NULL;
}

int llmk_oracle_sample_batch(int mode, const float* logits, uint32_t B,
                             uint32_t V, uint64_t row_stride,
                             const float* temperature, const int32_t* top_k,
                             const float* top_p, const float* min_p,
                             const float* repetition, const float* presence,
                             const float* frequency,
                             const uint32_t* hist_offsets,
                             const uint32_t* hist_tokens,
                             const uint32_t* mask, uint32_t mask_words,
                             const float* uniforms, uint32_t* out_tokens,
                             uint32_t* out_ids, float* out_probs,
                             uint32_t out_cap, uint32_t* out_count,
                             int nthreads) {
  if (V == 0 || B == 0) return -1;
  if (nthreads < 1) nthreads = 1;
  if ((uint32_t)nthreads > B) nthreads = (int)B;
  batch_job* jobs = (batch_job*)calloc((size_t)nthreads, sizeof(batch_job));
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  for (int t = 0; t < nthreads; ++t) {
    batch_job* j = &jobs[t];
    j->mode = mode;
    j->logits = logits;
    j->B = B;
    j->V = V;
    j->stride = row_stride;
    j->T = temperature;
    j->tk = top_k;
    j->tp = top_p;
    j->mp = min_p;
    j->rp = repetition;
    j->pp = presence;
    j->fp = frequency;
    j->ho = hist_offsets;
    j->ht = hist_tokens;
    j->mask = mask;
    j->mw = mask_words;
    j->u = uniforms;
    j->out_tokens = out_tokens;
    j->out_ids = out_ids;
    j->out_probs = out_probs;
    j->out_cap = out_cap;
    j->out_count = out_count;
    j->r0 = (uint32_t)(((uint64_t)B * t) / nthreads);
    j->r1 = (uint32_t)(((uint64_t)B * (t + 1)) / nthreads);
  }
  if (nthreads == 1) batch_worker(&jobs[0]);
  else {
    for (int t = 0; t < nthreads; ++t)
      pthread_create(&th[t], NULL, batch_worker, &jobs[t]);
    for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  }
  int status = 0;
  for (int t = 0; t < nthreads; ++t)
    if (jobs[t].status && !status) status = jobs[t].status;
  free(jobs);
  free(th);
  return status;
}

/* ------------------------------------------------------------------------ */
/* Mask-form helpers                                                         */
/* ------------------------------------------------------------------------ */

void llmk_oracle_apply_repetition_penalty(float* logits, uint32_t V,
                                          const uint32_t* hist, uint32_t H,
                                          float penalty) {
  apply_repetition(logits, V, hist, H, penalty);
}

void llmk_oracle_apply_temperature(float* logits, uint32_t V, float t) {
  apply_temperature(logits, V, t);
}

/* sampler.rs:160-173: threshold = k-th largest value; values below it are
 * masked, so ties at the threshold survive (more than k can remain). */
void llmk_oracle_apply_top_k(float* logits, uint32_t V, int64_t k) {
  if (k <= 0 || (uint64_t)k >= V) return;
  uint32_t* keys = (uint32_t*)malloc(sizeof(uint32_t) * V);
  for (uint32_t i = 0; i < V; ++i) {
    uint32_t b = f2u(logits[i]);
    keys[i] = (b & 0x80000000u) ? ~b : (b | 0x80000000u); /* ascending order key */
  }
  sort_u32(keys, V);
  uint32_t tk = keys[V - (uint32_t)k];
  uint32_t tb = (tk & 0x80000000u) ? (tk & 0x7fffffffu) : ~tk;
  float thr = u2f(tb);
  for (uint32_t i = 0; i < V; ++i)
    if (logits[i] < thr) logits[i] = -INFINITY;
  free(keys);
}

/* sampler.rs:176-216 */
void llmk_oracle_apply_top_p(int mode, float* logits, uint32_t V, float top_p) {
  if (top_p >= 1.0f || V == 0) return;
  float m = -INFINITY;
  for (uint32_t i = 0; i < V; ++i) m = fmaxf(m, logits[i]);
  float* e = (float*)malloc(sizeof(float) * V);
  for (uint32_t i = 0; i < V; ++i) {
    if (logits[i] == -INFINITY) e[i] = 0.0f;
    else if (mode == LLMK_ORACLE_MIRROR)  /* NaN acts as -inf, as on the GPU */
      e[i] = isnan(logits[i]) ? 0.0f : llmk_oracle_exp_ref(logits[i] - m);
    else
      e[i] = expf(logits[i] - m);
  }
  /* the sequential f32 sum in index order, :190 (top-k is off here) */
  float S = 0.0f;
  for (uint32_t i = 0; i < V; ++i) S += e[i];
  if (!(S > 0.0f)) {
    free(e);
    return;
  }
  for (uint32_t i = 0; i < V; ++i) e[i] = e[i] / S;
  uint64_t* keys = (uint64_t*)malloc(sizeof(uint64_t) * V);
  for (uint32_t i = 0; i < V; ++i) keys[i] = pkey(e[i], i);
  sort_u64(keys, V);
  float cum = 0.0f;
  uint32_t cut = V;
  for (uint32_t j = 0; j < V; ++j) {
    cum += u2f(~(uint32_t)(keys[j] >> 32));
    if (cum >= top_p) {
      cut = j + 1;
      break;
    }
  }
  unsigned char* keep = (unsigned char*)calloc(V, 1);
  for (uint32_t j = 0; j < cut; ++j) keep[keys[j] & 0xffffffffu] = 1;
  for (uint32_t i = 0; i < V; ++i)
    if (!keep[i]) logits[i] = -INFINITY;
  free(keep);
  free(keys);
  free(e);
}

uint32_t llmk_oracle_sample_simple(int mode, const float* logits, uint32_t V,
                                   float temperature, float u) {
  llmk_oracle_params p = {temperature, 0, 1.0f, 0.0f, 1.0f, 0.0f, 0.0f};
  uint32_t tok = 0, cnt = 0;
  if (llmk_oracle_sample_row(mode, logits, V, &p, NULL, 0, NULL, u, &tok, NULL,
                             NULL, 0, &cnt) != 0)
    return 0; /* sampler.rs:227 unwrap_or(0) */
  return tok;
}

/* ------------------------------------------------------------------------ */
/* final_logit_softcapping (candle.rs:1803-1807)                              */
/* ------------------------------------------------------------------------ */

static inline float f_bits(uint32_t b) {
  float x;
  memcpy(&x, &b, 4);
  return x;
}
static inline uint32_t bits_f(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  return b;
}

/* expm1 and tanh as glibc 2.35's expm1f / tanhf compute them (sysdeps/
 * ieee754/flt-32/s_expm1f.c, s_tanhf.c: Sun's fdlibm method in float, no
 * fused operations).  expm1: x = k ln2 + r, ln2 as a 16-bit head plus a
 * tail; k = +-1 between 0.5 ln2 and 1.5 ln2, else trunc(x/ln2 +- 1/2), the
 * reduction's rounding error carried in c; expm1(r) by fdlibm's rational form
 * with the quintic Q1..Q5 in r^2/2; 2^k (1 + expm1(r)) - 1 rebuilt per case
 * of k.  tanh: 1 - 2/(expm1(2|x|) + 2) from |x| = 1, -t/(t + 2) with
 * t = expm1(-2|x|) below, x(1 + x) below 2^-55, 1 from 22, sign last.
 * llmk_oracle_tanh_scan checks both against the host's functions. */
float llmk_oracle_expm1_ref(float x) {
  const float ln2_head = f_bits(0x3f317180u), ln2_tail = f_bits(0x3717f7d1u);
  const float inv_ln2 = f_bits(0x3fb8aa3bu);
  const float q1 = f_bits(0xbd088889u), q2 = f_bits(0x3ad00d01u), q3 = f_bits(0xb8a670cdu),
              q4 = f_bits(0x36867e54u), q5 = f_bits(0xb457edbbu);
  const uint32_t b = bits_f(x), mag = b & 0x7fffffffu;
  const int neg = (int)(b >> 31);
  if (mag >= 0x4195b844u) {
    if (mag >= 0x42b17218u) {
      if (mag > 0x7f800000u) return x + x;
      if (mag == 0x7f800000u) return neg ? -1.0f : x;
      if (x > f_bits(0x42b17180u)) return INFINITY;
    }
    if (neg) return -1.0f;
  }
  int k = 0;
  float c = 0.0f;
  if (mag > 0x3eb17218u) {
    float head, tail;
    if (mag < 0x3f851592u) {
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
  } else if (mag < 0x33000000u) {
    return x;
  }
  const float half_x = 0.5f * x, hx2 = x * half_x;
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
    return f_bits(bits_f(y) + ((uint32_t)k << 23)) - 1.0f;
  }
  if (k < 23) {
    t = f_bits(0x3f800000u - (0x1000000u >> k));
    y = t - (e - x);
  } else {
    t = f_bits((uint32_t)(0x7f - k) << 23);
    y = x - (e + t);
    y = y + 1.0f;
  }
  return f_bits(bits_f(y) + ((uint32_t)k << 23));
}

float llmk_oracle_tanh_ref(float x) {
  const uint32_t b = bits_f(x), mag = b & 0x7fffffffu;
  const int neg = (int)(b >> 31);
  if (mag >= 0x7f800000u) return neg ? 1.0f / x - 1.0f : 1.0f / x + 1.0f;
  float z;
  if (mag >= 0x41b00000u) {
    z = 1.0f;
  } else if (mag == 0) {
    return x;
  } else if (mag < 0x24000000u) {
    return x * (1.0f + x);
  } else if (mag >= 0x3f800000u) {
    const float t = llmk_oracle_expm1_ref(2.0f * fabsf(x));
    z = 1.0f - 2.0f / (t + 2.0f);
  } else {
    const float t = llmk_oracle_expm1_ref(-2.0f * fabsf(x));
    z = -t / (t + 2.0f);
  }
  return neg ? -z : z;
}

/* x rounded to nearest even into the dtype (0 f32, 1 bf16, 2 f16), as a
 * float: a 16-bit dtype keeps p = 8 or 11 significant bits, its subnormals a
 * fixed quantum, and overflows to infinity past its largest finite value. */
static double round_fmt(double x, int fmt) {
  if (fmt == 0) return (double)(float)x;
  if (x == 0.0 || isnan(x) || isinf(x)) return x;
  const int p = fmt == 1 ? 8 : 11, emin = fmt == 1 ? -126 : -14, emax = fmt == 1 ? 127 : 15;
  int e = 0;
  (void)frexp(x, &e);
  const int lead = e - 1 < emin ? emin : e - 1;
  const double quantum = ldexp(1.0, lead - p + 1);
  const double r = nearbyint(x / quantum) * quantum;
  const double maxf = ldexp(2.0 - ldexp(1.0, 1 - p), emax);
  if (fabs(r) > maxf) return r > 0 ? INFINITY : -INFINITY;
  return r;
}

/* candle.rs:1803-1807, (x / cap).tanh() * cap on the logits tensor, as
 * candle's CPU ops evaluate it: each scalar operation is the tensor's affine
 * map v * m + 0 with m = 1/cap or cap (an f64 made the dtype's value), tanh
 * is glibc's tanhf, and in a 16-bit dtype every operation rounds to it.
 * logits: the dtype's values as floats; rewritten in place. */
void llmk_oracle_softcap(int dtype, float* logits, uint32_t n, float cap) {
  const int fmt = dtype;
  const float m = (float)round_fmt(1.0 / (double)cap, fmt);
  const float c = (float)round_fmt((double)cap, fmt);
  for (uint32_t i = 0; i < n; ++i) {
    float y = (float)round_fmt((double)(logits[i] * m), fmt);
    y = (float)round_fmt((double)(y + 0.0f), fmt);
    float t = (float)round_fmt((double)llmk_oracle_tanh_ref(y), fmt);
    t = (float)round_fmt((double)(t * c), fmt);
    logits[i] = (float)round_fmt((double)(t + 0.0f), fmt);
  }
}

/* Every float bit pattern in [lo, hi]: mismatches of tanh_ref against the
 * host's tanhf and of expm1_ref against its expm1f (NaN results match any
 * NaN). */
void llmk_oracle_tanh_scan(uint32_t lo, uint32_t hi, uint64_t* n_tanh, uint64_t* n_expm1) {
  uint64_t a = 0, b = 0;
  for (uint64_t u = lo; u <= hi; ++u) {
    const float x = f_bits((uint32_t)u);
    const float r1 = tanhf(x), m1 = llmk_oracle_tanh_ref(x);
    if (bits_f(r1) != bits_f(m1) && !(isnan(r1) && isnan(m1))) ++a;
    const float r2 = expm1f(x), m2 = llmk_oracle_expm1_ref(x);
    if (bits_f(r2) != bits_f(m2) && !(isnan(r2) && isnan(m2))) ++b;
  }
  *n_tanh = a;
  *n_expm1 = b;
}

/* ------------------------------------------------------------------------ */
/* Speculative-decoding verification                                          */
/* ------------------------------------------------------------------------ */

/* One row of the verification docs/mlc-contracts.md:83-84 describes (the
 * reference leaves the hook, llm-core/src/backend.rs:20-22, and no
 * implementation), over the target's processed kept list (ids/probs in
 * (p desc, idx asc) order, n entries; p = 0 outside it) and the draft
 * distribution q[0..V): accept d iff u_a * q[d] < p(d); otherwise draw from
 * max(p - q, 0) with sampler.rs:113-124's loop over the residuals divided by
 * their sequential sum R, falling back to the last positive residual; R = 0
 * draws from p with the same loop.  Returns 1 (token LLMK_INVALID) for an
 * empty list or d >= V. */
int llmk_oracle_verify_row(uint32_t n, const uint32_t* ids, const float* probs,
                           uint32_t d, const float* q, uint32_t V, float u_a,
                           float u_r, uint32_t* tok, uint32_t* accepted) {
  *accepted = 0;
  if (n == 0 || d >= V) {
    *tok = 0xffffffffu;
    return 1;
  }
  float pd = 0.0f;
  for (uint32_t j = 0; j < n; ++j)
    if (ids[j] == d) pd = probs[j];
  if (u_a * q[d] < pd) {
    *tok = d;
    *accepted = 1;
    return 0;
  }
  float R = 0.0f;
  for (uint32_t j = 0; j < n; ++j) {
    const float r = probs[j] - (ids[j] < V ? q[ids[j]] : 0.0f);
    R += r > 0.0f ? r : 0.0f;
  }
  float c = 0.0f;
  if (R > 0.0f) {
    uint32_t last = 0;
    for (uint32_t j = 0; j < n; ++j) {
      float r = probs[j] - (ids[j] < V ? q[ids[j]] : 0.0f);
      r = r > 0.0f ? r : 0.0f;
      if (r > 0.0f) last = j;
      c += r / R;
      if (u_r <= c) {
        *tok = ids[j];
        return 0;
      }
    }
    *tok = ids[last];
    return 0;
  }
  for (uint32_t j = 0; j < n; ++j) {
    c += probs[j];
    if (u_r <= c) {
      *tok = ids[j];
      return 0;
    }
  }
  *tok = ids[n - 1];
  return 0;
}

/* ------------------------------------------------------------------------ */
/* exp_ref exhaustive scan                                                     */
/* ------------------------------------------------------------------------ */

void llmk_oracle_exp_scan(uint32_t lo_bits, uint32_t hi_bits,
                          uint64_t* n_checked, uint64_t* n_mismatch,
                          uint64_t* n_nonmono, uint32_t* max_ulp) {
  uint64_t chk = 0, mis = 0, nm = 0;
  uint32_t mu = 0;
  float prev = 0.0f;
  int have_prev = 0;
  for (uint64_t b = lo_bits; b <= hi_bits; ++b) {
    float y = u2f((uint32_t)b);
    float a = llmk_oracle_exp_ref(y);
    float r = expf(y);
    ++chk;
    if (f2u(a) != f2u(r)) {
      ++mis;
      uint32_t d = f2u(a) > f2u(r) ? f2u(a) - f2u(r) : f2u(r) - f2u(a);
      if (d > mu) mu = d;
    }
    /* bit patterns ascend in magnitude for negative floats: e^y must not grow */
    if (have_prev && a > prev) ++nm;
    prev = a;
    have_prev = 1;
  }
  *n_checked = chk;
  *n_mismatch = mis;
  *n_nonmono = nm;
  *max_ulp = mu;
}
