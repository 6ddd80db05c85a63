/*
 * llmk_oracle.h — CPU oracle for the llm-rs token-sampling path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline), never as the thing measured or shipped.  The
 * product path (llm-rs_amd/csrc) never links or calls it.
 *
 * Two modes, one code path:
 *
 *   LLMK_ORACLE_REF    — a line-by-line restatement of
 *                        llm-core/src/sampler.rs:25-125 (sample_logits) and its
 *                        helpers :128-228: glibc expf (what Rust's f32::exp
 *                        lowers to on Linux), sequential f32 sums in index /
 *                        sorted order, a full sort of (p, idx) pairs.
 *   LLMK_ORACLE_MIRROR — what the GPU engine computes, bit for bit.  It is
 *                        the same algorithm with the same glibc expf
 *                        (llmk_oracle_exp_ref restates it bit for bit), and
 *                        differs from REF in one place: on rows where top-k
 *                        renormalises (0 < top_k < V, sampler.rs:80-89) the
 *                        softmax normaliser S, which cancels there in exact
 *                        arithmetic, is first taken as 1, and that result is
 *                        kept when llmk_oracle_band_certain proves each of
 *                        its decisions to be REF's; otherwise the row is
 *                        computed as REF.  Tokens, kept counts and kept ids
 *                        are therefore REF's on every row; probabilities
 *                        differ only in their last bits on rows kept at
 *                        S = 1.  Every other row is computed exactly as REF
 *                        (NaN logits aside: mirror reads them as -inf).
 *
 * Both modes: ties in probability are ordered by index ascending (the
 * reference's sort_unstable_by leaves tie order unspecified, sampler.rs:77),
 * and the random draw takes a caller-supplied uniform u in [0,1) instead of
 * rand::thread_rng (sampler.rs:113-114).
 *
 * Extensions with no reference function (presence/frequency penalty, allow
 * bitmask, min-p) are applied in this order, which reduces to the reference
 * order when they are off:
 *   repetition (sampler.rs:128-147) -> presence/frequency
 *   (llm-tests/tests/mlc_parity.rs:1083 formula) -> allow-mask -> greedy
 *   (sampler.rs:40-50) -> temperature (:150-157) -> softmax (:56-71) -> sort
 *   (:77) -> min-p -> top-k (:80-89) -> top-p (:92-110) -> draw (:113-124).
 */
#ifndef LLMK_ORACLE_H
#define LLMK_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { LLMK_ORACLE_REF = 0, LLMK_ORACLE_MIRROR = 1 };

/* Per-row sampling knobs.  Mirrors llm-core/src/types.rs:176-196 (SampleParams)
 * plus the extension fields; defaults T=1, top_k=0, top_p=1, min_p=0,
 * repetition=1, presence=0, frequency=0 leave the logits untouched. */
typedef struct {
  float temperature;
  int32_t top_k;
  float top_p;
  float min_p;
  float repetition_penalty;
  float presence_penalty;
  float frequency_penalty;
} llmk_oracle_params;

/* One row.  mask: NULL or ceil(V/32) u32 words, LSB-first.  Returns 0, or -1
 * for V == 0 (sampler.rs:30-32 bails on empty logits), -2 for bad params.
 * out_ids / out_probs (may be NULL) receive the final kept list in
 * (p desc, idx asc) order, up to out_cap entries; *out_count its full length.
 * Greedy rows report one entry with probability 1. */
int llmk_oracle_sample_row(int mode, const float* logits, uint32_t V,
                           const llmk_oracle_params* p, const uint32_t* hist,
                           uint32_t H, const uint32_t* mask, float u,
                           uint32_t* out_token, uint32_t* out_ids,
                           float* out_probs, uint32_t out_cap,
                           uint32_t* out_count);

/* The penalised (repetition, presence/frequency) and masked logits of one
 * row, before the greedy check and temperature.  Returns 0, -1, -2 as above. */
int llmk_oracle_process_logits(int mode, const float* logits, uint32_t V,
                               const llmk_oracle_params* p,
                               const uint32_t* hist, uint32_t H,
                               const uint32_t* mask, float* out);

/* 1 when the decisions of llmk_oracle_semantics on a list of e = p with
 * S = 1 (min-p cut, top-k set and order, top-p cut, drawn token) are the
 * reference's for every normaliser S it can hold (p = fl(e / S), then its
 * renormalisations), 0 when one lies in the rounding band.  e_sorted[0..E)
 * in (p desc, idx asc) order, exact; entries past E (of full) are <= ptail. */
int llmk_oracle_band_certain(const float* e_sorted, const uint32_t* idx, uint32_t E,
                             uint32_t full, float ptail,
                             const llmk_oracle_params* prm, float u);
/* The first n entries (n <= V) of a row's list with S = 1 (e = exp_ref of
 * the processed logits over T, less their maximum) in (e desc, idx asc)
 * order.  Returns 0, -1, -2 as llmk_oracle_sample_row. */
int llmk_oracle_sorted_e(const float* logits, uint32_t V, const llmk_oracle_params* prm,
                         const uint32_t* hist, uint32_t H, const uint32_t* mask,
                         uint32_t n, float* e_out, uint32_t* idx_out);
/* The steps after the sort — min-p, top-k, top-p, draw — on a list already
 * in (p desc, idx asc) order (p_sorted[n], idx[n]).  Outputs as above. */
int llmk_oracle_semantics(const float* p_sorted, const uint32_t* idx, uint32_t n,
                          const llmk_oracle_params* p, float u,
                          uint32_t* out_token, uint32_t* out_ids,
                          float* out_probs, uint32_t out_cap,
                          uint32_t* out_count);

/* Batch over rows with nthreads host threads (rows split in contiguous
 * blocks).  Array arguments follow the device ABI layout: params as [B]
 * arrays (NULL = default), history as CSR (offsets[B+1], tokens), mask as
 * [B][mask_words] (NULL = none).  out_ids/out_probs are [B][out_cap]. */
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
                             int nthreads);

/* Mask-form helpers, in place on one row (sampler.rs:128-216). */
void llmk_oracle_apply_repetition_penalty(float* logits, uint32_t V,
                                          const uint32_t* hist, uint32_t H,
                                          float penalty);
void llmk_oracle_apply_temperature(float* logits, uint32_t V, float t);
void llmk_oracle_apply_top_k(float* logits, uint32_t V, int64_t k);
void llmk_oracle_apply_top_p(int mode, float* logits, uint32_t V, float top_p);
/* sampler.rs:219-228 `sample(logits, t)` with the draw's uniform supplied. */
uint32_t llmk_oracle_sample_simple(int mode, const float* logits, uint32_t V,
                                   float temperature, float u);

/* final_logit_softcapping (candle.rs:1803-1807) as candle's CPU ops evaluate
 * it in the logits' dtype (0 f32, 1 bf16, 2 f16; values as floats), in
 * place; and the glibc-exact tanhf / expm1f it uses, with an exhaustive
 * comparison against the host's. */
void llmk_oracle_softcap(int dtype, float* logits, uint32_t n, float cap);
float llmk_oracle_tanh_ref(float x);
float llmk_oracle_expm1_ref(float x);
void llmk_oracle_tanh_scan(uint32_t lo, uint32_t hi, uint64_t* n_tanh, uint64_t* n_expm1);

/* Speculative-decoding verification of one row (docs/mlc-contracts.md:
 * 83-84) over the target's kept list and the draft distribution q[0..V). */
int llmk_oracle_verify_row(uint32_t n, const uint32_t* ids, const float* probs,
                           uint32_t d, const float* q, uint32_t V, float u_a,
                           float u_r, uint32_t* tok, uint32_t* accepted);

/* Numerics. */
/* e^x exactly as glibc's expf (>= 2.28, x86-64 FMA build) computes it, for
 * x <= 0 (-inf and x < -0x1.9fe368p6 give +0). */
float llmk_oracle_exp_ref(float x);
float llmk_oracle_libm_expf(float y); /* the host's expf, for comparisons */

/* Exhaustive check of exp_ref over the float bit patterns [lo, hi] of
 * non-positive inputs (sign bit set, ascending magnitude): counts inputs
 * where exp_ref differs from the host's expf, and adjacent pairs where it is
 * not monotone.  max_ulp receives the largest difference in ulps. */
void llmk_oracle_exp_scan(uint32_t lo_bits, uint32_t hi_bits,
                          uint64_t* n_checked, uint64_t* n_mismatch,
                          uint64_t* n_nonmono, uint32_t* max_ulp);

#ifdef __cplusplus
}
#endif
#endif
