/*
 * llmk_sampler.h — C ABI of the MI355X batched token-sampling engine for
 * llm-rs.  One call samples a whole batch on one GPU, asynchronously on a HIP
 * stream, and replaces the per-row host loop of
 *   llm-scheduler/src/scheduler.rs:138-145  (for each row: backend.sample(..))
 * whose body is
 *   llm-core/src/backend.rs:23-24           (LlmBackend::sample)
 *   llm-core/src/backends/candle.rs:2033-2035 (CandleBackend::sample)
 *   llm-core/src/sampler.rs:25-125          (sample_logits).
 *
 * Conventions follow llm-ffi/src/lib.rs: plain `extern "C"` symbols, an opaque
 * handle with explicit create/destroy (lib.rs:38-84), `#[repr(C)]`-compatible
 * structs (lib.rs:10-29).  Unlike llm-ffi's null/0 sentinels, every call
 * returns a status code (0 = success, negative = error) and
 * llmk_last_error() gives the message for the calling thread.
 *
 * Semantics per row (identical to sampler.rs when the extension fields are
 * at their defaults): repetition penalty (sampler.rs:128-147) -> presence and
 * frequency penalty -> allow-bitmask -> greedy if temperature <= 1e-5
 * (sampler.rs:40-50) -> temperature (sampler.rs:150-157) -> softmax
 * (sampler.rs:56-71) -> order by (probability desc, index asc) (sampler.rs:77)
 * -> min-p -> top-k (sampler.rs:80-89) -> top-p (sampler.rs:92-110) -> draw
 * with the caller's uniform (sampler.rs:113-124).
 *
 * Memory: every pointer in llmk_sample_batch_args is DEVICE memory owned by
 * the caller and must stay valid until the stream reaches the call.
 */
#ifndef LLMK_SAMPLER_H
#define LLMK_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLMK_OK 0
#define LLMK_ERR_INVALID_ARGUMENT (-1)
#define LLMK_ERR_EMPTY_LOGITS (-2) /* sampler.rs:30-32 "Empty logits" */
#define LLMK_ERR_CAPACITY (-3)     /* batch/vocab above the handle's maxima */
#define LLMK_ERR_HIP (-4)
#define LLMK_ERR_ALIGNMENT (-5)
#define LLMK_ERR_UNSUPPORTED (-6)

/* Token written for a row whose parameters are invalid (NaN temperature,
 * negative top_k, non-finite penalties, ...). */
#define LLMK_INVALID_TOKEN 0xffffffffu

/* Bits of the device status word (llmk_sampler_status). */
#define LLMK_STATUS_INVALID_PARAMS 0x1u
/* More than 8192 distinct history tokens fell in one vocabulary segment of a
 * row (the fast path's LDS tables): the row was sampled by the slow path over
 * its materialised logits, every history token penalised by its count.  The
 * result is exact; the bit reports only that the row took the slower path. */
#define LLMK_STATUS_HISTORY_OVERFLOW 0x2u
#define LLMK_STATUS_SLOT_TIMEOUT 0x4u /* slow-path scratch slot not acquired */
/* llmk_history_append found a row's history buffer full (its token was not
 * appended). */
#define LLMK_STATUS_HISTORY_FULL 0x8u
/* A sampling row held a logit that makes the reference's probabilities NaN
 * (NaN itself, or +inf: l - max = inf - inf), outside the allow-mask's
 * disallowed tokens: the device analogue of sampler.rs's NAN_WARNED
 * warn-once flag (sampler.rs:7-9, :74-76).  The engine reads NaN as -inf
 * and samples on; results for such rows are outside the parity contract. */
#define LLMK_STATUS_NAN_LOGITS 0x10u

typedef struct llmk_sampler llmk_sampler; /* opaque; owns device workspace */

/* Logit element types.  bf16 and f16 (IEEE half, the lm_head output of
 * half-precision models) are converted exactly to f32 as they are read, as
 * candle's to_dtype(F32) does before sampling (candle.rs:2007-2010). */
typedef enum { LLMK_F32 = 0, LLMK_BF16 = 1, LLMK_F16 = 2 } llmk_dtype;

typedef struct {
  /* logits[b * row_stride + v], v < vocab; row_stride in elements, rows at
   * any element offset.  Rows that do not start 16-byte aligned (fp32:
   * row_stride not a multiple of 4, bf16 and f16: not of 8, or a base
   * address off 16 bytes) are first copied to aligned rows in the handle's
   * staging buffer, which llmk_sample_batch allocates (once, and again when
   * a call needs more); llmk_sample_batch_static, which allocates nothing,
   * returns LLMK_ERR_ALIGNMENT for them. */
  const void* logits;
  int32_t dtype; /* llmk_dtype */
  uint32_t batch;
  uint32_t vocab;
  uint64_t row_stride;
  /* Per-row parameters, [batch] each; NULL = the SampleParams default
   * (llm-core/src/types.rs:186-195): temperature 1, top_k 0 (off), top_p 1,
   * repetition 1; extensions: min_p 0, presence 0, frequency 0. */
  const float* temperature;
  const int32_t* top_k;
  const float* top_p;
  const float* min_p;
  const float* repetition_penalty;
  const float* presence_penalty;
  const float* frequency_penalty;
  /* Token history as CSR: hist_offsets[batch+1], hist_tokens[...].  NULL =
   * empty histories.  Ids >= vocab are ignored (sampler.rs:138). */
  const uint32_t* hist_offsets;
  const uint32_t* hist_tokens;
  /* Grammar allow-bitmask, [batch][mask_words_per_row] u32, LSB-first (token
   * t allowed iff bit t&31 of word t>>5 is set); NULL = everything allowed. */
  const uint32_t* allow_mask;
  uint32_t mask_words_per_row;
  /* One uniform in [0,1) per row; replaces rand::thread_rng (sampler.rs:113). */
  const float* uniforms;
  uint32_t* out_tokens; /* [batch] */
  /* Optional processed distribution: the kept candidates after top-p
   * renormalisation, in (p desc, idx asc) order, [batch][out_cap] each; and
   * the kept count per row.  NULL / out_cap 0 = not requested. */
  uint32_t* out_ids;
  float* out_probs;
  uint32_t out_cap;
  uint32_t* out_count;
  /* Optional, [batch]: row b's history is hist_tokens[hist_offsets[b] ..
   * hist_offsets[b] + hist_lengths[b]) (hist_offsets then needs [batch]
   * entries).  This lets the history live in per-row buffers with room to
   * grow, appended to on the device by llmk_history_append.  NULL = CSR. */
  const uint32_t* hist_lengths;
  /* final_logit_softcapping (candle.rs:1803-1807, models whose metadata sets
   * it, candle.rs:606): > 0 = the logits are the lm_head output before the
   * cap, and each is read as cap * tanh(l / cap) evaluated as candle's CPU
   * ops do in the logits' dtype (l * (1/cap) + 0, glibc's tanhf, * cap + 0,
   * each rounded to the dtype); 0 = off.  Fused into the sampling pass: the
   * capped logits are never written. */
  float softcap;
  /* Optional: the count-table form of the history (the per-row counts the
   * scheduler's token push, scheduler.rs:147, accumulates), indexed like
   * hist_tokens: entry i stands for hist_counts[i] occurrences of token
   * hist_tokens[i] (0 is read as 1).  Penalties are those of the history that
   * lists each token that many times (sampler.rs:128-147; the frequency
   * penalty's count).  Entries may come in any order; a token listed twice
   * has the sum of its counts.  llmk_history_count_append keeps such tables
   * sorted and distinct on the device, so a step reads each distinct token
   * once instead of every occurrence.  NULL = one occurrence per entry. */
  const uint32_t* hist_counts;
} llmk_sample_batch_args;

/* Create a sampler on `device` able to serve batches up to max_batch rows of
 * up to max_vocab logits; all device workspace is allocated here.
 * Replaces nothing in the reference (its sampler keeps no state). */
int llmk_sampler_create(llmk_sampler** out, int device, uint32_t max_batch,
                        uint32_t max_vocab);

/* Sample every row of the batch; enqueued on `hip_stream` (a hipStream_t, NULL
 * = default stream) and returns without waiting.  Allocates nothing.
 * Replaces the per-row loop scheduler.rs:138-145 over sampler.rs:25-125.
 * One handle serves one stream at a time (calls on a handle are serialised
 * by stream order; concurrent calls on two streams race on the workspace). */
int llmk_sample_batch(llmk_sampler* s, const llmk_sample_batch_args* args,
                      void* hip_stream);

/* llmk_sample_batch with no handle and no allocation of any kind.  It has no
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, semantics and results as
 * llmk_sample_batch, on the current device; its workspace is a static
 * device array of 108 MiB that each GPU the library runs on holds
 * until the process ends, sized for batch <= 256 and vocab <= 262144 (larger
 * calls fail with LLMK_ERR_CAPACITY).  `status`: optional device u32 into
 * which the call ORs its LLMK_STATUS_* bits (the caller clears it); NULL =
 * the bits are dropped.  Every call on one GPU shares that workspace: calls
 * that overlap on one GPU (two streams, or two threads) race and give wrong
 * results; calls in one stream's order are safe. */
int llmk_sample_batch_static(const llmk_sample_batch_args* args, uint32_t* status,
                             void* hip_stream);

/* Mask-form top-k, batched and in place: replaces apply_top_k
 * (llm-core/src/sampler.rs:160-173) called on each row.  In row b every
 * logit below the top_k[b]-th largest value becomes -inf; values equal to
 * that threshold stay, so more than top_k[b] can remain.  Rows with
 * top_k[b] <= 0 or >= vocab are left as they are (sampler.rs:161-163).
 * logits: device f32 [batch][row_stride] (the reference's &mut [f32]; any
 * stride, no alignment beyond the f32 one); top_k: device [batch].  Enqueued on hip_stream;
 * allocates nothing; uses no workspace of the handle. */
int llmk_apply_top_k(llmk_sampler* s, float* logits, uint32_t batch, uint32_t vocab,
                     uint64_t row_stride, const int32_t* top_k, void* hip_stream);

/* Mask-form top-p, batched and in place: replaces apply_top_p
 * (llm-core/src/sampler.rs:176-216) called on each row.  Softmax of the row,
 * order by (probability desc, index asc), keep the shortest prefix whose
 * sequential f32 running sum reaches top_p[b], set every other logit to
 * -inf.  Rows with top_p[b] >= 1 or NaN, or whose probabilities sum to 0
 * (every logit -inf), are left as they are.  The probabilities are those of
 * llmk_sample_batch at temperature 1 (the same exp and normaliser), and the
 * kept set is what llmk_sample_batch keeps with that top_p alone.  f32 rows
 * at any element offset and stride; batch and vocab within the handle's
 * maxima; uses the handle's workspace (stream order, like
 * llmk_sample_batch).  Allocates nothing, except that rows not starting
 * 16-byte aligned are read through the handle's staging buffer, allocated
 * as llmk_sample_batch does. */
int llmk_apply_top_p(llmk_sampler* s, float* logits, uint32_t batch, uint32_t vocab,
                     uint64_t row_stride, const float* top_p, void* hip_stream);

/* Logit bias (the OpenAI logit_bias map), batched and in place: no
 * function of the reference has it; its formula is the one its test
 * llm-tests/tests/mlc_parity.rs:1060-1072 applies, logits[idx] += bias (f32).
 * Row b's pairs are bias_tokens[j], bias_values[j] for j in
 * [bias_offsets[b], bias_offsets[b+1]) (device CSR, like the history); ids
 * >= vocab are ignored.  The tokens of a row are the keys of a map: a token
 * listed twice gets both biases in an unspecified order.  Run it before
 * llmk_sample_batch on the same stream.  logits: device f32
 * [batch][row_stride], any stride.  Allocates nothing. */
int llmk_apply_logit_bias(llmk_sampler* s, float* logits, uint32_t batch, uint32_t vocab,
                          uint64_t row_stride, const uint32_t* bias_offsets,
                          const uint32_t* bias_tokens, const float* bias_values,
                          void* hip_stream);

/* Appends each row's sampled token to its device-resident history, as the
 * scheduler pushes it (llm-scheduler/src/scheduler.rs:147):
 * hist_tokens[hist_offsets[b] + hist_lengths[b]] = tokens[b] and
 * hist_lengths[b] += 1, for rows whose token is not LLMK_INVALID_TOKEN.  A
 * row already holding `capacity` tokens is left as it is and raises
 * LLMK_STATUS_HISTORY_FULL.  With hist_lengths in llmk_sample_batch_args
 * the next step then reads the grown histories without a host round trip.
 * Enqueued on hip_stream; allocates nothing. */
int llmk_history_append(llmk_sampler* s, uint32_t batch, const uint32_t* hist_offsets,
                        uint32_t* hist_lengths, uint32_t* hist_tokens, uint32_t capacity,
                        const uint32_t* tokens, void* hip_stream);

/* The token push of scheduler.rs:147 on a count-table history: row b's
 * entries hist_tokens/hist_counts[hist_offsets[b] .. + hist_lengths[b]) hold
 * its distinct tokens in ascending order with their occurrences.  A token
 * already listed gets count + 1; a new token is inserted in order with count
 * 1 (hist_lengths[b] += 1), or, when the row already holds `capacity`
 * entries, the row is left as it is and LLMK_STATUS_HISTORY_FULL is raised.
 * Rows whose token is LLMK_INVALID_TOKEN are left as they are.  Pass the same
 * arrays as hist_offsets / hist_tokens / hist_lengths / hist_counts of
 * llmk_sample_batch_args.  Enqueued on hip_stream; allocates nothing. */
int llmk_history_count_append(llmk_sampler* s, uint32_t batch, const uint32_t* hist_offsets,
                              uint32_t* hist_lengths, uint32_t* hist_tokens,
                              uint32_t* hist_counts, uint32_t capacity,
                              const uint32_t* tokens, void* hip_stream);

/* Speculative-decoding verification, batched: the residual resampling that
 * docs/mlc-contracts.md:83-84 describes (BatchVerifyDraftTokensWithProb-
 * AfterTopP) at the hook the reference leaves for it (llm-core/src/
 * backend.rs:20-22, "so the scheduler can apply speculative decoding"); the
 * reference itself has no implementation.  Row b verifies draft token
 * draft_tokens[b] against the target distribution p that llmk_sample_batch
 * returned for the row: its kept list ids/probs[b * list_cap ..] (in
 * (p desc, idx asc) order) and counts[b], i.e. out_ids/out_probs/out_count
 * with out_cap = list_cap; p is 0 outside the list.  draft_probs[b *
 * draft_stride + t] is the draft model's probability of token t (an id >= vocab
 * in a list, which the sampler never writes, reads q = 0).
 *   accept iff u_accept[b] * q(d) < p(d)  (the contract's reject when
 *   r >= p/q): out_tokens[b] = d, out_accepted[b] = 1;
 *   else out_accepted[b] = 0 and out_tokens[b] is drawn from the residual
 *   max(p - q, 0) over the kept list (one f32 subtraction each): R = its
 *   sequential f32 sum in list order; the first entry whose running sum of
 *   residual/R reaches u_resample[b] (the reference's `r <= cumulative`,
 *   sampler.rs:113-124), else the last entry with a positive residual; when
 *   R = 0, the same draw over p itself.
 * A chain of k draft tokens is k rows, one per position; the caller keeps
 * the accepted prefix and the first resampled token.  A row whose count is 0
 * or above list_cap (the list was cut) or whose draft token is >= vocab gets
 * LLMK_INVALID_TOKEN and raises LLMK_STATUS_INVALID_PARAMS.  Device arrays;
 * enqueued on hip_stream; allocates nothing. */
int llmk_verify_batch(llmk_sampler* s, uint32_t batch, uint32_t vocab, const uint32_t* ids,
                      const float* probs, uint32_t list_cap, const uint32_t* counts,
                      const uint32_t* draft_tokens, const float* draft_probs,
                      uint64_t draft_stride, const float* u_accept, const float* u_resample,
                      uint32_t* out_tokens, uint32_t* out_accepted, void* hip_stream);

/* Reads and clears the device status word (OR of LLMK_STATUS_* bits raised by
 * calls since the last read).  Synchronises `hip_stream`. */
int llmk_sampler_status(llmk_sampler* s, void* hip_stream, uint32_t* status);

void llmk_sampler_destroy(llmk_sampler* s);

/* Message of the last error on the calling thread ("" if none). */
const char* llmk_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
