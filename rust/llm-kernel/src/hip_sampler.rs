//! Binding of `libllmk_sampler.so`, the MI355X batched token sampler
//! (C ABI: `include/llmk_sampler.h`).
//!
//! One `HipSampler::sample_batch` call samples every row of a decode step on
//! the GPU, stream-ordered, in place of the scheduler's per-row loop
//! (llm-scheduler/src/scheduler.rs:138-145) over `LlmBackend::sample`
//! (llm-core/src/backend.rs:23-24) and `sample_logits`
//! (llm-core/src/sampler.rs:25-125).  Built only with the `hip-sampler`
//! feature, which also makes `build.rs` link the library.
//!
//! Every pointer handed to these calls is device memory (or, for the
//! handle-free calls, as documented) that stays valid until the HIP stream
//! reaches the call: the calls enqueue work and return.

use std::ffi::{c_void, CStr};
use std::os::raw::{c_char, c_int};

/// `llmk_dtype`: element type of the logits.
pub const LLMK_F32: i32 = 0;
pub const LLMK_BF16: i32 = 1;
pub const LLMK_F16: i32 = 2;

/// Return codes.
pub const LLMK_OK: i32 = 0;
pub const LLMK_ERR_INVALID_ARGUMENT: i32 = -1;
pub const LLMK_ERR_EMPTY_LOGITS: i32 = -2;
pub const LLMK_ERR_CAPACITY: i32 = -3;
pub const LLMK_ERR_HIP: i32 = -4;
pub const LLMK_ERR_ALIGNMENT: i32 = -5;
pub const LLMK_ERR_UNSUPPORTED: i32 = -6;

/// Token written for a row whose parameters are invalid.
pub const LLMK_INVALID_TOKEN: u32 = 0xffff_ffff;

/// Bits of the device status word (`HipSampler::status`).
pub const LLMK_STATUS_INVALID_PARAMS: u32 = 0x1;
pub const LLMK_STATUS_HISTORY_OVERFLOW: u32 = 0x2;
pub const LLMK_STATUS_SLOT_TIMEOUT: u32 = 0x4;
pub const LLMK_STATUS_HISTORY_FULL: u32 = 0x8;
pub const LLMK_STATUS_NAN_LOGITS: u32 = 0x10;

/// `llmk_sample_batch_args`, field for field.  Null pointers select the
/// `SampleParams` defaults (llm-core/src/types.rs:186-195) or switch the
/// optional inputs and outputs off.
#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct LlmkSampleBatchArgs {
    /// `[batch][row_stride]` f32, bf16 or f16; rows at any element offset.
    pub logits: *const c_void,
    pub dtype: i32,
    pub batch: u32,
    pub vocab: u32,
    /// Elements between the starts of consecutive rows.
    pub row_stride: u64,
    pub temperature: *const f32,
    pub top_k: *const i32,
    pub top_p: *const f32,
    pub min_p: *const f32,
    pub repetition_penalty: *const f32,
    pub presence_penalty: *const f32,
    pub frequency_penalty: *const f32,
    /// History as CSR: `hist_offsets[batch + 1]` into `hist_tokens`.
    pub hist_offsets: *const u32,
    pub hist_tokens: *const u32,
    /// `[batch][mask_words_per_row]`, token t allowed iff bit `t & 31` of
    /// word `t >> 5` is set.
    pub allow_mask: *const u32,
    pub mask_words_per_row: u32,
    /// One U[0, 1) per row, in place of `rand::thread_rng` (sampler.rs:113).
    pub uniforms: *const f32,
    pub out_tokens: *mut u32,
    pub out_ids: *mut u32,
    pub out_probs: *mut f32,
    pub out_cap: u32,
    pub out_count: *mut u32,
    /// Per-row history lengths (per-row buffers at `hist_offsets[b]`).
    pub hist_lengths: *const u32,
    /// `final_logit_softcapping` (candle.rs:1803-1807), 0 = off.
    pub softcap: f32,
    /// Occurrences per `hist_tokens` entry (count tables).
    pub hist_counts: *const u32,
}

impl Default for LlmkSampleBatchArgs {
    fn default() -> Self {
        let n = std::ptr::null::<f32>();
        let nu = std::ptr::null::<u32>();
        Self {
            logits: std::ptr::null(),
            dtype: LLMK_F32,
            batch: 0,
            vocab: 0,
            row_stride: 0,
            temperature: n,
            top_k: std::ptr::null(),
            top_p: n,
            min_p: n,
            repetition_penalty: n,
            presence_penalty: n,
            frequency_penalty: n,
            hist_offsets: nu,
            hist_tokens: nu,
            allow_mask: nu,
            mask_words_per_row: 0,
            uniforms: n,
            out_tokens: std::ptr::null_mut(),
            out_ids: std::ptr::null_mut(),
            out_probs: std::ptr::null_mut(),
            out_cap: 0,
            out_count: std::ptr::null_mut(),
            hist_lengths: nu,
            softcap: 0.0,
            hist_counts: nu,
        }
    }
}

/// The opaque `llmk_sampler`.
#[repr(C)]
pub struct LlmkSampler {
    _private: [u8; 0],
}

extern "C" {
    pub fn llmk_sampler_create(out: *mut *mut LlmkSampler, device: c_int, max_batch: u32,
                               max_vocab: u32) -> c_int;
    pub fn llmk_sample_batch(s: *mut LlmkSampler, args: *const LlmkSampleBatchArgs,
                             hip_stream: *mut c_void) -> c_int;
    pub fn llmk_sample_batch_static(args: *const LlmkSampleBatchArgs, status: *mut u32,
                                    hip_stream: *mut c_void) -> c_int;
    pub fn llmk_apply_top_k(s: *mut LlmkSampler, logits: *mut f32, batch: u32, vocab: u32,
                            row_stride: u64, top_k: *const i32, hip_stream: *mut c_void) -> c_int;
    pub fn llmk_apply_top_p(s: *mut LlmkSampler, logits: *mut f32, batch: u32, vocab: u32,
                            row_stride: u64, top_p: *const f32, hip_stream: *mut c_void) -> c_int;
    pub fn llmk_apply_logit_bias(s: *mut LlmkSampler, logits: *mut f32, batch: u32, vocab: u32,
                                 row_stride: u64, bias_offsets: *const u32,
                                 bias_tokens: *const u32, bias_values: *const f32,
                                 hip_stream: *mut c_void) -> c_int;
    pub fn llmk_history_append(s: *mut LlmkSampler, batch: u32, hist_offsets: *const u32,
                               hist_lengths: *mut u32, hist_tokens: *mut u32, capacity: u32,
                               tokens: *const u32, hip_stream: *mut c_void) -> c_int;
    pub fn llmk_history_count_append(s: *mut LlmkSampler, batch: u32, hist_offsets: *const u32,
                                     hist_lengths: *mut u32, hist_tokens: *mut u32,
                                     hist_counts: *mut u32, capacity: u32, tokens: *const u32,
                                     hip_stream: *mut c_void) -> c_int;
    pub fn llmk_verify_batch(s: *mut LlmkSampler, batch: u32, vocab: u32, ids: *const u32,
                             probs: *const f32, list_cap: u32, counts: *const u32,
                             draft_tokens: *const u32, draft_probs: *const f32,
                             draft_stride: u64, u_accept: *const f32, u_resample: *const f32,
                             out_tokens: *mut u32, out_accepted: *mut u32,
                             hip_stream: *mut c_void) -> c_int;
    pub fn llmk_sampler_status(s: *mut LlmkSampler, hip_stream: *mut c_void,
                               status: *mut u32) -> c_int;
    pub fn llmk_sampler_destroy(s: *mut LlmkSampler);
    pub fn llmk_last_error() -> *const c_char;
}

/// An error from the library: its return code and `llmk_last_error()`.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct LlmkError {
    pub code: i32,
    pub message: String,
}

impl std::fmt::Display for LlmkError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "llmk error {}: {}", self.code, self.message)
    }
}

impl std::error::Error for LlmkError {}

fn check(rc: c_int) -> Result<(), LlmkError> {
    if rc == LLMK_OK {
        return Ok(());
    }
    // SAFETY: llmk_last_error returns a NUL-terminated string owned by the
    // library's thread-local state, valid until the next call on this thread.
    let message = unsafe { CStr::from_ptr(llmk_last_error()) }.to_string_lossy().into_owned();
    Err(LlmkError { code: rc, message })
}

/// The sampler of one GPU: owns the device workspace sized for
/// `max_batch` rows of up to `max_vocab` logits.  One handle serves one
/// stream at a time (its calls are ordered by that stream).
pub struct HipSampler {
    raw: *mut LlmkSampler,
}

// The handle holds device memory and no thread-bound state.
unsafe impl Send for HipSampler {}

impl HipSampler {
    pub fn new(device: i32, max_batch: u32, max_vocab: u32) -> Result<Self, LlmkError> {
        let mut raw = std::ptr::null_mut();
        // SAFETY: `raw` is a valid out-pointer; the call allocates on `device`.
        check(unsafe { llmk_sampler_create(&mut raw, device, max_batch, max_vocab) })?;
        Ok(Self { raw })
    }

    /// Enqueues one batched sampling step on `stream` (a `hipStream_t`, null
    /// for the default stream).
    ///
    /// # Safety
    /// Every pointer in `args` is device memory of the documented shape that
    /// stays valid until `stream` reaches the call.
    pub unsafe fn sample_batch(&self, args: &LlmkSampleBatchArgs, stream: *mut c_void)
        -> Result<(), LlmkError> {
        check(llmk_sample_batch(self.raw, args, stream))
    }

    /// `apply_top_k` (sampler.rs:160-173) on `batch` device rows, in place.
    ///
    /// # Safety
    /// `logits` holds `batch` f32 rows of `row_stride` elements and `top_k`
    /// `batch` entries, on the device, valid until `stream` reaches the call.
    pub unsafe fn apply_top_k(&self, logits: *mut f32, batch: u32, vocab: u32, row_stride: u64,
                              top_k: *const i32, stream: *mut c_void) -> Result<(), LlmkError> {
        check(llmk_apply_top_k(self.raw, logits, batch, vocab, row_stride, top_k, stream))
    }

    /// `apply_top_p` (sampler.rs:176-216) on `batch` device rows, in place.
    ///
    /// # Safety
    /// As `apply_top_k`, with `top_p` for `top_k`.
    pub unsafe fn apply_top_p(&self, logits: *mut f32, batch: u32, vocab: u32, row_stride: u64,
                              top_p: *const f32, stream: *mut c_void) -> Result<(), LlmkError> {
        check(llmk_apply_top_p(self.raw, logits, batch, vocab, row_stride, top_p, stream))
    }

    /// `logits[t] += bias` per row from a device CSR of (token, bias) pairs.
    ///
    /// # Safety
    /// Device arrays: `bias_offsets[batch + 1]`, tokens and values as long as
    /// the last offset; valid until `stream` reaches the call.
    pub unsafe fn apply_logit_bias(&self, logits: *mut f32, batch: u32, vocab: u32,
                                   row_stride: u64, bias_offsets: *const u32,
                                   bias_tokens: *const u32, bias_values: *const f32,
                                   stream: *mut c_void) -> Result<(), LlmkError> {
        check(llmk_apply_logit_bias(self.raw, logits, batch, vocab, row_stride, bias_offsets,
                                    bias_tokens, bias_values, stream))
    }

    /// The scheduler's token push (scheduler.rs:147) on per-row device
    /// history buffers.
    ///
    /// # Safety
    /// Device arrays of `batch` rows (`capacity` tokens per row buffer).
    pub unsafe fn history_append(&self, batch: u32, hist_offsets: *const u32,
                                 hist_lengths: *mut u32, hist_tokens: *mut u32, capacity: u32,
                                 tokens: *const u32, stream: *mut c_void)
        -> Result<(), LlmkError> {
        check(llmk_history_append(self.raw, batch, hist_offsets, hist_lengths, hist_tokens,
                                  capacity, tokens, stream))
    }

    /// The same push on count tables (sorted distinct tokens + counts).
    ///
    /// # Safety
    /// As `history_append`, plus `hist_counts` shaped like `hist_tokens`.
    pub unsafe fn history_count_append(&self, batch: u32, hist_offsets: *const u32,
                                       hist_lengths: *mut u32, hist_tokens: *mut u32,
                                       hist_counts: *mut u32, capacity: u32,
                                       tokens: *const u32, stream: *mut c_void)
        -> Result<(), LlmkError> {
        check(llmk_history_count_append(self.raw, batch, hist_offsets, hist_lengths,
                                        hist_tokens, hist_counts, capacity, tokens, stream))
    }

    /// Speculative decoding: accept or resample one draft token per row
    /// against the kept lists `sample_batch` returned (`out_ids`,
    /// `out_probs`, `out_count` with `out_cap = list_cap`).
    ///
    /// # Safety
    /// Device arrays of `batch` rows as `llmk_verify_batch` documents.
    #[allow(clippy::too_many_arguments)]
    pub unsafe fn verify_batch(&self, batch: u32, vocab: u32, ids: *const u32,
                               probs: *const f32, list_cap: u32, counts: *const u32,
                               draft_tokens: *const u32, draft_probs: *const f32,
                               draft_stride: u64, u_accept: *const f32, u_resample: *const f32,
                               out_tokens: *mut u32, out_accepted: *mut u32,
                               stream: *mut c_void) -> Result<(), LlmkError> {
        check(llmk_verify_batch(self.raw, batch, vocab, ids, probs, list_cap, counts,
                                draft_tokens, draft_probs, draft_stride, u_accept, u_resample,
                                out_tokens, out_accepted, stream))
    }

    /// Reads and clears the device status word (`LLMK_STATUS_*` bits raised
    /// since the last read); synchronises `stream`.
    pub fn status(&self, stream: *mut c_void) -> Result<u32, LlmkError> {
        let mut s = 0u32;
        // SAFETY: the handle is live and `s` a valid out-pointer.
        check(unsafe { llmk_sampler_status(self.raw, stream, &mut s) })?;
        Ok(s)
    }

    /// The raw handle, for callers that pass it on through a C ABI.
    pub fn as_raw(&self) -> *mut LlmkSampler {
        self.raw
    }
}

impl Drop for HipSampler {
    fn drop(&mut self) {
        // SAFETY: `raw` came from llmk_sampler_create and is freed once.
        unsafe { llmk_sampler_destroy(self.raw) }
    }
}

/// `llmk_sample_batch` without a handle and without any allocation, for
/// code under HIP graph capture or loops that must not allocate: batch
/// <= 256, vocab <= 262144, rows 16-byte aligned; overlapping calls on one
/// GPU race.  `status` is an optional device `u32` the call ORs its bits
/// into.
///
/// # Safety
/// As `HipSampler::sample_batch`; `status` is null or device memory.
pub unsafe fn sample_batch_static(args: &LlmkSampleBatchArgs, status: *mut u32,
                                  stream: *mut c_void) -> Result<(), LlmkError> {
    check(llmk_sample_batch_static(args, status, stream))
}

/// `SampleParams::top_k` (a `usize`, types.rs:181) as the engine's `i32`:
/// values the engine cannot hold are above any vocabulary, which means off
/// (sampler.rs:80), as `i32::MAX` does.
pub fn top_k_as_i32(top_k: usize) -> i32 {
    i32::try_from(top_k).unwrap_or(i32::MAX)
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn args_layout_matches_the_c_header() {
        // offsetof/sizeof of llmk_sample_batch_args on x86_64 and aarch64
        assert_eq!(std::mem::size_of::<LlmkSampleBatchArgs>(), 192);
        assert_eq!(std::mem::align_of::<LlmkSampleBatchArgs>(), 8);
    }

    #[test]
    fn host_checks_run_without_a_device() {
        let args = LlmkSampleBatchArgs::default();
        let rc = unsafe { llmk_sample_batch(std::ptr::null_mut(), &args, std::ptr::null_mut()) };
        assert_eq!(rc, LLMK_ERR_INVALID_ARGUMENT);
        let err = HipSampler::new(0, 0, 1000).err().expect("max_batch 0 is refused");
        assert_eq!(err.code, LLMK_ERR_INVALID_ARGUMENT);
        assert!(err.message.contains("max_batch"));
        assert_eq!(top_k_as_i32(usize::MAX), i32::MAX);
        assert_eq!(top_k_as_i32(40), 40);
    }
}
