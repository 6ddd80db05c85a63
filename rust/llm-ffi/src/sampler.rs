//! The batched GPU sampler for C and Python callers that embed llm-rs
//! without its scheduler, in llm-ffi's style (lib.rs: opaque handles,
//! `#[no_mangle] extern "C"`, null / 0 sentinels for failure).  Built with
//! the `hip-sampler` feature.

use std::ffi::c_void;
use llm_kernel::hip_sampler::{HipSampler, LlmkSampleBatchArgs, LLMK_ERR_INVALID_ARGUMENT};

/// A sampler on `device` for batches up to `max_batch` rows of up to
/// `max_vocab` logits; null on failure.
#[no_mangle]
pub extern "C" fn llm_sampler_create(device: i32, max_batch: u32, max_vocab: u32) -> *mut c_void {
    match HipSampler::new(device, max_batch, max_vocab) {
        Ok(s) => Box::into_raw(Box::new(s)) as *mut c_void,
        Err(_) => std::ptr::null_mut(),
    }
}

/// One batched sampling step on `stream`: 0 on success, else the library's
/// error code.
/// # SAFETY: `sampler` from llm_sampler_create; `args` valid, its device
/// pointers alive until the stream reaches the call.
#[no_mangle]
pub unsafe extern "C" fn llm_sample_batch(sampler: *mut c_void, args: *const LlmkSampleBatchArgs,
                                          stream: *mut c_void) -> i32 {
    if sampler.is_null() || args.is_null() {
        return LLMK_ERR_INVALID_ARGUMENT;
    }
    let s = &*(sampler as *const HipSampler);
    match s.sample_batch(&*args, stream) {
        Ok(()) => 0,
        Err(e) => e.code,
    }
}

/// Speculative-decoding verification of one draft token per row (see
/// `HipSampler::verify_batch`): 0 on success, else the error code.
/// # SAFETY: as llm_sample_batch; every array is device memory.
#[no_mangle]
pub unsafe extern "C" fn llm_verify_batch(sampler: *mut c_void, batch: u32, vocab: u32,
                                          ids: *const u32, probs: *const f32, list_cap: u32,
                                          counts: *const u32, draft_tokens: *const u32,
                                          draft_probs: *const f32, draft_stride: u64,
                                          u_accept: *const f32, u_resample: *const f32,
                                          out_tokens: *mut u32, out_accepted: *mut u32,
                                          stream: *mut c_void) -> i32 {
    if sampler.is_null() {
        return LLMK_ERR_INVALID_ARGUMENT;
    }
    let s = &*(sampler as *const HipSampler);
    match s.verify_batch(batch, vocab, ids, probs, list_cap, counts, draft_tokens, draft_probs,
                         draft_stride, u_accept, u_resample, out_tokens, out_accepted, stream) {
        Ok(()) => 0,
        Err(e) => e.code,
    }
}

/// Reads and clears the status bits raised since the last read; 0 also
/// when the handle is null or the read fails.
/// # SAFETY: `sampler` from llm_sampler_create or null.
#[no_mangle]
pub unsafe extern "C" fn llm_sampler_status(sampler: *mut c_void, stream: *mut c_void) -> u32 {
    if sampler.is_null() {
        return 0;
    }
    let s = &*(sampler as *const HipSampler);
    s.status(stream).unwrap_or(0)
}

/// Frees a sampler from llm_sampler_create (null: nothing).
/// # SAFETY: `sampler` from llm_sampler_create, not used afterwards.
#[no_mangle]
pub unsafe extern "C" fn llm_sampler_destroy(sampler: *mut c_void) {
    if !sampler.is_null() {
        drop(Box::from_raw(sampler as *mut HipSampler));
    }
}
