//! `send_request` with every sampling knob.  `ChatRequest` and
//! `send_request` (lib.rs) stay as they are for existing C callers, which
//! pass the struct by value; a caller that wants top-k, the penalties,
//! min-p, a seed or a logit bias fills `ChatRequestV2` instead.

use std::ffi::CStr;
use std::os::raw::c_char;

use libc::c_void;
use llm_core::types::{InferRequest, SampleParams};

use crate::FfiEngineContext;

#[repr(C)]
pub struct ChatRequestV2 {
    pub prompt: *const c_char,
    pub temperature: f32,
    pub top_p: f32,
    pub max_tokens: usize,
    /// 40 reproduces send_request's fixed value; 0 = off.
    pub top_k: usize,
    /// 1.1 reproduces send_request's fixed value; 1.0 = off.
    pub repetition_penalty: f32,
    /// `l -= presence + count * frequency` for tokens already generated.
    pub presence_penalty: f32,
    pub frequency_penalty: f32,
    /// Keep tokens with p >= min_p * p_max; 0 = off.
    pub min_p: f32,
    /// The request's uniforms come from a generator seeded with `seed` when
    /// `has_seed` is set.
    pub seed: u64,
    pub has_seed: bool,
    /// `logit_bias_len` pairs (token id, bias) added to the logits; the
    /// arrays may be null when the length is 0.
    pub logit_bias_tokens: *const u32,
    pub logit_bias_values: *const f32,
    pub logit_bias_len: usize,
}

impl ChatRequestV2 {
    /// # Safety
    /// The logit-bias arrays hold `logit_bias_len` entries (or the length is 0).
    unsafe fn sample_params(&self) -> SampleParams {
        let logit_bias = if self.logit_bias_len == 0
            || self.logit_bias_tokens.is_null()
            || self.logit_bias_values.is_null()
        {
            Vec::new()
        } else {
            let toks = std::slice::from_raw_parts(self.logit_bias_tokens, self.logit_bias_len);
            let vals = std::slice::from_raw_parts(self.logit_bias_values, self.logit_bias_len);
            toks.iter().copied().zip(vals.iter().copied()).collect()
        };
        SampleParams {
            temperature: self.temperature,
            top_p: self.top_p,
            top_k: self.top_k,
            repetition_penalty: self.repetition_penalty,
            max_new_tokens: self.max_tokens,
            presence_penalty: self.presence_penalty,
            frequency_penalty: self.frequency_penalty,
            min_p: self.min_p,
            seed: if self.has_seed { Some(self.seed) } else { None },
            logit_bias,
        }
    }
}

/// Queue a generation request; returns its sequence id, 0 on failure.
/// # SAFETY: `engine` from create_engine; `request.prompt` a valid
/// NUL-terminated string; the logit-bias arrays as documented.
#[no_mangle]
pub unsafe extern "C" fn send_request_v2(engine: *mut c_void, request: ChatRequestV2) -> u64 {
    if engine.is_null() || request.prompt.is_null() {
        return 0;
    }
    let prompt = match CStr::from_ptr(request.prompt).to_str() {
        Ok(p) => p,
        Err(_) => return 0,
    };
    let context = &mut *(engine as *mut FfiEngineContext);
    let seq_id = rand::random::<u64>();
    let infer_req = InferRequest {
        seq_id,
        // the same character-level stand-in tokenisation as send_request
        prompt_tokens: prompt.chars().map(u32::from).collect(),
        sample_params: request.sample_params(),
        max_new_tokens: request.max_tokens,
    };
    match context.engine.add_request(infer_req) {
        Ok(_) => seq_id,
        Err(_) => 0,
    }
}
