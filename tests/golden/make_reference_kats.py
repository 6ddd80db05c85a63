"""Writes reference_kats.json: the known-answer vectors of the reference's own
sampler tests, transcribed as data (inputs and expected outputs) with the
file:line of the test each comes from.  The reference is Rust and cannot be
built here, so its tests are not run; their literal vectors are the fixture.

  python tests/golden/make_reference_kats.py
"""
import json
import math
import os

import numpy as np

f32 = np.float32

T = "llm-tests/tests/mlc_test.rs"
P = "llm-tests/tests/mlc_parity.rs"

KATS = [
    # sampler::sample(logits, 0.0) == argmax (sampler.rs:219-228, :40-50)
    dict(name="greedy_argmax", src=f"{T}:630-635", op="sample_simple",
         logits=[0.1, 0.5, 3.0, 0.2], temperature=0.0, expect_token=2),
    dict(name="greedy_index_zero", src=f"{T}:637-642", op="sample_simple",
         logits=[10.0, 1.0, 0.5], temperature=0.0, expect_token=0),
    dict(name="temperature_zero_is_greedy", src=f"{T}:644-649", op="sample_simple",
         logits=[1.0, 2.0, 5.0, 0.5], temperature=0.0, expect_token=2),
    # LlmBackend::sample contract: argmax for a deterministic backend
    dict(name="backend_sample_argmax", src="llm-tests/tests/mlc_test.rs:877-883", op="sample_simple",
         logits=[0.1, 5.0, 0.3, 0.2], temperature=0.0, expect_token=1),
    # apply_repetition_penalty (sampler.rs:128-147)
    dict(name="repetition_positive", src=f"{T}:651-661", op="repetition",
         logits=[0.0, 1.0, 2.0, 0.0], history=[2], penalty=2.0,
         expect=[0.0, 1.0, 1.0, 0.0], tol=1e-5),
    dict(name="repetition_negative", src=f"{T}:663-670", op="repetition",
         logits=[0.0, -2.0, 0.0], history=[1], penalty=2.0,
         expect=[0.0, -4.0, 0.0], tol=1e-5),
    dict(name="repetition_no_history", src=f"{T}:672-677", op="repetition",
         logits=[1.0, 2.0, 3.0], history=[], penalty=1.5,
         expect=[1.0, 2.0, 3.0], tol=1e-5),
    # apply_temperature (sampler.rs:150-157)
    dict(name="temperature_halves", src=f"{T}:679-684", op="temperature",
         logits=[2.0, 4.0, 6.0], t=2.0, expect=[1.0, 2.0, 3.0], tol=1e-5),
    dict(name="temperature_one_noop", src=f"{T}:686-692", op="temperature",
         logits=[1.5, 0.3, -0.7], t=1.0, expect=[1.5, 0.3, -0.7], tol=1e-5),
    dict(name="temperature_half_exact", src=f"{P}:1036-1044", op="temperature",
         logits=[1.0, 2.0, 3.0], t=0.5, expect=[2.0, 4.0, 6.0], tol=0.0),
    # apply_top_k (sampler.rs:160-173)
    dict(name="top_k_three", src=f"{T}:694-707", op="top_k",
         logits=[1.0, 5.0, 3.0, 2.0, 4.0], k=3, expect_finite=[1, 2, 4], expect_masked=[0, 3]),
    dict(name="top_k_zero_noop", src=f"{T}:709-714", op="top_k",
         logits=[1.0, 2.0, 3.0], k=0, expect=[1.0, 2.0, 3.0], tol=1e-5),
    # apply_top_p (sampler.rs:176-216)
    dict(name="top_p_dominant", src=f"{T}:716-725", op="top_p",
         logits=[10.0, 0.0, 0.0, 0.0], top_p=0.85, expect_finite=[0], min_masked=2),
    dict(name="top_p_one_keeps_all", src=f"{T}:727-741", op="top_p",
         logits=[1.0, 2.0, 3.0], top_p=1.0, expect_finite=[0, 1, 2], min_masked=0),
    # softmax properties (sampler.rs:56-71)
    dict(name="softmax_sums_to_one", src=f"{T}:743-749", op="softmax",
         logits=[1.0, 2.0, 3.0, 0.0, -1.0], sum_tol=1e-5),
    dict(name="softmax_non_negative", src=f"{T}:751-758", op="softmax",
         logits=[-5.0, -1.0, 0.0, 3.0, 10.0], sum_tol=1e-5),
    dict(name="softmax_two_stage_max", src=f"{T}:1412-1417", op="softmax",
         logits=[1.0, 4.0, 2.0, -1.0], sum_tol=1e-6, expect_argmax=1),
    dict(name="softmax_sum_1e6", src=f"{T}:1419-1425", op="softmax",
         logits=[1.0, 4.0, 2.0, -1.0], sum_tol=1e-6),
    dict(name="softmax_largest_prob", src=f"{T}:1427-1435", op="softmax",
         logits=[1.0, 4.0, 2.0, -1.0], sum_tol=1e-6, expect_argmax=1),
    dict(name="softmax_mlc_hf_match", src=f"{P}:669-679", op="softmax",
         logits=[1.2, -0.4, 2.5, 0.0], sum_tol=1e-6, fp64_tol=1e-6),
    dict(name="softmax_two_stage", src=f"{P}:1705-1716", op="softmax",
         logits=[1.0, 2.0, 3.0], sum_tol=1e-5),
    # top-p renormalisation (sampler.rs:92-110): p = [.05,.15,.30,.50], 0.8 keeps {3, 2}
    dict(name="top_p_renormalised", src=f"{T}:1437-1459", op="top_p_probs",
         probs=[0.05, 0.15, 0.30, 0.50], top_p=0.8, expect_ids=[3, 2], sum_tol=1e-5),
    # presence / frequency (extension formula): count 2 -> 2 - (0.5 + 2*0.2), count 0 unchanged
    dict(name="presence_frequency", src=f"{P}:1074-1089", op="presence_frequency",
         logits=[2.0, 2.0], history=[0, 0], presence=0.5, frequency=0.2,
         # the test's assert_eq!(logits[0], 2.0 - (0.5 + 0.4)), evaluated in f32
         expect=[float(f32(2.0) - (f32(0.5) + f32(0.4))), 2.0], tol=0.0),
    # the same formula, logits[i] -= presence + (count as f32 * freq), on
    # inputs where its f32 evaluation order is visible: (l - p) - c*f differs
    dict(name="presence_frequency_f32_order", src=f"{P}:1083 (formula, new inputs)",
         op="presence_frequency",
         logits=[3.7883238792419434, 0.5029208660125732, 1.0], history=[0, 0, 1],
         presence=1.09, frequency=0.94,
         expect=[float(f32(3.7883238792419434) - (f32(1.09) + f32(2) * f32(0.94))),
                 float(f32(0.5029208660125732) - (f32(1.09) + f32(1) * f32(0.94))), 1.0],
         tol=0.0),
    # logit bias (OpenAI logit_bias): logits[idx] += bias; the test's token
    # ids 10 and 20 sit at positions 1 and 2 of its three-entry vector
    dict(name="logit_bias", src=f"{P}:1060-1072", op="logit_bias",
         logits=[1.0, 1.0, 1.0], bias_tokens=[1, 2], bias_values=[2.5, -5.0],
         expect=[1.0, 3.5, -4.0], tol=0.0),
    # documented order: repetition before temperature
    dict(name="order_rep_then_temp_neg", src=f"{T}:760-791", op="rep_then_temp",
         logits=[-8.0, 0.0], history=[0], penalty=2.0, t=2.0, expect=[-8.0, 0.0], tol=1e-5),
    dict(name="order_rep_intermediate", src=f"{T}:793-799", op="repetition",
         logits=[6.0], history=[0], penalty=3.0, expect=[2.0], tol=1e-5),
    dict(name="order_temp_then_rep", src=f"{T}:801-811", op="temp_then_rep",
         logits=[6.0], history=[0], penalty=3.0, t=3.0, expect=[0.667], tol=1e-3),
    # final_logit_softcapping, cap * tanh(x / cap) (candle.rs:1803-1807): the
    # test's expected values are that closed form in f64, cast to f32
    dict(name="softcap_thirty", src=f"{T}:251-263", op="softcap",
         logits=[10.0, -20.0, 0.0], cap=30.0,
         expect=[float(f32(30.0 * math.tanh(10.0 / 30.0))), float(f32(30.0 * math.tanh(-20.0 / 30.0))), 0.0],
         tol=1e-4),
]


def main():
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_kats.json")
    with open(out, "w") as f:
        json.dump({"source": "mashriram/llm-rs test vectors (transcribed)", "kats": KATS}, f, indent=1)
    print(f"wrote {len(KATS)} vectors to {out}")


if __name__ == "__main__":
    main()
