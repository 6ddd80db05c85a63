"""Fused final_logit_softcapping (candle.rs:1803-1807) and the lm_head's
[B, S, V] layout (candle.rs:2007-2009 reads position S - 1 of each row),
through the C ABI: the engine reads the raw logits with softcap set and must
match the oracle sampling the capped logits (llmk_oracle_softcap, candle's CPU
evaluation in the logits' dtype), bit for bit, for f32, bf16 and f16 logits;
the [B, S, V] case passes the last position as a view (offset (S - 1) V,
row stride S V).  Marked gpu."""
import copy

import numpy as np
import pytest
import torch

import llmk
from llmk import synth
from oracle import llmk_oracle as O

from gpu_util import assert_bit_exact

pytestmark = pytest.mark.gpu

CAP = 64


@pytest.fixture(scope="module")
def sampler():
    s = llmk.HipSampler(max_batch=64, max_vocab=256000)
    yield s
    s.close()


def make(name, B, dtype):
    w = synth.make(name, B=B)
    if dtype == "f16" and w.dtype != "f16":
        h = w.logits.astype(np.float16)
        w.bf16_bits, w.logits, w.dtype = h.view(np.uint16), h.astype(np.float32), "f16"
    elif dtype == "bf16" and w.dtype != "bf16":
        w.bf16_bits = synth.to_bf16_bits(w.logits)
        w.logits, w.dtype = synth.bf16_bits_to_f32(w.bf16_bits), "bf16"
    return w


def capped(w, cap):
    c = copy.copy(w)
    c.logits = O.softcap(w.dtype, w.logits.reshape(-1), cap).reshape(w.logits.shape)
    return c


def run(sampler, w, cap, seq=1):
    db = w.to_device()
    if seq > 1:
        # the lm_head output [B, S, V]: the row's logits at position S - 1,
        # the other positions filled with values that must not be read
        lg = db.logits
        big = torch.full((w.B, seq, w.V), float("nan"), dtype=lg.dtype, device=lg.device)
        big[:, seq - 1, :] = lg
        db.logits = big[:, seq - 1, :]
        assert db.logits.stride(0) == seq * w.V
    db.softcap = cap
    r = sampler.sample_batch(db, out_cap=CAP)
    torch.cuda.synchronize()
    return (r.tokens.cpu().numpy().view(np.uint32), r.ids.cpu().numpy().view(np.uint32),
            r.probs.cpu().numpy(), r.count.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("name,B,dtype", [("C3", 24, "f32"), ("C2", 24, "bf16"), ("C5", 16, "bf16"),
                                          ("C3", 16, "f16"), ("C4", 16, "f32")])
def test_softcap_matches_oracle(sampler, name, B, dtype):
    w = make(name, B, dtype)
    print(f"[case] softcap 30 {name} B={B} {dtype}", flush=True)
    gpu = run(sampler, w, 30.0)
    orc = O.sample_workload(O.MIRROR, capped(w, 30.0), out_cap=CAP, nthreads=16)
    assert_bit_exact(w, gpu, orc, CAP, f"{name}-{dtype}-softcap")
    assert sampler.status() == 0


@pytest.mark.parametrize("cap", [0.0, 30.0])
def test_last_position_of_bsv_logits(sampler, cap):
    w = make("C3", 8, "f32")
    print(f"[case] [B,S,V] last position, softcap {cap}", flush=True)
    gpu = run(sampler, w, cap, seq=3)
    orc = O.sample_workload(O.MIRROR, capped(w, cap) if cap else w, out_cap=CAP, nthreads=16)
    assert_bit_exact(w, gpu, orc, CAP, f"bsv-{cap}")
    assert sampler.status() == 0


def test_reference_softcap_kat(sampler):
    """mlc_test.rs:251-263 ([10, -20, 0], cap 30, expected cap * tanh(x / cap)
    to 1e-4) through llmk_sample_batch with softcap = 30: the kept
    probabilities are the softmax of the test's expected values, and the row
    is bit-equal to the oracle sampling its own capped logits."""
    import json
    import os
    from gpu_util import workload
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_kats.json")) as f:
        kat = next(k for k in json.load(f)["kats"] if k["op"] == "softcap")
    lg = np.asarray(kat["logits"], np.float32)
    expect = np.asarray(kat["expect"], np.float64)
    e = np.exp(expect - expect.max())
    for u in (0.0, 0.5, 0.999):
        w = workload(lg, T=1.0, u=u, name="softcap_kat")
        print(f"[case] softcap KAT u={u}", flush=True)
        gpu = run(sampler, w, kat["cap"])
        orc = O.sample_workload(O.MIRROR, capped(w, kat["cap"]), out_cap=CAP, nthreads=1)
        assert_bit_exact(w, gpu, orc, CAP, "softcap-kat")
        n = int(gpu[3][0])
        assert n == 3
        d = np.zeros(3)
        d[gpu[1][0, :n]] = gpu[2][0, :n]
        np.testing.assert_allclose(d, e / e.sum(), atol=kat["tol"], rtol=0)
    assert sampler.status() == 0


def test_softcap_rejects_bad_values(sampler):
    w = make("C3", 2, "f32")
    db = w.to_device()
    for bad in (-1.0, float("nan"), float("inf")):
        db.softcap = bad
        with pytest.raises(llmk.SamplerError):
            sampler.sample_batch(db)
