"""GPU: rows that top-k renormalises are sampled as the reference samples
them for every uniform and top_p, through the C ABI.

The engine samples such a row with S = 1 (p = e) and keeps that result only
when its band check proves each decision to be the reference's; otherwise it
computes the reference's own normaliser S (llm-core/src/sampler.rs:66) and
samples the row again in the reference's arithmetic.  The uniforms and top_p
values here are chosen on the CPU between the reference's cumulative and
that of S = 1 for one entry (tests/band_util.py), where S = 1 alone draws
another token or keeps another count.  Tokens, kept counts and kept ids
must be the reference oracle's, and every output the mirror oracle's bit
for bit.  Marked gpu."""
import numpy as np
import pytest

import llmk
from llmk import synth
from oracle import llmk_oracle as O

import band_util as BU
from gpu_util import assert_bit_exact, run_gpu
from test_gpu_parity import assert_matches_ref

pytestmark = pytest.mark.gpu

CAP = 256


@pytest.fixture(scope="module")
def sampler():
    s = llmk.HipSampler(max_batch=64, max_vocab=256000)
    yield s
    s.close()


def _check(sampler, w, label):
    gpu = run_gpu(sampler, w, CAP)
    assert_bit_exact(w, gpu, O.sample_workload(O.MIRROR, w, out_cap=CAP, nthreads=16), CAP, label)
    assert_matches_ref(w, gpu, O.sample_workload(O.REF, w, out_cap=CAP, nthreads=16), CAP, label)
    assert sampler.status() == 0


@pytest.mark.parametrize("name,B", [("C3", 24), ("C5", 12)])
def test_uniforms_where_s1_draws_another_token(sampler, name, B):
    w = synth.make(name, B=B)
    hit = 0
    for r in range(w.B):
        u = BU.divergent_uniform(w, r, cap=CAP)
        if u is not None:
            w.uniforms[r] = np.float32(u)
            hit += 1
    print(f"[case] {name} B={w.B}: {hit} rows with a divergent uniform", flush=True)
    assert hit >= (6 if name == "C3" else 2)
    _check(sampler, w, f"{name} divergent uniforms")


def test_top_p_where_s1_cuts_elsewhere(sampler):
    w = synth.make("C3", B=24)
    hit = 0
    for r in range(w.B):
        t = BU.divergent_top_p(w, r, cap=CAP)
        if t is not None:
            w.top_p[r] = np.float32(t)
            hit += 1
    print(f"[case] C3 B={w.B}: {hit} rows with a divergent top_p", flush=True)
    assert hit >= 4
    _check(sampler, w, "C3 divergent top_p")


def test_k_above_the_fast_path(sampler):
    """top-k above the candidate path's reach (K > 1024) goes through the
    slow path, whose band check reads the sorted list in global memory."""
    w = synth.make("C3", B=8)
    w.top_k[:] = np.array([1500, 3000, 1100, 2000, 1500, 5000, 1025, 4096], np.int32)
    w.top_p[:] = np.float32(0.999)
    for r in range(0, w.B, 2):
        u = BU.divergent_uniform(w, r, cap=8192)
        if u is not None:
            w.uniforms[r] = np.float32(u)
    print("[case] C3 B=8, top-k 1025..5000", flush=True)
    gpu = run_gpu(sampler, w, 64)
    assert_bit_exact(w, gpu, O.sample_workload(O.MIRROR, w, out_cap=64, nthreads=16), 64,
                     "large K")
    assert_matches_ref(w, gpu, O.sample_workload(O.REF, w, out_cap=64, nthreads=16), 64,
                       "large K")


@pytest.mark.parametrize("dtype,cap", [("f32", 0.0), ("bf16", 0.0), ("f16", 0.0), ("f32", 30.0),
                                       ("bf16", 30.0)])
def test_deferred_rows_in_every_dtype(sampler, dtype, cap):
    """Rows whose band check fails in a call of 20 rows (at least 16: their
    S comes from the second launch, window by window on many workgroups)
    with f32, bf16 and f16 logits, and with the softcap fused into the
    reads: the same outputs as the oracles on the (capped) logits."""
    from test_gpu_softcap import capped, make
    w = make("C3", 20, dtype)
    c = capped(w, cap) if cap else w
    hit = 0
    for r in range(w.B):
        u = BU.divergent_uniform(c, r, cap=CAP)
        if u is not None:
            w.uniforms[r] = c.uniforms[r] = np.float32(u)
            hit += 1
    print(f"[case] deferred rows {dtype} softcap {cap}: {hit} rows", flush=True)
    assert hit >= 4
    db = w.to_device()
    db.softcap = cap
    r = sampler.sample_batch(db, out_cap=CAP)
    import torch
    torch.cuda.synchronize()
    gpu = (r.tokens.cpu().numpy().view(np.uint32), r.ids.cpu().numpy().view(np.uint32),
           r.probs.cpu().numpy(), r.count.cpu().numpy().view(np.uint32))
    assert_bit_exact(w, gpu, O.sample_workload(O.MIRROR, c, out_cap=CAP, nthreads=16), CAP,
                     f"deferred {dtype} {cap}")
    assert_matches_ref(w, gpu, O.sample_workload(O.REF, c, out_cap=CAP, nthreads=16), CAP,
                       f"deferred {dtype} {cap}")
    assert sampler.status() == 0


def test_phase1_waits_that_run_out(monkeypatch):
    """Phase 1's bounded waits forced to run out at once (LLMK_TEST_XS_SPIN=0,
    read when the handle is created): no window waits for the sums before it,
    so no window past the first bounds its start and none of its segments
    has pairs or runs from its window (the walk forms them from the exact
    sum), and a walker that is not window 0 does not wait for window 0's own
    walk but walks from zero over window 0's published terms and runs.  On
    rows whose band check fails (C3's parameters, 20 rows, f32), two calls in
    a row (both job-count parities): the same outputs as the oracles."""
    import torch
    from test_gpu_softcap import make
    monkeypatch.setenv("LLMK_TEST_XS_SPIN", "0")
    s = llmk.HipSampler(max_batch=64, max_vocab=256000)
    try:
        w = make("C3", 20, "f32")
        hit = 0
        for r in range(w.B):
            u = BU.divergent_uniform(w, r, cap=CAP)
            if u is not None:
                w.uniforms[r] = np.float32(u)
                hit += 1
        assert hit >= 4
        mirror = O.sample_workload(O.MIRROR, w, out_cap=CAP, nthreads=16)
        ref = O.sample_workload(O.REF, w, out_cap=CAP, nthreads=16)
        db = w.to_device()
        for call in range(2):
            print(f"[case] phase-1 waits run out, {hit} deferred rows, call {call}", flush=True)
            r = s.sample_batch(db, out_cap=CAP)
            torch.cuda.synchronize()
            gpu = (r.tokens.cpu().numpy().view(np.uint32), r.ids.cpu().numpy().view(np.uint32),
                   r.probs.cpu().numpy(), r.count.cpu().numpy().view(np.uint32))
            assert_bit_exact(w, gpu, mirror, CAP, f"waits run out, call {call}")
            assert_matches_ref(w, gpu, ref, CAP, f"waits run out, call {call}")
            assert s.status() == 0
    finally:
        s.close()


@pytest.mark.parametrize("V", [12000, 20000, 40000])
def test_deferred_rows_at_small_vocabularies(sampler, V):
    """Rows whose band check fails at vocabularies of one phase-1 window
    (12000: window 0 is the walker and sums from zero), two windows (20000:
    window 0 walks its own segments, the walker goes on from there) and
    three (40000), C3's parameters, 20 rows: the same outputs as the
    oracles."""
    import torch
    w = synth.make("C3", B=20, V=V)
    hit = 0
    for r in range(w.B):
        u = BU.divergent_uniform(w, r, cap=CAP)
        if u is not None:
            w.uniforms[r] = np.float32(u)
            hit += 1
    print(f"[case] deferred rows at V={V}: {hit} rows", flush=True)
    assert hit >= 4
    db = w.to_device()
    r = sampler.sample_batch(db, out_cap=CAP)
    torch.cuda.synchronize()
    gpu = (r.tokens.cpu().numpy().view(np.uint32), r.ids.cpu().numpy().view(np.uint32),
           r.probs.cpu().numpy(), r.count.cpu().numpy().view(np.uint32))
    assert_bit_exact(w, gpu, O.sample_workload(O.MIRROR, w, out_cap=CAP, nthreads=16), CAP,
                     f"deferred V={V}")
    assert_matches_ref(w, gpu, O.sample_workload(O.REF, w, out_cap=CAP, nthreads=16), CAP,
                       f"deferred V={V}")
    assert sampler.status() == 0
