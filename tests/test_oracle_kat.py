"""The CPU oracle against the reference's own known-answer vectors
(tests/golden/reference_kats.json, transcribed from llm-tests/tests/mlc_test.rs
and mlc_parity.rs with file:line per vector), in both oracle modes.  The
softcap vector (mlc_test.rs:251-263) pins the capped values to the test's
1e-4; the bit-level composition below that stays unpinned."""
import json
import math
import os

import numpy as np
import pytest

from oracle import llmk_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(HERE, "golden", "reference_kats.json")) as f:
    KATS = json.load(f)["kats"]

MODES = [O.REF, O.MIRROR]


def _dist(mode, logits, **kw):
    """Processed distribution as a dense per-index vector."""
    rc, tok, ids, probs, cnt = O.sample_row(mode, logits, O.params(**kw))
    assert rc == 0
    d = np.zeros(len(logits), np.float32)
    d[ids] = probs
    return d, ids, probs


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("kat", KATS, ids=[k["name"] for k in KATS])
def test_reference_kat(kat, mode):
    op = kat["op"]
    lg = np.asarray(kat.get("logits", []), np.float32)
    if op == "sample_simple":
        # the draw's uniform is irrelevant for greedy; try both ends
        for u in (0.0, 0.999999):
            assert O.sample_simple(mode, lg, kat["temperature"], u) == kat["expect_token"]
        # same through the full row entry point
        rc, tok, _, _, _ = O.sample_row(mode, lg, O.params(temperature=kat["temperature"]))
        assert rc == 0 and tok == kat["expect_token"]
    elif op == "repetition":
        out = O.apply_repetition_penalty(lg, kat["history"], kat["penalty"])
        np.testing.assert_array_less(np.abs(out - np.asarray(kat["expect"], np.float32)), kat["tol"] + 1e-30)
        # the full pipeline's penalty step gives the same logits
        pl = O.process_logits(mode, lg, O.params(repetition=kat["penalty"]), kat["history"])
        assert np.array_equal(pl, out)
    elif op == "temperature":
        out = O.apply_temperature(lg, kat["t"])
        exp = np.asarray(kat["expect"], np.float32)
        if kat["tol"] == 0.0:
            assert np.array_equal(out, exp)
        else:
            np.testing.assert_array_less(np.abs(out - exp), kat["tol"])
    elif op == "top_k":
        out = O.apply_top_k(lg, kat["k"])
        if "expect" in kat:
            assert np.array_equal(out, np.asarray(kat["expect"], np.float32))
        else:
            fin = np.nonzero(out > -np.inf)[0]
            assert sorted(fin.tolist()) == kat["expect_finite"]
            assert all(out[i] == -np.inf for i in kat["expect_masked"])
            assert np.array_equal(out[fin], lg[fin])
    elif op == "top_p":
        out = O.apply_top_p(mode, lg, kat["top_p"])
        for i in kat["expect_finite"]:
            assert out[i] > -np.inf
        assert int(np.sum(out == -np.inf)) >= kat["min_masked"]
    elif op == "softmax":
        d, ids, probs = _dist(mode, lg)
        # the reference sums with Iterator::sum, sequential in f32
        s = np.float32(0.0)
        for x in d:
            s = np.float32(s + x)
        assert abs(float(s) - 1.0) < kat["sum_tol"]
        assert np.all(d >= 0.0)
        if "expect_argmax" in kat:
            assert int(np.argmax(d)) == kat["expect_argmax"] and int(ids[0]) == kat["expect_argmax"]
        if "fp64_tol" in kat:
            x = lg.astype(np.float64)
            e = np.exp(x - x.max())
            np.testing.assert_allclose(d, e / e.sum(), atol=kat["fp64_tol"], rtol=0)
    elif op == "top_p_probs":
        # the test starts from probabilities: run the steps after the sort
        p = np.asarray(kat["probs"], np.float32)
        order = sorted(range(p.size), key=lambda i: (-p[i], i))
        rc, tok, ids, probs, cnt = O.semantics(p[order], order, O.params(top_p=kat["top_p"]))
        assert rc == 0
        assert ids.tolist() == kat["expect_ids"]
        s = np.float32(0.0)
        for x in probs:
            s = np.float32(s + x)
        assert abs(float(s) - 1.0) < kat["sum_tol"]
    elif op == "presence_frequency":
        prm = O.params(presence=kat["presence"], frequency=kat["frequency"])
        out = O.process_logits(mode, lg, prm, kat["history"])
        assert np.array_equal(out, np.asarray(kat["expect"], np.float32))
    elif op == "rep_then_temp":
        out = O.apply_temperature(O.apply_repetition_penalty(lg, kat["history"], kat["penalty"]), kat["t"])
        np.testing.assert_array_less(np.abs(out - np.asarray(kat["expect"], np.float32)), kat["tol"])
    elif op == "temp_then_rep":
        out = O.apply_repetition_penalty(O.apply_temperature(lg, kat["t"]), kat["history"], kat["penalty"])
        np.testing.assert_array_less(np.abs(out - np.asarray(kat["expect"], np.float32)), kat["tol"])
    elif op == "logit_bias":
        out = O.apply_logit_bias(lg, kat["bias_tokens"], kat["bias_values"])
        assert np.array_equal(out, np.asarray(kat["expect"], np.float32))
    elif op == "softcap":
        # the oracle's softcap in f32 logits (candle's CPU ops, llmk_oracle_softcap)
        out = O.softcap("f32", lg, kat["cap"])
        np.testing.assert_array_less(np.abs(out - np.asarray(kat["expect"], np.float32)), kat["tol"])
        # and the capped distribution the sampler then draws from
        d, ids, probs = _dist(mode, out)
        e = np.exp(np.asarray(kat["expect"], np.float64) - max(kat["expect"]))
        np.testing.assert_allclose(d, e / e.sum(), atol=kat["tol"], rtol=0)
    else:
        raise AssertionError(f"unknown op {op}")


def test_kat_fixture_matches_generator():
    """The committed fixture is what its generator writes."""
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "mk", os.path.join(HERE, "golden", "make_reference_kats.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    assert json.loads(json.dumps(mk.KATS)) == KATS


@pytest.mark.parametrize("mode", MODES)
def test_empty_logits_is_an_error(mode):
    """sampler.rs:30-32 bails on empty logits."""
    rc, *_ = O.sample_row(mode, np.zeros(0, np.float32), O.params())
    assert rc == -1


@pytest.mark.parametrize("mode", MODES)
def test_sample_wrapper_defaults(mode):
    """sampler.rs:219-228: sample() uses top_p 1, top_k 0, repetition 1 and
    no history, so at T=1 the kept list is the whole vocabulary."""
    lg = np.array([0.5, -1.0, 2.0, 0.0], np.float32)
    rc, tok, ids, probs, cnt = O.sample_row(mode, lg, O.params(temperature=1.0), u=0.0)
    assert rc == 0 and cnt == 4 and tok == 2
    assert O.sample_simple(mode, lg, 1.0, 0.0) == 2
    # u just below 1: the cumulative may fall short, then the last kept id wins
    assert O.sample_simple(mode, lg, 1.0, float(np.float32(1.0 - 2 ** -24))) in (int(ids[-1]),)
