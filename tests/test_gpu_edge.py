"""GPU edge cases through the C ABI, each compared bit for bit with the CPU
mirror oracle (tokens, kept counts, kept ids and probabilities): the
reference's known-answer vectors, tiny and ragged vocabularies, padded rows,
fully masked rows, top-k at and beyond its limits, extreme top-p and
uniforms, bf16 and f16 ties, f16 logits, history ids outside the vocabulary, invalid parameters
and the device status word.  Marked gpu."""
import json
import os

import numpy as np
import pytest

import llmk
from llmk import _lib, synth
from oracle import llmk_oracle as O

from gpu_util import assert_bit_exact, run_gpu, run_gpu_offset, run_gpu_strided, workload

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
CAP = 64


@pytest.fixture(scope="module")
def sampler():
    s = llmk.HipSampler(max_batch=512, max_vocab=256000)
    yield s
    s.close()


def check(sampler, w, cap=CAP, strided=False, label=""):
    print(f"[case] {label or w.name} B={w.B} V={w.V} dtype={w.dtype} strided={strided}", flush=True)
    gpu = (run_gpu_strided if strided else run_gpu)(sampler, w, cap)
    orc = O.sample_workload(O.MIRROR, w, out_cap=cap, nthreads=16)
    assert_bit_exact(w, gpu, orc, cap, label or w.name)
    return gpu, orc


def test_reference_kats_through_the_abi(sampler):
    with open(os.path.join(HERE, "golden", "reference_kats.json")) as f:
        kats = [k for k in json.load(f)["kats"] if k["op"] in ("sample_simple", "softmax")]
    for k in kats:
        lg = np.asarray(k["logits"], np.float32)
        T = k.get("temperature", 1.0)
        for u in (0.0, 0.37, 0.999):
            gpu, orc = check(sampler, workload(lg, T=T, u=u), cap=8, strided=True, label=k["name"])
            if "expect_token" in k:
                assert gpu[0][0] == k["expect_token"]
            if "sum_tol" in k:
                assert abs(float(np.sum(gpu[2][0, :gpu[3][0]], dtype=np.float32)) - 1) < k["sum_tol"]


@pytest.mark.parametrize("V", [1, 2, 3, 5, 63, 1023, 1024, 1025, 4097, 16385, 151937])
def test_ragged_vocabularies(sampler, V):
    rng = np.random.default_rng(V)
    B = 6
    lg = rng.normal(0, 3, (B, V)).astype(np.float32)
    T = np.array([0.0, 0.7, 1.0, 1.3, 0.7, 0.9], np.float32)
    K = np.array([0, 50, 0, 3, 1, 0], np.int32)
    P = np.array([1.0, 0.95, 0.9, 1.0, 0.5, 1.0], np.float32)
    hists = [rng.integers(0, V + 5, 40) for _ in range(B)]
    w = workload(lg, T=T, K=K, P=P, R=1.1, PR=0.2, FR=0.1, hists=hists,
                 u=rng.random(B).astype(np.float32))
    check(sampler, w, strided=True, label=f"ragged V={V}")


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_fully_masked_rows(sampler, dtype):
    V = 5000
    lg = np.random.default_rng(1).normal(0, 2, (5, V)).astype(np.float32)
    mask = np.zeros((5, (V + 31) // 32), np.uint32)
    mask[4] = 0xFFFFFFFF  # one ordinary row beside them
    w = workload(lg, T=[0.0, 0.8, 0.8, 0.8, 0.8], K=[0, 0, 7, 0, 20], P=[1.0, 0.9, 1.0, 1.0, 0.9],
                 u=[0.3, 0.0, 0.3, 0.3, 0.3], mask=mask, dtype=dtype)
    gpu, _ = check(sampler, w, label=f"masked {dtype}")
    assert gpu[0][:4].tolist() == [0, 0, 6, V - 1]


def test_top_k_limits(sampler):
    V = 20000
    rng = np.random.default_rng(2)
    lg = rng.normal(0, 3, (8, V)).astype(np.float32)
    K = np.array([1, 2, 1023, 1024, 1025, V - 1, V, V + 7], np.int32)
    w = workload(lg, T=0.8, K=K, P=1.0, u=rng.random(8).astype(np.float32))
    check(sampler, w, cap=1100, label="top-k limits")


def test_extreme_top_p_and_uniforms(sampler):
    V = 30000
    rng = np.random.default_rng(3)
    lg = rng.normal(0, 3, (8, V)).astype(np.float32)
    one_minus = np.float32(1.0 - 2.0 ** -24)
    w = workload(lg, T=0.9, K=[40, 40, 0, 0, 40, 40, 0, 0],
                 P=[1e-30, 1.0, 1e-30, 0.3, 0.95, 0.95, 0.95, 0.999],
                 u=[0.5, 0.5, 0.0, one_minus, 0.0, one_minus, one_minus, 0.999])
    check(sampler, w, label="extreme top-p / u")


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_ties(sampler, dtype):
    """Quantised logits make many equal probabilities: (p desc, idx asc)."""
    V = 40000
    rng = np.random.default_rng(4)
    lg = np.round(rng.normal(0, 2, (6, V)) * 2) / 2
    lg[:, :: 97] = 6.0  # a plateau of equal maxima
    lg[5] = 1.25  # all equal
    w = workload(lg.astype(np.float32), T=[0.7, 0.7, 1.0, 1.0, 0.0, 0.9], K=[50, 0, 200, 1, 0, 30],
                 P=[0.95, 0.9, 1.0, 1.0, 1.0, 1.0], MP=[0.0, 0.05, 0.0, 0.0, 0.0, 0.0],
                 u=rng.random(6).astype(np.float32), dtype=dtype)
    check(sampler, w, cap=256, label=f"ties {dtype}")


def test_min_p_rows(sampler):
    V = 50000
    rng = np.random.default_rng(5)
    lg = rng.normal(0, 3, (6, V)).astype(np.float32)
    lg[:, 7] = 12.0
    w = workload(lg, T=0.9, K=[0, 200, 0, 50, 0, 0], P=[1.0, 0.98, 0.9, 1.0, 1.0, 0.95],
                 MP=[0.02, 0.02, 0.1, 0.5, 1.0, 1e-4], u=rng.random(6).astype(np.float32))
    check(sampler, w, cap=256, label="min-p")


def test_wide_nuclei(sampler):
    """Flat rows whose nucleus holds 10^3..10^5 tokens: the slow path's
    choice of bins and its fallback, the exact running sums over long sorted
    lists (many binade crossings and rounding ties), a top-k above the fast
    path's limit and a min-p cut next to the chosen bins."""
    V = 151936
    rng = np.random.default_rng(11)
    lg = rng.normal(0, 0.8, (6, V)).astype(np.float32)
    w = workload(lg, T=[1.0, 1.2, 0.9, 1.0, 1.1, 1.0], K=[0, 0, 0, 0, 5000, 0],
                 P=[0.5, 0.9, 0.99, 0.9995, 0.95, 1.0], MP=[0.0, 0.0, 0.3, 0.0, 0.0, 0.02],
                 u=rng.random(6).astype(np.float32))
    check(sampler, w, cap=4096, label="wide nuclei")


def test_empty_and_out_of_vocab_histories(sampler):
    V = 30000
    rng = np.random.default_rng(6)
    lg = rng.normal(0, 3, (4, V)).astype(np.float32)
    hists = [[], [V, V + 1, 2 ** 31, 0xFFFFFFFE], rng.integers(0, V, 3000), [5] * 500]
    w = workload(lg, T=0.8, K=30, P=0.9, R=1.3, PR=0.4, FR=0.2, hists=hists,
                 u=rng.random(4).astype(np.float32))
    check(sampler, w, label="histories")
    # no history arrays at all
    db = w.to_device()
    db.hist_offsets = db.hist_tokens = None
    r = sampler.sample_batch(db, out_cap=0)
    w2 = workload(lg, T=0.8, K=30, P=0.9, R=1.3, PR=0.4, FR=0.2, u=w.uniforms)
    orc = O.sample_workload(O.MIRROR, w2, out_cap=0)
    assert np.array_equal(r.tokens.cpu().numpy().view(np.uint32), orc[1])


def test_invalid_parameters_and_status(sampler):
    V = 9000
    rng = np.random.default_rng(7)
    lg = rng.normal(0, 3, (6, V)).astype(np.float32)
    T = np.array([np.nan, 0.8, 0.8, np.inf, 0.8, 0.8], np.float32)
    K = np.array([0, -1, 10, 0, 10, 10], np.int32)
    P = np.array([1.0, 1.0, np.nan, 1.0, 1.0, 0.9], np.float32)
    R = np.array([1.0, 1.0, 1.0, 1.0, np.inf, 1.1], np.float32)
    w = workload(lg, T=T, K=K, P=P, R=R, u=0.4)
    sampler.status()  # clear what earlier calls raised
    print("[case] invalid params", flush=True)
    tok, ids, probs, cnt = run_gpu(sampler, w, 8)
    assert np.all(tok[:5] == _lib.LLMK_INVALID_TOKEN) and np.all(cnt[:5] == 0)
    ok = workload(lg[5:], T=0.8, K=10, P=0.9, R=1.1, u=0.4)
    orc = O.sample_workload(O.MIRROR, ok, out_cap=8)
    assert tok[5] == orc[1][0]
    assert sampler.status() == _lib.LLMK_STATUS_INVALID_PARAMS
    assert sampler.status() == 0  # reading clears it


def test_history_overflow_penalises_every_token(sampler):
    """Past 8192 distinct history tokens in one vocabulary segment (16384
    tokens a segment for rows of this vocabulary in a small batch) the row is
    materialised by the slow path: every one of the 20,000 distinct tokens
    is penalised, as the reference does (sampler.rs:132-146, no limit), and
    the status word says the row took that path.  A top-k row, a top-k-off
    row and a greedy row, each checked bit-exact against the oracle on the
    full history."""
    V = 151936
    lg = np.random.default_rng(8).normal(0, 3, (3, V)).astype(np.float32)
    hist = np.concatenate([np.arange(20000), [5, 5, 9000, 17000, 17000]])
    T = np.array([0.8, 0.8, 0.0], np.float32)
    K = np.array([40, 0, 0], np.int32)
    P = np.array([0.95, 0.9, 1.0], np.float32)
    w = workload(lg, hists=[hist] * 3, T=T, K=K, P=P, R=1.1, PR=0.3, FR=0.2, u=0.3)
    sampler.status()
    print("[case] history overflow: 20000 distinct tokens, top-k / top-p / greedy", flush=True)
    gpu = run_gpu(sampler, w, CAP)
    assert sampler.status() & _lib.LLMK_STATUS_HISTORY_OVERFLOW
    orc = O.sample_workload(O.MIRROR, w, out_cap=CAP, nthreads=16)
    assert_bit_exact(w, gpu, orc, CAP, "history overflow")
    ref = O.sample_workload(O.REF, w, out_cap=CAP, nthreads=16)
    assert np.array_equal(gpu[0], ref[1]), (gpu[0], ref[1])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("offset,extra", [(0, 0), (1, 3), (3, 5)])
def test_rows_at_any_offset(sampler, dtype, offset, extra):
    """Rows at any element offset and stride (GPT-2's 50257-token vocabulary
    at stride V, and views at odd offsets): copied to aligned rows, then
    sampled bit-exact against the oracle (sampler.rs:25-29 takes any
    &[f32])."""
    from llmk import synth
    w = synth.make("C3", B=4)
    V = 50257
    lg = np.ascontiguousarray(w.logits[:, :V])
    w2 = workload(lg, T=w.temperature, K=w.top_k, P=w.top_p, R=w.repetition,
                  PR=w.presence, FR=w.frequency, u=w.uniforms, dtype=dtype,
                  hists=[h[h < V] for h in np.split(w.hist_tokens, w.hist_offsets[1:-1])])
    print(f"[case] {dtype} V={V} offset={offset} stride=V+{extra}", flush=True)
    gpu = run_gpu_offset(sampler, w2, CAP, offset=offset, extra=extra)
    orc = O.sample_workload(O.MIRROR, w2, out_cap=CAP)
    assert_bit_exact(w2, gpu, orc, CAP, f"offset {offset}")


def test_host_errors(sampler):
    import torch
    w = workload(np.zeros((2, 100), np.float32))
    db = w.to_device()
    with pytest.raises(llmk.SamplerError) as e:
        db.vocab = 0
        sampler.sample_batch(db)
    assert e.value.code == _lib.LLMK_ERR_EMPTY_LOGITS
    db.vocab = 100
    big = workload(np.zeros((2, 300000), np.float32)).to_device()
    with pytest.raises(llmk.SamplerError) as e:
        sampler.sample_batch(big)
    assert e.value.code == _lib.LLMK_ERR_CAPACITY
    # the reference's per-row call and sample() wrapper
    lg = torch.tensor([0.1, 0.5, 3.0, 0.2], device="cuda:0")
    assert llmk.sample(sampler, lg, 0.0, 0.5) == 2
    with pytest.raises(llmk.SamplerError):
        sampler.sample(torch.zeros(0, device="cuda:0"), llmk.SampleParams(), [], 0.5)


@pytest.mark.parametrize("B", [1, 7, 9, 300])
def test_batch_shapes(sampler, B):
    """Batch sizes that change the segment count and the XCD mapping."""
    w = synth.make("C3", B=B, V=50000)
    check(sampler, w, label=f"C3 B={B} V=50000")


def test_f16_logits(sampler):
    """f16 logits (half-precision lm_head output) read and upcast exactly:
    C2's rows and parameters with the logits rounded to half."""
    c2 = synth.make("C2", B=32)
    hists = [c2.hist_tokens[c2.hist_offsets[b]:c2.hist_offsets[b + 1]] for b in range(c2.B)]
    w = workload(c2.logits, T=c2.temperature, K=c2.top_k, P=c2.top_p, MP=c2.min_p,
                 R=c2.repetition, PR=c2.presence, FR=c2.frequency, hists=hists,
                 u=c2.uniforms, dtype="f16", name="C2 f16")
    check(sampler, w, label="C2 rows, f16 logits")


@pytest.mark.parametrize("name", ["C1", "C2", "C4", "C5"])
def test_full_size_configs(sampler, name):
    w = synth.make(name)
    check(sampler, w, label=f"full {name}")


def test_repeated_calls_are_stable(sampler):
    """The workspace (arrival counters, slots) is left clean by every call."""
    w = synth.make("C2", B=16)
    first = run_gpu(sampler, w, CAP)
    for i in range(3):
        again = run_gpu(sampler, w, CAP)
        for a, b in zip(first, again):
            assert np.array_equal(a, b)


def test_history_buffers_and_device_append(sampler):
    """Per-row history buffers (hist_lengths) and llmk_history_append: two
    decode steps of C3 rows whose histories live in buffers of capacity
    2100, the sampled tokens appended on the device between the steps
    (scheduler.rs:147), each step bit-exact against the oracle on the
    compact CSR; a full row keeps its history and raises
    LLMK_STATUS_HISTORY_FULL; an invalid token is not pushed."""
    import torch
    w = synth.make("C3", B=24)
    cap = 2100
    B = w.B
    lens = np.diff(w.hist_offsets.astype(np.int64)).astype(np.int64)
    lens[3] = cap  # a full row: its history padded with repeats of its own tokens
    buf = np.zeros(B * cap, np.uint32)
    for b in range(B):
        h = w.hist_tokens[w.hist_offsets[b]:w.hist_offsets[b + 1]]
        hh = np.resize(h, int(lens[b])) if len(h) else np.zeros(int(lens[b]), np.uint32)
        buf[b * cap:b * cap + lens[b]] = hh
    offs = (np.arange(B) * cap).astype(np.uint32)
    d_off = torch.from_numpy(offs.view(np.int32)).cuda()
    d_len = torch.from_numpy(lens.astype(np.int32)).cuda()
    d_buf = torch.from_numpy(buf.view(np.int32)).cuda()
    assert sampler.status() == 0
    for step in range(2):
        # the compact CSR the oracle reads
        cur = d_buf.cpu().numpy().view(np.uint32)
        ln = d_len.cpu().numpy().astype(np.int64)
        w.hist_offsets = np.concatenate([[0], np.cumsum(ln)]).astype(np.uint32)
        w.hist_tokens = np.concatenate([cur[b * cap:b * cap + ln[b]] for b in range(B)]).astype(np.uint32)
        w.uniforms = np.random.default_rng(40 + step).random(B).astype(np.float32)
        print(f"[case] history buffers step {step}", flush=True)
        db = w.to_device()
        db.hist_offsets, db.hist_tokens, db.hist_lengths = d_off, d_buf, d_len
        r = sampler.sample_batch(db, out_cap=CAP)
        torch.cuda.synchronize()
        gpu = (r.tokens.cpu().numpy().view(np.uint32), r.ids.cpu().numpy().view(np.uint32),
               r.probs.cpu().numpy(), r.count.cpu().numpy().view(np.uint32))
        orc = O.sample_workload(O.MIRROR, w, out_cap=CAP, nthreads=16)
        assert_bit_exact(w, gpu, orc, CAP, f"history buffers step {step}")
        toks = r.tokens.clone()
        toks[5] = -1  # LLMK_INVALID_TOKEN: no push
        sampler.history_append(d_off, d_len, d_buf, cap, toks)
        torch.cuda.synchronize()
        ln2 = d_len.cpu().numpy().astype(np.int64)
        full = ln >= cap
        full[5] = True  # unchanged like a full row, without the status bit
        assert np.array_equal(ln2, np.where(full, ln, ln + 1))
        nb = d_buf.cpu().numpy().view(np.uint32)
        for b in np.nonzero(~full)[0]:
            assert nb[b * cap + ln[b]] == gpu[0][b]
        assert sampler.status() == _lib.LLMK_STATUS_HISTORY_FULL


def test_nan_logits_raise_the_status_bit(sampler):
    """NaN logits are read as -inf (as the mirror oracle does) and raise
    LLMK_STATUS_NAN_LOGITS, the device form of sampler.rs's NAN_WARNED
    (sampler.rs:7-9, :74-76): on the fast candidate path (top-k 50), the
    general one (top-k 600 over flat logits), the slow path (top-k off, a
    nucleus of ~10^4 tokens) and for a penalised history token.  A greedy row
    (whose reference branch returns before the warning) and a NaN under a
    disallowed mask bit raise nothing; +inf raises the bit too."""
    V = 30000
    rng = np.random.default_rng(21)
    cases = {
        "fast": dict(sd=3.0, T=0.8, K=50, P=0.95),
        "general": dict(sd=0.5, T=1.0, K=600, P=1.0),
        "slow": dict(sd=0.5, T=1.0, K=0, P=0.99),
        "history": dict(sd=3.0, T=0.8, K=40, P=0.9, R=1.3, hist=True),
    }
    for name, c in cases.items():
        lg = rng.normal(0, c["sd"], (3, V)).astype(np.float32)
        lg[:, [5, 999, 20001]] = np.nan
        hists = [[999, 3, 3, 20001] for _ in range(3)] if c.get("hist") else None
        w = workload(lg, T=c["T"], K=c["K"], P=c["P"], R=c.get("R", 1.0), hists=hists,
                     u=rng.random(3).astype(np.float32))
        sampler.status()
        check(sampler, w, cap=CAP, label=f"NaN {name}")
        assert sampler.status() & _lib.LLMK_STATUS_NAN_LOGITS, name
    # greedy rows: no warning (the reference returns before it); the token
    # is the first maximum, NaN read as -inf
    lg = rng.normal(0, 3, (2, V)).astype(np.float32)
    lg[:, 17] = np.nan
    sampler.status()
    check(sampler, workload(lg, T=0.0), cap=4, label="NaN greedy")
    assert not sampler.status() & _lib.LLMK_STATUS_NAN_LOGITS
    # a NaN at a disallowed token is -inf before anything reads it
    mask = np.full((2, (V + 31) // 32), 0xFFFFFFFF, np.uint32)
    mask[:, 17 >> 5] &= ~np.uint32(1 << (17 & 31))
    check(sampler, workload(lg, T=0.9, K=30, mask=mask), cap=8, label="NaN masked")
    assert not sampler.status() & _lib.LLMK_STATUS_NAN_LOGITS
    # +inf: l - max is inf - inf for the reference
    lg2 = lg.copy()
    lg2[:, 17] = np.inf
    print("[case] +inf logit", flush=True)
    run_gpu(sampler, workload(lg2, T=0.9, K=30), 8)
    assert sampler.status() & _lib.LLMK_STATUS_NAN_LOGITS
