"""GPU mask-form top-k and top-p (llmk_apply_top_k / llmk_apply_top_p, the
batched in-place forms of sampler.rs:160-216) through the C ABI, compared bit
for bit with the CPU oracle's apply_top_k and mirror-mode apply_top_p: the
reference's known-answer vectors, the benchmark shapes, ties at the threshold,
rows whose chosen radix digit holds more values than LDS gathers (so every
digit level runs), -inf entries, signed zeros, padded rows, no-op parameters
and tiny vocabularies.  NaN logits are left out (the reference's order is
undefined there).  Marked gpu."""
import json
import os

import numpy as np
import pytest
import torch

import llmk
from oracle import llmk_oracle as O

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def sampler():
    s = llmk.HipSampler(max_batch=64, max_vocab=270000)
    yield s
    s.close()


def run_mask(sampler, op, rows, params, pad=0):
    """rows [B, V] f32 (numpy); params [B]; returns the masked rows from the GPU."""
    B, V = rows.shape
    print(f"[case] {op} B={B} V={V} pad={pad} params={list(params)[:6]}", flush=True)
    buf = np.full((B, V + pad), 7.0, np.float32)
    buf[:, :V] = rows
    t = torch.from_numpy(buf).cuda()
    lg = t[:, :V] if pad else t
    if op == "k":
        sampler.apply_top_k(lg, torch.tensor(np.asarray(params, np.int64).clip(-2**31, 2**31 - 1)
                                              .astype(np.int32)).cuda())
    else:
        sampler.apply_top_p(lg, torch.tensor(np.asarray(params, np.float32)).cuda())
    out = t.cpu().numpy()
    if pad:
        assert np.all(out[:, V:] == 7.0), "padding was written"
    return out[:, :V]


def oracle_mask(op, rows, params):
    out = np.empty_like(rows)
    for i, (r, p) in enumerate(zip(rows, params)):
        out[i] = O.apply_top_k(r, int(p)) if op == "k" else O.apply_top_p(O.MIRROR, r, float(p))
    return out


def check(sampler, op, rows, params, pad=0):
    rows = np.ascontiguousarray(rows, np.float32)
    gpu = run_mask(sampler, op, rows, params, pad)
    orc = oracle_mask(op, rows, params)
    bad = np.nonzero(np.any(gpu.view(np.uint32) != orc.view(np.uint32), axis=1))[0]
    assert bad.size == 0, (
        f"{op}: rows {bad[:8].tolist()} differ; row {bad[0]}: param {params[bad[0]]}, "
        f"kept gpu {int(np.sum(gpu[bad[0]] > -np.inf))} oracle {int(np.sum(orc[bad[0]] > -np.inf))}")
    assert sampler.status() == 0
    return gpu


def test_reference_kats(sampler):
    with open(os.path.join(HERE, "golden", "reference_kats.json")) as f:
        kats = [k for k in json.load(f)["kats"] if k["op"] in ("top_k", "top_p")]
    assert len(kats) == 4
    for k in kats:
        lg = np.asarray(k["logits"], np.float32)[None, :]
        op = "k" if k["op"] == "top_k" else "p"
        out = check(sampler, op, lg, [k["k"] if op == "k" else k["top_p"]],
                    pad=(-lg.shape[1]) % 4)[0]
        if "expect" in k:
            assert np.array_equal(out, np.asarray(k["expect"], np.float32))
        fin = np.nonzero(out > -np.inf)[0].tolist()
        if op == "k" and "expect_finite" in k:
            assert fin == k["expect_finite"]
            assert all(out[i] == -np.inf for i in k["expect_masked"])
        if op == "p":
            assert set(k["expect_finite"]) <= set(fin)
            assert int(np.sum(out == -np.inf)) >= k["min_masked"]


def c3_rows(B, V, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.0, 3.0, (B, V)).astype(np.float32)
    hot = rng.random((B, V)) < 0.001
    x[hot] = rng.normal(8.0, 2.0, int(hot.sum())).astype(np.float32)
    return x


@pytest.mark.parametrize("pad", [0, 12])
def test_top_k_benchmark_shape(sampler, pad):
    V = 151936
    ks = [1, 2, 50, 200, 1000, 20000, 75968, V - 1, V, V + 5, 0, -3, 7, 40, 100, 5000]
    check(sampler, "k", c3_rows(len(ks), V, 11), ks, pad)


def test_top_k_ties_and_every_digit_level(sampler):
    rng = np.random.default_rng(12)
    V = 100000
    rows = [
        rng.integers(-5, 6, V).astype(np.float32),                       # ties: one key holds ~V/11
        np.full(V, 2.5, np.float32),                                     # all equal
        (1.0 + rng.random(V) * 2.0**-10).astype(np.float32),            # one top digit
        (1.0 + rng.integers(0, 4096, V) * 2.0**-23).astype(np.float32),  # top two digits shared
        np.where(rng.random(V) < 0.5, -np.inf, rng.normal(0, 1, V)).astype(np.float32),
        np.where(rng.random(V) < 0.5, np.float32(-0.0), np.float32(0.0)),  # signed zeros only
        np.concatenate([np.full(V - 10, -np.inf), np.arange(10)]).astype(np.float32),
        np.where(rng.random(V) < 0.3, np.float32(0.0), rng.normal(0, 1, V)).astype(np.float32),
    ]
    for ks in ([1, 3, 50000, 99999, 17, 60000, 5, 40000], [9091, 50000, 33, 2, 99990, 30000, 10, 1]):
        check(sampler, "k", np.stack(rows), ks)


def test_top_k_one_read_and_its_fallbacks(sampler):
    """apply_top_k's one-read path (top_k <= 1024, V <= 2^18: values gathered
    above a rising threshold, then a write-only mask pass) and each way back
    to the radix select: an ascending row whose every value passes the rising
    threshold (the gather buffer overflows), top_k 1025, and V above 2^18."""
    rng = np.random.default_rng(21)
    V = 151936
    asc = np.sort(rng.normal(0, 3, V)).astype(np.float32)
    rows = np.stack([asc, asc[::-1].copy(), c3_rows(1, V, 22)[0], c3_rows(1, V, 23)[0]])
    check(sampler, "k", rows, [1024, 1024, 1024, 1025])
    check(sampler, "k", rows, [1, 1000, 50, 1])
    for V in (1 << 18, (1 << 18) + 8):
        check(sampler, "k", c3_rows(2, V, V), [50, 1024])


@pytest.mark.parametrize("V", [1, 2, 3, 5, 7, 64, 4097])
def test_top_k_tiny_vocab(sampler, V):
    rng = np.random.default_rng(V)
    rows = np.stack([rng.normal(0, 1, V), rng.integers(0, 3, V)]).astype(np.float32)
    for k in range(0, min(V, 6) + 1):
        check(sampler, "k", rows, [k, k], pad=4 if V % 4 else 0)


@pytest.mark.parametrize("pad", [0, 4])
def test_top_p_benchmark_shape(sampler, pad):
    V = 128256
    tps = [0.9, 0.5, 0.95, 0.99, 0.999, 0.9999, 1e-6, 0.0, -1.0, -np.inf, np.nan, 1.0, 1.5,
           np.inf, 0.3, 0.7]
    rng = np.random.default_rng(13)
    rows = rng.normal(0.0, 3.0, (len(tps), V)).astype(np.float32)
    check(sampler, "p", rows, tps, pad)


def test_top_p_ties_flat_and_masked_rows(sampler):
    rng = np.random.default_rng(14)
    V = 50000
    rows = np.stack([
        rng.integers(-3, 4, V).astype(np.float32),            # p ties at every cut
        np.zeros(V, np.float32),                              # uniform
        np.full(V, -np.inf, np.float32),                      # sum 0: untouched
        np.where(rng.random(V) < 0.9, -np.inf, rng.normal(0, 2, V)).astype(np.float32),
        (rng.normal(0, 2, V).astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32),
        np.concatenate([[20.0], np.zeros(V - 1)]).astype(np.float32),  # one dominant
        rng.normal(0, 0.01, V).astype(np.float32),            # nearly flat: a wide nucleus
        np.where(rng.random(V) < 0.5, np.float32(-0.0), np.float32(0.0)),
    ])
    for tps in ([0.5, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5, 0.5],
                [0.9, 0.25, 0.9, 0.999, 0.95, 0.99, 0.99, 0.001],
                [0.123, 0.9999, 0.1, 0.2, 0.6, 0.999999, 0.5, 0.75]):
        check(sampler, "p", rows, tps)


@pytest.mark.parametrize("V", [1, 2, 3, 5, 7, 64, 4097])
def test_top_p_tiny_vocab(sampler, V):
    rng = np.random.default_rng(100 + V)
    rows = np.stack([rng.normal(0, 1, V), rng.integers(0, 3, V)]).astype(np.float32)
    for tp in (0.0, 0.3, 0.6, 0.9, 0.99):
        check(sampler, "p", rows, [tp, tp], pad=(-V) % 4 + 4 if V % 4 else 0)


def test_mask_forms_agree_with_sampling(sampler):
    """The kept set of apply_top_p is the kept list of a sampling call with
    that top_p alone (sampler.rs:92-110 against sampler.rs:176-216)."""
    V = 32000
    rows = c3_rows(8, V, 15)
    tps = np.asarray([0.5, 0.8, 0.9, 0.95, 0.99, 0.3, 0.7, 0.6], np.float32)
    out = check(sampler, "p", rows, tps)
    t = torch.from_numpy(rows).cuda()
    db = llmk.DeviceBatch(logits=t, uniforms=torch.zeros(8, device="cuda"),
                          top_p=torch.from_numpy(tps).cuda())
    r = sampler.sample_batch(db, out_cap=V)
    cnt = r.count.cpu().numpy()
    ids = r.ids.cpu().numpy()
    for i in range(8):
        assert set(np.nonzero(out[i] > -np.inf)[0].tolist()) == set(ids[i, :cnt[i]].tolist())


def test_invalid_arguments(sampler):
    t = torch.zeros(2, 16, device="cuda")
    k = torch.ones(2, dtype=torch.int32, device="cuda")
    with pytest.raises(llmk.SamplerError):
        sampler.apply_top_k(t.to(torch.bfloat16), k)
    with pytest.raises(llmk.SamplerError):
        sampler.apply_top_p(torch.zeros(2, 300000, device="cuda"), torch.ones(2, device="cuda"))
    with pytest.raises(llmk.SamplerError):
        sampler.apply_top_k(torch.zeros(16, device="cuda"), k)


@pytest.mark.parametrize("op", ["k", "p"])
def test_unaligned_rows(sampler, op):
    """Both mask forms take rows at any f32 offset: a stride of 4099 and a
    view starting one element in (scalar heads before the first 16-byte
    boundary; top-p's sampling step reads aligned copies of the rows)."""
    rng = np.random.default_rng(16)
    B, V = 6, 4096
    full = rng.normal(0, 3, (B, 4099)).astype(np.float32)
    rows = full[:, 1:1 + V]
    params = [1, 17, 400, 4095, 2048, 3] if op == "k" else [0.5, 0.9, 0.99, 0.1, 0.7, 0.95]
    t = torch.from_numpy(full).cuda()
    lg = t[:, 1:1 + V]
    print(f"[case] unaligned {op}", flush=True)
    if op == "k":
        sampler.apply_top_k(lg, torch.tensor(params, dtype=torch.int32).cuda())
    else:
        sampler.apply_top_p(lg, torch.tensor(params, dtype=torch.float32).cuda())
    out = t.cpu().numpy()
    assert np.array_equal(out[:, 0], full[:, 0]) and np.array_equal(out[:, 1 + V:], full[:, 1 + V:])
    orc = oracle_mask(op, rows, params)
    assert np.array_equal(out[:, 1:1 + V].view(np.uint32), orc.view(np.uint32))


def bias_case(B, V, seed, dup=False):
    rng = np.random.default_rng(seed)
    rows = rng.normal(0, 3, (B, V)).astype(np.float32)
    rows[0, :5] = [-np.inf, 0.0, -0.0, 1e-40, -1e-40]  # -inf, signed zeros, denormals
    n = rng.integers(0, 300, B)
    n[0] = 8
    off = np.concatenate([[0], np.cumsum(n)]).astype(np.uint32)
    tok, val = [], []
    for b in range(B):
        t = rng.choice(V + 50, int(n[b]), replace=dup)  # some ids >= V (ignored)
        if b == 0:
            t = np.array([0, 1, 2, 3, 4, V + 1, 7, 7 if dup else 8])
        tok.append(t)
        val.append(rng.normal(0, 5, int(n[b])).astype(np.float32))
    val[0][:5] = [3.0, 1e-40, -1e-40, 1e-40, 2e-40]
    return rows, off, np.concatenate(tok).astype(np.uint32), np.concatenate(val).astype(np.float32)


@pytest.mark.parametrize("dup", [False, True])
def test_logit_bias(sampler, dup):
    """llmk_apply_logit_bias against the oracle's restatement of the
    formula of mlc_parity.rs:1060-1072, bit for bit: ids beyond the
    vocabulary, -inf, signed zeros, denormal logits and biases, and (dup)
    tokens listed twice, whose two f32 additions are checked in either order."""
    B, V = 40, 32003
    rows, off, tok, val = bias_case(B, V, 17, dup)
    print(f"[case] logit_bias B={B} V={V} dup={dup}", flush=True)
    t = torch.from_numpy(rows.copy()).cuda()
    sampler.apply_logit_bias(t, torch.from_numpy(off.view(np.int32)).cuda(),
                             torch.from_numpy(tok.view(np.int32)).cuda(), torch.from_numpy(val).cuda())
    gpu = t.cpu().numpy()
    for b in range(B):
        tb, vb = tok[off[b]:off[b + 1]], val[off[b]:off[b + 1]]
        want = O.apply_logit_bias(rows[b], tb, vb)
        if not np.array_equal(gpu[b].view(np.uint32), want.view(np.uint32)):
            # a token listed twice: its biases may land in the other order
            alt = O.apply_logit_bias(rows[b], tb[::-1], vb[::-1])
            diff = np.nonzero(gpu[b].view(np.uint32) != want.view(np.uint32))[0]
            assert dup and np.array_equal(gpu[b][diff].view(np.uint32), alt[diff].view(np.uint32)), (b, diff[:5])


def test_logit_bias_then_sample(sampler):
    """Bias then sample on one stream equals the oracle sampling the biased
    rows (C3's parameters and histories)."""
    from llmk import synth
    from gpu_util import assert_bit_exact, run_gpu
    w = synth.make("C3", B=16)
    rng = np.random.default_rng(18)
    n = rng.integers(1, 50, w.B)
    off = np.concatenate([[0], np.cumsum(n)]).astype(np.uint32)
    tok = rng.choice(w.V, int(off[-1])).astype(np.uint32)
    val = rng.normal(0, 8, int(off[-1])).astype(np.float32)
    biased = np.stack([O.apply_logit_bias(w.logits[b], tok[off[b]:off[b + 1]], val[off[b]:off[b + 1]])
                       for b in range(w.B)])
    print("[case] logit_bias then C3 sampling B=16", flush=True)
    db = w.to_device()
    sampler.apply_logit_bias(db.logits, torch.from_numpy(off.view(np.int32)).cuda(),
                             torch.from_numpy(tok.view(np.int32)).cuda(), torch.from_numpy(val).cuda())
    assert np.array_equal(db.logits.cpu().numpy().view(np.uint32), biased.view(np.uint32))
    w.logits = biased
    gpu = run_gpu(sampler, w, 64)
    orc = O.sample_workload(O.MIRROR, w, out_cap=64, nthreads=16)
    assert_bit_exact(w, gpu, orc, 64, "bias+C3")


def random_rows(rng, B, V):
    kind = rng.integers(0, 5)
    if kind == 0:
        x = rng.normal(0, rng.uniform(0.01, 6), (B, V))
    elif kind == 1:
        x = rng.integers(-4, 5, (B, V))  # heavy ties
    elif kind == 2:
        x = rng.normal(0, 3, (B, V)).astype(np.float32)
        x = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)  # bf16-valued
    elif kind == 3:
        x = rng.standard_cauchy((B, V)).clip(-1e4, 1e4)  # heavy tails
    else:
        x = rng.normal(0, 2, (B, V))
        x[:, rng.integers(0, V, max(1, V // 100))] += rng.uniform(5, 15)  # spikes
    x = np.asarray(x, np.float32)
    if rng.random() < 0.4:
        x[rng.random((B, V)) < rng.uniform(0, 0.95)] = -np.inf
    return x


@pytest.mark.parametrize("seed", range(20))
def test_mask_forms_random(sampler, seed):
    """Seeded random shapes, distributions, parameters and paddings, both
    mask forms bit-exact against the oracle."""
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 33))
    V = int(rng.choice([int(rng.integers(1, 300)), int(rng.integers(300, 20000)),
                        int(rng.integers(20000, 200000))]))
    rows = random_rows(rng, B, V)
    ks = [int(rng.choice([0, 1, 2, rng.integers(1, V + 2), V - 1, V, rng.integers(1, 64)]))
          for _ in range(B)]
    tps = [float(rng.choice([rng.uniform(0, 1), rng.uniform(0.9, 1.0), 0.0, 1.0,
                             rng.uniform(0.99, 0.99999)])) for _ in range(B)]
    check(sampler, "k", rows, ks, pad=int(rng.integers(0, 9)))
    check(sampler, "p", rows, tps, pad=(-V) % 4 + 4 * int(rng.integers(0, 3)))


def test_mask_forms_properties_at_full_batch():
    """The whole C3 batch (256 rows of 151936, more than the oracle covers in
    seconds), checked row by row through properties that fix the mask forms
    whatever the row.  apply_top_k (sampler.rs:160-173): values only ever
    replaced by -inf; every masked value below every kept one; at least k
    values at or above the smallest kept value and fewer than k strictly
    above it, so the threshold is the k-th largest value and its ties stay;
    a second application changes nothing.  apply_top_p (sampler.rs:176-216):
    values only ever replaced by -inf; the kept values a top segment of the
    row's order (ties at the cut may split); the row's maximum kept; the kept
    softmax mass, in float64, at least top_p less the error bound of the
    reference's float32 arithmetic: its normaliser is a sequential float32
    sum of V terms and its cumulative sum one of the kept terms, each
    addition off by at most half an ulp of the running sum, so the relative
    error is below (V + kept) * 2^-24.  The bound is not slack: at this
    shape terms below half an ulp of the running sum (about 12) are dropped
    whole, so the float32 normaliser reads low and the kept mass falls short
    of top_p by about 2e-4."""
    B, V = 256, 151936
    rows = c3_rows(B, V, 31)
    rows[::4] = np.round(rows[::4] * 2.0) / 2.0  # heavy ties on every fourth row
    rows[1::8, : V // 3] = -np.inf                # -inf prefixes
    ks = np.array([[1, 50, 1000, 1024, 1025, 5000, 75968, V][i % 8] for i in range(B)])
    tps = np.array([[0.5, 0.9, 0.95, 0.999, 0.1, 0.8][i % 6] for i in range(B)], np.float32)
    s = llmk.HipSampler(max_batch=B, max_vocab=V)
    try:
        t = torch.from_numpy(rows.copy()).cuda()
        kt = torch.tensor(ks.astype(np.int32)).cuda()
        print(f"[case] top_k properties B={B} V={V}", flush=True)
        s.apply_top_k(t, kt)
        once = t.cpu().numpy()
        s.apply_top_k(t, kt)
        assert np.array_equal(t.cpu().numpy().view(np.uint32), once.view(np.uint32)), \
            "apply_top_k is not idempotent"
        t = torch.from_numpy(rows.copy()).cuda()
        print(f"[case] top_p properties B={B} V={V}", flush=True)
        s.apply_top_p(t, torch.tensor(tps).cuda())
        pmask = t.cpu().numpy()
    finally:
        s.close()
    for i in range(B):
        r, o, k = rows[i], once[i], int(ks[i])
        kept = o > -np.inf
        assert np.array_equal(o[kept], r[kept]) and np.all(np.isneginf(o[~kept])), f"row {i}"
        if k >= V:
            assert np.array_equal(o, r), f"row {i}: top_k {k} >= V masks nothing"
            continue
        lo = r[kept].min()
        assert np.all(r[~kept] < lo), f"row {i}: a masked value at or above a kept one"
        assert (r >= lo).sum() >= k > (r > lo).sum(), f"row {i}: threshold is not the {k}-th largest"
    for i in range(B):
        r, o, p = rows[i], pmask[i], float(tps[i])
        kept = o > -np.inf
        assert np.array_equal(o[kept], r[kept]) and np.all(np.isneginf(o[~kept])), f"row {i}"
        assert o[np.argmax(r)] == r.max(), f"row {i}: the maximum was masked"
        assert np.all(r[~kept] <= r[kept].min()), f"row {i}: kept values are not a top segment"
        e = np.exp(r.astype(np.float64) - r.max())
        tol = (V + int(kept.sum())) * 2.0**-24
        assert e[kept].sum() / e.sum() >= p - tol, f"row {i}: kept mass below top_p {p}"
