"""Pins the CPU oracle by what the mathematics fixes, independently of its own
code: closed forms and special cases (llm-core/src/sampler.rs:25-125), an
fp64 textbook pipeline, inverse-CDF boundaries found by bisection over the
2^-24 uniform grid, deterministic and chi-square draw frequencies, an
exhaustive scan of the mirror exp against glibc expf, the exp2 polynomial's
error bound and the mirror normaliser against an fp64 sum."""
import concurrent.futures as cf
import math

import numpy as np
import pytest

from oracle import llmk_oracle as O
from llmk import synth

MODES = [O.REF, O.MIRROR]
f32 = np.float32


# ---------------------------------------------------------------------------
# An independent fp64 restatement of the pipeline (textbook steps)
# ---------------------------------------------------------------------------
def fp64_pipeline(lg, T=1.0, K=0, P=1.0, MP=0.0, R=1.0, PR=0.0, FR=0.0, hist=(), mask=None):
    V = lg.size
    l = lg.astype(np.float64)
    h = np.asarray(hist, np.int64)
    h = h[h < V]
    if h.size:
        uniq, counts = np.unique(h, return_counts=True)
        if R != 1.0:
            l[uniq] = np.where(l[uniq] > 0, l[uniq] / R, l[uniq] * R)
        if PR != 0.0 or FR != 0.0:
            l[uniq] -= PR + counts * FR
    if mask is not None:
        bits = (mask[np.arange(V) >> 5] >> (np.arange(V) & 31)) & 1
        l[bits == 0] = -np.inf
    if T <= 1e-5:
        return np.array([int(np.argmax(l))]), np.array([1.0]), None
    x = l / T
    e = np.where(np.isneginf(x), 0.0, np.exp(x - np.max(x)))
    p = e / e.sum()
    order = np.lexsort((np.arange(V), -p))
    p, ids = p[order], order
    amb = 0.0  # distance of the top-p cut from its threshold
    if MP > 0:
        keep = p >= MP * p[0]
        n = int(np.argmin(keep)) if not keep.all() else V
        p, ids = p[:n] / p[:n].sum(), ids[:n]
    if 0 < K < p.size:
        p, ids = p[:K] / p[:K].sum(), ids[:K]
    if P < 1.0:
        c = np.cumsum(p)
        j = int(np.argmax(c >= P)) if (c >= P).any() else p.size - 1
        amb = abs(c[j] - P)
        if j > 0:
            amb = min(amb, abs(c[j - 1] - P))
        p, ids = p[:j + 1] / p[:j + 1].sum(), ids[:j + 1]
    return ids, p, amb


def rand_rows(seed, n, V):
    rng = np.random.default_rng(seed)
    lg = rng.normal(0, 3, size=(n, V)).astype(np.float32)
    for r in range(n):
        sp = rng.choice(V, 6, replace=False)
        lg[r, sp] += rng.uniform(4, 12, 6).astype(np.float32)
    return rng, lg


@pytest.mark.parametrize("mode", MODES)
def test_pipeline_matches_fp64_textbook(mode):
    rng, lg = rand_rows(1, 24, 3000)
    checked = 0
    for r in range(lg.shape[0]):
        T = float(f32(rng.uniform(0.5, 1.5)))
        K = int(rng.choice([0, 1, 5, 40, 200]))
        P = float(f32(rng.uniform(0.5, 1.0)))
        MP = float(f32(rng.choice([0.0, 0.02, 0.1])))
        R = float(f32(rng.choice([1.0, 1.1, 1.3])))
        PR, FR = float(f32(rng.choice([0.0, 0.5]))), float(f32(rng.choice([0.0, 0.3])))
        hist = rng.integers(0, 3200, size=int(rng.integers(0, 300)))  # some ids >= V
        ids64, p64, amb = fp64_pipeline(lg[r], T, K, P, MP, R, PR, FR, hist)
        if amb is not None and amb < 1e-5:
            continue  # the cut sits within rounding of the threshold
        rc, tok, ids, probs, cnt = O.sample_row(
            mode, lg[r], O.params(T, K, P, MP, R, PR, FR), hist, u=0.5)
        assert rc == 0
        assert cnt == ids64.size, f"row {r}: kept {cnt} vs fp64 {ids64.size}"
        assert np.array_equal(ids, ids64), f"row {r}: kept ids differ"
        np.testing.assert_allclose(probs, p64, rtol=1e-5, atol=1e-12)
        checked += 1
    assert checked >= 20


@pytest.mark.parametrize("mode", MODES)
def test_mask_and_greedy_match_fp64(mode):
    rng, lg = rand_rows(2, 8, 2000)
    for r in range(8):
        mask = rng.integers(0, 2 ** 32, size=(2000 + 31) // 32, dtype=np.uint64).astype(np.uint32)
        for T in (0.0, 0.8):
            ids64, p64, _ = fp64_pipeline(lg[r], T=T, K=20, mask=mask)
            rc, tok, ids, probs, cnt = O.sample_row(mode, lg[r], O.params(temperature=T, top_k=20),
                                                    mask=mask, u=0.0)
            assert rc == 0 and np.array_equal(ids, ids64)
            np.testing.assert_allclose(probs, p64, rtol=1e-5)
            assert tok == ids64[0]


# ---------------------------------------------------------------------------
# Closed forms and special cases
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("mode", MODES)
def test_top_k_one_and_tiny_top_p_give_argmax(mode):
    rng, lg = rand_rows(3, 16, 5000)
    for r in range(16):
        hist = rng.integers(0, 5000, 50)
        pl = O.process_logits(mode, lg[r], O.params(repetition=1.2), hist)
        am = int(np.argmax(pl))
        for T in (0.3, 1.0, 2.5):  # argmax is invariant under any T > 0
            for u in (0.0, 0.5, 0.9999):
                assert O.sample_row(mode, lg[r], O.params(T, top_k=1, repetition=1.2), hist, u=u)[1] == am
                assert O.sample_row(mode, lg[r], O.params(T, top_p=1e-30, repetition=1.2), hist, u=u)[1] == am
        # greedy (T <= 1e-5) is the first index of the maximum (sampler.rs:40-50)
        assert O.sample_row(mode, lg[r], O.params(0.0, repetition=1.2), hist)[1] == am


@pytest.mark.parametrize("mode", MODES)
def test_top_k_at_or_above_vocab_is_off(mode):
    rng, lg = rand_rows(4, 4, 700)
    for r in range(4):
        base = O.sample_row(mode, lg[r], O.params(0.9, top_k=0, top_p=0.9), u=0.3)
        for K in (700, 701, 10 ** 6):
            got = O.sample_row(mode, lg[r], O.params(0.9, top_k=K, top_p=0.9), u=0.3)
            assert got[1] == base[1] and np.array_equal(got[2], base[2]) and np.array_equal(got[3], base[3])


@pytest.mark.parametrize("mode", MODES)
def test_u_zero_takes_first_and_draw_is_monotone(mode):
    rng, lg = rand_rows(5, 6, 1500)
    us = np.sort(rng.random(200).astype(np.float32))
    for r in range(6):
        prm = O.params(0.8, top_k=50, top_p=0.95)
        rc, tok, ids, probs, cnt = O.sample_row(mode, lg[r], prm, u=0.0)
        assert tok == ids[0]
        pos = {int(i): j for j, i in enumerate(ids)}
        last = -1
        for u in us:
            t = O.sample_row(mode, lg[r], prm, u=float(u), out_cap=0)[1]
            assert pos[t] >= last
            last = pos[t]


@pytest.mark.parametrize("mode", MODES)
def test_all_equal_logits_are_uniform(mode):
    V = 3000
    lg = np.full(V, 1.25, np.float32)
    rc, tok, ids, probs, cnt = O.sample_row(mode, lg, O.params(0.7))
    assert cnt == V and np.array_equal(ids, np.arange(V))  # ties by index
    assert np.all(probs == probs[0])
    if mode == O.REF:  # sequential sum of V ones is exact
        assert probs[0] == f32(1.0) / f32(V)
    else:  # normaliser terms 2^(fma residual) are 1 to within an ulp
        assert abs(probs[0] * V - 1) < 2e-7
    rc, tok, ids, probs, cnt = O.sample_row(mode, lg, O.params(0.7, top_k=64))
    assert np.array_equal(ids, np.arange(64))
    np.testing.assert_allclose(probs, 1 / 64, rtol=1e-6)


@pytest.mark.parametrize("mode", MODES)
def test_two_token_distribution_by_hand(mode):
    lg = np.array([0.0, math.log(3.0)], np.float32)  # p = (1/4, 3/4)
    rc, tok, ids, probs, cnt = O.sample_row(mode, lg, O.params())
    assert ids.tolist() == [1, 0]
    np.testing.assert_allclose(probs, [0.75, 0.25], rtol=1e-6)
    for u, want in ((0.0, 1), (0.5, 1), (0.7499, 1), (0.7501, 0), (0.9999, 0)):
        assert O.sample_row(mode, lg, O.params(), u=u)[1] == want
    # top-p 0.7 keeps the first alone (0.75 >= 0.7), renormalised to 1
    rc, tok, ids, probs, cnt = O.sample_row(mode, lg, O.params(top_p=0.7), u=0.99)
    assert ids.tolist() == [1] and probs.tolist() == [1.0] and tok == 1


@pytest.mark.parametrize("mode", MODES)
def test_fully_masked_row(mode):
    """Every logit -inf: greedy returns index 0 (sampler.rs:41-49); sampling
    keeps all-zero probabilities in index order, u = 0 draws index 0 and any
    u > 0 falls through to the last kept id (sampler.rs:123-124)."""
    V = 100
    lg = np.random.default_rng(6).normal(size=V).astype(np.float32)
    mask = np.zeros((V + 31) // 32, np.uint32)
    assert O.sample_row(mode, lg, O.params(0.0), mask=mask)[1] == 0
    rc, tok, ids, probs, cnt = O.sample_row(mode, lg, O.params(0.8, top_p=0.9), mask=mask, u=0.0)
    assert cnt == V and np.array_equal(ids, np.arange(V)) and np.all(probs == 0) and tok == 0
    assert O.sample_row(mode, lg, O.params(0.8, top_p=0.9), mask=mask, u=0.3)[1] == V - 1
    assert O.sample_row(mode, lg, O.params(0.8, top_k=7), mask=mask, u=0.3)[1] == 6


@pytest.mark.parametrize("mode", MODES)
def test_history_ids_at_or_above_vocab_are_ignored(mode):
    """sampler.rs:138: only ids < V are penalised."""
    lg = np.array([1.0, -1.0, 2.0, 0.5], np.float32)
    pl = O.process_logits(mode, lg, O.params(repetition=2.0, presence=0.5, frequency=0.25), [4, 9, 1, 1, 2])
    assert pl.tolist() == [1.0, float(f32(-2.0) - (f32(0.5) + f32(2) * f32(0.25))),
                           float(f32(1.0) - (f32(0.5) + f32(0.25))), 0.5]


@pytest.mark.parametrize("mode", MODES)
def test_min_p_keeps_ties_at_the_threshold(mode):
    """min-p keeps p >= min_p * p_max: with min_p = 1 exactly the maxima stay."""
    lg = np.array([0.5, 2.0, 2.0, 1.0, 2.0], np.float32)
    rc, tok, ids, probs, cnt = O.sample_row(mode, lg, O.params(0.8, min_p=1.0), u=0.9)
    assert ids.tolist() == [1, 2, 4] and cnt == 3 and tok == 4
    np.testing.assert_allclose(probs, 1 / 3, rtol=1e-6)
    rc, tok, ids, probs, cnt = O.sample_row(mode, np.full(9, -3.0, np.float32), O.params(1.3, min_p=1.0))
    assert cnt == 9


def test_min_p_against_fp64():
    rng, lg = rand_rows(7, 10, 4000)
    for r in range(10):
        for MP in (0.02, 0.2):
            ids64, p64, _ = fp64_pipeline(lg[r], T=0.9, MP=MP)
            for mode in MODES:
                rc, tok, ids, probs, cnt = O.sample_row(mode, lg[r], O.params(0.9, min_p=MP))
                assert np.array_equal(ids, ids64)
                np.testing.assert_allclose(probs, p64, rtol=1e-5)


# ---------------------------------------------------------------------------
# The draw: inverse-CDF boundaries on the 2^-24 grid, and frequencies
# ---------------------------------------------------------------------------
GRID = 1 << 24


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("V", [2, 5, 8])
def test_draw_boundaries_on_uniform_grid(mode, V):
    """For a tiny row, find by bisection over u = i / 2^24 the first grid
    point that draws each position of the kept list; it must sit at the fp64
    cumulative probability (sampler.rs:115-121 is an inverse CDF)."""
    rng = np.random.default_rng(100 + V)
    lg = rng.normal(0, 1.5, V).astype(np.float32)
    prm = O.params(0.9)
    rc, tok, ids, probs, cnt = O.sample_row(mode, lg, prm)
    pos = {int(i): j for j, i in enumerate(ids)}
    draw = lambda i: pos[O.sample_row(mode, lg, prm, u=float(f32(i / GRID)), out_cap=0)[1]]
    _, p64, _ = fp64_pipeline(lg, T=0.9)
    cum = np.cumsum(p64)
    for j in range(1, V):
        lo, hi = 0, GRID - 1  # draw(lo) < j <= draw(hi)
        assert draw(lo) < j <= draw(hi)
        while hi - lo > 1:
            mid = (lo + hi) // 2
            if draw(mid) >= j:
                hi = mid
            else:
                lo = mid
        assert abs(hi / GRID - cum[j - 1]) < 4e-7, f"boundary {j}: {hi / GRID} vs {cum[j - 1]}"


@pytest.mark.parametrize("mode", MODES)
def test_draw_frequencies(mode):
    """Deterministic grid of uniforms: counts within 2 of N p; random
    uniforms: chi-square at p > 1e-4."""
    from scipy import stats
    V, N = 12, 60000
    lg = np.random.default_rng(8).normal(0, 1, V).astype(np.float32)
    _, p64, _ = fp64_pipeline(lg, T=1.0)
    ids64 = fp64_pipeline(lg, T=1.0)[0]
    rows = np.repeat(lg[None, :], N, axis=0)
    u = ((np.arange(N) + 0.5) / N).astype(np.float32)
    rc, tok, _, _, _ = O.sample_batch(mode, rows, uniforms=u, nthreads=8)
    cnt = np.bincount(tok, minlength=V)[ids64]
    assert np.max(np.abs(cnt - N * p64)) <= 2
    u = np.random.default_rng(9).random(N).astype(np.float32)
    rc, tok, _, _, _ = O.sample_batch(mode, rows, uniforms=u, nthreads=8)
    cnt = np.bincount(tok, minlength=V)[ids64]
    assert stats.chisquare(cnt, N * p64).pvalue > 1e-4


# ---------------------------------------------------------------------------
# Mirror numerics
# ---------------------------------------------------------------------------
def test_exp_m_exhaustive_against_glibc():
    """Every float y in [-110, -0]: exp_m differs from glibc expf by at most
    1 ulp, on under 1 input in 10^4, and is monotone."""
    lo, hi = 0x80000000, 0xC2DC0000  # -0.0 .. -110.0
    edges = np.linspace(lo, hi, 65).astype(np.int64)
    chunks = [(int(edges[i]) + (1 if i else 0), int(edges[i + 1])) for i in range(64)]
    with cf.ThreadPoolExecutor(8) as ex:
        res = list(ex.map(lambda c: O.exp_scan(*c), chunks))
    n = sum(r[0] for r in res)
    mism = sum(r[1] for r in res)
    nonmono = sum(r[2] for r in res)
    assert n == hi - lo + 1 - 0  # every pattern checked once
    assert max(r[3] for r in res) <= 1
    assert nonmono == 0
    assert mism / n < 1e-4


def test_exp_m_special_values():
    assert O.exp_m(0.0) == 1.0 and O.exp_m(-0.0) == 1.0
    assert O.exp_m(-200.0) == 0.0 and O.exp_m(float("-inf")) == 0.0
    assert O.exp_m(-1.0) == f32(math.exp(-1.0))
    assert 0 < O.exp_m(-100.0) < 1e-43


def test_exp2_f_error_bound_and_clamp():
    d = np.concatenate([np.linspace(-125, 0, 200001), -np.random.default_rng(10).random(20000) * 8])
    d = d.astype(np.float32)
    got = np.array([O.exp2_f(x) for x in d[::7]], np.float64)
    want = np.exp2(d[::7].astype(np.float64))
    assert np.max(np.abs(got / want - 1)) < 2.0e-7
    for k in range(0, 126):  # integers are exact (the polynomial is 1 at 0)
        assert O.exp2_f(-float(k)) == 2.0 ** -k
    assert O.exp2_f(float("-inf")) == 2.0 ** -125 and O.exp2_f(float("nan")) == 2.0 ** -125
    assert O.exp2_f(-1000.0) == 2.0 ** -125


@pytest.mark.parametrize("hist", [False, True])
@pytest.mark.parametrize("V,where", [(151936, "first"), (151936, "last"), (4097, "last"),
                                     (1000, "mid"), (256000, "mid")])
def test_normalizer_against_fp64(V, where, hist):
    """The mirror normaliser (tiles of 1024, virtual tiles for history tokens,
    fixed trees) equals the fp64 sum of exp((l - max)/T) to 1e-5 relative,
    wherever the maximum sits, also when it is a history token."""
    rng = np.random.default_rng(V)
    lg = rng.normal(0, 3, V).astype(np.float32)
    i = {"first": 3, "last": V - 2, "mid": V // 2}[where]
    lg[i] = 20.0
    lg[rng.choice(V, V // 50, replace=False)] = -np.inf
    is_hist = None
    if hist:
        is_hist = np.zeros(V, np.uint8)
        is_hist[rng.choice(V, min(V, 3000), replace=False)] = 1
        is_hist[i] = 1
    for T in (0.7, 1.0, 1.9):
        S = O.normalizer(lg, T, is_hist)
        x = lg.astype(np.float64) / np.float64(f32(T))
        want = np.sum(np.where(np.isneginf(x), 0.0, np.exp(x - x.max())))
        assert abs(S / want - 1) < 1e-5, (T, S, want)


def test_mirror_and_ref_agree():
    """The two modes differ only in exp's last bit and the normaliser's
    summation order: probabilities within 1e-5 relative, tokens equal on
    nearly every row."""
    w = synth.make("C3", B=48, V=20000)
    _, tr, ir, pr, cr = O.sample_workload(O.REF, w, out_cap=64, nthreads=8)
    _, tm, im, pm, cm = O.sample_workload(O.MIRROR, w, out_cap=64, nthreads=8)
    assert np.mean(tr == tm) >= 0.95
    same = (cr == cm)
    assert np.mean(same) >= 0.95
    for b in np.nonzero(same)[0]:
        n = min(int(cr[b]), 64)
        if np.array_equal(ir[b, :n], im[b, :n]):
            np.testing.assert_allclose(pm[b, :n], pr[b, :n], rtol=1e-5)
