"""Pins the CPU oracle by what the mathematics fixes, independently of its own
code: closed forms and special cases (llm-core/src/sampler.rs:25-125), an
fp64 textbook pipeline, inverse-CDF boundaries found by bisection over the
2^-24 uniform grid, deterministic and chi-square draw frequencies, an
exhaustive scan of the engine's expf against the host's glibc expf, its table
recomputed from 2^(i/32), and the one difference of the two oracle modes
(S = 1 on rows that top-k renormalises) measured on the full configs."""
import concurrent.futures as cf
import math
import os

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
    assert probs[0] == f32(1.0) / f32(V)  # the sequential sum of V ones is exact
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
# The engine's expf and the two modes
# ---------------------------------------------------------------------------
def test_exp_ref_exhaustive_against_glibc():
    """Every float x in [-104, -0]: exp_ref equals the host's expf (what
    Rust's f32::exp calls, sampler.rs:61) bit for bit, and is monotone."""
    lo, hi = 0x80000000, 0xC2D00000  # -0.0 .. -104.0
    edges = np.linspace(lo, hi, 65).astype(np.int64)
    chunks = [(int(edges[i]) + (1 if i else 0), int(edges[i + 1])) for i in range(64)]
    with cf.ThreadPoolExecutor(8) as ex:
        res = list(ex.map(lambda c: O.exp_scan(*c), chunks))
    n = sum(r[0] for r in res)
    assert n == hi - lo + 1  # every pattern checked once
    assert sum(r[1] for r in res) == 0
    assert sum(r[2] for r in res) == 0


def test_exp_ref_special_values():
    assert O.exp_ref(0.0) == 1.0 and O.exp_ref(-0.0) == 1.0
    assert O.exp_ref(float("-inf")) == 0.0 and O.exp_ref(-1e30) == 0.0
    # the underflow edge: below -0x1.9fe368p6 glibc returns +0, above it the
    # smallest subnormals
    edge = float(np.float32(-float.fromhex("0x1.9fe368p6")))
    assert O.exp_ref(float(np.nextafter(np.float32(edge), np.float32(-200)))) == 0.0
    assert O.exp_ref(edge) == O.libm_expf(edge)
    assert O.exp_ref(-103.0) > 0
    assert O.exp_ref(-1.0) == f32(math.exp(-1.0))


def test_exp_table_recomputed_from_mathematics():
    """EXP_TAB (oracle) and kExpTab (device) both hold bits(2^(i/32)) - (i << 47)
    with 2^(i/32) correctly rounded, recomputed here to 80 digits."""
    import re
    from oracle import gen_constants
    want = gen_constants.exp_table()
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for path, name in (("oracle/llmk_oracle.c", "EXP_TAB"),
                       ("llm-rs_amd/csrc/llmk_numerics.h", "kExpTab")):
        text = open(os.path.join(root, path)).read()
        body = text[text.index(name):]
        body = body[body.index("{") + 1:body.index("}")]
        got = [int(x, 16) for x in re.findall(r"0x[0-9a-fA-F]+", body)]
        assert got == want, path


def _rows_topk(w):
    return (w.top_k > 0) & (w.top_k < w.V)


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
def test_mirror_against_ref_on_full_configs(name):
    """The full benchmark configurations in both modes.  Rows without top-k
    (C2's top_k = 0 rows, every C4 row) and greedy rows: identical, bit for
    bit.  Rows that top-k renormalises (mirror's S = 1): the same tokens and
    kept ids, probabilities within 1e-5 relative."""
    w = synth.make(name)
    cap = 256
    rr = O.sample_workload(O.REF, w, out_cap=cap, nthreads=8)
    rm = O.sample_workload(O.MIRROR, w, out_cap=cap, nthreads=8)
    assert rr[0] == 0 and rm[0] == 0
    topk = _rows_topk(w) & (w.temperature > 1e-5)
    for b in range(w.B):
        n = min(int(rr[4][b]), cap)
        assert rr[1][b] == rm[1][b], f"{name} row {b}: token {rm[1][b]} vs ref {rr[1][b]}"
        assert rr[4][b] == rm[4][b], f"{name} row {b}: kept {rm[4][b]} vs ref {rr[4][b]}"
        assert np.array_equal(rr[2][b, :n], rm[2][b, :n]), f"{name} row {b}: kept ids differ"
        if topk[b]:
            np.testing.assert_allclose(rm[3][b, :n], rr[3][b, :n], rtol=1e-5, atol=1e-30)
        else:
            assert np.array_equal(rr[3][b, :n].view(np.uint32), rm[3][b, :n].view(np.uint32)), \
                f"{name} row {b}: probabilities differ"


def test_mirror_equals_ref_without_top_k():
    """Random rows without top-k (every knob else, masks, histories, bf16-
    shaped ties): the two modes agree bit for bit."""
    rng = np.random.default_rng(31)
    for r in range(40):
        V = int(rng.choice([7, 300, 5000, 40000]))
        lg = rng.normal(0, rng.uniform(0.5, 5), V).astype(np.float32)
        if r % 3 == 0:
            lg = np.round(lg * 8) / 8  # many exact ties
        hist = rng.integers(0, V + 10, size=int(rng.integers(0, 200)))
        mask = None
        if r % 4 == 1:
            mask = rng.integers(0, 2 ** 32, size=(V + 31) // 32, dtype=np.uint64).astype(np.uint32)
        prm = O.params(float(f32(rng.uniform(0.3, 1.8))), int(rng.choice([0, V, V + 5])),
                       float(f32(rng.uniform(0.5, 1.0))), float(f32(rng.choice([0.0, 0.05]))),
                       float(f32(rng.choice([1.0, 1.2]))), float(f32(rng.choice([0.0, 0.4]))),
                       float(f32(rng.choice([0.0, 0.2]))))
        u = float(f32(rng.random()))
        a = O.sample_row(O.REF, lg, prm, hist, mask, u)
        b = O.sample_row(O.MIRROR, lg, prm, hist, mask, u)
        assert a[1] == b[1] and a[4] == b[4] and np.array_equal(a[2], b[2])
        assert np.array_equal(a[3].view(np.uint32), b[3].view(np.uint32))


# ---------------------------------------------------------------------------
# The mask-form apply_top_p (sampler.rs:176-216), on its own cut loop
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("mode", [O.REF, O.MIRROR])
def test_apply_top_p_against_fp64_kept_set(mode):
    """Random rows and thresholds: the kept set is the shortest prefix of the
    (p desc, idx asc) order whose fp64 running sum reaches top_p, on every
    row whose cut is decided by more than 3e-4 (an f32 sequential sum of at
    most 3000 probabilities drifts by less than 3000 * 2^-24 = 1.8e-4); kept
    logits are unchanged, the others -inf."""
    rng = np.random.default_rng(11)
    checked = 0
    for _ in range(200):
        V = int(rng.integers(50, 3000))
        lg = (rng.normal(0, rng.choice([0.5, 2.0, 4.0]), V)).astype(np.float32)
        tp = float(np.float32(rng.uniform(0.05, 0.995)))
        p = np.exp(lg.astype(np.float64) - lg.max())
        p /= p.sum()
        order = sorted(range(V), key=lambda i: (-p[i], i))
        cum = np.cumsum(p[order])
        j = int(np.searchsorted(cum, tp))  # first j with cum[j] >= tp
        lo = cum[j - 1] if j > 0 else 0.0
        if abs(cum[j] - tp) < 3e-4 or abs(lo - tp) < 3e-4:
            continue
        out = O.apply_top_p(mode, lg, tp)
        kept = set(np.nonzero(out > -np.inf)[0].tolist())
        assert kept == set(order[:j + 1]), (V, tp, len(kept), j + 1)
        assert np.array_equal(out[sorted(kept)], lg[sorted(kept)])
        checked += 1
    assert checked >= 100


@pytest.mark.parametrize("mode", [O.REF, O.MIRROR])
def test_apply_top_p_cut_is_at_or_above(mode):
    """sampler.rs:98: the cut is the first running sum >= top_p.  With top_p
    equal to the first probability itself, exactly one token stays; one f32
    step above it, two.  A `>` in the cut loop keeps two in the first case."""
    lg = np.array([3.0, 1.0, 0.5, -1.0, 0.25], np.float32)
    exp = O.exp_ref if mode == O.MIRROR else O.libm_expf
    e = np.array([exp(np.float32(x - lg.max())) for x in lg], np.float32)
    S = np.float32(0)
    for x in e:  # the sequential f32 sum in index order
        S = np.float32(S + x)
    p0 = np.float32(e[0] / S)
    assert np.count_nonzero(O.apply_top_p(mode, lg, float(p0)) > -np.inf) == 1
    above = float(np.nextafter(p0, np.float32(1)))
    assert np.count_nonzero(O.apply_top_p(mode, lg, above) > -np.inf) == 2
