"""The rounding band of S = 1 on rows that top-k renormalises (CPU).

The engine samples such a row with S = 1 (p = e) and keeps that result only
when llmk_oracle_band_certain (its CPU restatement; band_certain_wave on the
device) proves every decision to be the reference's whatever its normaliser
S; otherwise the row is sampled with the reference's own S.  Pinned here:

* the certificate against its definition: on rows it certifies, every one of
  many normalisers S (the reference's arithmetic p = fl(e / S), its sort and
  its renormalisations) gives the same token, kept count and kept ids as
  S = 1, with uniforms and top_p placed within a few ulps of the S = 1
  cumulatives, where a loose bound would be caught;
* closed cases: top_p or the uniform exactly at an S = 1 cumulative, ids
  inverted between entries within 2^-20, an entry below 2^-100 and min_p at
  an entry are uncertain; a spread-out list far from every boundary is
  certain;
* the mirror oracle against the reference on C3 rows, at uniforms and top_p
  values found on rand's 2^-24 grid between the two cumulatives of one entry
  (where S = 1 alone draws another token or keeps another count): the same
  token, count and ids.
"""
import numpy as np
import pytest

from llmk import synth
from oracle import llmk_oracle as O

import band_util as BU

U24 = 2.0 ** -24


def _f32(x):
    return np.float32(x)


def s_semantics(es, ix, prm, u, S, cap):
    """The reference's steps on the list with normaliser S: p = fl(e / S),
    sorted (p desc, idx asc), then min-p / top-k / top-p / draw."""
    p = (es / np.float32(S)).astype(np.float32)
    order = np.lexsort((ix, -p.astype(np.float64)))
    _, tok, ids, probs, cnt = O.semantics(p[order], ix[order], prm, u, out_cap=cap)
    return tok, cnt, ids[:min(cnt, cap)]


def random_list(rng, n):
    """A sorted e list as the engine sees it: e_0 = 1, the rest exp of
    negative offsets, some exact ties, indices random."""
    x = -np.abs(rng.normal(0, rng.uniform(1.0, 4.0), n - 1)).astype(np.float32)
    if rng.random() < 0.3:
        x = (np.round(x * 16) / 16).astype(np.float32)
    e = np.concatenate([[1.0], np.exp(x.astype(np.float64))]).astype(np.float32)
    idx = rng.permutation(200000)[:n].astype(np.uint32)
    order = np.lexsort((idx, -e.astype(np.float64)))
    return e[order], idx[order]


def near(rng, c, lo, hi):
    """c moved by a random number of its ulps in [lo, hi] either way."""
    d = int(rng.integers(lo, hi + 1)) * (1 if rng.random() < 0.5 else -1)
    return float(np.float32(np.float64(c) + d * np.spacing(np.float32(c), dtype=np.float32)))


def near_boundaries(rng, es, ix, prm, cap, lo, hi, k=3):
    """top_p values a few ulps from the cumulatives of the S = 1 list after
    top-k (where top-p cuts), uniforms a few ulps from those of the final
    list (where the draw decides)."""
    p1 = O.params(prm.temperature, prm.top_k, 1.0, prm.min_p)
    _, _, _, pk, ck = O.semantics(es, ix, p1, 0.5, out_cap=cap)
    ck_ = BU.cumulative(pk[:min(ck, cap)])
    _, _, _, pf, cf = O.semantics(es, ix, prm, 0.5, out_cap=cap)
    cf_ = BU.cumulative(pf[:min(cf, cap)])
    tps = [near(rng, ck_[rng.integers(0, len(ck_) - 1)], lo, hi) for _ in range(k)
           if len(ck_) > 1]
    us = [near(rng, cf_[rng.integers(0, len(cf_) - 1)], lo, hi) for _ in range(k)
          if len(cf_) > 1]
    return [t for t in tps if t < 1.0], us


def test_certificate_holds_for_every_normaliser():
    """Lists certified for top_p / uniforms 1-16 ulps off the S = 1
    cumulatives: 64 normalisers each must decide as S = 1 does.  A bound
    short of the reference's rounding (e.g. without the running sums' half
    ulps, or without the renormalising sum's error) certifies values there
    that some normaliser decides differently."""
    rng = np.random.default_rng(4242)
    certified = uncertain = 0
    for trial in range(160):
        n = int(rng.integers(30, 200))
        es, ix = random_list(rng, n)
        K = int(rng.integers(2, min(n - 1, 80)))
        mp = float(rng.choice([0.0, 0.0, 0.01, 0.05]))
        prm = O.params(0.8, K, 0.95, mp)
        tps, us = near_boundaries(rng, es, ix, prm, n, 1, 16)
        for tp in tps[:2] + [float(rng.uniform(0.5, 1.0))]:
            for u in us[:2] + [float(rng.random())]:
                q = O.params(0.8, K, tp, mp)
                ok = O.band_certain(es, ix, q, u, E=n, full=n + 1000, ptail=0.0)
                base = s_semantics(es, ix, q, u, 1.0, n)
                if not ok:
                    uncertain += 1
                    continue
                certified += 1
                for S in np.exp(rng.uniform(0.0, 9.0, 64)).astype(np.float32):
                    got = s_semantics(es, ix, q, u, float(S), n)
                    assert got[0] == base[0] and got[1] == base[1] and \
                        np.array_equal(got[2], base[2]), \
                        f"trial {trial}: certified, but S={S} gives {got[:2]} vs S=1 {base[:2]}"
    assert certified > 300 and uncertain > 100, (certified, uncertain)


def test_closed_cases():
    e = np.array([1.0, 0.5, 0.25, 0.125, 0.0625, 0.03125], np.float32)
    ix = np.arange(6, dtype=np.uint32)
    # far from every boundary: certain
    assert O.band_certain(e, ix, O.params(1.0, 4, 0.7), 0.3, full=100)
    # top_p equal to an S = 1 cumulative of the top-k list: uncertain
    _, _, _, p, c = O.semantics(e, ix, O.params(1.0, 4, 1.0), 0.5, out_cap=6)
    c2 = BU.cumulative(p[:c])
    assert not O.band_certain(e, ix, O.params(1.0, 4, float(c2[1])), 0.3, full=100)
    # the uniform equal to a cumulative of the final list: uncertain
    _, _, _, p, c = O.semantics(e, ix, O.params(1.0, 4, 0.7), 0.5, out_cap=6)
    c3 = BU.cumulative(p[:c])
    assert not O.band_certain(e, ix, O.params(1.0, 4, 0.7), float(c3[0]), full=100)
    # two entries within 2^-20 with their indices inverted: uncertain; in
    # index order, or exactly equal: certain
    e2 = e.copy()
    e2[2] = np.float32(e2[1] * (1 - 2.0 ** -22))
    inv = np.array([0, 2, 1, 3, 4, 5], np.uint32)
    assert not O.band_certain(e2, inv, O.params(1.0, 4, 0.7), 0.3, full=100)
    assert O.band_certain(e2, ix, O.params(1.0, 4, 0.7), 0.3, full=100)
    e3 = e.copy()
    e3[2] = e3[1]
    assert O.band_certain(e3, ix, O.params(1.0, 4, 0.7), 0.3, full=100)
    # the same across the top-k boundary (entries 3 and 4 with K = 4)
    e4 = e.copy()
    e4[4] = np.float32(e4[3] * (1 - 2.0 ** -22))
    inv4 = np.array([0, 1, 2, 4, 3, 5], np.uint32)
    assert not O.band_certain(e4, inv4, O.params(1.0, 4, 0.7), 0.3, full=100)
    # an entry below 2^-100 among the first K + 1: uncertain
    e5 = e.copy()
    e5[3:] = np.float32(2.0 ** -110)
    assert not O.band_certain(e5, ix, O.params(1.0, 4, 0.7), 0.3, full=100)
    # min_p at an entry (e_0 = 1, so the S = 1 threshold is min_p): uncertain
    assert not O.band_certain(e, ix, O.params(1.0, 5, 0.99, 0.125), 0.3, full=100)
    assert O.band_certain(e, ix, O.params(1.0, 5, 0.99, 0.1), 0.3, full=100)
    # an unknown entry K (past the exact prefix) close to the K-th: uncertain
    assert not O.band_certain(e[:4], ix[:4], O.params(1.0, 4, 0.7), 0.3, E=4, full=100,
                              ptail=float(e[3]))
    assert O.band_certain(e[:4], ix[:4], O.params(1.0, 4, 0.7), 0.3, E=4, full=100,
                          ptail=float(e[4]))


@pytest.fixture(scope="module")
def c3():
    return synth.make("C3", B=24)


def test_mirror_is_reference_where_s1_draws_another_token(c3):
    """On C3 rows, a uniform on the 2^-24 grid between REF's and S = 1's
    cumulative of one entry draws different tokens from the two; there the
    mirror (the engine's arithmetic) draws REF's token, keeps REF's count
    and ids."""
    found = 0
    for r in range(c3.B):
        u = BU.divergent_uniform(c3, r, cap=256)
        if u is None:
            continue
        found += 1
        prm = BU.row_params(c3, r)
        ref = BU.kept(O.REF, c3, r, prm, u, 256)
        mir = BU.kept(O.MIRROR, c3, r, prm, u, 256)
        assert ref[0] == mir[0] and ref[1] == mir[1], f"row {r} u={u}: {mir[:2]} vs ref {ref[:2]}"
        assert np.array_equal(ref[2][:ref[1]], mir[2][:mir[1]])
        np.testing.assert_array_equal(ref[3][:ref[1]].view(np.uint32),
                                      mir[3][:mir[1]].view(np.uint32))
    assert found >= 10, found


def test_mirror_is_reference_where_s1_cuts_top_p_elsewhere(c3):
    found = 0
    for r in range(c3.B):
        t = BU.divergent_top_p(c3, r, cap=256)
        if t is None:
            continue
        found += 1
        prm = BU.row_params(c3, r, top_p=t)
        for u in (0.25, 0.9):
            ref = BU.kept(O.REF, c3, r, prm, u, 256)
            mir = BU.kept(O.MIRROR, c3, r, prm, u, 256)
            assert ref[0] == mir[0] and ref[1] == mir[1], f"row {r} top_p={t}"
            assert np.array_equal(ref[2][:ref[1]], mir[2][:mir[1]])
    assert found >= 5, found


def test_mirror_tokens_are_reference_on_a_dense_uniform_grid(c3):
    """Every uniform of a dense grid around each S = 1 cumulative (+-64 ulps)
    of four C3 rows: the mirror's token is REF's."""
    for r in range(4):
        prm = BU.row_params(c3, r)
        _, rc, _, rp = BU.kept(O.REF, c3, r, prm, 0.5, 256)
        cr = BU.cumulative(rp[:rc])
        grid = sorted({float(np.float32(np.floor(c * BU.GRID + d) / BU.GRID))
                       for c in cr[:-1] for d in range(-64, 65, 8)})
        w1 = synth.Workload("grid", len(grid), c3.V, "f32",
                            np.repeat(c3.logits[r:r + 1], len(grid), 0), None,
                            np.full(len(grid), c3.temperature[r], np.float32),
                            np.full(len(grid), c3.top_k[r], np.int32),
                            np.full(len(grid), c3.top_p[r], np.float32),
                            np.full(len(grid), c3.min_p[r], np.float32),
                            np.full(len(grid), c3.repetition[r], np.float32),
                            np.full(len(grid), c3.presence[r], np.float32),
                            np.full(len(grid), c3.frequency[r], np.float32),
                            *synth._csr([BU.row_hist(c3, r)] * len(grid)), None,
                            np.array(grid, np.float32))
        rr = O.sample_workload(O.REF, w1, nthreads=8)
        rm = O.sample_workload(O.MIRROR, w1, nthreads=8)
        bad = np.nonzero(rr[1] != rm[1])[0]
        assert bad.size == 0, f"row {r}: tokens differ at u={np.array(grid)[bad[:5]]}"
