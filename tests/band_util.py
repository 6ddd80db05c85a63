"""Rows on which sampling with S = 1 and the reference's S draw different
tokens or cut top-p at different places (test infrastructure).

On a row that top-k renormalises, the reference divides every e by its
sequential sum S before renormalising (llm-core/src/sampler.rs:66-71, :83-88);
S cancels in exact arithmetic but not in f32, so its cumulative sums differ
from those of S = 1 in the last bits.  A uniform on rand's 2^-24 grid that
lies between the two cumulatives of one entry draws different tokens, and a
top_p between them keeps different counts.  These helpers find such values
with the CPU oracle: REF (the reference's arithmetic) against the semantics
of the S = 1 list (llmk_oracle_sorted_e + llmk_oracle_semantics)."""
import numpy as np

from oracle import llmk_oracle as O

GRID = 1 << 24


def row_params(w, r, **over):
    kw = dict(temperature=float(w.temperature[r]), top_k=int(w.top_k[r]),
              top_p=float(w.top_p[r]), min_p=float(w.min_p[r]),
              repetition=float(w.repetition[r]), presence=float(w.presence[r]),
              frequency=float(w.frequency[r]))
    kw.update(over)
    return O.params(**kw)


def row_hist(w, r):
    return w.hist_tokens[w.hist_offsets[r]:w.hist_offsets[r + 1]]


def row_mask(w, r):
    return None if w.mask is None else w.mask[r]


def cumulative(probs):
    """The reference's running sum (sampler.rs:93-96, :115-117), in f32."""
    c = np.float32(0.0)
    out = np.zeros(len(probs), np.float32)
    for j, p in enumerate(probs):
        c = np.float32(c + np.float32(p))
        out[j] = c
    return out


def kept(mode_or_s1, w, r, prm, u, cap, es=None, ix=None):
    """(token, count, ids, probs) of one row: O.REF / O.MIRROR, or "s1" for
    the S = 1 list's semantics (es, ix: its sorted e and indices)."""
    if mode_or_s1 == "s1":
        _, tok, ids, probs, cnt = O.semantics(es, ix, prm, u, out_cap=cap)
    else:
        _, tok, ids, probs, cnt = O.sample_row(mode_or_s1, w.logits[r], prm, row_hist(w, r),
                                               row_mask(w, r), u, out_cap=cap)
    return tok, cnt, ids, probs


def grid_between(a, b):
    """A multiple of 2^-24 in (min, max] of two cumulatives, or None."""
    lo, hi = (a, b) if a < b else (b, a)
    g = np.floor(np.float64(hi) * GRID) / GRID
    return float(g) if g > lo and g <= hi else None


def divergent_uniform(w, r, cap=1024):
    """A uniform on the 2^-24 grid that draws different tokens from REF and
    from S = 1 on row r at its own parameters, or None."""
    prm = row_params(w, r)
    es, ix = O.sorted_e(w.logits[r], prm, row_hist(w, r), row_mask(w, r), n=cap)
    _, rc, rids, rp = kept(O.REF, w, r, prm, 0.5, cap)
    _, sc, sids, sp = kept("s1", w, r, prm, 0.5, cap, es, ix)
    if rc != sc or not np.array_equal(rids[:rc], sids[:sc]):
        return None
    cr, cs = cumulative(rp[:rc]), cumulative(sp[:sc])
    for j in range(rc - 1):
        u = grid_between(cr[j], cs[j])
        if u is not None and u < 1.0:
            if kept(O.REF, w, r, prm, u, cap)[0] != kept("s1", w, r, prm, u, cap, es, ix)[0]:
                return u
    return None


def divergent_top_p(w, r, cap=1024):
    """A top_p that REF and S = 1 cut at different places on row r (its
    other parameters as they are), or None."""
    prm = row_params(w, r, top_p=1.0)
    es, ix = O.sorted_e(w.logits[r], prm, row_hist(w, r), row_mask(w, r), n=cap)
    _, rc, rids, rp = kept(O.REF, w, r, prm, 0.5, cap)
    _, sc, sids, sp = kept("s1", w, r, prm, 0.5, cap, es, ix)
    cr, cs = cumulative(rp[:rc]), cumulative(sp[:sc])
    for j in range(min(rc, sc) - 1):
        t = grid_between(cr[j], cs[j])
        if t is not None and 0.5 < t < 1.0:
            p2 = row_params(w, r, top_p=t)
            if kept(O.REF, w, r, p2, 0.5, cap)[1] != kept("s1", w, r, p2, 0.5, cap, es, ix)[1]:
                return t
    return None
