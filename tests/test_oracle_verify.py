"""The oracle's speculative-decoding verification (llmk_oracle_verify_row,
docs/mlc-contracts.md:83-84), pinned by what the mathematics fixes:

* the output of "accept d ~ q with probability min(1, p(d)/q(d)), else draw
  from max(p - q, 0)" is distributed as p (the speculative-sampling
  theorem): enumerated over every draft token and a fine grid of both
  uniforms, the output frequencies match p to the grid's resolution.  A
  swapped residual (q - p), an inverted test or a missing normalisation
  fails it;
* closed cases: q = p always accepts, p(d) = 0 always rejects, q(d) = 0 with
  p(d) > 0 always accepts, the R = 0 branch is the reference's draw over p,
  invalid rows.
No GPU."""
import numpy as np
import pytest

from oracle import llmk_oracle as O

INVALID = 0xFFFFFFFF


def kept_list(p_full):
    """(ids, probs) of the nonzero entries of p in (p desc, idx asc) order."""
    ids = [i for i in range(len(p_full)) if p_full[i] > 0]
    ids.sort(key=lambda i: (-p_full[i], i))
    return np.array(ids, np.uint32), np.array([p_full[i] for i in ids], np.float32)


def output_distribution(p_full, q, G=400):
    ids, probs = kept_list(p_full)
    V = len(q)
    out = np.zeros(V)
    grid = (np.arange(G) + 0.5) / G
    for d in range(V):
        if q[d] == 0:
            continue
        acc_tok = None
        for ua in grid:
            tok, acc = O.verify_row(ids, probs, d, q, ua, 0.0)
            if acc:
                out[d] += q[d] / G
            else:
                # the rejection branch does not depend on u_a: sweep u_r once
                if acc_tok is None:
                    acc_tok = np.zeros(V)
                    for ur in grid:
                        t, a = O.verify_row(ids, probs, d, q, 1.0, ur)
                        assert a == 0
                        acc_tok[t] += 1.0 / G
                out += q[d] / G * acc_tok
    return out


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_output_is_distributed_as_the_target(seed):
    rng = np.random.default_rng(seed)
    V = 7
    p = rng.random(V).astype(np.float64)
    p[rng.integers(V)] = 0.0          # a token outside the target's kept list
    p = (p / p.sum()).astype(np.float32)
    q = rng.random(V)
    q = (q / q.sum()).astype(np.float32)
    out = output_distribution(p, q)
    np.testing.assert_allclose(out, p, atol=0.01)


def test_equal_distributions_always_accept():
    p = np.array([0.5, 0.25, 0.125, 0.125], np.float32)
    ids, probs = kept_list(p)
    for d in range(4):
        for ua in (0.0, 0.3, 0.999999):
            assert O.verify_row(ids, probs, d, p, ua, 0.5) == (d, 1)


def test_token_outside_the_list_is_rejected():
    p = np.array([0.6, 0.4, 0.0, 0.0], np.float32)
    q = np.array([0.1, 0.1, 0.7, 0.1], np.float32)
    ids, probs = kept_list(p)
    for ua in (0.0, 0.5):
        tok, acc = O.verify_row(ids, probs, 2, q, ua, 0.0)
        assert acc == 0 and tok in (0, 1)
    # residual (0.5, 0.3) / 0.8: u_r 0.6 < 0.625 draws token 0, 0.7 token 1
    assert O.verify_row(ids, probs, 2, q, 0.5, 0.6) == (0, 0)
    assert O.verify_row(ids, probs, 2, q, 0.5, 0.7) == (1, 0)


def test_draft_probability_zero_accepts():
    p = np.array([0.7, 0.3], np.float32)
    q = np.array([1.0, 0.0], np.float32)
    ids, probs = kept_list(p)
    assert O.verify_row(ids, probs, 1, q, 0.999, 0.1) == (1, 1)


def test_residual_draw_is_the_reference_loop():
    """Residuals r = max(p - q, 0) in list order, divided by their sequential
    sum, then the first running sum >= u; a plain restatement at float32."""
    rng = np.random.default_rng(9)
    for _ in range(200):
        V = 12
        p = rng.random(V) ** 3
        p[rng.random(V) < 0.3] = 0
        if p.sum() == 0:
            continue
        p = (p / p.sum()).astype(np.float32)
        q = rng.random(V).astype(np.float32)
        q /= q.sum()
        ids, probs = kept_list(p)
        d = int(rng.integers(V))
        ua, ur = np.float32(rng.random()), np.float32(rng.random())
        tok, acc = O.verify_row(ids, probs, d, q, ua, ur)
        pd = np.float32(p[d])
        if np.float32(ua * q[d]) < pd:
            assert (tok, acc) == (d, 1)
            continue
        r = np.maximum(probs - q[ids], np.float32(0)).astype(np.float32)
        R = np.float32(0)
        for x in r:
            R = np.float32(R + x)
        c = np.float32(0)
        want = None
        if R > 0:
            for j, x in enumerate(r):
                c = np.float32(c + np.float32(x / R))
                if ur <= c:
                    want = ids[j]
                    break
            if want is None:
                want = ids[np.nonzero(r > 0)[0][-1]]
        else:
            for j, x in enumerate(probs):
                c = np.float32(c + x)
                if ur <= c:
                    want = ids[j]
                    break
            if want is None:
                want = ids[-1]
        assert (tok, acc) == (int(want), 0)


def test_zero_residual_draws_from_the_target():
    """q = 2p (not normalised) rejects for u_a >= 1/2 with every residual 0:
    the draw falls back to p itself."""
    p = np.array([0.5, 0.3, 0.2], np.float32)
    q = 2 * p
    ids, probs = kept_list(p)
    assert O.verify_row(ids, probs, 1, q, 0.4, 0.1) == (1, 1)
    assert O.verify_row(ids, probs, 1, q, 0.6, 0.1) == (0, 0)
    assert O.verify_row(ids, probs, 1, q, 0.6, 0.7) == (1, 0)
    assert O.verify_row(ids, probs, 1, q, 0.6, 0.95) == (2, 0)


def test_invalid_rows():
    p = np.array([1.0], np.float32)
    assert O.verify_row([], [], 0, p, 0.5, 0.5)[0] == INVALID
    assert O.verify_row([0], [1.0], 1, p, 0.5, 0.5)[0] == INVALID
