"""The runs scheme of the exact sequential sums (seg_runs / runs_walk in
llmk_sampler.hip), restated in Python and checked against the sequential f32
sum it replaces, on the CPU.

A wave holds 64 lanes of Q consecutive terms.  Each lane bounds the running
sums over its terms from an interval [clo, chi] that holds the sum entering
the wave and the exact prefix of the lanes' f32 sums: k additions from c stay
within k u (1.001) of the exact sum (u = 2^-24; plus 2^-150 per addition
below 2^-126), a lane's own f32 sum within Q u of its terms'.  A lane whose
bounds share one binade forms its pair of quantum increments there (from an
even and from an odd count, a tie going to the even sum); consecutive such
lanes form a run, scanned with row shifts and row broadcasts as on the
device.  The walk adds a run at once and every other lane one f32 addition a
term.  The result must be the sequential f32 sum exactly, whatever the
interval's width, and the runs must never disagree with the sum they are
applied to (no fallback).  The terms mimic the kernel's: exponentials of
normal logits, subnormal ones, ties at the quantum, zeros; and terms that
each round away just below a power of two while their exact sum passes it
(the case the drift bound exists for)."""
import math

import numpy as np
import pytest

f32 = np.float32
SAT = 1 << 24


def binade_of(c):
    return -126 if c < f32(2.0 ** -126) else math.frexp(float(c))[1] - 1


def binade_d(x):
    return -1023 if x <= 0 else math.frexp(x)[1] - 1


def lane_pair(e, eb):
    s0, s1 = 0, 1
    for v in e:
        x = float(f32(min(float(v) * 2.0 ** (23 - eb), 2.0 ** 25)))
        k = math.floor(x)
        fr = x - k
        r = k + 1 if fr > 0.5 else k
        t = 1 if fr == 0.5 else 0
        s0 += r + (t & ((s0 ^ r) & 1))
        s1 += r + (t & ((s1 ^ r) & 1))
    return min(s0, SAT), min(s1 - 1, SAT)


def sat_then(f, g):
    a0 = f[0] + (g[1] if f[0] & 1 else g[0])
    a1 = f[1] + (g[0] if f[1] & 1 else g[1])
    return min(a0, SAT), min(a1, SAT)


def shifted(xs, step):
    """The device's DPP sources: row_shr 1, 2, 4, 8 within rows of 16, then
    row_bcast 15 (rows 1 and 3) and row_bcast 31 (rows 2 and 3); (0, 0)
    elsewhere."""
    out = [(0, 0)] * 64
    for lane in range(64):
        row, i = divmod(lane, 16)
        if step in (1, 2, 4, 8):
            if i >= step:
                out[lane] = xs[lane - step]
        elif step == 15:
            if row in (1, 3):
                out[lane] = xs[16 * row - 1]
        elif row in (2, 3):
            out[lane] = xs[31]
    return out


def runs_sum(c, lanes, nl, Q, clo, chi):
    c = f32(c)
    ls = []
    for lane in lanes:
        s = f32(0)
        for v in lane:
            s = f32(s + v)
        ls.append(float(s))
    pre = np.cumsum([0.0] + ls[:-1])
    ok, eb = [], []
    for lane in range(64):
        d = (Q * (lane + 2) + 4) * 2.0 ** -24 * 1.02 + 2.0 ** -45
        ab = Q * (lane + 1) * 2.0 ** -150
        lo = (clo + pre[lane]) * (1 - d) - ab
        hi = (chi + pre[lane] + ls[lane]) * (1 + d) + ab
        e = binade_d(lo)
        ok.append(lane < nl and lo >= 2.0 ** -126 and hi < 2.0 ** 120 and binade_d(hi) == e)
        eb.append(e)
    key = [eb[i] + 512 if ok[i] else 0 for i in range(64)]
    head = [(not ok[i]) or i == 0 or key[i - 1] != key[i] for i in range(64)]
    rs, cur = [], 0
    for i in range(64):
        cur = i if head[i] else cur
        rs.append(cur)
    xs = [lane_pair(lanes[i], eb[i] if ok[i] else 0) for i in range(64)]
    conds = ((1, lambda i: rs[i] + 1 <= i), (2, lambda i: rs[i] + 2 <= i),
             (4, lambda i: rs[i] + 4 <= i), (8, lambda i: rs[i] + 8 <= i),
             (15, lambda i: rs[i] + 1 <= (i & ~15)), (31, lambda i: rs[i] <= 31))
    for step, cond in conds:
        ys = shifted(xs, step)
        xs = [sat_then(ys[i], xs[i]) if cond(i) else xs[i] for i in range(64)]
    pos = 0
    while pos < nl:
        if not ok[pos]:
            for v in lanes[pos]:
                c = f32(c + v)
            pos += 1
            continue
        end = next((j for j in range(pos + 1, 64) if head[j]), 64)
        last = min(end, nl) - 1
        assert c >= f32(2.0 ** -126) and binade_of(c) == eb[pos], "a run's binade is wrong"
        C = int(float(c) * 2.0 ** (23 - eb[pos]))
        inc = xs[last][1] if C & 1 else xs[last][0]
        assert C + inc < SAT, "a run leaves its binade"
        c = f32((C + inc) * 2.0 ** (eb[pos] - 23))
        pos = last + 1
    return c


def terms(rng, kind, n):
    if kind == 0:   # exponentials of normal logits at T 0.7 (C3's distribution)
        t = np.exp(rng.normal(-13, 2.86, n))
    elif kind == 1:  # subnormal and near-subnormal terms
        t = np.exp(rng.normal(-90, 10, n))
    elif kind == 2:  # zeros among uniform terms
        t = np.where(rng.random(n) < 0.5, 0.0, rng.random(n))
    elif kind == 3:  # small multiples of 2^-24: ties at the quantum
        t = 2.0 ** -24 * rng.integers(1, 4, n)
    elif kind == 4:  # wide exponent spread
        t = rng.random(n) * 2.0 ** rng.integers(-30, 5, n)
    else:           # terms that each round away under 1 - 2^-21 (below)
        t = np.full(n, 0.4 * 2.0 ** -24)
    return t.astype(f32)


@pytest.mark.parametrize("Q", [4, 16])
@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4, 5])
def test_runs_reproduce_the_sequential_sum(Q, kind):
    rng = np.random.default_rng(1000 * Q + kind)
    for it in range(4):
        n = 64 * Q if it == 0 else int(rng.integers(1, 64 * Q + 1))
        t = terms(rng, kind, n)
        c0 = f32(0) if it % 2 == 0 else f32(rng.random() * 10.0 ** rng.uniform(-8, 2))
        if kind == 5:
            # the exact sum passes 1 after a few lanes while every f32 addition
            # rounds back to 1 - 2^-21: a lane bounded without the drift would
            # be given binade 0 while the sum stays in binade -1
            n, c0 = 64 * Q, f32(1.0 - 2.0 ** -21)
            t = terms(rng, kind, n)
        width = 0.0 if it < 2 else float(rng.uniform(0, 0.02))  # the start known to 2 %
        lanes = [[f32(0)] * Q for _ in range(64)]
        for i, v in enumerate(t):
            lanes[i // Q][i % Q] = v
        want = c0
        for v in t:
            want = f32(want + v)
        got = runs_sum(c0, lanes, (n + Q - 1) // Q, Q, float(c0) * (1 - width),
                       float(c0) * (1 + width))
        assert got == want, (Q, kind, it, got, want)
