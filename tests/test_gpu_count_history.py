"""The count-table form of the token history (hist_counts) and its device
push, llmk_history_count_append: each row's history as its distinct tokens
with their occurrence counts, the form the scheduler's per-row counts take
(llm-scheduler/src/scheduler.rs:147 pushes one token per step; the penalties
of llm-core/src/sampler.rs:128-147 and the frequency penalty read only the
set of tokens and their counts).  Every result is checked bit for bit
against the CPU mirror oracle run on the expanded history (each token
repeated `count` times).  Marked gpu."""
import numpy as np
import pytest
import torch

import llmk
from llmk import _lib, synth
from oracle import llmk_oracle as O

from gpu_util import assert_bit_exact, workload

pytestmark = pytest.mark.gpu
CAP = 64


@pytest.fixture(scope="module")
def sampler():
    s = llmk.HipSampler(max_batch=512, max_vocab=256000)
    yield s
    s.close()


def rows_of(w):
    return [w.hist_tokens[w.hist_offsets[b]:w.hist_offsets[b + 1]] for b in range(w.B)]


def count_tables(hists, shuffle_seed=None, split=False):
    """(offsets, tokens, counts) of each row's distinct tokens, ascending, with
    their occurrences; shuffled and with one token split over two entries
    when asked (the sampler sums duplicates and reads any order)."""
    rng = np.random.default_rng(shuffle_seed)
    toks, cnts = [], []
    for h in hists:
        u, c = np.unique(np.asarray(h, np.uint32), return_counts=True)
        u, c = u.astype(np.uint32), c.astype(np.uint32)
        if split:
            big = np.nonzero(c >= 2)[0]
            if big.size:
                i = int(big[0])
                u = np.append(u, u[i])
                c = np.append(c, np.uint32(1))
                c[i] -= 1
        if shuffle_seed is not None:
            p = rng.permutation(u.size)
            u, c = u[p], c[p]
        toks.append(u)
        cnts.append(c)
    offs, tk = synth._csr(toks)
    _, ct = synth._csr(cnts)
    return offs, tk, ct


def run_counts(sampler, w, offs, toks, cnts, cap=CAP):
    db = w.to_device()
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a if a.size else np.zeros(1, np.uint32))
                                   .view(np.int32)).cuda()
    db.hist_offsets, db.hist_tokens, db.hist_counts = T(offs), T(toks), T(cnts)
    r = sampler.sample_batch(db, out_cap=cap)
    torch.cuda.synchronize()
    return (r.tokens.cpu().numpy().view(np.uint32), r.ids.cpu().numpy().view(np.uint32),
            r.probs.cpu().numpy(), r.count.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("name,B,shuffle,split", [
    ("C3", 32, None, False), ("C3", 16, 7, True), ("C5", 16, None, False),
    ("C2", 24, 3, True), ("C4", 16, None, False), ("C1", 1, None, False)])
def test_count_table_equals_the_expanded_history(sampler, name, B, shuffle, split):
    """hist_counts over each row's distinct tokens gives the tokens, kept ids
    and probabilities of the plain history (C2 and C4 rows also take the
    whole-row history tables of the exact normaliser and the slow path)."""
    w = synth.make(name, B=B)
    offs, toks, cnts = count_tables(rows_of(w), shuffle, split)
    print(f"[case] count table {name} B={B} shuffle={shuffle} split={split} "
          f"entries={toks.size} of {w.hist_tokens.size}", flush=True)
    gpu = run_counts(sampler, w, offs, toks, cnts)
    orc = O.sample_workload(O.MIRROR, w, out_cap=CAP, nthreads=16)
    assert_bit_exact(w, gpu, orc, CAP, f"count table {name}")


def test_count_table_with_many_distinct_tokens(sampler):
    """One segment per row (B 256) with more distinct tokens than one pass of
    the token waves (2048) and than the LDS rank tables (8192): the
    multi-pass and the all-waves table builds weigh each entry by its count,
    and the 9000-token rows are materialised by the slow path (status bit),
    every token penalised by its count.  All rows are checked against the
    oracle on the full histories."""
    rng = np.random.default_rng(91)
    B, V = 256, 151936
    lg = rng.normal(0, 3, (B, V)).astype(np.float32)
    hists = []
    for b in range(B):
        n = (3000, 6000, 9000)[b % 3]
        u = np.sort(rng.choice(V, n, replace=False)).astype(np.uint32)
        c = rng.integers(1, 7, n)
        hists.append(np.repeat(u, c))
    K = np.where(np.arange(B) % 2 == 0, 50, 0).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    args = dict(T=0.8, K=K, P=0.95, R=1.1, PR=0.5, FR=0.3, u=u)
    w = workload(lg, hists=hists, name="many distinct", **args)
    offs, toks, cnts = count_tables(hists)
    print("[case] many distinct: 3000 / 6000 / 9000 distinct tokens per row", flush=True)
    sampler.status()
    gpu = run_counts(sampler, w, offs, toks, cnts)
    assert sampler.status() & _lib.LLMK_STATUS_HISTORY_OVERFLOW  # the 9000-token rows
    orc = O.sample_workload(O.MIRROR, w, out_cap=CAP, nthreads=16)
    assert_bit_exact(w, gpu, orc, CAP, "many distinct")


def test_device_count_append_over_decode_steps(sampler):
    """Three decode steps of C3 rows on count tables in buffers of fixed
    capacity: each step is bit-exact against the oracle on the expanded
    history, and llmk_history_count_append between steps raises the count
    of a token already listed or inserts a new one in order; a full row
    keeps its table and raises LLMK_STATUS_HISTORY_FULL; an invalid token
    changes nothing."""
    w = synth.make("C3", B=24)
    B = w.B
    hists = [list(h) for h in rows_of(w)]
    tables = []
    for h in hists:
        u, c = np.unique(np.asarray(h, np.uint32), return_counts=True)
        tables.append((u.astype(np.uint32), c.astype(np.uint32)))
    cap = max(len(u) for u, _ in tables) + 2
    full_row = 3
    # fill row 3 to capacity with tokens it does not list (the highest ids)
    u, c = tables[full_row]
    extra = np.setdiff1d(np.arange(w.V, dtype=np.uint32), u)[-(cap - len(u)):]
    hists[full_row] += list(extra)
    u, c = np.unique(np.asarray(hists[full_row], np.uint32), return_counts=True)
    tables[full_row] = (u.astype(np.uint32), c.astype(np.uint32))
    assert len(u) == cap
    tok_buf = np.zeros(B * cap, np.uint32)
    cnt_buf = np.zeros(B * cap, np.uint32)
    for b, (u, c) in enumerate(tables):
        tok_buf[b * cap:b * cap + len(u)] = u
        cnt_buf[b * cap:b * cap + len(u)] = c
    d_off = torch.from_numpy((np.arange(B) * cap).astype(np.int32)).cuda()
    d_len = torch.from_numpy(np.array([len(u) for u, _ in tables], np.int32)).cuda()
    d_tok = torch.from_numpy(tok_buf.view(np.int32)).cuda()
    d_cnt = torch.from_numpy(cnt_buf.view(np.int32)).cuda()
    assert sampler.status() == 0
    for step in range(3):
        w.hist_offsets, w.hist_tokens = synth._csr([np.asarray(h, np.uint32) for h in hists])
        w.uniforms = np.random.default_rng(70 + step).random(B).astype(np.float32)
        print(f"[case] count append step {step}", flush=True)
        db = w.to_device()
        db.hist_offsets, db.hist_tokens, db.hist_lengths, db.hist_counts = d_off, d_tok, d_len, d_cnt
        r = sampler.sample_batch(db, out_cap=CAP)
        torch.cuda.synchronize()
        gpu = (r.tokens.cpu().numpy().view(np.uint32), r.ids.cpu().numpy().view(np.uint32),
               r.probs.cpu().numpy(), r.count.cpu().numpy().view(np.uint32))
        orc = O.sample_workload(O.MIRROR, w, out_cap=CAP, nthreads=16)
        assert_bit_exact(w, gpu, orc, CAP, f"count append step {step}")
        toks = r.tokens.clone()
        toks[5] = -1  # LLMK_INVALID_TOKEN: no push
        # the full row is offered a token it does not list
        toks[full_row] = int(np.setdiff1d(np.arange(4096, dtype=np.uint32), tables[full_row][0])[0])
        if step == 1:
            toks[7] = int(tables[7][0][0])  # a token already listed: its count rises
        sampler.history_count_append(d_off, d_len, d_tok, d_cnt, cap, toks)
        torch.cuda.synchronize()
        pushed = toks.cpu().numpy().view(np.uint32)
        ln = d_len.cpu().numpy()
        tb = d_tok.cpu().numpy().view(np.uint32)
        cb = d_cnt.cpu().numpy().view(np.uint32)
        for b in range(B):
            u, c = tables[b]
            t = pushed[b]
            if t != _lib.LLMK_INVALID_TOKEN:
                if t in u:
                    c = c.copy()
                    c[np.searchsorted(u, t)] += 1
                    hists[b].append(t)
                elif len(u) < cap:
                    i = np.searchsorted(u, t)
                    u, c = np.insert(u, i, t), np.insert(c, i, np.uint32(1))
                    hists[b].append(t)
            tables[b] = (u, c)
            assert ln[b] == len(u), f"row {b}"
            assert np.array_equal(tb[b * cap:b * cap + len(u)], u), f"row {b} tokens"
            assert np.array_equal(cb[b * cap:b * cap + len(u)], c), f"row {b} counts"
        assert sampler.status() == _lib.LLMK_STATUS_HISTORY_FULL


def test_count_append_long_tables(sampler):
    """Tables longer than one pass of the push kernel (2048 entries per
    chunk): insertion at the front, the middle and the end moves every entry
    above it once, and counts follow their tokens."""
    rng = np.random.default_rng(5)
    n, cap = 5000, 5003
    base = np.sort(rng.choice(np.arange(1, 200000, 2), n, replace=False)).astype(np.uint32)
    cnt = rng.integers(1, 9, n).astype(np.uint32)
    new = np.array([0, base[2500] + 1, 400001, base[17]], np.uint32)  # front, middle, end, repeat
    B = len(new)
    buf_t = np.zeros(B * cap, np.uint32)
    buf_c = np.zeros(B * cap, np.uint32)
    for b in range(B):
        buf_t[b * cap:b * cap + n] = base
        buf_c[b * cap:b * cap + n] = cnt
    d_off = torch.from_numpy((np.arange(B) * cap).astype(np.int32)).cuda()
    d_len = torch.full((B,), n, dtype=torch.int32, device="cuda:0")
    d_tok = torch.from_numpy(buf_t.view(np.int32)).cuda()
    d_cnt = torch.from_numpy(buf_c.view(np.int32)).cuda()
    toks = torch.from_numpy(new.view(np.int32)).cuda()
    print("[case] long count tables", flush=True)
    sampler.history_count_append(d_off, d_len, d_tok, d_cnt, cap, toks)
    torch.cuda.synchronize()
    tb = d_tok.cpu().numpy().view(np.uint32)
    cb = d_cnt.cpu().numpy().view(np.uint32)
    ln = d_len.cpu().numpy()
    for b, t in enumerate(new):
        u, c = base, cnt.copy()
        if t in u:
            c[np.searchsorted(u, t)] += 1
        else:
            i = np.searchsorted(u, t)
            u, c = np.insert(u, i, t), np.insert(c, i, np.uint32(1))
        assert ln[b] == len(u)
        assert np.array_equal(tb[b * cap:b * cap + len(u)], u), f"row {b}"
        assert np.array_equal(cb[b * cap:b * cap + len(u)], c), f"row {b}"


def test_count_append_to_a_zero_count_entry(sampler):
    """A listed token with count 0 is read as one occurrence (the sampler
    weighs a listed entry at least 1); appending it once more makes 2, and
    the next step's frequency penalty sees 2 occurrences."""
    cap = 8
    base = np.array([3, 7, 11], np.uint32)
    cnt = np.array([0, 2, 0], np.uint32)
    buf_t = np.zeros(cap, np.uint32)
    buf_c = np.zeros(cap, np.uint32)
    buf_t[:3], buf_c[:3] = base, cnt
    d_off = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    d_len = torch.full((1,), 3, dtype=torch.int32, device="cuda:0")
    d_tok = torch.from_numpy(buf_t.view(np.int32)).cuda()
    d_cnt = torch.from_numpy(buf_c.view(np.int32)).cuda()
    print("[case] append to a zero-count entry", flush=True)
    sampler.history_count_append(d_off, d_len, d_tok, d_cnt, cap,
                                 torch.tensor([3], dtype=torch.int32, device="cuda:0"))
    torch.cuda.synchronize()
    cb = d_cnt.cpu().numpy().view(np.uint32)
    assert list(cb[:3]) == [2, 2, 0], cb[:3]
    assert int(d_len.cpu()[0]) == 3
