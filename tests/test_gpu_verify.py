"""llmk_verify_batch (speculative-decoding verification, docs/mlc-contracts.md:
83-84) through the C ABI against the oracle's llmk_oracle_verify_row, bit for
bit (tokens and accept flags), on the target lists llmk_sample_batch itself
returns: mixed parameters, draft tokens inside and outside the kept lists,
draft probabilities of zero, a not-normalised draft (the R = 0 branch), long
lists (top-p alone) and invalid rows.  Marked gpu."""
import numpy as np
import pytest
import torch

import llmk
from llmk import _lib
from oracle import llmk_oracle as O

from gpu_util import workload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    s = llmk.HipSampler(max_batch=64, max_vocab=32000)
    yield s
    s.close()


def target_lists(sampler, w, cap):
    db = w.to_device()
    r = sampler.sample_batch(db, out_cap=cap)
    torch.cuda.synchronize()
    return r.ids, r.probs, r.count


def softmax32(x):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return (e / e.sum(axis=1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("seed,V", [(0, 4096), (1, 32000), (2, 32000)])
def test_verify_matches_oracle(sampler, seed, V):
    rng = np.random.default_rng(seed)
    B = 48
    lg = rng.normal(0, 3, (B, V)).astype(np.float32)
    T = rng.choice([0.7, 1.0, 1.3], B).astype(np.float32)
    K = rng.choice([0, 20, 50, 200], B).astype(np.int32)
    P = rng.choice([1.0, 0.9, 0.95], B).astype(np.float32)
    w = workload(lg, T=T, K=K, P=P, u=rng.random(B).astype(np.float32), name=f"verify{seed}")
    cap = V
    ids, probs, cnt = target_lists(sampler, w, cap)
    # draft: a perturbed softmax; row kinds by b % 4: 0 a draft from q, 1 the
    # target's own top token, 2 a token outside the kept list, 3 a draft q of
    # 2p on the kept list (not normalised: R = 0 on rejection)
    q = softmax32(lg / T[:, None] + rng.normal(0, 1.0, (B, V)).astype(np.float32))
    hid, hp, hc = ids.cpu().numpy().view(np.uint32), probs.cpu().numpy(), cnt.cpu().numpy()
    d = np.zeros(B, np.uint32)
    for b in range(B):
        n = int(hc[b])
        kind = b % 4
        if kind == 0:
            pp = q[b].astype(np.float64)
            d[b] = rng.choice(V, p=pp / pp.sum())
        elif kind == 1:
            d[b] = hid[b, 0]
        elif kind == 2:
            outside = np.setdiff1d(np.arange(V), hid[b, :n])
            d[b] = outside[rng.integers(outside.size)] if outside.size else hid[b, 0]
        else:
            q[b] = 0.0
            q[b, hid[b, :n]] = 2.0 * hp[b, :n]
            d[b] = hid[b, rng.integers(n)]
        if b % 7 == 3:
            q[b, d[b]] = 0.0  # a draft that gives its own token zero mass
    ua = rng.random(B).astype(np.float32)
    ur = rng.random(B).astype(np.float32)
    ua[::5] = 0.999
    dev = "cuda:0"
    print(f"[case] verify seed={seed} V={V} B={B}", flush=True)
    tok, acc = sampler.verify_batch(ids, probs, cnt, torch.from_numpy(d.view(np.int32)).to(dev),
                                    torch.from_numpy(q).to(dev), torch.from_numpy(ua).to(dev),
                                    torch.from_numpy(ur).to(dev))
    torch.cuda.synchronize()
    gt, ga = tok.cpu().numpy().view(np.uint32), acc.cpu().numpy()
    kinds = {"accepted": 0, "resampled": 0}
    for b in range(B):
        n = int(hc[b])
        want = O.verify_row(hid[b, :n], hp[b, :n], int(d[b]), q[b], ua[b], ur[b])
        assert (int(gt[b]), int(ga[b])) == want, f"row {b}: gpu {(gt[b], ga[b])} oracle {want}"
        kinds["accepted" if want[1] else "resampled"] += 1
    assert kinds["accepted"] > 0 and kinds["resampled"] > 0
    assert sampler.status() == 0


def test_verify_invalid_rows(sampler):
    V = 1000
    lg = np.random.default_rng(5).normal(0, 2, (4, V)).astype(np.float32)
    w = workload(lg, T=1.0, P=0.99, name="verify-invalid")
    ids, probs, cnt = target_lists(sampler, w, 8)  # top-p 0.99 keeps more than 8
    dev = "cuda:0"
    d = torch.tensor([0, 1, 2, V + 3], dtype=torch.int32, device=dev)
    q = torch.full((4, V), 1.0 / V, device=dev)
    u = torch.full((4,), 0.5, device=dev)
    print("[case] verify invalid rows", flush=True)
    tok, acc = sampler.verify_batch(ids, probs, cnt, d, q, u, u)
    torch.cuda.synchronize()
    assert (tok.cpu().numpy().view(np.uint32) == _lib.LLMK_INVALID_TOKEN).all()
    assert (acc.cpu().numpy() == 0).all()
    assert sampler.status() & _lib.LLMK_STATUS_INVALID_PARAMS
