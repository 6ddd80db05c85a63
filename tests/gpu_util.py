"""Helpers shared by the GPU tests: move a synth.Workload to cuda:0, run the
engine through the C ABI, run the CPU mirror oracle, compare."""
import numpy as np
import torch

import llmk
from oracle import llmk_oracle as O


def to_device(w, dev="cuda:0"):
    return w.to_device(dev)


def run_gpu(sampler, w, out_cap=64):
    db = to_device(w)
    r = sampler.sample_batch(db, out_cap=out_cap)
    torch.cuda.synchronize()
    tok = r.tokens.cpu().numpy().view(np.uint32)
    cnt = r.count.cpu().numpy().view(np.uint32)
    ids = r.ids.cpu().numpy().view(np.uint32) if out_cap else None
    probs = r.probs.cpu().numpy() if out_cap else None
    return tok, ids, probs, cnt


def assert_bit_exact(w, gpu, orc, out_cap, label=""):
    tok, ids, probs, cnt = gpu
    rc, otok, oids, oprobs, ocnt = orc
    assert rc == 0
    bad = np.nonzero(tok != otok)[0]
    assert bad.size == 0, f"{label}: token mismatch rows {bad[:10]} gpu={tok[bad[:10]]} oracle={otok[bad[:10]]}"
    bad = np.nonzero(cnt != ocnt)[0]
    assert bad.size == 0, f"{label}: kept-count mismatch rows {bad[:10]} gpu={cnt[bad[:10]]} oracle={ocnt[bad[:10]]}"
    if out_cap:
        for b in range(w.B):
            n = min(int(ocnt[b]), out_cap)
            assert np.array_equal(ids[b, :n], oids[b, :n]), f"{label}: row {b} ids differ"
            assert np.array_equal(probs[b, :n].view(np.uint32), oprobs[b, :n].view(np.uint32)), \
                f"{label}: row {b} probs differ: {probs[b, :n][:8]} vs {oprobs[b, :n][:8]}"
