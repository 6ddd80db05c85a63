"""Helpers shared by the GPU tests: move a synth.Workload to cuda:0, run the
engine through the C ABI, run the CPU mirror oracle, compare."""
import numpy as np
import torch

import llmk
from oracle import llmk_oracle as O


def to_device(w, dev="cuda:0"):
    T = lambda a, dt=None: torch.from_numpy(
        np.ascontiguousarray(a) if dt is None else np.ascontiguousarray(a).view(dt)).to(dev)
    if w.dtype == "bf16":
        lg = T(w.bf16_bits, np.int16).view(torch.bfloat16)
    else:
        lg = T(w.logits)
    ht = w.hist_tokens if w.hist_tokens.size else np.zeros(1, np.uint32)
    return llmk.DeviceBatch(
        logits=lg, uniforms=T(w.uniforms), vocab=w.V, temperature=T(w.temperature),
        top_k=T(w.top_k), top_p=T(w.top_p), min_p=T(w.min_p),
        repetition_penalty=T(w.repetition), presence_penalty=T(w.presence),
        frequency_penalty=T(w.frequency), hist_offsets=T(w.hist_offsets, np.int32),
        hist_tokens=T(ht, np.int32),
        allow_mask=None if w.mask is None else T(w.mask, np.int32))


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
