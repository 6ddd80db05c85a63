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


def workload(logits, T=1.0, K=0, P=1.0, MP=0.0, R=1.0, PR=0.0, FR=0.0, hists=None, mask=None,
             u=0.5, dtype="f32", name="case"):
    """A synth.Workload from explicit per-row values (scalars broadcast)."""
    from llmk import synth
    lg = np.atleast_2d(np.asarray(logits, np.float32))
    B, V = lg.shape
    bf = None
    if dtype == "bf16":
        bf = synth.to_bf16_bits(lg)
        lg = synth.bf16_bits_to_f32(bf)
    elif dtype == "f16":  # round to half, keep its exact upcast
        h = lg.astype(np.float16)
        bf = h.view(np.uint16)
        lg = h.astype(np.float32)
    col = lambda x, dt=np.float32: np.broadcast_to(np.asarray(x, dt), (B,)).copy()
    hists = hists if hists is not None else [[] for _ in range(B)]
    offs, toks = synth._csr([np.asarray(h, np.uint32) for h in hists])
    return synth.Workload(name, B, V, dtype, lg, bf, col(T), col(K, np.int32), col(P), col(MP),
                          col(R), col(PR), col(FR), offs, toks, mask, col(u))


def run_gpu_strided(sampler, w, out_cap=64, extra=4):
    """Like run_gpu, with each row padded to a stride above V (a multiple of
    8 elements) and the padding filled with +inf, which must never be read."""
    import torch
    db = w.to_device()
    stride = ((w.V + extra + 7) // 8) * 8
    if w.dtype in ("bf16", "f16"):
        pad = np.full((w.B, stride), 0x7F80 if w.dtype == "bf16" else 0x7C00, np.uint16)
        pad[:, :w.V] = w.bf16_bits
        lg = torch.from_numpy(pad.view(np.int16)).to("cuda:0").view(
            torch.bfloat16 if w.dtype == "bf16" else torch.float16)
    else:
        pad = np.full((w.B, stride), np.inf, np.float32)
        pad[:, :w.V] = w.logits
        lg = torch.from_numpy(pad).to("cuda:0")
    db.logits = lg
    db.vocab = w.V
    r = sampler.sample_batch(db, out_cap=out_cap)
    torch.cuda.synchronize()
    tok = r.tokens.cpu().numpy().view(np.uint32)
    cnt = r.count.cpu().numpy().view(np.uint32)
    ids = r.ids.cpu().numpy().view(np.uint32) if out_cap else None
    probs = r.probs.cpu().numpy() if out_cap else None
    return tok, ids, probs, cnt


def run_gpu_offset(sampler, w, out_cap=64, offset=1, extra=3):
    """Like run_gpu, with row b at element offset + b * (V + extra) of one
    buffer (rows at any alignment), the rest of the buffer +inf, which must
    never be read."""
    import torch
    db = w.to_device()
    stride = w.V + extra
    n = w.B * stride + offset + 8
    if w.dtype in ("bf16", "f16"):
        buf = np.full(n, 0x7F80 if w.dtype == "bf16" else 0x7C00, np.uint16)
        for b in range(w.B):
            buf[offset + b * stride:offset + b * stride + w.V] = w.bf16_bits[b]
        t = torch.from_numpy(buf.view(np.int16)).to("cuda:0").view(
            torch.bfloat16 if w.dtype == "bf16" else torch.float16)
    else:
        buf = np.full(n, np.inf, np.float32)
        for b in range(w.B):
            buf[offset + b * stride:offset + b * stride + w.V] = w.logits[b]
        t = torch.from_numpy(buf).to("cuda:0")
    db.logits = t.as_strided((w.B, w.V), (stride, 1), offset)
    db.vocab = w.V
    r = sampler.sample_batch(db, out_cap=out_cap)
    torch.cuda.synchronize()
    tok = r.tokens.cpu().numpy().view(np.uint32)
    cnt = r.count.cpu().numpy().view(np.uint32)
    ids = r.ids.cpu().numpy().view(np.uint32) if out_cap else None
    probs = r.probs.cpu().numpy() if out_cap else None
    return tok, ids, probs, cnt
