"""ctypes binding of the CPU oracle (oracle/_build/libllmk_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker / CPU baseline.  The product path
(llm-rs_amd) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libllmk_oracle.so")
REF, MIRROR = 0, 1

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB):
        build()
    lib = ctypes.CDLL(LIB)
    P = ctypes.c_void_p
    u32, i32, f32 = ctypes.c_uint32, ctypes.c_int32, ctypes.c_float
    lib.llmk_oracle_sample_batch.argtypes = [
        ctypes.c_int, P, u32, u32, ctypes.c_uint64, P, P, P, P, P, P, P, P, P, P, u32,
        P, P, P, P, u32, P, ctypes.c_int]
    lib.llmk_oracle_sample_batch.restype = ctypes.c_int
    lib.llmk_oracle_sample_row.argtypes = [ctypes.c_int, P, u32, P, P, u32, P, f32, P, P, P, u32, P]
    lib.llmk_oracle_sample_row.restype = ctypes.c_int
    lib.llmk_oracle_process_logits.argtypes = [ctypes.c_int, P, u32, P, P, u32, P, P]
    lib.llmk_oracle_process_logits.restype = ctypes.c_int
    lib.llmk_oracle_sorted_e.argtypes = [P, u32, P, P, u32, P, u32, P, P]
    lib.llmk_oracle_sorted_e.restype = ctypes.c_int
    lib.llmk_oracle_band_certain.argtypes = [P, P, u32, u32, f32, P, f32]
    lib.llmk_oracle_band_certain.restype = ctypes.c_int
    lib.llmk_oracle_semantics.argtypes = [P, P, u32, P, f32, P, P, P, u32, P]
    lib.llmk_oracle_semantics.restype = ctypes.c_int
    lib.llmk_oracle_exp_ref.argtypes = [f32]
    lib.llmk_oracle_exp_ref.restype = f32
    lib.llmk_oracle_libm_expf.argtypes = [f32]
    lib.llmk_oracle_libm_expf.restype = f32
    lib.llmk_oracle_apply_repetition_penalty.argtypes = [P, u32, P, u32, f32]
    lib.llmk_oracle_apply_temperature.argtypes = [P, u32, f32]
    lib.llmk_oracle_apply_top_k.argtypes = [P, u32, ctypes.c_int64]
    lib.llmk_oracle_apply_top_p.argtypes = [ctypes.c_int, P, u32, f32]
    lib.llmk_oracle_sample_simple.argtypes = [ctypes.c_int, P, u32, f32, f32]
    lib.llmk_oracle_sample_simple.restype = u32
    lib.llmk_oracle_verify_row.argtypes = [u32, P, P, u32, P, u32, f32, f32,
                                           ctypes.POINTER(u32), ctypes.POINTER(u32)]
    lib.llmk_oracle_verify_row.restype = ctypes.c_int
    lib.llmk_oracle_softcap.argtypes = [ctypes.c_int, P, u32, f32]
    lib.llmk_oracle_tanh_ref.argtypes = [f32]
    lib.llmk_oracle_tanh_ref.restype = f32
    lib.llmk_oracle_expm1_ref.argtypes = [f32]
    lib.llmk_oracle_expm1_ref.restype = f32
    lib.llmk_oracle_tanh_scan.argtypes = [u32, u32, ctypes.POINTER(ctypes.c_uint64),
                                          ctypes.POINTER(ctypes.c_uint64)]
    u64p = ctypes.POINTER(ctypes.c_uint64)
    lib.llmk_oracle_exp_scan.argtypes = [u32, u32, u64p, u64p, u64p, ctypes.POINTER(u32)]
    _lib = lib
    return lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def sample_batch(mode, logits, temperature=None, top_k=None, top_p=None, min_p=None,
                 repetition=None, presence=None, frequency=None, hist_offsets=None,
                 hist_tokens=None, mask=None, uniforms=None, out_cap=0, nthreads=1, V=None):
    """Returns (tokens, ids, probs, counts) as numpy arrays.  logits: float32 [B, stride]."""
    lib = load()
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    B, stride = logits.shape
    V = stride if V is None else V
    c = lambda a, dt: None if a is None else np.ascontiguousarray(a, dtype=dt)
    T, K, TP, MP = c(temperature, np.float32), c(top_k, np.int32), c(top_p, np.float32), c(min_p, np.float32)
    R, PR, FR = c(repetition, np.float32), c(presence, np.float32), c(frequency, np.float32)
    HO, HT = c(hist_offsets, np.uint32), c(hist_tokens, np.uint32)
    if HT is not None and HT.size == 0:
        HT = np.zeros(1, np.uint32)
    M = c(mask, np.uint32)
    U = c(uniforms if uniforms is not None else np.zeros(B), np.float32)
    tok = np.zeros(B, np.uint32)
    cnt = np.zeros(B, np.uint32)
    ids = np.zeros((B, max(out_cap, 1)), np.uint32)
    probs = np.zeros((B, max(out_cap, 1)), np.float32)
    rc = lib.llmk_oracle_sample_batch(
        mode, _p(logits), B, V, stride, _p(T), _p(K), _p(TP), _p(MP), _p(R), _p(PR), _p(FR),
        _p(HO), _p(HT), _p(M), 0 if M is None else M.shape[1], _p(U), _p(tok),
        _p(ids) if out_cap else None, _p(probs) if out_cap else None, out_cap, _p(cnt), nthreads)
    return rc, tok, ids[:, :out_cap], probs[:, :out_cap], cnt


def sample_workload(mode, w, out_cap=0, nthreads=1, rows=None):
    """Run the oracle on an llmk.synth.Workload (optionally a subset of rows)."""
    sel = slice(None) if rows is None else rows
    lg = w.logits[sel]
    ho, ht = w.hist_offsets, w.hist_tokens
    if rows is not None:
        idx = np.arange(w.B)[sel]
        hs = [ht[ho[i]:ho[i + 1]] for i in idx]
        ho = np.zeros(len(hs) + 1, np.uint32)
        for i, h in enumerate(hs):
            ho[i + 1] = ho[i] + len(h)
        ht = np.concatenate(hs).astype(np.uint32) if ho[-1] else np.zeros(0, np.uint32)
    return sample_batch(mode, lg, w.temperature[sel], w.top_k[sel], w.top_p[sel], w.min_p[sel],
                        w.repetition[sel], w.presence[sel], w.frequency[sel], ho, ht,
                        None if w.mask is None else w.mask[sel], w.uniforms[sel], out_cap, nthreads)


class Params(ctypes.Structure):
    """llmk_oracle_params (oracle/llmk_oracle.h)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32),
                ("top_p", ctypes.c_float), ("min_p", ctypes.c_float),
                ("repetition_penalty", ctypes.c_float), ("presence_penalty", ctypes.c_float),
                ("frequency_penalty", ctypes.c_float)]


def params(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repetition=1.0, presence=0.0,
           frequency=0.0):
    return Params(temperature, top_k, top_p, min_p, repetition, presence, frequency)


def sample_row(mode, logits, prm, hist=(), mask=None, u=0.0, out_cap=None):
    """One row.  Returns (rc, token, ids, probs, count); out_cap defaults to V."""
    lib = load()
    l = _f32p(logits)
    V = l.size
    cap = V if out_cap is None else out_cap
    h = np.ascontiguousarray(hist, dtype=np.uint32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
    tok, cnt = ctypes.c_uint32(), ctypes.c_uint32()
    ids = np.zeros(max(cap, 1), np.uint32)
    probs = np.zeros(max(cap, 1), np.float32)
    rc = lib.llmk_oracle_sample_row(mode, _p(l) if V else None, V, ctypes.byref(prm),
                                    _p(h) if h.size else None, h.size, _p(m), u,
                                    ctypes.byref(tok), _p(ids), _p(probs), cap, ctypes.byref(cnt))
    n = min(cnt.value, cap)
    return rc, tok.value, ids[:n], probs[:n], cnt.value


def semantics(p_sorted, idx, prm, u=0.0, out_cap=None):
    """min-p / top-k / top-p / draw on a sorted list.  Returns (rc, token, ids, probs, count)."""
    lib = load()
    p = _f32p(p_sorted)
    ix = np.ascontiguousarray(idx, dtype=np.uint32)
    n = p.size
    cap = n if out_cap is None else out_cap
    tok, cnt = ctypes.c_uint32(), ctypes.c_uint32()
    ids = np.zeros(max(cap, 1), np.uint32)
    probs = np.zeros(max(cap, 1), np.float32)
    rc = lib.llmk_oracle_semantics(_p(p), _p(ix), n, ctypes.byref(prm), u, ctypes.byref(tok),
                                   _p(ids), _p(probs), cap, ctypes.byref(cnt))
    k = min(cnt.value, cap)
    return rc, tok.value, ids[:k], probs[:k], cnt.value


def sorted_e(logits, prm, hist=(), mask=None, n=None):
    """The row's first n entries with S = 1, (e, idx) in (e desc, idx asc)
    order (llmk_oracle_sorted_e)."""
    l = _f32p(logits)
    n = l.size if n is None else min(n, l.size)
    h = np.ascontiguousarray(hist, dtype=np.uint32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
    e = np.zeros(n, np.float32)
    ix = np.zeros(n, np.uint32)
    rc = load().llmk_oracle_sorted_e(_p(l), l.size, ctypes.byref(prm), _p(h) if h.size else None,
                                     h.size, _p(m), n, _p(e), _p(ix))
    if rc != 0:
        raise ValueError(f"oracle rc {rc}")
    return e, ix


def band_certain(e_sorted, idx, prm, u, E=None, full=None, ptail=0.0):
    """llmk_oracle_band_certain: True when S = 1's decisions on the sorted
    list are the reference's for every normaliser S."""
    e = _f32p(e_sorted)
    ix = np.ascontiguousarray(idx, dtype=np.uint32)
    E = e.size if E is None else E
    full = e.size if full is None else full
    return bool(load().llmk_oracle_band_certain(_p(e), _p(ix), E, full, float(ptail),
                                                ctypes.byref(prm), float(u)))


def process_logits(mode, logits, prm, hist=(), mask=None):
    """Penalised + masked logits of one row (before greedy / temperature)."""
    lib = load()
    l = _f32p(logits)
    out = np.zeros_like(l)
    h = np.ascontiguousarray(hist, dtype=np.uint32)
    m = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint32)
    rc = lib.llmk_oracle_process_logits(mode, _p(l), l.size, ctypes.byref(prm),
                                        _p(h) if h.size else None, h.size, _p(m), _p(out))
    if rc != 0:
        raise ValueError(f"oracle rc {rc}")
    return out


def _f32p(x):
    return np.ascontiguousarray(x, dtype=np.float32)


def apply_repetition_penalty(logits, hist, penalty):
    l = _f32p(logits).copy()
    h = np.ascontiguousarray(hist, dtype=np.uint32)
    load().llmk_oracle_apply_repetition_penalty(_p(l), l.size, _p(h) if h.size else None, h.size, penalty)
    return l


def apply_temperature(logits, t):
    l = _f32p(logits).copy()
    load().llmk_oracle_apply_temperature(_p(l), l.size, t)
    return l


def apply_top_k(logits, k):
    l = _f32p(logits).copy()
    load().llmk_oracle_apply_top_k(_p(l), l.size, k)
    return l


def apply_top_p(mode, logits, top_p):
    l = _f32p(logits).copy()
    load().llmk_oracle_apply_top_p(mode, _p(l), l.size, top_p)
    return l


def apply_logit_bias(logits, tokens, values):
    """Logit bias, the formula of llm-tests/tests/mlc_parity.rs:1060-1072
    (logits[idx] += bias, in f32), for each (token, bias) pair in list order;
    ids >= len(logits) are ignored."""
    l = _f32p(logits).copy()
    for t, v in zip(tokens, values):
        if int(t) < l.size:
            l[int(t)] = np.float32(l[int(t)] + np.float32(v))
    return l


def sample_simple(mode, logits, t, u):
    l = _f32p(logits)
    return int(load().llmk_oracle_sample_simple(mode, _p(l), l.size, t, u))


def exp_ref(y):
    return np.float32(load().llmk_oracle_exp_ref(float(y)))


def libm_expf(y):
    return np.float32(load().llmk_oracle_libm_expf(float(y)))


def exp_scan(lo_bits, hi_bits):
    a, b, c = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    d = ctypes.c_uint32()
    load().llmk_oracle_exp_scan(lo_bits, hi_bits, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c), ctypes.byref(d))
    return a.value, b.value, c.value, d.value


def verify_row(ids, probs, d, q, u_a, u_r):
    """Speculative verification of one row (docs/mlc-contracts.md:83-84):
    the target's kept list (ids, probs), draft token d, draft distribution q
    over the vocabulary; returns (token, accepted), token 0xffffffff for an
    invalid row."""
    i = np.ascontiguousarray(ids, dtype=np.uint32)
    p = np.ascontiguousarray(probs, dtype=np.float32)
    qq = np.ascontiguousarray(q, dtype=np.float32)
    tok, acc = ctypes.c_uint32(), ctypes.c_uint32()
    load().llmk_oracle_verify_row(i.size, _p(i), _p(p), int(d), _p(qq), qq.size, float(u_a),
                                  float(u_r), ctypes.byref(tok), ctypes.byref(acc))
    return tok.value, acc.value


DTYPES = {"f32": 0, "bf16": 1, "f16": 2}


def softcap(dtype, logits, cap):
    """final_logit_softcapping (candle.rs:1803-1807) in the logits' dtype
    ("f32", "bf16", "f16"; values given as float32), as a new array."""
    l = np.ascontiguousarray(logits, dtype=np.float32).copy()
    load().llmk_oracle_softcap(DTYPES[dtype], _p(l), l.size, float(cap))
    return l


def tanh_ref(x):
    return np.float32(load().llmk_oracle_tanh_ref(float(x)))


def tanh_scan(lo_bits, hi_bits):
    a, b = ctypes.c_uint64(), ctypes.c_uint64()
    load().llmk_oracle_tanh_scan(lo_bits, hi_bits, ctypes.byref(a), ctypes.byref(b))
    return a.value, b.value
