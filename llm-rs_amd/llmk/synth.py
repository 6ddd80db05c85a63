"""Seeded synthetic sampling workloads (numpy only).

The five configurations of the benchmark contract, with the distributions the
task statement fixes (logit laws, spikes, Zipf histories, bitmask runs).  Where
it leaves a value open (C2/C4 penalties) the choice is recorded in
CONFIG_NOTES.  Seeds: numpy PCG64(0x11A50000 + config index), overridable.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

CONFIG_NOTES = {
    "C2": "penalties not fixed by the task: repetition 1.1 on every non-greedy row, "
          "presence 0.2 and frequency 0.1 on every fourth row",
    "C4": "penalties not fixed by the task: repetition 1.1",
}


@dataclass
class Workload:
    name: str
    B: int
    V: int
    dtype: str                 # "f32", "bf16" or "f16"
    logits: np.ndarray         # float32 [B,V] (for bf16: the exact upcast of bf16_bits)
    bf16_bits: Optional[np.ndarray]  # uint16 [B,V]: the 16-bit logits when dtype is "bf16" or "f16"
    temperature: np.ndarray
    top_k: np.ndarray          # int32
    top_p: np.ndarray
    min_p: np.ndarray
    repetition: np.ndarray
    presence: np.ndarray
    frequency: np.ndarray
    hist_offsets: np.ndarray   # uint32 [B+1]
    hist_tokens: np.ndarray    # uint32
    mask: Optional[np.ndarray] # uint32 [B, words]
    uniforms: np.ndarray       # float32 [B], multiples of 2^-24 like rand 0.8's gen::<f32>()

    @property
    def mask_words(self) -> int:
        return 0 if self.mask is None else self.mask.shape[1]

    def to_device(self, dev="cuda:0"):
        """The workload as an llmk.DeviceBatch of torch CUDA tensors."""
        import torch
        from .sampler import DeviceBatch
        T = lambda a, dt=None: torch.from_numpy(
            np.ascontiguousarray(a) if dt is None else np.ascontiguousarray(a).view(dt)).to(dev)
        if self.dtype == "bf16":
            lg = T(self.bf16_bits, np.int16).view(torch.bfloat16)
        elif self.dtype == "f16":
            lg = T(self.bf16_bits, np.int16).view(torch.float16)
        else:
            lg = T(self.logits)
        ht = self.hist_tokens if self.hist_tokens.size else np.zeros(1, np.uint32)
        return DeviceBatch(
            logits=lg, uniforms=T(self.uniforms), vocab=self.V, temperature=T(self.temperature),
            top_k=T(self.top_k), top_p=T(self.top_p), min_p=T(self.min_p),
            repetition_penalty=T(self.repetition), presence_penalty=T(self.presence),
            frequency_penalty=T(self.frequency), hist_offsets=T(self.hist_offsets, np.int32),
            hist_tokens=T(ht, np.int32),
            allow_mask=None if self.mask is None else T(self.mask, np.int32))

    def algorithmic_bytes(self) -> int:
        """HBM bytes one step must move at minimum (logits once, histories,
        mask, per-row params/uniform/output)."""
        esz = 4 if self.dtype == "f32" else 2
        b = self.B * self.V * esz + 4 * int(self.hist_offsets[-1])
        if self.mask is not None:
            b += 4 * self.B * ((self.V + 31) // 32)
        b += self.B * (28 + 4 + 4)
        return b


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def uniforms_24bit(rng, n) -> np.ndarray:
    return (rng.integers(0, 1 << 24, size=n).astype(np.float64) / (1 << 24)).astype(np.float32)


def zipf_history(rng, V, H, s, perm) -> np.ndarray:
    ranks = np.arange(1, V + 1, dtype=np.float64)
    p = ranks ** (-s)
    p /= p.sum()
    r = rng.choice(V, size=H, p=p)
    return perm[r].astype(np.uint32)


def _csr(hists):
    offs = np.zeros(len(hists) + 1, dtype=np.uint32)
    for i, h in enumerate(hists):
        offs[i + 1] = offs[i] + len(h)
    toks = np.concatenate(hists).astype(np.uint32) if offs[-1] else np.zeros(0, np.uint32)
    return offs, toks


def make(name: str, seed: Optional[int] = None, B: Optional[int] = None,
         V: Optional[int] = None) -> Workload:
    """Build config `name` in {"C1".."C5"}; B/V may be shrunk for tests."""
    idx = int(name[1])
    rng = np.random.Generator(np.random.PCG64(0x11A50000 + idx if seed is None else seed))
    if name == "C1":
        B_, V_ = 1, 151936
    elif name == "C2":
        B_, V_ = 64, 151936
    elif name == "C3":
        B_, V_ = 256, 151936
    elif name == "C4":
        B_, V_ = 128, 128256
    elif name == "C5":
        B_, V_ = 512, 256000
    else:
        raise ValueError(name)
    B = B_ if B is None else B
    V = V_ if V is None else V
    f = lambda v: np.full(B, v, dtype=np.float32)
    mask = None
    bf16 = None
    if name == "C1":
        lg = rng.normal(0.0, 3.0, size=(B, V)).astype(np.float32)
        for b in range(B):
            sp = rng.choice(V, size=min(8, V), replace=False)
            lg[b, sp] += rng.uniform(8, 15, size=len(sp)).astype(np.float32)
        T, K, P, MP = f(0.8), np.full(B, 40, np.int32), f(0.95), f(0.0)
        R, PR, FR = f(1.1), f(0.0), f(0.0)
        hists = [rng.integers(0, V, size=64).astype(np.uint32) for _ in range(B)]
        dtype = "f32"
    elif name == "C2":
        lg = rng.normal(0.0, 2.5, size=(B, V)).astype(np.float32)
        for b in range(B):
            ns = int(rng.integers(4, 17))
            sp = rng.choice(V, size=min(ns, V), replace=False)
            lg[b, sp] += rng.uniform(6, 14, size=len(sp)).astype(np.float32)
        bf16 = to_bf16_bits(lg)
        lg = bf16_bits_to_f32(bf16)
        greedy = rng.random(B) < 0.25
        T = np.where(greedy, 0.0, rng.uniform(0.5, 1.2, size=B)).astype(np.float32)
        K = rng.choice(np.array([0, 20, 50, 100], np.int32), size=B).astype(np.int32)
        P = rng.uniform(0.8, 1.0, size=B).astype(np.float32)
        MP = rng.choice(np.array([0.0, 0.05], np.float32), size=B).astype(np.float32)
        R = np.where(greedy, 1.0, 1.1).astype(np.float32)
        quarter = (np.arange(B) % 4) == 3
        PR = np.where(quarter, 0.2, 0.0).astype(np.float32)
        FR = np.where(quarter, 0.1, 0.0).astype(np.float32)
        perm = rng.permutation(V)
        hists = [zipf_history(rng, V, int(rng.integers(256, 1025)), 1.1, perm) for _ in range(B)]
        dtype = "bf16"
    elif name == "C3":
        lg = rng.normal(0.0, 3.0, size=(B, V)).astype(np.float32)
        heavy = rng.random((B, V)) < 0.001
        lg[heavy] = rng.normal(8.0, 2.0, size=int(heavy.sum())).astype(np.float32)
        T, K, P, MP = f(0.7), np.full(B, 50, np.int32), f(0.95), f(0.0)
        R, PR, FR = f(1.1), f(0.5), f(0.3)
        perm = rng.permutation(V)
        hists = [zipf_history(rng, V, 2048, 1.1, perm) for _ in range(B)]
        dtype = "f32"
    elif name == "C4":
        lg = rng.normal(0.0, 3.0, size=(B, V)).astype(np.float32)
        T, K, P, MP = f(1.0), np.zeros(B, np.int32), f(0.9), f(0.0)
        R, PR, FR = f(1.1), f(0.0), f(0.0)
        perm = rng.permutation(V)
        hists = [zipf_history(rng, V, 512, 1.1, perm) for _ in range(B)]
        words = (V + 31) // 32
        mask = np.zeros((B, words), dtype=np.uint32)
        for b in range(B):
            target = int(rng.uniform(0.01, 0.05) * V)
            allowed = np.zeros(V, dtype=bool)
            while allowed.sum() < target:
                L = int(rng.integers(8, 65))
                s0 = int(rng.integers(0, max(1, V - L)))
                allowed[s0:s0 + L] = True
            bits = np.packbits(allowed.astype(np.uint8), bitorder="little")
            pad = np.zeros(words * 4, dtype=np.uint8)
            pad[:len(bits)] = bits
            mask[b] = pad.view(np.uint32)
        dtype = "f32"
    else:  # C5
        lg = rng.normal(0.0, 4.0, size=(B, V)).astype(np.float32)
        for b in range(B):
            sp = rng.choice(V, size=min(32, V), replace=False)
            lg[b, sp] += rng.uniform(10, 20, size=len(sp)).astype(np.float32)
        bf16 = to_bf16_bits(lg)
        lg = bf16_bits_to_f32(bf16)
        T, K, P, MP = f(0.9), np.full(B, 200, np.int32), f(0.98), f(0.02)
        R, PR, FR = f(1.0), f(0.0), f(0.5)
        perm = rng.permutation(V)
        hists = [zipf_history(rng, V, 4096, 1.05, perm) for _ in range(B)]
        dtype = "bf16"
    offs, toks = _csr(hists)
    u = uniforms_24bit(rng, B)
    return Workload(name, B, V, dtype, lg, bf16, T, K, P, MP, R, PR, FR, offs, toks, mask, u)
