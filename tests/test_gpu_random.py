"""A seeded sweep of random workloads through the C ABI, each compared bit
for bit with the CPU mirror oracle (tokens, kept counts, kept ids and
probabilities): random batch and vocabulary sizes, f32, bf16 and f16 logits of
several shapes (flat, peaked, quantised, with spikes), per-row parameters
mixing greedy rows, top-k from 1 to beyond V, top-p, min-p, all three
penalties, histories with duplicates and out-of-vocabulary ids, allow-masks
in runs, and edge uniforms.  It reaches the fast and general candidate paths,
the probability bins, the slow path and its fallback.  Marked gpu."""
import numpy as np
import pytest

import llmk

from gpu_util import assert_bit_exact, run_gpu, run_gpu_strided, workload
from oracle import llmk_oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sampler():
    s = llmk.HipSampler(max_batch=64, max_vocab=70000)
    yield s
    s.close()


def make_case(seed):
    rng = np.random.default_rng(0x5EED0000 + seed)
    B = int(rng.integers(1, 49))
    V = int(rng.choice([700, 1024, 4097, 20000, 33333, 65536, 69999]))
    shape = seed % 5
    if shape == 0:
        lg = rng.normal(0, 3, (B, V))
    elif shape == 1:
        lg = rng.normal(0, 0.4, (B, V))           # flat: wide nuclei
    elif shape == 2:
        lg = np.round(rng.normal(0, 2, (B, V)) * 4) / 4  # quantised: ties
    elif shape == 3:
        lg = rng.normal(0, 1.5, (B, V))
        for b in range(B):                          # spikes
            lg[b, rng.integers(0, V, 8)] += rng.uniform(5, 15, 8)
    else:
        lg = rng.normal(0, 6, (B, V))              # peaked
    lg = lg.astype(np.float32)
    T = np.where(rng.random(B) < 0.15, 0.0, rng.uniform(0.3, 1.5, B)).astype(np.float32)
    K = rng.choice([0, 0, 1, 5, 50, 300, 2000, V + 1], B).astype(np.int32)
    P = np.where(rng.random(B) < 0.3, 1.0, rng.uniform(0.3, 1.0, B)).astype(np.float32)
    MP = rng.choice([0.0, 0.0, 0.01, 0.1], B).astype(np.float32)
    R = np.where(rng.random(B) < 0.5, 1.0, rng.uniform(1.0, 1.5, B)).astype(np.float32)
    PR = np.where(rng.random(B) < 0.5, 0.0, rng.uniform(0, 1, B)).astype(np.float32)
    FR = np.where(rng.random(B) < 0.5, 0.0, rng.uniform(0, 0.5, B)).astype(np.float32)
    hists = []
    for b in range(B):
        n = int(rng.choice([0, 5, 200, 3000]))
        h = rng.zipf(1.1, n) % (V + 50)           # duplicates; some ids >= V
        hists.append(h.astype(np.uint32))
    mask = None
    if seed % 3 == 0:
        words = (V + 31) // 32
        bits = np.zeros((B, words * 32), np.uint8)
        for b in range(B):
            dens = rng.choice([0.01, 0.05, 0.5])
            for _ in range(max(1, int(V * dens / 32))):
                s0 = int(rng.integers(0, V))
                bits[b, s0:s0 + int(rng.integers(8, 65))] = 1
        mask = np.packbits(bits, axis=1, bitorder="little").view(np.uint32)
    u = rng.random(B).astype(np.float32)
    u[rng.random(B) < 0.1] = 0.0
    u[rng.random(B) < 0.1] = np.float32(1.0 - 2.0 ** -24)
    dtype = ("f32", "bf16", "f16")[(seed // 3) % 3]
    w = workload(lg, T=T, K=K, P=P, MP=MP, R=R, PR=PR, FR=FR, hists=hists, mask=mask, u=u,
                 dtype=dtype, name=f"random-{seed}")
    cap = int(rng.choice([0, 16, 300]))
    return w, cap


@pytest.mark.parametrize("seed", range(60))
def test_random_workloads(sampler, seed):
    w, cap = make_case(seed)
    print(f"[case] random seed={seed} B={w.B} V={w.V} dtype={w.dtype} cap={cap} "
          f"mask={w.mask is not None}", flush=True)
    # rows whose length breaks the 16-byte alignment go through a padded
    # stride (the padding holds +inf, which must never be read)
    gpu = (run_gpu_strided if w.V % 8 else run_gpu)(sampler, w, cap)
    orc = O.sample_workload(O.MIRROR, w, out_cap=cap, nthreads=16)
    assert_bit_exact(w, gpu, orc, cap, f"random-{seed}")
    assert sampler.status() == 0
