"""Batches above 512 rows: rows b and b + 512 share one slow-path scratch slot
(row b uses slot b mod min(max_batch, 512)), taken under a bounded spin
lock.  Slow rows (top-k off, a nucleus of thousands of tokens) sit on both
sides of the wrap, fast rows between them; every row must match the mirror
oracle bit for bit and no slot may time out.  Marked gpu."""
import numpy as np
import pytest

import llmk
from llmk import _lib
from oracle import llmk_oracle as O

from gpu_util import assert_bit_exact, run_gpu, workload

pytestmark = pytest.mark.gpu


def test_rows_sharing_slow_slots():
    B, V = 520, 16384
    rng = np.random.default_rng(21)
    lg = rng.normal(0, 0.5, (B, V)).astype(np.float32)
    K = np.full(B, 50, np.int32)
    P = np.full(B, 0.95, np.float32)
    slow = [0, 1, 2, 3, 7, 100, 512, 513, 514, 515, 519]
    K[slow] = 0
    P[slow] = 0.99
    w = workload(lg, T=1.0, K=K, P=P, R=1.1, hists=[rng.integers(0, V, 64) for _ in range(B)],
                 u=rng.random(B).astype(np.float32), name="slots")
    s = llmk.HipSampler(max_batch=B, max_vocab=V)
    try:
        print(f"[case] B={B} V={V} slow rows {slow}", flush=True)
        gpu = run_gpu(s, w, 64)
        orc = O.sample_workload(O.MIRROR, w, out_cap=64, nthreads=16)
        assert_bit_exact(w, gpu, orc, 64, "slots")
        # the slow rows' nuclei are far above the candidate path's 4096
        assert (gpu[3][slow] > 4096).all(), gpu[3][slow]
        st = s.status()
        assert not st & _lib.LLMK_STATUS_SLOT_TIMEOUT
        assert st == 0
    finally:
        s.close()
