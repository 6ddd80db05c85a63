"""GPU parity: the HIP engine (through the C ABI) against the CPU mirror oracle,
bit for bit (tokens, kept counts, kept ids and probabilities), on the five
benchmark configurations.  Marked gpu."""
import numpy as np
import pytest

import llmk
from llmk import synth
from oracle import llmk_oracle as O

from gpu_util import assert_bit_exact, run_gpu

pytestmark = pytest.mark.gpu

CAP = 64


@pytest.fixture(scope="module")
def sampler():
    s = llmk.HipSampler(max_batch=512, max_vocab=256000)
    yield s
    s.close()


@pytest.mark.parametrize("name,B", [("C1", None), ("C2", 16), ("C3", 32), ("C4", 16), ("C5", 16)])
def test_config_rows_match_mirror(sampler, name, B):
    w = synth.make(name, B=B)
    print(f"[case] {name} B={w.B} V={w.V}", flush=True)
    gpu = run_gpu(sampler, w, CAP)
    orc = O.sample_workload(O.MIRROR, w, out_cap=CAP, nthreads=16)
    assert_bit_exact(w, gpu, orc, CAP, name)
    assert sampler.status() == 0


@pytest.mark.parametrize("name", ["C3"])
def test_full_size_matches_mirror(sampler, name):
    w = synth.make(name)
    print(f"[case] full {name} B={w.B} V={w.V}", flush=True)
    gpu = run_gpu(sampler, w, CAP)
    orc = O.sample_workload(O.MIRROR, w, out_cap=CAP, nthreads=16)
    assert_bit_exact(w, gpu, orc, CAP, name)
