"""llmk_sample_batch_static, the sampling call that allocates nothing, against
llmk_sample_batch on a handle: the same tokens, kept counts, kept ids and
probability bits, on two calls in a row (the second smaller, so it runs on
what the first left in the static workspace), plus its status word and its
size limits.  Marked gpu; every call goes through the C ABI."""
import numpy as np
import pytest
import torch

import llmk
from llmk import _lib, synth

pytestmark = pytest.mark.gpu

CAP = 64


def outputs(B, dev="cuda:0"):
    return (torch.empty(B, dtype=torch.int32, device=dev),
            torch.empty(B, CAP, dtype=torch.int32, device=dev),
            torch.empty(B, CAP, dtype=torch.float32, device=dev),
            torch.empty(B, dtype=torch.int32, device=dev))


def host(outs):
    tok, ids, probs, cnt = (t.cpu().numpy() for t in outs)
    return tok.view(np.uint32), ids.view(np.uint32), probs, cnt.view(np.uint32)


def assert_same(w, a, b, label):
    tok, ids, probs, cnt = a
    rtok, rids, rprobs, rcnt = b
    bad = np.nonzero(tok != rtok)[0]
    assert bad.size == 0, f"{label}: token mismatch rows {bad[:10]}: {tok[bad[:10]]} vs {rtok[bad[:10]]}"
    assert np.array_equal(cnt, rcnt), f"{label}: kept counts differ"
    for r in range(w.B):
        n = min(int(cnt[r]), CAP)
        assert np.array_equal(ids[r, :n], rids[r, :n]), f"{label}: row {r} ids differ"
        assert np.array_equal(probs[r, :n].view(np.uint32), rprobs[r, :n].view(np.uint32)), \
            f"{label}: row {r} probabilities differ"


@pytest.fixture(scope="module")
def sampler():
    s = llmk.HipSampler(max_batch=256, max_vocab=151936)
    yield s
    s.close()


def test_static_matches_handle_on_two_calls(sampler):
    # C3 at full size (256 rows, fp32), then 24 rows of C2 (bf16, mixed
    # parameters with rows on the slow path)
    for name, B in (("C3", None), ("C2", 24)):
        w = synth.make(name, B=B)
        print(f"[case] static vs handle {name} B={w.B} V={w.V}", flush=True)
        db = w.to_device()
        ref = outputs(w.B)
        sampler.launch(db, *ref)
        torch.cuda.synchronize()
        assert sampler.status() == 0
        got = outputs(w.B)
        status = torch.zeros(1, dtype=torch.int32, device="cuda:0")
        free0 = torch.cuda.mem_get_info()[0]
        llmk.sample_batch_static(db, *got, status=status)
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        assert_same(w, host(got), host(ref), name)
        assert int(status.item()) == 0
        if name == "C2":  # the workspace is resident since the first call
            assert free1 == free0, f"device memory moved by {free0 - free1} bytes"


def test_static_every_row_on_the_slow_path(sampler):
    """256 rows that all take the slow path (top-k off, a nucleus of most of
    the vocabulary) queue 32 deep on each of the static workspace's 8
    slow-path slots, where the handle has a slot per row: the same results,
    and no slot wait runs out (LLMK_STATUS_SLOT_TIMEOUT)."""
    from gpu_util import workload
    rng = np.random.default_rng(256)
    B, V = 256, 151936
    lg = rng.normal(0.0, 2.0, (B, V)).astype(np.float32)
    hists = [rng.integers(0, V, 64) for _ in range(B)]
    w = workload(lg, T=1.0, K=0, P=0.999, R=1.1, hists=hists,
                 u=rng.random(B).astype(np.float32), name="slow256")
    print(f"[case] static vs handle, every row slow, B={B} V={V}", flush=True)
    db = w.to_device()
    ref = outputs(B)
    sampler.launch(db, *ref)
    torch.cuda.synchronize()
    assert sampler.status() == 0
    got = outputs(B)
    status = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    llmk.sample_batch_static(db, *got, status=status)
    torch.cuda.synchronize()
    assert int(status.item()) & _lib.LLMK_STATUS_SLOT_TIMEOUT == 0
    assert int(status.item()) == 0
    h, r = host(got), host(ref)
    assert_same(w, h, r, "slow256")
    # the nuclei are wide: every kept list overflows the 64 entries returned
    assert np.all(h[3] > 1000), "a row did not keep a wide nucleus"


def test_static_status_word():
    """A NaN logit raises LLMK_STATUS_NAN_LOGITS in the caller's status word;
    the call without a status pointer drops the bits."""
    V = 4096
    lg = np.random.default_rng(3).normal(0, 3, (4, V)).astype(np.float32)
    lg[2, 77] = np.nan
    from gpu_util import workload
    w = workload(lg, T=0.8, P=0.9)
    db = w.to_device()
    print("[case] static status word, NaN in row 2", flush=True)
    status = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    llmk.sample_batch_static(db, *outputs(4), status=status)
    torch.cuda.synchronize()
    assert int(status.item()) == _lib.LLMK_STATUS_NAN_LOGITS
    llmk.sample_batch_static(db, *outputs(4))
    torch.cuda.synchronize()


def test_static_limits():
    """Above batch 256 or vocab 262144 the call fails before any launch."""
    lib = _lib.load()
    a = _lib.SampleBatchArgs()
    a.batch, a.vocab, a.row_stride = 257, 1000, 1000
    rc = lib.llmk_sample_batch_static(a, None, None)
    assert rc == _lib.LLMK_ERR_CAPACITY
    assert "batch <= 256" in _lib.last_error()
    a.batch, a.vocab, a.row_stride = 4, (1 << 18) + 1, (1 << 18) + 8
    assert lib.llmk_sample_batch_static(a, None, None) == _lib.LLMK_ERR_CAPACITY
    assert lib.llmk_sample_batch_static(None, None, None) == _lib.LLMK_ERR_INVALID_ARGUMENT
    # rows off 16 bytes: the handle copies them to aligned rows, the static
    # call (which allocates nothing) refuses them before sampling
    import ctypes
    a.batch, a.vocab, a.row_stride, a.dtype = 2, 101, 101, _lib.LLMK_F32
    a.logits = ctypes.c_void_p(0x1004)
    a.uniforms = ctypes.c_void_p(0x2000)
    a.out_tokens = ctypes.c_void_p(0x3000)
    assert lib.llmk_sample_batch_static(a, None, None) == _lib.LLMK_ERR_ALIGNMENT
