"""The oracle's final_logit_softcapping (candle.rs:1803-1807) and the
glibc-exact tanhf it uses, pinned without the GPU:

* tanh_ref and expm1_ref against the host's tanhf and expm1f on every one of
  the 2^32 float bit patterns (the functions Rust's f32::tanh and candle's CPU
  tanh call);
* the dtype rounding against numpy's float16 conversion and the bf16
  round-to-nearest-even of the synthetic data;
* softcap against its closed form cap * tanh(x / cap) (float64) to within a
  few units in the last place of the dtype, its special values (+-inf ->
  +-cap, -0 -> +0) and monotonicity."""
import concurrent.futures as cf

import numpy as np
import pytest

from llmk import synth
from oracle import llmk_oracle as O


def test_tanh_and_expm1_exhaustive_against_glibc():
    edges = np.linspace(0, 1 << 32, 129).astype(np.int64)
    chunks = [(int(edges[i]), int(edges[i + 1]) - 1) for i in range(128)]
    with cf.ThreadPoolExecutor(8) as ex:
        res = list(ex.map(lambda c: O.tanh_scan(*c), chunks))
    assert sum(r[0] for r in res) == 0, "tanh_ref differs from tanhf"
    assert sum(r[1] for r in res) == 0, "expm1_ref differs from expm1f"


def f16_values(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def bf16_values(x):
    return synth.bf16_bits_to_f32(synth.to_bf16_bits(np.asarray(x, np.float32)))


def test_dtype_rounding_matches_numpy_and_bf16_rne():
    """The oracle's rounding into a 16-bit dtype, seen through softcap(+inf):
    tanh(+inf) = 1 exactly, so the result is cap as the dtype's value.
    Compared with numpy's float16 conversion and the bf16 round-to-nearest-
    even of the synthetic data, over normal, subnormal and overflowing caps."""
    rng = np.random.default_rng(0)
    # values spanning normals, subnormals and overflow of f16 and bf16
    x = np.concatenate([rng.normal(0, 1, 2000), rng.normal(0, 1e-6, 500), rng.normal(0, 1e5, 500),
                        np.ldexp(rng.random(200), -24), [65504.0, 65519.9, 65520.0, 7e4]])
    x = x.astype(np.float32)
    for cap in x[np.isfinite(x) & (np.abs(x) > 0)][:400]:
        cap = abs(float(cap))
        for dt, ref in (("f16", f16_values), ("bf16", bf16_values)):
            got = O.softcap(dt, np.array([np.inf], np.float32), cap)[0]
            want = ref(np.float32(cap))
            if np.isinf(want):
                assert np.isinf(got)
            else:
                # cap rounded to the dtype, times tanh(+inf) = 1, plus 0
                assert got == want, (dt, cap, got, want)


@pytest.mark.parametrize("dt,ulps", [("f32", 4), ("bf16", 3), ("f16", 3)])
def test_softcap_closed_form(dt, ulps):
    rng = np.random.default_rng(1)
    cap = 30.0
    x = np.concatenate([rng.normal(0, 10, 4000), rng.normal(0, 60, 2000), [0.0, 1e-30, -1e-30]])
    x = x.astype(np.float32)
    if dt == "bf16":
        x = bf16_values(x)
    elif dt == "f16":
        x = f16_values(x)
    got = O.softcap(dt, x, cap).astype(np.float64)
    want = cap * np.tanh(x.astype(np.float64) / cap)
    if dt == "f32":
        ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    else:
        # one unit of the dtype at |want| (its significand: 8 or 11 bits)
        p = 8 if dt == "bf16" else 11
        e = np.floor(np.log2(np.maximum(np.abs(want), 1e-30)))
        ulp = np.ldexp(1.0, (e - p + 1).astype(int))  # every step rounds once
    assert np.all(np.abs(got - want) <= ulps * ulp + 1e-45), np.max(np.abs(got - want) / ulp)
    # the result is a value of the dtype
    if dt == "bf16":
        assert np.array_equal(bf16_values(got.astype(np.float32)), got.astype(np.float32))
    if dt == "f16":
        assert np.array_equal(f16_values(got.astype(np.float32)), got.astype(np.float32))


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_softcap_special_values_and_order(dt):
    cap = 50.0
    s = O.softcap(dt, np.array([np.inf, -np.inf, -0.0, 0.0], np.float32), cap)
    assert s[0] == 50.0 and s[1] == -50.0
    # candle's affine maps add +0: -0 comes out as +0
    assert s[2] == 0.0 and not np.signbit(s[2]) and not np.signbit(s[3])
    x = np.sort(np.random.default_rng(2).normal(0, 80, 20000).astype(np.float32))
    if dt == "bf16":
        x = bf16_values(x)
    elif dt == "f16":
        x = f16_values(x)
    y = O.softcap(dt, x, cap)
    assert np.all(np.diff(y) >= 0), "softcap is not monotone"
    assert np.all(np.abs(y) <= cap)
