"""Derive the numeric constants shared (by value) between the oracle and the HIP kernels.

Test infrastructure: prints C literals; nothing here is imported at run time.

exp2 polynomial: 2^f on f in [-1/2, 1/2] with the constant term pinned to 1,
fitted by Lawson's iteratively reweighted least squares (which converges to the
minimax / Chebyshev-equioscillating solution of the relative error), coefficients
then rounded to fp32 and re-checked with fp32 Horner evaluation.
"""
import math
import numpy as np


def fit_exp2(deg, iters=200):
    x = np.cos(np.linspace(0, np.pi, 4001)) * 0.5          # Chebyshev-spaced grid
    y = np.exp2(x)
    A = np.stack([x ** k for k in range(1, deg + 1)], axis=1)   # c0 = 1 pinned
    w = np.ones_like(x)
    for _ in range(iters):
        W = np.sqrt(w) / y                                      # relative error weighting
        c, *_ = np.linalg.lstsq(A * W[:, None], (y - 1.0) * W, rcond=None)
        err = np.abs((1.0 + A @ c - y) / y)
        w = w * err
        w /= w.sum()
    return c


def horner32(c32, f):
    p = np.float32(c32[-1]) * np.ones_like(f, dtype=np.float32)
    for ck in reversed(c32[:-1]):
        p = (p.astype(np.float64) * f + np.float64(ck)).astype(np.float32)  # fma: one rounding
    p = (p.astype(np.float64) * f + 1.0).astype(np.float32)
    return p


if __name__ == "__main__":
    for deg in (5, 6):
        c = fit_exp2(deg)
        c32 = [np.float32(v) for v in c]
        f = np.linspace(-0.5, 0.5, 2_000_001).astype(np.float32)
        p = horner32(c32, f.astype(np.float64))
        rel = np.abs(p.astype(np.float64) / np.exp2(f.astype(np.float64)) - 1.0)
        print(f"deg {deg}: max rel err {rel.max():.3e} (fp32 ulp ~ 5.96e-08)")
        for k, v in enumerate(c32, start=1):
            print(f"  C{k} = {float(v).hex()}f  /* {float(v):.9e} */")
