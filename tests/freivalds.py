"""Whole-output checks for products too large for an fp64 reference of every
element: fp64 row and column checksums of C against the same checksums of
the exact product, computed as A.(B.v) and (u^T.A).B (Freivalds' check).

v and u are random +-1 vectors.  With e = C - A.B and every element within the
north-star bound |e_ij| <= tau = TOL * sqrt(K) * max|A| * max|B|:
  * rigorously, |(e.v)_i| <= ||v||_1 * tau = N * tau;
  * for any fixed e, v drawn independently of it gives
    P(|(e.v)_i| > 8 * ||e_i||_2) <= 2 exp(-32) (Hoeffding), and
    ||e_i||_2 <= sqrt(N) * tau, so |(e.v)_i| <= 8 sqrt(N) tau except with
    negligible probability.
Both bounds are asserted.  The second is the sharp one: a single output tile
computed from the wrong operands (errors of the size of C's entries over a
32 x 32 block) exceeds it by orders of magnitude, and so does any element off
by more than 8 sqrt(N) tau.  Every output element enters one row checksum and
one column checksum.
"""
from __future__ import annotations

import math

import numpy as np


def signs(n: int, seed: int) -> np.ndarray:
    """Random +-1 vector (float64)."""
    rng = np.random.default_rng(seed)
    return rng.integers(0, 2, n).astype(np.float64) * 2.0 - 1.0


def reference(orc, a: np.ndarray, b: np.ndarray, v: np.ndarray, u: np.ndarray):
    """fp64 (A.B).v = A.(B.v) and u^T.(A.B) = (u^T.A).B for fp32 operands (any
    non-negative strides: transposed views are read in place)."""
    cv = orc.matvec(a, orc.matvec(b, v))
    utc = orc.matvec(b.T, orc.matvec(a.T, u))
    return cv, utc


def check(orc, cv, utc, ref_cv, ref_utc, K: int, amax: float, bmax: float, what: str = ""):
    """Assert the checksum bounds of the module docstring; returns the worst
    row/column deviation in units of the sharp bound."""
    cv, utc = np.asarray(cv, np.float64), np.asarray(utc, np.float64)
    ref_cv, ref_utc = np.asarray(ref_cv, np.float64), np.asarray(ref_utc, np.float64)
    assert cv.shape == ref_cv.shape and utc.shape == ref_utc.shape
    assert np.all(np.isfinite(cv)) and np.all(np.isfinite(utc)), f"{what}: non-finite checksum"
    tau = orc.TOL * math.sqrt(max(K, 1)) * amax * bmax
    n_cols, n_rows = utc.shape[-1], cv.shape[-1]
    worst = 0.0
    for name, got, ref, n in (("row", cv, ref_cv, n_cols), ("column", utc, ref_utc, n_rows)):
        d = float(np.max(np.abs(got - ref))) if got.size else 0.0
        assert d <= n * tau, f"{what}: {name} checksum off by {d:.3e} > ||v||_1 tau = {n * tau:.3e}"
        sharp = 8.0 * math.sqrt(n) * tau
        assert d <= sharp, f"{what}: {name} checksum off by {d:.3e} > 8 sqrt(n) tau = {sharp:.3e}"
        worst = max(worst, d / sharp)
    return worst
