"""The compact actor's product arithmetic on the CPU: the two-piece fp16
split of an fp32 operand and the three cross terms the matrix cores sum.

For x scaled into [2^14, 2^15) by a power of two (the kernel scales each
operand row so that its largest magnitude lies there), hi = fp16(x) and
lo = fp16(x - hi), both rounded to nearest even.  Then x - hi is exact in
fp32, and hi*hi + hi*lo + lo*hi misses the true product by at most
3 * 2^-22 of |w x| while the pieces are normal fp16 values.  These checks
restate that arithmetic in numpy (float16 rounds to nearest even) and hold
it to the bound, and show that the bound is tight enough to catch a dropped
cross term or an operand left unscaled.
"""
from __future__ import annotations

import numpy as np

BOUND = 3 * 2.0 ** -22


def split(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.asarray(x, np.float32)
    hi = x.astype(np.float16)
    rest = (x - hi.astype(np.float32)).astype(np.float32)
    return hi.astype(np.float64), rest.astype(np.float16).astype(np.float64)


def scaled(x: np.ndarray) -> np.ndarray:
    """x times the power of two that brings max |x| into [2^14, 2^15)."""
    m = np.abs(x).max()
    e = int(np.frexp(np.float64(m))[1]) - 1  # m in [2^e, 2^(e+1))
    return np.ldexp(x.astype(np.float32), 14 - e).astype(np.float32)


def three_terms(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    wh, wl = split(w)
    xh, xl = split(x)
    return wh * xh + wh * xl + wl * xh


def test_subtraction_is_exact():
    rng = np.random.default_rng(1)
    x = scaled(rng.standard_normal(1 << 16).astype(np.float32))
    hi = x.astype(np.float16).astype(np.float64)
    assert np.array_equal((x - hi.astype(np.float32)).astype(np.float64), x.astype(np.float64) - hi)


def test_three_terms_within_bound():
    rng = np.random.default_rng(2)
    n = 1 << 18
    # rows at their kernel scale: magnitudes spread over 2^-13 .. 2^15, so
    # both pieces of every value stay normal fp16
    w = scaled((rng.choice([-1.0, 1.0], n) * 2.0 ** rng.uniform(-13, 15, n)).astype(np.float32))
    x = scaled((rng.choice([-1.0, 1.0], n) * 2.0 ** rng.uniform(-13, 15, n)).astype(np.float32))
    keep = (np.abs(w) >= 2.0 ** -3) & (np.abs(x) >= 2.0 ** -3)  # lo pieces normal
    w, x = w[keep], x[keep]
    exact = w.astype(np.float64) * x.astype(np.float64)
    err = np.abs(three_terms(w, x) - exact)
    assert np.all(err <= BOUND * np.abs(exact))
    # the bound is not loose by orders of magnitude
    assert err.max() / np.abs(exact[np.argmax(err)]) > BOUND / 16


def test_a_dropped_cross_term_fails_the_bound():
    rng = np.random.default_rng(3)
    w = scaled(rng.uniform(0.5, 1.0, 4096).astype(np.float32))
    x = scaled(rng.uniform(0.5, 1.0, 4096).astype(np.float32))
    wh, wl = split(w)
    xh, xl = split(x)
    exact = w.astype(np.float64) * x.astype(np.float64)
    two_terms = wh * xh + wh * xl
    assert np.any(np.abs(two_terms - exact) > BOUND * np.abs(exact))


def test_an_unscaled_operand_fails_the_bound():
    """Without the row scale, small operands put their low piece below fp16's
    normal range (2^-14) and lose it."""
    rng = np.random.default_rng(4)
    w = rng.uniform(1e-4, 2e-4, 4096).astype(np.float32)
    x = scaled(rng.uniform(0.5, 1.0, 4096).astype(np.float32))
    exact = w.astype(np.float64) * x.astype(np.float64)
    assert np.any(np.abs(three_terms(w, x) - exact) > BOUND * np.abs(exact))
    assert np.all(np.abs(three_terms(scaled(w), x) - scaled(w).astype(np.float64)
                         * x.astype(np.float64))
                  <= BOUND * np.abs(scaled(w).astype(np.float64) * x.astype(np.float64)))
