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


def scale_exponent(x: np.ndarray) -> int:
    """The kernel's row exponent t: max |x| 2^t in [2^14, 2^15)."""
    m = np.abs(x).max()
    return 14 - (int(np.frexp(np.float64(m))[1]) - 1)


def split_dot(w: np.ndarray, x: np.ndarray) -> float:
    """sum_k w_k x_k as the kernel forms it from one weight row and one
    feature row: each row scaled by its own power of two, split, the three
    cross terms summed (exactly, in float64 here) and unscaled."""
    tw, tx = scale_exponent(w), scale_exponent(x)
    ws = np.ldexp(w.astype(np.float32), tw).astype(np.float32)
    xs = np.ldexp(x.astype(np.float32), tx).astype(np.float32)
    return float(np.ldexp(three_terms(ws, xs).sum(), -(tw + tx)))


def subnormal_term(w: np.ndarray, x: np.ndarray) -> float:
    """sum_k |x_k| min(|w_k|, 2^-39 max|w|) + |w_k| min(|x_k|, 2^-39 max|x|):
    the absolute error the pieces' subnormal rounding may add to the sum."""
    aw, ax = np.abs(w.astype(np.float64)), np.abs(x.astype(np.float64))
    sub = 2.0 ** -39
    return float((ax * np.minimum(aw, sub * aw.max())).sum()
                 + (aw * np.minimum(ax, sub * ax.max())).sum())


def test_an_anticorrelated_row_needs_the_subnormal_term():
    """The row's largest weight (2^20) meets a zero feature and a weight 2^30
    below it meets 2^10: at the row's scale that weight is an fp16
    subnormal, and its rounding error is about 1e-3 of the sum, far above
    any multiple of u sum|w x|, but within the subnormal term."""
    w = np.array([2.0 ** 20, 1.23 * 2.0 ** -10], np.float32)
    x = np.array([0.0, 2.0 ** 10], np.float32)
    exact = float(w.astype(np.float64) @ x.astype(np.float64))
    err = abs(split_dot(w, x) - exact)
    assert err > 1e-4 * abs(exact)
    assert err <= BOUND * abs(exact) + subnormal_term(w, x)


def test_rows_across_the_float_range_within_the_two_terms():
    """Dot products of one weight row and one feature row at random scales
    (2^-30 .. 2^30), in both signs.  Even trials: both rows spread over
    2^-50 .. 1 of their largest entry.  Odd trials, anticorrelated: one weight
    dominates a row spread over 2^-45 .. 2^-20 of it (so most weights are
    fp16 subnormals at the row's scale) and meets a zero feature, the other
    features spread over 2^-10 .. 1.  Every sum is within 3 * 2^-22 sum|w x|
    plus the subnormal term, and the anticorrelated ones need that term."""
    rng = np.random.default_rng(5)
    n = 142
    needed = 0

    def row(lo, hi):
        return (rng.choice([-1.0, 1.0], n) * 2.0 ** rng.uniform(lo, hi, n)
                * 2.0 ** rng.uniform(-30, 30))

    for trial in range(2000):
        if trial % 2 == 0:
            w, x = row(-50, 0), row(-50, 0)
        else:
            w, x = row(-45, -20), row(-10, 0)
            j = int(rng.integers(n))
            w[j] = np.abs(w).max() * 2.0 ** 20
            x[j] = 0.0
        w, x = w.astype(np.float32), x.astype(np.float32)
        exact = float(w.astype(np.float64) @ x.astype(np.float64))
        mag = float(np.abs(w.astype(np.float64) * x.astype(np.float64)).sum())
        err = abs(split_dot(w, x) - exact)
        assert err <= BOUND * mag + subnormal_term(w, x)
        needed += err > BOUND * mag
    assert needed > 500
