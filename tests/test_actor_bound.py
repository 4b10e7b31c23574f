"""The compact actor's raw-output bound, eps (1 + S2 + J), held by the GPU
parity tests (tests/test_gpu_sac_actor.py `conditioning`), checked on the CPU.

J = sum over both hidden layers and units n of |d out / d p_n| S_n, where p_n
is the unit's pre-activation and S_n = |b_n| + sum_k |w_nk x_k| the magnitude
of its summands, plus the fp16 subnormal pieces' term (summand_scales).  Its
derivatives are hand-derived (tanh' = 1 - h^2 through the later layers);
here they are compared with central differences of a float64 forward pass in
which each pre-activation is perturbed on its own, so a transposed weight, a
dropped tanh' or an absolute value taken inside the sum instead of outside
fails.
"""
from __future__ import annotations

import numpy as np

from tests.test_gpu_sac_actor import conditioning, random_weights, summand_scales

HIDDEN = 8


def forward(weights, x, shift0=None, shift1=None):
    """float64 network with optional perturbations of the two pre-activations."""
    w0, b0, w1, b1, w2, b2 = (np.asarray(a, np.float64) for a in weights)
    p0 = x @ w0.T + b0
    if shift0 is not None:
        p0 = p0 + shift0
    h0 = np.tanh(p0)
    p1 = h0 @ w1.T + b1
    if shift1 is not None:
        p1 = p1 + shift1
    h1 = np.tanh(p1)
    return h1 @ w2.T + b2, h0, h1


def case(seed=3):
    w = random_weights(HIDDEN, seed=seed, gain=2.0)
    x = np.random.default_rng(seed).uniform(-2, 2, (5, 142)).astype(np.float32)
    return w, x


def finite_difference_j(w, x, step=1e-6):
    xd = x.astype(np.float64)
    _, h0, h1 = forward(w, xd)
    s0, s1, _ = summand_scales(w, xd, h0, h1)
    j = np.zeros((x.shape[0], 30))
    for layer, s in ((0, s0), (1, s1)):
        for n in range(HIDDEN):
            e = np.zeros(HIDDEN)
            e[n] = step
            kw = ("shift0", "shift1")[layer]
            up = forward(w, xd, **{kw: e})[0]
            down = forward(w, xd, **{kw: -e})[0]
            j += np.abs((up - down) / (2 * step)) * s[:, n:n + 1]
    return j


def last_layer_scale(w, x):
    xd = x.astype(np.float64)
    _, h0, h1 = forward(w, xd)
    return summand_scales(w, xd, h0, h1)[2]


def test_jacobian_term_matches_central_differences():
    w, x = case()
    j = conditioning(w, x) - 1 - last_layer_scale(w, x)
    np.testing.assert_allclose(j, finite_difference_j(w, x), rtol=1e-6, atol=1e-9)


def test_absolute_values_inside_the_sum_fail():
    """The first-layer derivative is |sum_m w2 g1 w1| g0: the sum of absolute
    products (|w2| g1 |w1|) is a looser bound that the check must reject."""
    w, x = case()
    xd = x.astype(np.float64)
    w0, b0, w1, b1, w2, b2 = (np.asarray(a, np.float64) for a in w)
    _, h0, h1 = forward(w, xd)
    g0, g1 = 1 - h0 * h0, 1 - h1 * h1
    s0, s1, _ = summand_scales(w, xd, h0, h1)
    loose = ((g1 * s1) @ np.abs(w2).T
             + np.einsum("om,em,mn,en->eo", np.abs(w2), g1, np.abs(w1), g0 * s0))
    fd = finite_difference_j(w, x)
    assert not np.allclose(loose, fd, rtol=1e-3)
    assert np.all(loose >= fd * (1 - 1e-9))
