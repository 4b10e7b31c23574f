"""GPU parity of the batched compact SAC actor (tb_hip_sac_actor_pack_device
+ tb_hip_sac_actor_act_device) against the CPU oracle, which reproduces
tb_sac_act_features bit for bit (tests/test_sac_actor_oracle.py).

The matrix cores sum in another order than the reference's sequential loop,
each product is formed from two-piece fp16 splits of its operands with the
lo*lo cross term (at most 2^-22 of the product) left out, each instruction's
block sum drops the bits of its products that lie more than 2^-24 below the
largest of their group of eight before rounding (tests/csrc/check_mfma_sum.hip:
at most 3.8 u sum|p| per instruction over 262,144 random outputs, 0.4 u on
average, u = 2^-24, where the reference's sequential fp32 sum rounds every
step to nearest), and tanhf / expf / logf are the device library's.  So each
output is held to a bound set by its own conditioning:
  * raw outputs: eps (1 + S2 + J), eps = 1e-6 (about 17 u), the first-order
    effect of an error of at most eps S_l in every pre-activation of every
    layer l, where S_l = |b_l| + sum_k |w_lk x_k| is the magnitude of that
    layer's summands: S2 for the output layer itself, and
    J = sum over hidden layers and units n of |d out / d p_ln| S_ln, with
    the network's own float64 derivatives.  A hidden unit far from
    saturation whose summands cancel (S_ln >> |p_ln|, as with features over
    ten decades against first-layer weights over ten more) passes the error
    of its sum on to the output on both sides, the reference's included.
    S_l also carries the fp16 subnormal pieces' absolute error (SUBNORMAL):
    an operand more than 2^28 below its row's largest is rounded to fp16's
    subnormal grid, an error of up to 2^-39 of that largest magnitude (and no
    more than the operand itself), however small the operand's own product
    (tests/test_split_products.py);
  * actions: (1 - a^2) dz + 2.4e-7, dz the raw bound of the mean plus the
    exp-rounding of std * eps (tanh' = 1 - a^2; 2.4e-7 = tanh rounding);
  * log-probability: 1e-4 (1 + |lp|) plus, per action, the log-std bound and
    the reference formula's sensitivity to the action, 2|a| / (1 - a^2 + 1e-6),
    times the action bound.  Near |a| = 1 log(1 - a^2 + 1e-6) amplifies one
    ulp of the action by ~1e6, so a flat bound would be loose or wrong;
  * deterministic calls: log-probability exactly 0, as the reference leaves it.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

import oracle
from tests.test_sac_actor_oracle import random_features, reference_agent
from turbinator_c_amd import actor

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def random_weights(hidden: int, seed: int, gain: float = 1.0) -> list[np.ndarray]:
    rng = np.random.default_rng(seed)
    out = []
    for (o, i), b in actor.layer_shapes(hidden):
        out.append((rng.standard_normal((o, i)) * gain * np.sqrt(2.0 / (o + i))).astype(
            np.float32))
        out.append((rng.standard_normal(b) * 0.1 * gain).astype(np.float32))
    return out


def run_gpu(torch, weights, hidden, feats, draws, want_raw=True):
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()   # noqa: E731
    b = feats.shape[0]
    nbytes = actor.packed_bytes(hidden)
    assert nbytes > 0
    packed = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda")
    dw = [dev(w) for w in weights]
    s = torch.cuda.current_stream()
    assert actor.pack_device(*dw, hidden, packed, s) == 1
    f = dev(feats)
    n = None if draws is None else dev(draws)
    act = torch.full((b, 15), float("nan"), dtype=torch.float32, device="cuda")
    lp = torch.full((b,), float("nan"), dtype=torch.float32, device="cuda")
    raw = torch.full((b, 30), float("nan"), dtype=torch.float32, device="cuda") \
        if want_raw else None
    assert actor.act_device(packed, hidden, f, n, act, lp, raw, b, s) == 1
    torch.cuda.synchronize()
    return act.cpu().numpy(), lp.cpu().numpy(), None if raw is None else raw.cpu().numpy()


RAW_EPS = 1e-6
# A scaled operand's piece below fp16's normal range (2^-14) is rounded to
# the subnormal grid: an absolute error of at most 2^-25 at the row's scale,
# which is 2^-39 of the row's largest magnitude (of 1 for hidden
# activations, whose scale is a fixed 2^14), and never more than the value
# itself.  It follows the row's largest magnitude rather than the product,
# so when a row's largest weight meets a zero feature and a weight 2^30
# below it meets a large one, that product carries an error far above
# eps |w x|.
SUBNORMAL = 2.0 ** -39


def summand_scales(weights, x, h0, h1, subnormal=True):
    """S_l per (row, unit) of the three layers, in float64: |b| + sum_k |w_k x_k|,
    plus (with `subnormal`) the subnormal pieces' absolute error in units of
    RAW_EPS: sum_k |x_k| min(|w_k|, 2^-39 max|w|) + |w_k| min(|x_k|, 2^-39 max|x|),
    max|x| = 1 for the hidden activations (tests/test_split_products.py holds
    the two-piece split to this).  Infinite features have no pieces (the kernel
    adds their products in fp32), so they count as 0 in that term."""
    w0, b0, w1, b1, w2, b2 = (np.asarray(a, np.float64) for a in weights)
    s0 = np.abs(b0) + np.abs(x) @ np.abs(w0).T
    s1 = np.abs(b1) + np.abs(h0) @ np.abs(w1).T
    s2 = np.abs(b2) + np.abs(h1) @ np.abs(w2).T
    if subnormal:
        def term(a, w, a_max):
            aw = np.abs(w)
            floor_w = np.minimum(aw, SUBNORMAL * aw.max(1, keepdims=True))
            return (a @ floor_w.T + np.minimum(a, SUBNORMAL * a_max) @ aw.T) / RAW_EPS

        ax = np.where(np.isfinite(x), np.abs(x), 0.0)
        s0 = s0 + term(ax, w0, ax.max(1, keepdims=True))
        s1 = s1 + term(np.abs(h0), w1, 1.0)
        s2 = s2 + term(np.abs(h1), w2, 1.0)
    return s0, s1, s2


def conditioning(weights, feats, subnormal=True) -> np.ndarray:
    """1 + S2 + J per (row, output), in float64: S2 = |b2| + |h1| @ |w2|^T, and
    J = sum_n |d out / d p0_n| S0_n + sum_m |d out / d p1_m| S1_m, each S_l with
    the subnormal pieces' term of summand_scales.  Units fed an infinite
    feature are saturated (tanh' = 0) and contribute nothing."""
    w0, b0, w1, b1, w2, b2 = (np.asarray(x, np.float64) for x in weights)
    x = feats.astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        h0 = np.tanh(x @ w0.T + b0)
        h1 = np.tanh(h0 @ w1.T + b1)
        s0, s1, s2 = summand_scales(weights, x, h0, h1, subnormal)
        g0, g1 = 1 - h0 * h0, 1 - h1 * h1
        # d out_o / d p1_m = w2[o, m] g1_m;  d out_o / d p0_n = sum_m w2[o, m] g1_m w1[m, n] g0_n
        t1 = (g1 * s1) @ np.abs(w2).T
        s0g = np.where(g0 == 0, 0.0, g0 * s0)
        t0 = np.empty_like(t1)
        for r in range(0, len(x), 512):  # [rows, out, hidden] slabs of at most ~30 MB
            d0 = np.abs((w2[None] * g1[r:r + 512, None, :]) @ w1)
            t0[r:r + 512] = np.einsum("eon,en->eo", d0, s0g[r:r + 512])
        out = 1 + s2 + t0 + t1
    return np.nan_to_num(out, nan=1.0, posinf=1.0)


def check(got, want, weights, feats, draws, label, subnormal=True):
    (ga, glp, graw), (wa, wlp, wraw) = got, want
    scale = np.ones(15)
    scale[14] = 0.15
    eps = np.zeros(wa.shape) if draws is None else np.abs(draws * scale)
    raw_tol = RAW_EPS * conditioning(weights, feats, subnormal)
    if graw is not None:
        finite = np.isfinite(wraw)
        assert np.array_equal(finite, np.isfinite(graw)), f"{label}: raw finiteness"
        bad = finite & (np.abs(np.where(finite, graw - wraw, 0)) > raw_tol)
        assert not bad.any(), f"{label}: raw {np.argwhere(bad)[:3]}"
    a = wa.astype(np.float64)
    std = np.exp(np.clip(np.nan_to_num(wraw[:, 15:].astype(np.float64)), -3.5, -1.6))
    # mean error + std * eps error (expf rounding and the log-std error)
    dz = raw_tol[:, :15] + std * eps * (1e-6 + raw_tol[:, 15:])
    tol_a = (1 - a * a) * dz + 2.4e-7
    da = np.abs(ga - a)
    assert np.all(da <= tol_a), f"{label}: action {np.argwhere(da > tol_a)[:3]}"
    if draws is None:
        assert np.all(glp == 0), label
        return {"action_max": float(da.max())}
    sens = 2 * np.abs(a) / (1 - a * a + 1e-6)
    tol = 1e-4 * (1 + np.abs(wlp)) + (raw_tol[:, 15:] + sens * tol_a).sum(1)
    dl = np.abs(glp.astype(np.float64) - wlp)
    assert np.all(dl <= tol), f"{label}: log_prob env {np.argmax(dl - tol)}"
    return {"action_max": float(da.max()), "logp_max": float(dl.max())}


@pytest.mark.parametrize("hidden", [16, 37, 80, 128, 200, 256])
def test_random_weights(torch_cuda, hip, hidden):
    note(f"sac actor hidden {hidden}, 1000 envs")
    w = random_weights(hidden, seed=hidden)
    feats = random_features(1000, seed=7 * hidden)
    draws = np.random.default_rng(hidden).standard_normal((1000, 15)).astype(np.float32)
    ow = oracle.SacActorWeights(*w)
    for d in (None, draws):
        got = run_gpu(torch_cuda, w, hidden, feats, d)
        stats = check(got, oracle.sac_actor(ow, feats, d), w, feats, d, f"h{hidden}")
        note(f"hidden {hidden} {'det' if d is None else 'stoch'}: {stats}")


def test_saturating_and_special_rows(torch_cuda, hip):
    """Large weights push z past +-8 and log-std past both clamps; NaN / Inf
    features propagate to the raw outputs, which the sampler maps to 0."""
    note("sac actor saturation and special rows")
    hidden = 64
    w = random_weights(hidden, seed=3, gain=12.0)
    feats = random_features(256, seed=11)
    feats[3, 5] = np.nan
    feats[4, 7] = np.inf
    feats[5] = 1e30
    draws = np.random.default_rng(4).standard_normal((256, 15)).astype(np.float32) * 3
    ow = oracle.SacActorWeights(*w)
    got = run_gpu(torch_cuda, w, hidden, feats, draws)
    stats = check(got, oracle.sac_actor(ow, feats, draws), w, feats, draws, "saturating")
    note(f"saturating: {stats}")


def f32_bits(u: int) -> np.float32:
    return np.frombuffer(np.uint32(u).tobytes(), np.float32)[0]


@pytest.mark.parametrize("hidden", [37, 128])
def test_extreme_and_infinite_features(torch_cuda, hip, hidden):
    """Features at the ends of the float range.  Finite ones go through the
    split at a per-row scale; infinite ones have no split and the kernel adds
    their products in fp32.  Rows: 0x1.ffp127 of each sign, FLT_MAX, -inf and
    +inf in one row (per output +-inf or NaN, as the reference's sum falls),
    two FLT_MAX, 0x1.ffp127 beside the largest float below it, a row of
    -FLT_MAX / 64 only, and +inf in the last feature.  Every partial sum of
    the reference's loop stays finite here: a row whose sequential sum
    overflows partway (142 terms of FLT_MAX) ends at an infinity that depends
    on the summation order, which no parallel sum reproduces."""
    note(f"sac actor extreme features, hidden {hidden}")
    w = random_weights(hidden, seed=5)
    feats = random_features(64, seed=13)
    big, below = f32_bits(0x7F7F8000), f32_bits(0x7F7F7FFF)
    fmax = np.finfo(np.float32).max
    feats[0, 0] = big
    feats[1, 141] = -big
    feats[2, 70] = fmax
    feats[3, 3], feats[3, 9] = -np.inf, np.inf
    feats[4, 10] = feats[4, 11] = fmax
    feats[5, 20], feats[5, 21] = big, below
    feats[6, :] = -fmax / 64
    feats[7, 141] = np.inf
    draws = np.random.default_rng(6).standard_normal((64, 15)).astype(np.float32)
    ow = oracle.SacActorWeights(*w)
    for d in (None, draws):
        got = run_gpu(torch_cuda, w, hidden, feats, d)
        want = oracle.sac_actor(ow, feats, d)
        stats = check(got, want, w, feats, d, f"extreme h{hidden}")
        note(f"extreme hidden {hidden} {'det' if d is None else 'stoch'}: {stats}")


def wide_range_case(seed: int = 21):
    """Operand rows across the float range, for the matrix cores' per-row
    scaling: first-layer weight rows at scales 10^U(-15, 15) and feature
    rows at 10^U(-15, 15), each with entries spread over 10^U(-10, 0) of
    their row's scale; hidden-layer rows at their usual scale but spread over
    10^U(-8, 0) (the low pieces of the smallest are fp16 subnormals at the
    row's scale); an all-zero weight row per layer and an all-zero feature
    row.  Products stay below 1e30, so the reference's sums stay finite.
    Hidden-layer weights keep their usual scale because larger ones amplify
    the hidden tanh's own rounding (about 2e-7 absolute here, an ulp in the
    reference) past a bound on the last layer's sum."""
    hidden = 128
    rng = np.random.default_rng(seed)
    w = random_weights(hidden, seed=seed)
    for li, (lo, hi) in ((0, (-15, 15)), (2, (0, 0)), (4, (0, 0))):
        rows = w[li].shape[0]
        row_scale = 10.0 ** rng.uniform(lo, hi, (rows, 1))
        spread = 10.0 ** rng.uniform(-10 if li == 0 else -8, 0, w[li].shape)
        w[li] = (w[li] * row_scale * spread).astype(np.float32)
        w[li][rows // 2] = 0.0
    feats = (rng.choice([-1.0, 1.0], (256, 142)) * 10.0 ** rng.uniform(-15, 15, (256, 1))
             * 10.0 ** rng.uniform(-10, 0, (256, 142))).astype(np.float32)
    feats[7] = 0.0
    return hidden, w, feats


def test_wide_dynamic_range(torch_cuda, hip):
    note("sac actor wide dynamic range, hidden 128")
    hidden, w, feats = wide_range_case()
    draws = np.random.default_rng(22).standard_normal((256, 15)).astype(np.float32)
    ow = oracle.SacActorWeights(*w)
    for d in (None, draws):
        got = run_gpu(torch_cuda, w, hidden, feats, d)
        stats = check(got, oracle.sac_actor(ow, feats, d), w, feats, d, "wide range")
        note(f"wide range {'det' if d is None else 'stoch'}: {stats}")


def anticorrelated_case(seed: int = 31):
    """First-layer rows whose largest weight (2^20) meets a zero feature while
    a weight 2^30 .. 2^37 below it meets a feature of +-2^10: that weight's
    scaled pieces are fp16 subnormals, rounded by up to 2^-25 at the row's
    scale (2^-9 of the unit's pre-activation, which is about 2^-7 .. 1 here),
    and the unit stays unsaturated, so the error reaches the outputs.  Units
    0..15 are such rows; the rest keep random weights."""
    hidden = 128
    rng = np.random.default_rng(seed)
    w = random_weights(hidden, seed=seed)
    for n in range(16):
        w[0][n] = 0.0
        w[0][n, 0] = 2.0 ** 20
        w[0][n, 1 + n] = np.float32((1.0 + rng.uniform(0.0, 0.99)) * 2.0 ** (-10 - (n % 8)))
    feats = random_features(128, seed=seed + 1)
    feats[:, 0] = 0.0
    feats[:, 1:17] = rng.choice([-1.0, 1.0], (128, 16)) * 2.0 ** 10
    return hidden, w, feats


def test_anticorrelated_subnormal_pieces(torch_cuda, hip):
    """The subnormal term is what holds these rows: without it the bound
    fails on them, with it the outputs pass."""
    note("sac actor anticorrelated rows, subnormal weight pieces, hidden 128")
    hidden, w, feats = anticorrelated_case()
    draws = np.random.default_rng(32).standard_normal((128, 15)).astype(np.float32)
    ow = oracle.SacActorWeights(*w)
    for d in (None, draws):
        got = run_gpu(torch_cuda, w, hidden, feats, d)
        want = oracle.sac_actor(ow, feats, d)
        stats = check(got, want, w, feats, d, "anticorrelated")
        with pytest.raises(AssertionError):
            check(got, want, w, feats, d, "anticorrelated, no subnormal term", subnormal=False)
        note(f"anticorrelated {'det' if d is None else 'stoch'}: {stats}")


@pytest.mark.parametrize("batch", [1, 15, 63, 65, 16384])
def test_batch_tails(torch_cuda, hip, batch):
    note(f"sac actor batch {batch}")
    hidden = 128
    w = random_weights(hidden, seed=batch)
    feats = random_features(batch, seed=batch + 1) if batch > 3 else \
        np.random.default_rng(batch).uniform(-1, 1, (batch, 142)).astype(np.float32)
    draws = np.random.default_rng(batch).standard_normal((batch, 15)).astype(np.float32)
    got = run_gpu(torch_cuda, w, hidden, feats, draws)
    pick = np.arange(batch) if batch <= 1024 else \
        np.random.default_rng(2).choice(batch, 1024, replace=False)
    want = oracle.sac_actor(oracle.SacActorWeights(*w), feats[pick], draws[pick])
    check(tuple(g[pick] for g in got), want, w, feats[pick], draws[pick], f"batch{batch}")


def test_reference_checkpoint(torch_cuda, hip, tmp_path):
    """A checkpoint the reference wrote, its own random stream: the GPU batch
    equals consecutive tb_sac_act_features calls within the tolerances."""
    if oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built")
    note("sac actor from a reference checkpoint")
    ref, agent, path = reference_agent(tmp_path, 128, seed=5)
    try:
        weights, hidden, rng = actor.read_checkpoint_actor(str(path))
        feats = random_features(300, seed=21)
        draws, _ = actor.normals(rng, 300 * 15)
        draws = draws.reshape(300, 15)
        want_a = np.empty((300, 15), np.float32)
        want_lp = np.empty(300, np.float32)
        for e in range(300):
            assert ref.tb_sac_act_features(agent, feats[e].ctypes.data, 0,
                                           want_a[e].ctypes.data, want_lp[e:].ctypes.data) == 1
        got = run_gpu(torch_cuda, weights, hidden, feats, draws)
        want = oracle.sac_actor(oracle.SacActorWeights(*weights), feats, draws)
        assert np.array_equal(want[0].view(np.uint32), want_a.view(np.uint32))
        assert np.array_equal(want[1].view(np.uint32), want_lp.view(np.uint32))
        check(got, want, weights, feats, draws, "checkpoint")
    finally:
        ref.tb_sac_destroy(agent)


def test_argument_validation(hip):
    lib = hip.hip_lib()
    d = ctypes.c_void_p(256)
    odd = ctypes.c_void_p(264)
    pack, act = lib.tb_hip_sac_actor_pack_device, lib.tb_hip_sac_actor_act_device
    assert pack(None, d, d, d, d, d, 128, d, None) == 0
    assert pack(d, d, d, d, d, d, 15, d, None) == 0
    assert pack(d, d, d, d, d, d, 128, odd, None) == 0
    assert act(None, 128, d, None, d, None, None, 1, None) == 0
    assert act(d, 257, d, None, d, None, None, 1, None) == 0
    assert act(odd, 128, d, None, d, None, None, 1, None) == 0
    assert act(d, 128, None, None, d, None, None, 1, None) == 0
    assert act(d, 128, d, None, None, None, None, 1, None) == 0
    assert act(d, 128, d, None, d, None, None, 0, None) == 0
