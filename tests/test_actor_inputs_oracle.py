"""Pins the CPU oracle of the 618M actor's sensor preparation
(oracle/actor_inputs_oracle.c) before it is trusted.

Each output is checked against a formulation computed another way:
  * LiDAR channels against numpy float32 array arithmetic on a
    (head, row, az) reshape.  A channel taking head c // 2 instead of c % 2,
    a wrong clamp or a wrong sentinel value fails;
  * luma against b * fl(1/255) - 0.5 formed exactly in double precision and
    rounded once to float: the fused multiply-add nvcc makes of
    network_gpu.cu:482 by default.  Two roundings (product, then difference)
    fail for 158 of the 256 bytes;
  * the 52 symlog scalars against float64 log1p, within 2 ulp, including the
    scale table of network_gpu.cu:287-293, probed one input at a time;
  * mission / tactical / prior placement against orc_onboard_env, whose own
    goldens are pinned in tests/test_onboard_oracle.py.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from turbinator_c_amd import synth


def reference_scales() -> np.ndarray:
    """network_gpu.cu:287-293: symlog scale per scalar index."""
    s = np.ones(52, np.float32)
    s[0:3] = 0.05
    s[3:6] = 0.10
    s[10:13] = 0.20
    s[13:16] = 0.10
    s[28:32] = 0.50
    s[32:36] = 0.20
    return s


def numpy_lidar_channels(obs: np.ndarray) -> np.ndarray:
    b = obs.shape[0]
    r = obs[:, 48:4144].reshape(b, 2, 16, 128)
    valid = (r > 0) & np.isfinite(r)
    clamped = np.fmax(np.float32(0.05), np.fmin(np.float32(30.0), r))
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(valid, np.float32(1.0) / np.fmax(np.float32(0.2), clamped), 0)
        ratio = np.where(valid, clamped / np.float32(30.0), 1)
    out = np.empty((b, 6, 16, 128), np.float32)
    out[:, 0:2] = inv
    out[:, 2:4] = ratio
    out[:, 4:6] = valid
    return out


def exact_luma(cameras: np.ndarray) -> np.ndarray:
    c = np.float64(np.float32(1.0) / np.float32(255.0))
    # b * c is exact in double (8 x 24 significant bits, a multiple of 2^-31
    # below 2), and so is b * c - 0.5: the one cast is the fused
    # multiply-add's single rounding.
    return (cameras.astype(np.float64) * c - 0.5).astype(np.float32).reshape(
        cameras.shape[0], 4, 64, 64)


def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ia = a.astype(np.float32).view(np.int32).astype(np.int64)
    ib = b.astype(np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7fffffff), ia)
    ib = np.where(ib < 0, -(ib & 0x7fffffff), ib)
    return np.abs(ia - ib)


def float64_symlog(obs: np.ndarray) -> np.ndarray:
    raw = np.concatenate([obs[:, :48], obs[:, 4144:4148]], axis=1).astype(np.float32)
    raw = np.where(np.isfinite(raw), np.fmax(np.float32(-1000), np.fmin(np.float32(1000), raw)),
                   np.float32(0))
    x = np.abs(raw * reference_scales()).astype(np.float32)   # float32 product
    sym = np.copysign(np.log1p(x.astype(np.float64)), raw)
    return sym / np.sqrt(np.float64(np.float32(1.0001)))


@pytest.mark.parametrize("variant", [0, 1, 2, 3, 4, 5])
def test_lidar_and_luma_closed_forms(variant):
    b = synth.make_batch(12, seed=500 + variant, variant=variant)
    got = oracle.actor_inputs(b.obs, b.mission, b.cameras)
    assert np.array_equal(got["lidar"].view(np.uint32),
                          numpy_lidar_channels(b.obs).view(np.uint32))
    assert np.array_equal(got["luma"].view(np.uint32), exact_luma(b.cameras).view(np.uint32))


def test_luma_rounding_matters():
    """The two-rounding evaluation (product rounded, then the difference)
    differs from the fused multiply-add for 158 bytes, so the closed form
    above decides between them."""
    b = np.arange(256, dtype=np.float64)
    c = np.float64(np.float32(1) / np.float32(255))
    two = ((b * c).astype(np.float32).astype(np.float64) - 0.5).astype(np.float32)
    cams = np.tile(np.arange(256, dtype=np.uint8), 64)[None, :]
    obs = np.zeros((1, 4148), np.float32)
    got = oracle.actor_inputs(obs, np.zeros((1, 10), np.float32), cams)["luma"].ravel()[:256]
    assert int((got != two).sum()) == 158
    # 255 * fl(1/255) is just above 1: the fused form keeps the excess, the
    # product's own rounding gives exactly 1.
    assert got[0] == -0.5 and got[255] == np.nextafter(np.float32(0.5), np.float32(1))
    assert two[255] == 0.5


@pytest.mark.parametrize("variant", [0, 4, 5])
def test_symlog_scalars_within_2_ulp(variant):
    b = synth.make_batch(16, seed=520 + variant, variant=variant)
    got = oracle.actor_inputs(b.obs, b.mission, b.cameras)["proprio"][:, :52]
    want = float64_symlog(b.obs)
    assert ulp_distance(got, want.astype(np.float32)).max() <= 2


def test_symlog_scale_table_by_probe():
    """Raw value 1 at one index at a time: the output is log1p(scale) /
    sqrt(1.0001); zeros elsewhere stay zero."""
    obs = np.zeros((52, 4148), np.float32)
    for i in range(52):
        obs[i, i if i < 48 else 4144 + i - 48] = 1.0
    got = oracle.actor_inputs(obs, np.zeros((52, 10), np.float32), None)["proprio"][:, :52]
    want = np.log1p(reference_scales().astype(np.float64)) / np.sqrt(
        np.float64(np.float32(1.0001)))
    assert ulp_distance(np.diag(got), want.astype(np.float32)).max() <= 2
    off = got[~np.eye(52, dtype=bool)]
    assert np.all(off == 0)


def test_symlog_clamps_and_non_finite():
    obs = np.zeros((1, 4148), np.float32)
    obs[0, 6:10] = [np.nan, np.inf, -np.inf, -0.0]      # scale 1 at 6..9 and 16..27
    obs[0, 16:18] = [1e30, -1e30]
    got = oracle.actor_inputs(obs, np.zeros((1, 10), np.float32), None)["proprio"][0]
    big = np.float32(np.log1p(1000.0) / np.sqrt(np.float64(np.float32(1.0001))))
    assert got[6] == 0 and got[7] == 0 and got[8] == 0
    assert got[9] == 0 and np.signbit(got[9])
    assert ulp_distance(got[16:18], np.array([big, -big])).max() <= 2


@pytest.mark.parametrize("variant", [0, 5])
def test_mission_and_onboard_placement(variant):
    b = synth.make_batch(8, seed=540 + variant, variant=variant)
    got = oracle.actor_inputs(b.obs, b.mission, b.cameras)
    tac, pri, _ = oracle.onboard(b.obs, b.mission)
    u = lambda a: np.ascontiguousarray(a).view(np.uint32)   # noqa: E731
    assert np.array_equal(u(got["tactical"]), u(tac)) and np.array_equal(u(got["prior"]), u(pri))
    assert np.array_equal(u(got["proprio"][:, 52:76]), u(tac))
    assert np.array_equal(u(got["proprio"][:, 76:91]), u(pri))
    assert np.array_equal(u(got["mission"][:, 10:34]), u(tac))
    assert np.array_equal(u(got["mission"][:, 34:49]), u(pri))
    want_m = np.where(np.isfinite(b.mission), b.mission, np.float32(0))
    assert np.array_equal(u(got["mission"][:, :10]), u(want_m))
