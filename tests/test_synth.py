"""The seeded generator produces the configured distributions and edge cases."""
from __future__ import annotations

import numpy as np

from turbinator_c_amd import synth


def test_deterministic_and_thread_invariant():
    a = synth.make_batch(40, seed=5, threads=1)
    b = synth.make_batch(40, seed=5, threads=6)
    for x, y in ((a.obs, b.obs), (a.mission, b.mission), (a.cameras, b.cameras)):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8))
    c = synth.make_batch(40, seed=6)
    assert not np.array_equal(a.obs, c.obs)


def test_ordinary_distributions():
    b = synth.make_batch(64, seed=42, with_depth=True)
    lidar = b.obs[:, 48:4144]
    sentinel = lidar == -1.0
    assert abs(sentinel.mean() - 0.10) < 0.01
    valid = lidar[~sentinel]
    assert valid.min() >= 0.2 and valid.max() < 300.0
    state = np.concatenate([b.obs[:, :48], b.obs[:, 4144:]], axis=1)
    assert abs(state.mean()) < 0.1 and abs(state.std() - 1.0) < 0.1
    far = b.depth == 200.0
    assert abs(far.mean() - 0.15) < 0.01
    assert b.depth.min() >= 0.5
    assert np.all(b.cameras[far] == 0)
    arena = b.mission[:, 6]
    assert set(np.unique(arena)) <= {0.0, 1.0}
    assert np.all(np.abs(b.mission) <= 1.5)


def test_edge_quarters():
    b = synth.make_batch(64, seed=42, variant=synth.EDGE_QUARTERS)
    q1, q2, q3, q4 = (slice(0, 16), slice(16, 32), slice(32, 48), slice(48, 64))
    assert np.all(b.obs[q1, 48:4144] == -1.0)
    assert np.all(b.cameras[q2] == 207)
    lidar3 = b.obs[q3, 48:4144].reshape(16, 2, 4, 4, 8, 16)  # env,head,es,el,as,az
    sectors = lidar3.transpose(0, 1, 2, 4, 3, 5).reshape(16, 64, 64)
    for e in range(16):
        for s in range(64):
            vals = sectors[e, s]
            valid = vals[vals >= 0]
            tie = 0.75 if s & 1 else 0.5
            assert valid.min() == tie
    lidar4 = b.obs[q4, 48:4144]
    for v in (0.2, 120.0, 300.0):
        assert (lidar4 == np.float32(v)).sum() > 100


def test_special_values_present():
    b = synth.make_batch(12, seed=3, variant=synth.SPECIAL)
    assert np.isnan(b.obs).any() and np.isinf(b.obs).any()
    assert np.isnan(b.mission).any()
    assert (np.signbit(b.obs) & (b.obs == 0)).any()
