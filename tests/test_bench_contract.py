"""CPU checks of bench.py's contract: one GPU only, and the onboard leg's
byte accounting (which scan rays each mission's controller uses)."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np

import oracle

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr


def test_onboard_ray_bytes_by_mission_class():
    # (m4, m5) -> rays used: none, dodge (m5 > 0.75), slalom (m4 > 0.75,
    # m5 <= 0.25), lateral (m4 > 0.75, m5 > 0.25: none), and the thresholds
    # and non-finite values on both sides.
    cases = [((0.0, 0.0), 0), ((0.0, 1.0), 4096), ((1.0, 0.0), 6144), ((1.0, 0.5), 0),
             ((1.0, 0.8), 4096), ((0.75, 0.0), 0), ((0.0, 0.75), 0),
             ((0.0, float(np.nextafter(np.float32(0.75), np.float32(2)))), 4096),
             ((1.0, 0.25), 6144), ((float("inf"), float("nan")), 6144),
             ((float("nan"), float("inf")), 4096), ((-float("inf"), 1.2), 4096)]
    mission = np.zeros((len(cases), 10), np.float32)
    for i, ((m4, m5), _) in enumerate(cases):
        mission[i, 4], mission[i, 5] = m4, m5
    got = bench.onboard_scan_ray_bytes(mission)
    assert got.tolist() == [want for _, want in cases]


def test_onboard_ray_bytes_match_what_the_prior_reads():
    """The accounting's classes agree with the oracle's prior: an
    environment counted as using no scan rays gives the same prior whatever
    its LiDAR holds, one counted as dodge whatever rows 4..5 hold."""
    rng = np.random.default_rng(5)
    n = 256
    obs = rng.normal(size=(n, 4148)).astype(np.float32)
    obs[:, 48:4144] = rng.uniform(0.3, 12.0, size=(n, 4096)).astype(np.float32)
    mission = rng.uniform(-1.5, 1.5, size=(n, 10)).astype(np.float32)
    used = bench.onboard_scan_ray_bytes(mission)
    base = oracle.onboard(obs, mission)[1]
    other = obs.copy()
    other[:, 48:4144] = rng.uniform(0.3, 12.0, size=(n, 4096)).astype(np.float32)
    none = used == 0
    assert none.any() and (~none).any()
    changed = oracle.onboard(other, mission)[1]
    assert np.array_equal(base[none], changed[none])
    assert not np.array_equal(base[~none], changed[~none])
    # Dodge: only elevation rows 0..3 of each head are read.
    upper = obs.copy()
    for head in range(2):
        lo = 48 + (16 * head + 4) * 128
        upper[:, lo:lo + 2 * 128] = rng.uniform(0.3, 12.0, size=(n, 256)).astype(np.float32)
    dodge = used == 4096
    assert dodge.any()
    assert np.array_equal(base[dodge], oracle.onboard(upper, mission)[1][dodge])
