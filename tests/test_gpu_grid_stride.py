"""GPU checks of the grid-stride loops, through the C-ABI.

Every kernel's grid is capped, and a batch past the cap makes the first
workgroups take a second environment (row, value) in the same launch, which
runs the loop's carried state and, in the feature kernel, the barrier that
guards the LDS stage between environments.  The caps:

  * feature kernel (device, diagnostics, depth, indexed entries):
    2^20 workgroups of one environment -> batches above 1,048,576;
  * actor plane kernel (tb_hip_actor_inputs_device): 2^20 workgroups of one
    environment -> above 1,048,576;
  * compact SAC actor: 65,536 workgroups of 64 rows -> above 4,194,304 rows;
  * LiDAR transform: 2^20 workgroups of 256 values -> above 2^28 values.
  (The onboard controller's cap, 4,096 workgroups of 64 environments, is
  passed by the 263,144-row cases of test_gpu_onboard / test_gpu_actor_inputs.)

Each case tiles a few thousand distinct inputs on the device to a batch just
past its cap, and every output row must equal, bit for bit, the same input's
row from the small call; the small call is checked against the CPU oracle
(or numpy closed forms).  Comparison stays on the device, slab by slab.  The
largest case holds about 105 GB of device memory.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
from tests.conftest import assert_feature_parity
from tests.test_actor_inputs_oracle import exact_luma, numpy_lidar_channels
from tests.test_gpu_sac_actor import check
from tests.test_sac_actor_oracle import random_features
from turbinator_c_amd import actor, synth

pytestmark = pytest.mark.gpu

FEATURE_CAP = 1 << 20


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def release_device_memory(torch_cuda):
    torch_cuda.cuda.empty_cache()
    yield
    torch_cuda.cuda.synchronize()
    torch_cuda.cuda.empty_cache()


def tile(x, batch):
    """Rows of x repeated to `batch` rows, contiguous, on the device."""
    reps = (batch + x.shape[0] - 1) // x.shape[0]
    shape = (reps,) + (1,) * (x.dim() - 1)
    return x.repeat(*shape)[:batch].contiguous()


def assert_tiled_equal(torch, big, small, label, rows=None):
    """big[i] == small[rows[i]] as 32-bit words for every i; rows defaults to
    i mod len(small)."""
    n = small.shape[0]
    words = lambda t: t.reshape(t.shape[0], -1).view(torch.int32)   # noqa: E731
    bw, sw = words(big), words(small)
    if rows is not None:
        want = sw[rows]
        if not torch.equal(bw, want):
            bad = (bw != want).any(1).nonzero().flatten()[:5].tolist()
            raise AssertionError(f"{label}: rows {bad} differ")
        return
    for start in range(0, bw.shape[0], n):
        stop = min(start + n, bw.shape[0])
        if not torch.equal(bw[start:stop], sw[:stop - start]):
            bad = (bw[start:stop] != sw[:stop - start]).any(1).nonzero().flatten()[:5]
            raise AssertionError(f"{label}: rows {(bad + start).tolist()} differ")


def nan_rows(torch, n, *shape):
    return torch.full((n,) + shape, float("nan"), dtype=torch.float32, device="cuda")


def test_features_device_and_diagnostics(torch_cuda, hip):
    torch = torch_cuda
    distinct, batch = 4096, FEATURE_CAP + 4096
    note(f"features + diagnostics: {batch} envs tiled from {distinct}")
    b = synth.make_batch(distinct, seed=2024, variant=synth.EDGE_QUARTERS, threads=16)
    obs, mis = torch.from_numpy(b.obs).cuda(), torch.from_numpy(b.mission).cuda()
    cam = torch.from_numpy(b.cameras).cuda()
    s = torch.cuda.current_stream()

    def run(o, m, c):
        n = o.shape[0]
        out, out2 = nan_rows(torch, n, 142), nan_rows(torch, n, 142)
        diag = torch.full((n, oracle.DIAG_BYTES), 0xa5, dtype=torch.uint8, device="cuda")
        assert hip.extract_features_device(o, m, c, out, n, s) == 1
        assert hip.extract_features_diagnostics_device(o, m, c, out2, diag, n, s) == 1
        assert hip.synchronize(s) == 1
        return out, out2, diag

    small = run(obs, mis, cam)
    assert_feature_parity(small[0].cpu().numpy(), oracle.features(b.obs, b.mission, b.cameras),
                          "small")
    assert torch.equal(small[0].view(torch.int32), small[1].view(torch.int32))
    assert np.array_equal(small[2].cpu().numpy(), oracle.diagnostics(b.obs, b.cameras))
    big_obs, big_mis, big_cam = tile(obs, batch), tile(mis, batch), tile(cam, batch)
    big = run(big_obs, big_mis, big_cam)
    del big_obs, big_mis, big_cam
    for g, w, name in zip(big, small, ("features", "diag features", "diagnostics")):
        assert_tiled_equal(torch, g, w, name)


def test_features_depth_cameras(torch_cuda, hip):
    torch = torch_cuda
    distinct, batch = 1024, FEATURE_CAP + 1024
    note(f"features from fp32 depth: {batch} envs tiled from {distinct}")
    b = synth.make_batch(distinct, seed=2025, with_depth=True, threads=16)
    obs, mis = torch.from_numpy(b.obs).cuda(), torch.from_numpy(b.mission).cuda()
    dep = torch.from_numpy(b.depth).cuda()
    s = torch.cuda.current_stream()

    def run(o, m, d):
        out = nan_rows(torch, o.shape[0], 142)
        assert hip.extract_features_depth_device(o, m, d, out, o.shape[0], s) == 1
        assert hip.synchronize(s) == 1
        return out

    small = run(obs, mis, dep)
    assert_feature_parity(small.cpu().numpy(),
                          oracle.features(b.obs, b.mission, oracle.depth_to_luma(b.depth)),
                          "small depth")
    big_obs, big_mis, big_dep = tile(obs, batch), tile(mis, batch), tile(dep, batch)
    big = run(big_obs, big_mis, big_dep)
    del big_obs, big_mis, big_dep
    assert_tiled_equal(torch, big, small, "depth features")


def test_features_indexed_with_invalid_rows(torch_cuda, hip):
    """1,052,672 sampled indices into 4,096 stored environments, every 97th
    out of range (NaN row, nothing read): workgroups that loop meet valid and
    invalid environments in either order."""
    torch = torch_cuda
    cap, n = 4096, FEATURE_CAP + 4096
    note(f"indexed features: {n} samples of {cap} slots")
    b = synth.make_batch(cap, seed=2026, threads=16)
    obs, mis = torch.from_numpy(b.obs).cuda(), torch.from_numpy(b.mission).cuda()
    cam = torch.from_numpy(b.cameras).cuda()
    idx = np.random.default_rng(3).integers(0, cap, n).astype(np.uint32)
    idx[::97] = cap + 11
    d_idx = torch.from_numpy(idx.view(np.int32)).cuda()
    s = torch.cuda.current_stream()
    every = nan_rows(torch, cap, 142)
    assert hip.extract_features_device(obs, mis, cam, every, cap, s) == 1
    out = torch.zeros((n, 142), dtype=torch.float32, device="cuda")
    assert hip.extract_features_indexed_device(obs, 16592, mis, 40, cam, 16384, cap, d_idx,
                                               out, n, s) == 1
    assert hip.synchronize(s) == 1
    bad = idx >= cap
    got_bad = out[torch.from_numpy(bad).cuda()]
    assert bool(torch.isnan(got_bad).all()), "out-of-range rows must be NaN"
    ok = torch.from_numpy(~bad).cuda()
    rows = torch.from_numpy(idx[~bad].astype(np.int64)).cuda()
    assert_tiled_equal(torch, out[ok], every, "indexed features", rows=rows)
    sample = np.flatnonzero(~bad)[-512:]          # rows of the looping workgroups' pass
    assert_feature_parity(out[torch.from_numpy(sample).cuda()].cpu().numpy(),
                          oracle.features(b.obs[idx[sample]], b.mission[idx[sample]],
                                          b.cameras[idx[sample]]), "indexed sample")


@pytest.mark.parametrize("planes", ["lidar", "luma"])
def test_actor_planes(torch_cuda, hip, planes):
    torch = torch_cuda
    distinct, batch = 4096, FEATURE_CAP + 4096
    note(f"actor inputs ({planes} planes): {batch} envs tiled from {distinct}")
    b = synth.make_batch(distinct, seed=2027, variant=synth.EDGE_QUARTERS, threads=16)
    obs, mis = torch.from_numpy(b.obs).cuda(), torch.from_numpy(b.mission).cuda()
    cam = torch.from_numpy(b.cameras).cuda() if planes == "luma" else None
    s = torch.cuda.current_stream()

    def run(o, m, c):
        n = o.shape[0]
        out = [nan_rows(torch, n, w) for w in (91, 49, 24, 15)]
        plane = nan_rows(torch, n, 6, 16, 128) if planes == "lidar" else \
            nan_rows(torch, n, 4, 64, 64)
        lidar, luma = (plane, None) if planes == "lidar" else (None, plane)
        assert hip.actor_inputs_device(o, m, c, *out, lidar, luma, n, s) == 1
        assert hip.synchronize(s) == 1
        return out + [plane]

    small = run(obs, mis, cam)
    want = numpy_lidar_channels(b.obs) if planes == "lidar" else exact_luma(b.cameras)
    assert np.array_equal(small[4].cpu().numpy().view(np.uint32), want.view(np.uint32))
    big_obs, big_mis = tile(obs, batch), tile(mis, batch)
    big_cam = None if cam is None else tile(cam, batch)
    big = run(big_obs, big_mis, big_cam)
    del big_obs, big_mis, big_cam
    for g, w, name in zip(big, small, ("proprio", "mission", "tactical", "prior", planes)):
        assert_tiled_equal(torch, g, w, name)


def test_sac_actor(torch_cuda, hip):
    torch = torch_cuda
    hidden, distinct = 128, 4096
    batch = 65536 * 64 + distinct
    note(f"compact actor: {batch} rows tiled from {distinct}")
    rng = np.random.default_rng(2028)
    weights = []
    for (o, i), nb in actor.layer_shapes(hidden):
        weights.append((rng.standard_normal((o, i)) * np.sqrt(2.0 / (o + i))).astype(np.float32))
        weights.append((rng.standard_normal(nb) * 0.1).astype(np.float32))
    feats = random_features(distinct, seed=2029)
    draws = rng.standard_normal((distinct, 15)).astype(np.float32)
    s = torch.cuda.current_stream()
    packed = torch.empty(actor.packed_bytes(hidden) // 4, dtype=torch.float32, device="cuda")
    dw = [torch.from_numpy(w).cuda() for w in weights]
    assert actor.pack_device(*dw, hidden, packed, s) == 1
    f, d = torch.from_numpy(feats).cuda(), torch.from_numpy(draws).cuda()

    def run(fe, dr):
        n = fe.shape[0]
        act, lp, raw = nan_rows(torch, n, 15), nan_rows(torch, n), nan_rows(torch, n, 30)
        assert actor.act_device(packed, hidden, fe, dr, act, lp, raw, n, s) == 1
        assert hip.synchronize(s) == 1
        return act, lp, raw

    small = run(f, d)
    check(tuple(t.cpu().numpy() for t in small),
          oracle.sac_actor(oracle.SacActorWeights(*weights), feats, draws), weights, feats, draws,
          "small")
    big = run(tile(f, batch), tile(d, batch))
    for g, w, name in zip(big, small, ("actions", "log_prob", "raw")):
        assert_tiled_equal(torch, g, w, name)


def test_lidar_transform(torch_cuda, hip):
    torch = torch_cuda
    distinct = 1 << 18
    count = (1 << 28) + distinct
    note(f"LiDAR transform: {count} values tiled from {distinct}")
    rng = np.random.default_rng(2030)
    vals = rng.uniform(-5, 130, distinct).astype(np.float32)
    vals[::101] = np.array([np.nan, np.inf, -np.inf, -0.0, 0.0, 120.0, 1e-40],
                           np.float32)[np.arange(vals[::101].size) % 7]
    v = torch.from_numpy(vals).cuda()
    s = torch.cuda.current_stream()

    def run(x):
        out = torch.full_like(x, float("nan"))
        assert hip.lidar_transform_device(x, out, x.numel(), s) == 1
        assert hip.synchronize(s) == 1
        return out

    small = run(v)
    got, want = small.cpu().numpy(), oracle.lidar_feature(vals)
    valid = (vals >= 0) & np.isfinite(vals)
    assert np.all(got[~valid] == -1.0)
    ulp = np.abs(got[valid].view(np.int32).astype(np.int64) -
                 want[valid].view(np.int32).astype(np.int64))
    assert ulp.max() <= 4
    big = run(tile(v.view(-1, 1024), count // 1024).view(-1))
    assert_tiled_equal(torch, big.view(-1, 1024), small.view(-1, 1024), "lidar transform")
