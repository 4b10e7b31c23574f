"""GPU parity of the 142-feature path against the CPU oracle, through the C-ABI.

Cases: the reference's 3-env fixture through the host batch object, the
golden sets, configuration 2 (1,024 envs), configuration 4 (4,096-env edge
quarters), configuration 3 at its full 16,384 envs, configuration 5's
66,672-byte replay records (aligned, 4-byte-aligned next_obs and byte-aligned
cameras), NULL cameras, non-finite inputs, a non-default stream, and the
reference's own tests/test_cuda_features.c linked against this library.
Tolerance classes are defined in tests/conftest.py.
"""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from tests.conftest import assert_feature_parity
from tests.golden.make_golden import fixture_sets
from turbinator_c_amd import synth

pytestmark = pytest.mark.gpu

GOLDEN = np.load(oracle.HERE.parent / "tests" / "golden" / "features_golden.npz")

# Replay transition record, field order of tb_gpu_host_batch
# (reference include/turbinator/gpu/replay.h:17-30).
RECORD = 66672
OFF_OBS, OFF_MISSION, OFF_CAM = 0, 16592, 16632
OFF_NEXT_OBS, OFF_NEXT_MISSION, OFF_NEXT_CAM = 33396, 49988, 50028


def note(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def run_device(torch, hip, obs, mission, cameras, stream=None):
    b = obs.shape[0]
    d_obs = torch.from_numpy(np.ascontiguousarray(obs)).cuda()
    d_mis = torch.from_numpy(np.ascontiguousarray(mission)).cuda()
    d_cam = None if cameras is None else torch.from_numpy(np.ascontiguousarray(cameras)).cuda()
    out = torch.full((b, 142), float("nan"), dtype=torch.float32, device="cuda")
    s = stream or torch.cuda.current_stream()
    torch.cuda.synchronize()
    assert hip.extract_features_device(d_obs, d_mis, d_cam, out, b, s) == 1
    assert hip.synchronize(s) == 1
    return out.cpu().numpy()


def test_reference_fixture_through_host_object(hip):
    note("ref3 via tb_cuda_extract_features_host")
    sets = {n: inputs for n, inputs, _ in fixture_sets()}
    obs, mission, cams = sets["ref3"]
    batch = hip.FeatureBatch.create(0, 3)
    assert batch is not None
    try:
        out = np.full((3, 142), np.nan, np.float32)
        assert batch.extract_host(obs, mission, cams, 3, out) == 1, batch.error()
        assert batch.error() == ""
    finally:
        batch.destroy()
    stats = assert_feature_parity(out, GOLDEN["ref3"], "ref3")
    note(f"ref3 stats {stats}")


@pytest.mark.parametrize("name", ["c1", "c4", "special"])
def test_golden_sets_device(torch_cuda, hip, name):
    note(f"golden {name}")
    sets = {n: inputs for n, inputs, _ in fixture_sets()}
    obs, mission, cams = sets[name]
    got = run_device(torch_cuda, hip, obs, mission, cams)
    stats = assert_feature_parity(got, GOLDEN[name], name)
    note(f"{name} stats {stats}")


def test_config2_1024_envs(torch_cuda, hip):
    note("config 2: 1024 envs")
    b = synth.make_batch(1024, seed=42)
    got = run_device(torch_cuda, hip, b.obs, b.mission, b.cameras)
    stats = assert_feature_parity(got, oracle.features(b.obs, b.mission, b.cameras), "c2")
    note(f"c2 stats {stats}")


def test_config4_edge_quarters(torch_cuda, hip):
    note("config 4: 4096 envs edge quarters")
    b = synth.make_batch(4096, seed=42, variant=synth.EDGE_QUARTERS)
    got = run_device(torch_cuda, hip, b.obs, b.mission, b.cameras)
    want = oracle.features(b.obs, b.mission, b.cameras)
    stats = assert_feature_parity(got, want, "c4")
    assert np.all(got[:1024, 62:126] == -1.0)                       # Q1 all no-return
    assert np.all(got[1024:2048, 126:142] == np.float32(207) / np.float32(255))  # Q2
    note(f"c4 stats {stats}")


def test_config3_full_16384(torch_cuda, hip):
    note("config 3: 16384 envs full parity")
    b = synth.make_batch(16384, seed=42, threads=16)
    got = run_device(torch_cuda, hip, b.obs, b.mission, b.cameras)
    stats = assert_feature_parity(got, oracle.features(b.obs, b.mission, b.cameras, threads=16),
                                  "c3")
    note(f"c3 stats {stats}")


def test_null_cameras(torch_cuda, hip):
    note("NULL cameras")
    b = synth.make_batch(64, seed=11)
    got = run_device(torch_cuda, hip, b.obs, b.mission, None)
    assert_feature_parity(got, oracle.features(b.obs, b.mission, None), "nocam")
    assert np.all(got[:, 126:142].view(np.uint32) == 0)


def test_special_values(torch_cuda, hip):
    note("non-finite / signed-zero inputs, 256 envs")
    b = synth.make_batch(256, seed=99, variant=synth.SPECIAL)
    got = run_device(torch_cuda, hip, b.obs, b.mission, b.cameras)
    assert_feature_parity(got, oracle.features(b.obs, b.mission, b.cameras), "special")


def test_nondefault_stream(torch_cuda, hip):
    note("non-default stream")
    torch = torch_cuda
    b = synth.make_batch(300, seed=12)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        got = run_device(torch, hip, b.obs, b.mission, b.cameras, stream=s)
    assert_feature_parity(got, oracle.features(b.obs, b.mission, b.cameras), "stream")


def strided_case(torch, hip, batch, record, obs_off, mis_off, cam_off, label):
    buf = np.zeros(batch * record, np.uint8)
    synth.fill_records(buf, batch, record, obs_off, mis_off, cam_off, seed=77, threads=16)
    want = oracle.features_strided(buf, batch, record, obs_off, mis_off, cam_off, threads=16)
    d = torch.from_numpy(buf).cuda()
    out = torch.full((batch, 142), float("nan"), dtype=torch.float32, device="cuda")
    base = d.data_ptr()
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    assert hip.extract_features_strided_device(base + obs_off, record, base + mis_off, record,
                                               base + cam_off, record, out, batch, s) == 1
    assert hip.synchronize(s) == 1
    got = out.cpu().numpy()
    del d
    return assert_feature_parity(got, want, label)


@pytest.mark.parametrize("which", ["obs", "next_obs"])
def test_replay_records_small(torch_cuda, hip, which):
    note(f"replay records, 512 envs, {which}")
    offs = (OFF_OBS, OFF_MISSION, OFF_CAM) if which == "obs" else \
        (OFF_NEXT_OBS, OFF_NEXT_MISSION, OFF_NEXT_CAM)
    strided_case(torch_cuda, hip, 512, RECORD, *offs, f"replay-{which}")


def test_eight_byte_aligned_rows(torch_cuda, hip):
    note("strided, 8-byte aligned obs and camera rows")
    strided_case(torch_cuda, hip, 300, 33032, 0, 16600, 16640, "eight-byte")


def test_byte_aligned_cameras(torch_cuda, hip):
    note("strided, byte-aligned camera rows")
    strided_case(torch_cuda, hip, 257, 33020, 0, 16592, 16633, "byte-aligned")


def test_config5_replay_65536(torch_cuda, hip):
    note("config 5: 65536 records x 66672 B")
    stats = strided_case(torch_cuda, hip, 65536, RECORD, OFF_OBS, OFF_MISSION, OFF_CAM, "c5")
    note(f"c5 stats {stats}")


def test_lidar_transform_accuracy(torch_cuda, hip):
    note("per-bin transform over a strided sweep of [0,120] and specials")
    torch = torch_cuda
    top = np.float32(120.0).view(np.uint32)
    bits = np.arange(0, int(top) + 1, 61, dtype=np.uint32)
    specials = np.array([0.0, -0.0, 1e-45, 1e-38, 1e-30, 1e-8, 0.05, 0.2, 1.0, 2.0, 119.99, 120.0,
                         120.5, 300.0, 3e38, np.inf, -np.inf, np.nan, -1.0, -1e-30],
                        np.float32)
    xs = np.concatenate([bits.view(np.float32), specials])
    d_in = torch.from_numpy(xs).cuda()
    d_out = torch.empty_like(d_in)
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    assert hip.lidar_transform_device(d_in, d_out, xs.size, s) == 1
    assert hip.synchronize(s) == 1
    got = d_out.cpu().numpy()
    want = oracle.lidar_feature(xs)
    valid = (xs >= 0) & np.isfinite(xs)
    assert np.all(got[~valid] == -1.0)
    g, w = got[valid], want[valid]
    assert np.array_equal(np.signbit(g[w == 0]), np.signbit(w[w == 0]))
    ulp = np.abs(g.view(np.int32).astype(np.int64) - w.view(np.int32).astype(np.int64))
    note(f"transform: {valid.sum()} values, max ulp {ulp.max()}, "
         f"exact {np.mean(ulp == 0):.4f}, <=1ulp {np.mean(ulp <= 1):.6f}")
    assert ulp.max() <= 4


def test_abi_errors_with_device(hip):
    note("ABI error paths with a device present")
    assert hip.FeatureBatch.create(4096, 8) is None        # no such device
    b = hip.FeatureBatch.create(0, 4)
    assert b is not None
    try:
        obs = np.zeros((8, 4148), np.float32)
        mis = np.zeros((8, 10), np.float32)
        cam = np.zeros((8, 16384), np.uint8)
        out = np.zeros((8, 142), np.float32)
        assert b.extract_host(obs, mis, cam, 0, out) == 0
        assert b.extract_host(obs, mis, cam, 5, out) == 0     # above max_batch
        assert b.error() == ""
        assert b.extract_host(obs, mis, cam, 4, out) == 1
        assert b.error() == ""
        assert np.all(out[:4, 62:126] == 0.0) and np.all(out[4:] == 0.0)
    finally:
        b.destroy()


def test_reference_test_binary_drop_in():
    """The reference's own tests/test_cuda_features.c + training.c, compiled
    from the reference sources by oracle/Makefile (droptest) and linked
    against libturbinator_hip.so."""
    exe = oracle.HERE / "_ref" / "test_cuda_features_dropin"
    if not exe.exists():
        pytest.skip("drop-in binary not built (reference tree absent at build time)")
    note("reference test_cuda_features.c linked against libturbinator_hip.so")
    env = dict(os.environ, TB_CUDA_TEST_DEVICE="0")
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    note(f"drop-in: rc={proc.returncode} out={proc.stdout.strip()} err={proc.stderr.strip()}")
    assert proc.returncode == 0
    assert "matches C11 extraction" in proc.stdout


def run_diag(torch, hip, obs, mission, cameras):
    b = obs.shape[0]
    d_obs = torch.from_numpy(np.ascontiguousarray(obs)).cuda()
    d_mis = torch.from_numpy(np.ascontiguousarray(mission)).cuda()
    d_cam = None if cameras is None else torch.from_numpy(np.ascontiguousarray(cameras)).cuda()
    out = torch.full((b, 142), float("nan"), dtype=torch.float32, device="cuda")
    diag = torch.full((b, oracle.DIAG_BYTES), 0xa5, dtype=torch.uint8, device="cuda")
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    assert hip.extract_features_diagnostics_device(d_obs, d_mis, d_cam, out, diag, b, s) == 1
    assert hip.synchronize(s) == 1
    return out.cpu().numpy(), diag.cpu().numpy()


@pytest.mark.parametrize("variant,batch", [(synth.EDGE_QUARTERS, 4096), (synth.SPECIAL, 512),
                                           (synth.ORDINARY, 1024)])
def test_diagnostics_bit_exact(torch_cuda, hip, variant, batch):
    note(f"diagnostics variant {variant}, {batch} envs")
    b = synth.make_batch(batch, seed=4242, variant=variant, threads=16)
    feats, diag = run_diag(torch_cuda, hip, b.obs, b.mission, b.cameras)
    assert_feature_parity(feats, oracle.features(b.obs, b.mission, b.cameras), "diag-features")
    want = oracle.diagnostics(b.obs, b.cameras)
    bad = np.argwhere(diag != want)
    assert not bad.size, f"diag word {bad[0]}: gpu {diag[tuple(bad[0])]:#x} " \
                         f"cpu {want[tuple(bad[0])]:#x} ({len(bad)} words differ)"
    if variant == synth.EDGE_QUARTERS:
        assert np.all(diag[:1024, 256:384:2] == 0xff)             # Q1: no valid bin
        assert np.all(diag[:1024, 257:384:2] == 0)                # ... and no count
        assert np.all(diag[1024:2048, 384:400] == 207)            # Q2: constant camera


def test_diagnostics_null_cameras(torch_cuda, hip):
    note("diagnostics, NULL cameras")
    b = synth.make_batch(128, seed=5)
    feats, diag = run_diag(torch_cuda, hip, b.obs, b.mission, None)
    assert np.array_equal(diag, oracle.diagnostics(b.obs, None))
    assert np.all(diag[:, 384:] == 0)


def run_depth(torch, hip, obs, mission, depth):
    b = obs.shape[0]
    d_obs = torch.from_numpy(np.ascontiguousarray(obs)).cuda()
    d_mis = torch.from_numpy(np.ascontiguousarray(mission)).cuda()
    d_dep = torch.from_numpy(np.ascontiguousarray(depth)).cuda()
    out = torch.full((b, 142), float("nan"), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    assert hip.extract_features_depth_device(d_obs, d_mis, d_dep, out, b, s) == 1
    assert hip.synchronize(s) == 1
    return out.cpu().numpy()


def test_depth_cameras_config2(torch_cuda, hip):
    note("fp32 depth cameras, 1024 envs")
    b = synth.make_batch(1024, seed=42, with_depth=True, threads=16)
    got = run_depth(torch_cuda, hip, b.obs, b.mission, b.depth)
    want = oracle.features(b.obs, b.mission, oracle.depth_to_luma(b.depth))
    assert_feature_parity(got, want, "depth")


def test_config4_edge_quarters_depth(torch_cuda, hip):
    """Configuration 4 with its cameras as BASELINE states them, fp32 depth:
    quarter 2 holds 37.5 m in every pixel, which quantises to luma 207
    (255 (1 - 37.5 / 200) = 207.19), so its quadrant means are 207/255
    exactly (training.c:128-141).  The depth entry must also equal the u8
    entry on the generator's own luma bytes, bit for bit."""
    note("config 4: 4096 envs edge quarters, fp32 depth cameras")
    b = synth.make_batch(4096, seed=42, variant=synth.EDGE_QUARTERS, with_depth=True,
                         threads=16)
    assert np.all(b.depth[1024:2048] == np.float32(37.5))
    luma = oracle.depth_to_luma(b.depth)
    assert np.all(luma[1024:2048] == 207)
    got = run_depth(torch_cuda, hip, b.obs, b.mission, b.depth)
    stats = assert_feature_parity(got, oracle.features(b.obs, b.mission, luma), "c4-depth")
    assert np.all(got[:1024, 62:126] == -1.0)                       # Q1 all no-return
    assert np.all(got[1024:2048, 126:142] == np.float32(207) / np.float32(255))  # Q2
    u8 = run_device(torch_cuda, hip, b.obs, b.mission, b.cameras)
    assert np.array_equal(got.view(np.uint32), u8.view(np.uint32))
    note(f"c4 depth stats {stats}")


def test_config3_depth_full_16384(torch_cuda, hip):
    """Configuration 3 as BASELINE states it (16,384 environments of
    4 x 64 x 64 fp32 depth cameras, 1.07 GB of depth), every environment
    against the oracle on the quantised bytes."""
    note("config 3: 16384 envs, fp32 depth cameras, full parity")
    b = synth.make_batch(16384, seed=42, with_depth=True, threads=16)
    got = run_depth(torch_cuda, hip, b.obs, b.mission, b.depth)
    want = oracle.features(b.obs, b.mission, oracle.depth_to_luma(b.depth), threads=16)
    stats = assert_feature_parity(got, want, "c3-depth")
    note(f"c3 depth stats {stats}")


def test_depth_cameras_special_values(torch_cuda, hip):
    note("fp32 depth cameras, special depth values")
    b = synth.make_batch(64, seed=8, with_depth=True)
    depth = b.depth.copy()
    rng = np.random.default_rng(1)
    specials = np.array([np.nan, np.inf, -np.inf, -0.0, 0.0, -3.0, 200.0, 250.0, 1e-40, 3e38,
                         37.5, 100.0], np.float32)
    mask = rng.random(depth.shape) < 0.2
    depth[mask] = rng.choice(specials, mask.sum())
    got = run_depth(torch_cuda, hip, b.obs, b.mission, depth)
    want = oracle.features(b.obs, b.mission, oracle.depth_to_luma(depth))
    assert_feature_parity(got, want, "depth-special")


def reference_sampler(seed: int, count: int, size: int) -> np.ndarray:
    """Index stream of the reference replay (src/gpu/replay.cu:18-25,153):
    xorshift64* modulo the current size."""
    state, out = seed or 1, np.empty(count, np.uint32)
    mask = (1 << 64) - 1
    for i in range(count):
        x = state
        x ^= x >> 12
        x ^= (x << 25) & mask
        x ^= x >> 27
        state = x
        out[i] = ((x * 2685821657736338717) & mask) % size
    return out


def test_indexed_soa_replay(torch_cuda, hip):
    note("fused replay sampling: SoA storage, 4096 slots, 2048 samples")
    torch = torch_cuda
    cap, n = 4096, 2048
    b = synth.make_batch(cap, seed=31, threads=16)
    idx = reference_sampler(42, n, cap)
    idx[::97] = cap + 5                      # out-of-range rows -> NaN, nothing read
    d_obs, d_mis = torch.from_numpy(b.obs).cuda(), torch.from_numpy(b.mission).cuda()
    d_cam = torch.from_numpy(b.cameras).cuda()
    d_idx = torch.from_numpy(idx.view(np.int32)).cuda()
    out = torch.zeros((n, 142), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    assert hip.extract_features_indexed_device(d_obs, 16592, d_mis, 40, d_cam, 16384, cap, d_idx,
                                               out, n, s) == 1
    assert hip.synchronize(s) == 1
    got = out.cpu().numpy()
    bad = idx >= cap
    assert np.all(np.isnan(got[bad]))
    ok = ~bad
    want = oracle.features(b.obs[idx[ok]], b.mission[idx[ok]], b.cameras[idx[ok]])
    assert_feature_parity(got[ok], want, "indexed-soa")


def test_indexed_aos_records(torch_cuda, hip):
    note("fused replay sampling: 66,672-byte records, next_obs fields")
    torch = torch_cuda
    cap, n = 1024, 700
    buf = np.zeros(cap * RECORD, np.uint8)
    synth.fill_records(buf, cap, RECORD, OFF_NEXT_OBS, OFF_NEXT_MISSION, OFF_NEXT_CAM, seed=9,
                       threads=16)
    idx = reference_sampler(7, n, cap)
    full = oracle.features_strided(buf, cap, RECORD, OFF_NEXT_OBS, OFF_NEXT_MISSION,
                                   OFF_NEXT_CAM, threads=16)
    d = torch.from_numpy(buf).cuda()
    base = d.data_ptr()
    d_idx = torch.from_numpy(idx.view(np.int32)).cuda()
    out = torch.zeros((n, 142), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    assert hip.extract_features_indexed_device(base + OFF_NEXT_OBS, RECORD,
                                               base + OFF_NEXT_MISSION, RECORD,
                                               base + OFF_NEXT_CAM, RECORD, cap, d_idx, out, n,
                                               s) == 1
    assert hip.synchronize(s) == 1
    assert_feature_parity(out.cpu().numpy(), full[idx], "indexed-aos")


@pytest.mark.parametrize("batch", [1, 2, 5, 63, 65, 257])
def test_ragged_batches_every_entry(torch_cuda, hip, batch):
    """Batches that are not a multiple of the 8 XCDs (the workgroup-to-
    environment mapping falls back to the identity for the last ids) through
    the device, diagnostics, depth, strided and indexed entries."""
    note(f"ragged batch {batch}: every feature entry")
    torch = torch_cuda
    b = synth.make_batch(batch, seed=900 + batch, variant=synth.EDGE_QUARTERS if batch > 3 else
                         synth.ORDINARY, with_depth=True)
    want = oracle.features(b.obs, b.mission, b.cameras)
    assert_feature_parity(run_device(torch, hip, b.obs, b.mission, b.cameras), want, "device")
    feats, diag = run_diag(torch, hip, b.obs, b.mission, b.cameras)
    assert_feature_parity(feats, want, "diagnostics")
    assert np.array_equal(diag, oracle.diagnostics(b.obs, b.cameras))
    assert_feature_parity(run_depth(torch, hip, b.obs, b.mission, b.depth),
                          oracle.features(b.obs, b.mission, oracle.depth_to_luma(b.depth)),
                          "depth")
    strided_case(torch, hip, batch, RECORD, OFF_NEXT_OBS, OFF_NEXT_MISSION, OFF_NEXT_CAM,
                 "strided")
    # Indexed: every environment once, in reverse order, plus one invalid row.
    idx = np.concatenate([np.arange(batch)[::-1], [batch]]).astype(np.uint32)
    d_obs, d_mis = torch.from_numpy(b.obs).cuda(), torch.from_numpy(b.mission).cuda()
    d_cam = torch.from_numpy(b.cameras).cuda()
    d_idx = torch.from_numpy(idx.view(np.int32)).cuda()
    out = torch.zeros((idx.size, 142), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    assert hip.extract_features_indexed_device(d_obs, 16592, d_mis, 40, d_cam, 16384, batch,
                                               d_idx, out, idx.size, s) == 1
    assert hip.synchronize(s) == 1
    got = out.cpu().numpy()
    assert np.all(np.isnan(got[-1]))
    assert_feature_parity(got[:-1], want[::-1], "indexed")
