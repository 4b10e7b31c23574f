"""GPU parity of the 618M actor's fused sensor preparation, through the
C-ABI entry tb_hip_actor_inputs_device, against the CPU oracle
(oracle/actor_inputs_oracle.c, restating network_gpu.cu:274-304, 467-483).

Classes:
  * LiDAR channels, camera luma and mission_vec[0..9]: bit-exact;
  * the 52 symlog scalars: |gpu - cpu| <= 1e-5 |cpu| + 1e-6 (log1p is this
    backend's own evaluation, as in the LiDAR feature means);
  * tactical / prior: the onboard bar (5e-5 + 2e-6 relative, tests/conftest.py)
    and the same NaN pattern; their copies in proprio / mission_vec equal the GPU's own
    tactical / prior bit-for-bit.
At the 16,384-environment configuration the channels and luma are checked
against numpy closed forms for every environment and the rest against the
oracle on a sample of environments.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

import oracle
from tests.conftest import h2_over
from tests.test_actor_inputs_oracle import exact_luma, numpy_lidar_channels, ulp_distance
from turbinator_c_amd import synth

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def u32(a):
    return np.ascontiguousarray(a).view(np.uint32)


def run_actor(torch, hip, obs, mission, cameras, lidar=True, luma=True):
    b = obs.shape[0]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()   # noqa: E731
    nan = lambda *shape: torch.full(shape, float("nan"), dtype=torch.float32,  # noqa: E731
                                    device="cuda")
    d_obs, d_mis = dev(obs), dev(mission)
    d_cam = None if cameras is None else dev(cameras)
    out = {"proprio": nan(b, 91), "mission": nan(b, 49), "tactical": nan(b, 24),
           "prior": nan(b, 15), "lidar": nan(b, 6, 16, 128) if lidar else None,
           "luma": nan(b, 4, 64, 64) if luma else None}
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    assert hip.actor_inputs_device(d_obs, d_mis, d_cam, out["proprio"], out["mission"],
                                   out["tactical"], out["prior"], out["lidar"], out["luma"],
                                   b, s) == 1
    assert hip.synchronize(s) == 1
    return {k: None if v is None else v.cpu().numpy() for k, v in out.items()}


def check_h2(got, want, label):
    for name in ("tactical", "prior"):
        g, w = got[name], want[name]
        assert np.array_equal(np.isnan(g), np.isnan(w)), f"{label}: {name} NaN pattern"
        bad = h2_over(g, w)
        assert not bad.size, f"{label}: {name} {bad[:3]}"


def check_copies(got, label):
    assert np.array_equal(u32(got["proprio"][:, 52:76]), u32(got["tactical"])), label
    assert np.array_equal(u32(got["proprio"][:, 76:91]), u32(got["prior"])), label
    assert np.array_equal(u32(got["mission"][:, 10:34]), u32(got["tactical"])), label
    assert np.array_equal(u32(got["mission"][:, 34:49]), u32(got["prior"])), label


def check_symlog(got, want, label) -> int:
    g, w = got[:, :52].astype(np.float64), want[:, :52].astype(np.float64)
    bad = np.abs(g - w) > 1e-5 * np.abs(w) + 1e-6
    assert not bad.any(), f"{label}: symlog {np.argwhere(bad)[:3]}"
    return int(ulp_distance(got[:, :52], want[:, :52]).max())


def finite_scalars(b):
    """Variant SPECIAL with its 3e38 scalars replaced: huge finite inputs make
    the onboard controller ill-conditioned (covered in test_gpu_onboard)."""
    obs, mission = b.obs.copy(), b.mission.copy()
    for sl in (np.s_[:, :48], np.s_[:, 4144:]):
        v = obs[sl]
        v[np.abs(v) == np.float32(3e38)] = np.float32(7.5)
        obs[sl] = v
    mission[np.abs(mission) == np.float32(3e38)] = np.float32(0.25)
    return obs, mission


@pytest.mark.parametrize("variant", [0, 1, 2, 3, 4, 5])
def test_variants_against_oracle(torch_cuda, hip, variant):
    note(f"actor inputs variant {variant}, 256 envs")
    b = synth.make_batch(256, seed=600 + variant, variant=variant, threads=16)
    obs, mission = finite_scalars(b)
    got = run_actor(torch_cuda, hip, obs, mission, b.cameras)
    want = oracle.actor_inputs(obs, mission, b.cameras)
    assert np.array_equal(u32(got["lidar"]), u32(want["lidar"])), "lidar channels"
    assert np.array_equal(u32(got["luma"]), u32(want["luma"])), "luma"
    assert np.array_equal(u32(got["mission"][:, :10]), u32(want["mission"][:, :10]))
    ulps = check_symlog(got["proprio"], want["proprio"], f"variant{variant}")
    check_h2(got, want, f"variant{variant}")
    check_copies(got, f"variant{variant}")
    note(f"variant {variant}: symlog max {ulps} ulp")


def test_symlog_dense_sweep(torch_cuda, hip):
    """Every scalar slot over magnitudes 1e-30 .. 1e3 (both signs), zeros,
    and non-finite values."""
    note("actor inputs symlog sweep")
    vals = np.concatenate([np.logspace(-30, 3, 3000).astype(np.float32), [0, -0.0, np.nan,
                                                                           np.inf, -np.inf]])
    vals = np.concatenate([vals, -vals]).astype(np.float32)
    n = (vals.size + 51) // 52
    flat = np.resize(vals, n * 52).reshape(n, 52)
    obs = np.zeros((n, 4148), np.float32)
    obs[:, :48] = flat[:, :48]
    obs[:, 4144:] = flat[:, 48:]
    mission = np.zeros((n, 10), np.float32)
    got = run_actor(torch_cuda, hip, obs, mission, None, lidar=False, luma=False)
    want = oracle.actor_inputs(obs, mission, None)
    ulps = check_symlog(got["proprio"], want["proprio"], "sweep")
    note(f"symlog sweep: max {ulps} ulp over {n * 52} values")


def test_optional_outputs_and_ragged(torch_cuda, hip):
    note("actor inputs without lidar/luma outputs, batches 1 and 3")
    for n in (1, 3):
        b = synth.make_batch(n, seed=650 + n)
        got = run_actor(torch_cuda, hip, b.obs, b.mission, None, lidar=False, luma=False)
        want = oracle.actor_inputs(b.obs, b.mission, None)
        check_symlog(got["proprio"], want["proprio"], f"ragged{n}")
        check_h2(got, want, f"ragged{n}")
        check_copies(got, f"ragged{n}")


def test_config_16384(torch_cuda, hip):
    """The benchmark's 16,384-environment batch: channels and luma bit-exact for
    every environment against numpy; the rest against the oracle on 512
    sampled environments."""
    note("actor inputs 16384 envs")
    b = synth.make_batch(16384, seed=1, variant=synth.EDGE_QUARTERS, threads=16)
    got = run_actor(torch_cuda, hip, b.obs, b.mission, b.cameras)
    assert np.array_equal(u32(got["lidar"]), u32(numpy_lidar_channels(b.obs)))
    assert np.array_equal(u32(got["luma"]), u32(exact_luma(b.cameras)))
    check_copies(got, "16384")
    pick = np.random.default_rng(5).choice(16384, 512, replace=False)
    want = oracle.actor_inputs(b.obs[pick], b.mission[pick], b.cameras[pick])
    sub = {k: got[k][pick] for k in ("proprio", "mission", "tactical", "prior")}
    check_symlog(sub["proprio"], want["proprio"], "16384")
    assert np.array_equal(u32(sub["mission"][:, :10]), u32(want["mission"][:, :10]))
    check_h2(sub, want, "16384")


@pytest.mark.parametrize("n", [300, 1024, 2048, 2560])
def test_lidar_or_luma_alone(torch_cuda, hip, n):
    """The scan kernel writes the channel planes of elevation rows 0..5 and
    the plane kernel the other rows: each plane output requested alone, at a
    one-stream batch and at one that overlaps the two streams, is complete
    and bit-exact against numpy for every environment."""
    note(f"actor inputs, lidar or luma alone, {n} envs")
    b = synth.make_batch(n, seed=700 + n, threads=16)
    got = run_actor(torch_cuda, hip, b.obs, b.mission, None, lidar=True, luma=False)
    assert np.array_equal(u32(got["lidar"]), u32(numpy_lidar_channels(b.obs)))
    check_copies(got, f"lidar{n}")
    got = run_actor(torch_cuda, hip, b.obs, b.mission, b.cameras, lidar=False, luma=True)
    assert np.array_equal(u32(got["luma"]), u32(exact_luma(b.cameras)))
    check_copies(got, f"luma{n}")


def _call_all(torch, hip, d_in, out, n, stream_arg, s_sync):
    assert hip.actor_inputs_device(*d_in, *out, n, stream_arg) == 1
    assert hip.synchronize(s_sync) == 1
    return [t[:n].cpu().numpy().view(np.uint32).copy() for t in out]


def _device_batch(torch, n, seed):
    b = synth.make_batch(n, seed=seed, threads=16)
    d_in = [torch.from_numpy(a).cuda() for a in (b.obs, b.mission, b.cameras)]
    out = [torch.full(shape, float("nan"), dtype=torch.float32, device="cuda")
           for shape in ((n, 91), (n, 49), (n, 24), (n, 15), (n, 6, 16, 128), (n, 4, 64, 64))]
    return d_in, out


def test_mode_thresholds_and_null_stream(torch_cuda, hip):
    """The entry picks its mode by batch: one stream below 1,792
    environments, with the scan kernel writing its rows' LiDAR channels from
    512; two streams from 1,792, with that split from 2,560.  Every call on
    either side of each threshold must equal the 2,560-row call on their
    common rows, bit for bit, and a call on the null stream must equal one on
    a torch stream."""
    torch = torch_cuda
    names = ("proprio", "mission", "tactical", "prior", "lidar", "luma")
    note("actor inputs: mode thresholds 512 / 1792 / 2560, null stream")
    d_in, out = _device_batch(torch, 2560, seed=2560)
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    full = _call_all(torch, hip, d_in, out, 2560, s, s)
    for n in (511, 512, 1791, 1792, 2559):
        for t in out:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        part = _call_all(torch, hip, d_in, out, n, s, s)
        for name, g, w in zip(names, full, part):
            assert np.array_equal(g[:n], w), f"{name}: {n}-row call differs from 2560-row call"
    for t in out:
        t.fill_(float("nan"))
    torch.cuda.synchronize()
    null = _call_all(torch, hip, d_in, out, 2560, None, None)
    for name, g, w in zip(names, null, full):
        assert np.array_equal(g, w), f"{name}: null-stream call differs"


def test_concurrent_callers_on_their_own_streams(torch_cuda, hip):
    """Two host threads, each on its own stream, call the entry at 4,096
    environments three times each at once: the calls share the device's
    second stream one fork ... join at a time, and every result must equal
    the same call made alone."""
    import threading

    torch = torch_cuda
    note("actor inputs: two host threads, 4096 envs, own streams")
    jobs = [_device_batch(torch, 4096, seed=4096 + k) for k in range(2)]
    s0 = torch.cuda.current_stream()
    torch.cuda.synchronize()
    alone = [_call_all(torch, hip, d_in, out, 4096, s0, s0) for d_in, out in jobs]
    for _, out in jobs:
        for t in out:
            t.fill_(float("nan"))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in jobs]
    results, errors = [None, None], []

    def worker(k):
        try:
            d_in, out = jobs[k]
            for _ in range(3):
                assert hip.actor_inputs_device(*d_in, *out, 4096, streams[k]) == 1
            assert hip.synchronize(streams[k]) == 1
            results[k] = [t.cpu().numpy().view(np.uint32).copy() for t in out]
        except Exception as exc:  # reported below, on the test's thread
            errors.append(repr(exc))

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a caller thread did not finish"
    assert not errors, errors
    for k in range(2):
        for name, g, w in zip(("proprio", "mission", "tactical", "prior", "lidar", "luma"),
                              results[k], alone[k]):
            assert np.array_equal(g, w), f"thread {k}: {name} differs from the call made alone"


def test_graph_capture_with_the_second_stream(torch_cuda, hip):
    """A call captured into a HIP graph after the device's second stream
    exists: the fork and join events bring that stream into the capture.
    Each of three replays, with eager work and a refill of the outputs
    between them, must equal the eager call bit for bit."""
    torch = torch_cuda
    note("actor inputs: graph capture at 4096 envs, 3 replays")
    d_in, out = _device_batch(torch, 4096, seed=4242)
    s0 = torch.cuda.current_stream()
    torch.cuda.synchronize()
    eager = _call_all(torch, hip, d_in, out, 4096, s0, s0)   # also makes the second stream
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cs = torch.cuda.current_stream()
        assert hip.actor_inputs_device(*d_in, *out, 4096, cs) == 1
    scratch = torch.zeros(1 << 20, device="cuda")
    for rep in range(3):
        for t in out:
            t.fill_(float("nan"))
        scratch.add_(1.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t.cpu().numpy().view(np.uint32).copy() for t in out]
        for name, g, w in zip(("proprio", "mission", "tactical", "prior", "lidar", "luma"),
                              got, eager):
            assert np.array_equal(g, w), f"replay {rep}: {name} differs from the eager call"


def test_more_than_64_environments_per_scan_wave(torch_cuda, hip):
    """As for the onboard entry: 263,144 rows tiled from 4,096 distinct
    environments (the scan waves form a second group of 64 frames, and the
    control kernel's workgroups, which also write the symlog scalars, loop
    past their 4,096-workgroup cap); proprio, mission, tactical and prior
    rows must equal the 4,096-row call's bit for bit, and so must the LiDAR
    channels (the scan waves write those of their rays), compared on the
    device.  Luma is left out (no scan wave writes it)."""
    torch = torch_cuda
    distinct, batch = 4096, 64 * 4096 + 1000
    note(f"actor inputs {batch} envs tiled from {distinct}")
    b = synth.make_batch(distinct, seed=272, threads=16)
    obs = torch.from_numpy(b.obs).cuda()
    mission = torch.from_numpy(b.mission).cuda()
    reps = (batch + distinct - 1) // distinct

    def run(o, m):
        n = o.shape[0]
        out = [torch.full((n, w), float("nan"), dtype=torch.float32, device="cuda")
               for w in (91, 49, 24, 15)]
        lidar = torch.full((n, 6, 16, 128), float("nan"), dtype=torch.float32, device="cuda")
        s = torch.cuda.current_stream()
        assert hip.actor_inputs_device(o, m, None, *out, lidar, None, n, s) == 1
        assert hip.synchronize(s) == 1
        return [t.cpu().numpy().view(np.uint32) for t in out], lidar

    small, small_lidar = run(obs, mission)
    big_obs = obs.repeat(reps, 1)[:batch].contiguous()
    big_mis = mission.repeat(reps, 1)[:batch].contiguous()
    big, big_lidar = run(big_obs, big_mis)
    del big_obs, big_mis
    rows = np.arange(batch) % distinct
    for g, w, name in zip(big, small, ("proprio", "mission", "tactical", "prior")):
        bad = np.argwhere((g != w[rows]).any(1)).ravel()
        assert not bad.size, f"{name} differs at rows {bad[:5]}"
    for k in range(reps):
        n = min(distinct, batch - k * distinct)
        assert torch.equal(big_lidar[k * distinct:k * distinct + n].view(torch.int32),
                           small_lidar[:n].view(torch.int32)), f"lidar differs in tile {k}"


def test_argument_validation(hip):
    lib = hip.hip_lib()
    d = ctypes.c_void_p(256)
    odd = ctypes.c_void_p(260)
    f = lib.tb_hip_actor_inputs_device
    assert f(None, d, d, d, d, d, d, d, d, 1, None) == 0          # obs NULL
    assert f(d, d, d, None, d, d, d, d, d, 1, None) == 0          # proprio NULL
    assert f(d, d, None, d, d, d, d, d, d, 1, None) == 0          # luma without cameras
    assert f(odd, d, d, d, d, d, d, d, d, 1, None) == 0           # misaligned obs
    assert f(d, d, d, d, d, d, d, odd, d, 1, None) == 0           # misaligned channels
    assert f(d, d, d, d, d, d, d, d, d, 0, None) == 0             # empty batch
