#!/usr/bin/env python3
"""Benchmark of the batched sensor-feature path on one MI355X.

Workload: 16,384 environments per call, each
4x64x64 uint8 cameras + 4,148-float observation (4,096 LiDAR bins, 52 state
values) + 10-float mission -> 142 float features.  One "step" is one call of
tb_cuda_extract_features_device over the whole resident batch; inputs rotate
over several buffer sets (each 550 MB, together far above the 256 MB
Infinity Cache) so no step is served from cache.

Prints ONE JSON line (the driver's contract) with a `roofline` object (the
feature kernel's algorithmic HBM bytes / its average duration, HIP events on
the launch stream) and a `cpu_baseline` object (the CPU oracle timed on this
host's cores over a bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "sensor-feature envs/sec and achieved HBM GB/s (% of peak) at 16,384 envs"
BATCH = 16384
OBS_B, MISSION_B, CAMERA_B, OUT_B = 4148 * 4, 10 * 4, 16384, 142 * 4
BYTES_PER_ENV = OBS_B + MISSION_B + CAMERA_B + OUT_B          # 33,584 algorithmic bytes
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "traffic_features_16384.json"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


CPU_THREAD_CAP = 16  # the GPU box's CPU share for one GPU


def affinity_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def host_threads() -> int:
    return max(1, min(affinity_cores(), CPU_THREAD_CAP))


def make_sets(torch, nsets: int, threads: int):
    from turbinator_c_amd import synth
    sets = []
    host0 = None
    for k in range(nsets):
        b = synth.make_batch(BATCH, seed=42 + k, threads=threads)
        if k == 0:
            host0 = b
        sets.append((torch.from_numpy(b.obs).cuda(), torch.from_numpy(b.mission).cuda(),
                     torch.from_numpy(b.cameras).cuda(),
                     torch.empty((BATCH, 142), dtype=torch.float32, device="cuda")))
    torch.cuda.synchronize()
    return sets, host0


def time_gpu(torch, sets, steps: int, warmup: int):
    from turbinator_c_amd import features
    stream = torch.cuda.current_stream()
    n = len(sets)

    def call(i):
        o, m, c, out = sets[i % n]
        if features.extract_features_device(o, m, c, out, BATCH, stream) != 1:
            raise RuntimeError("tb_cuda_extract_features_device launch failed")

    # Device ramp before the W warm-up calls: after the host-side input
    # generation the GPU's first ~30 ms of work run slower (10 warm-up calls
    # measured 87.1-88.7 us per call, 400 measured 85.9-86.0 us on the same
    # box), so the feature kernel runs for at least RAMP_S first.
    ramp_calls, t_ramp = 0, time.perf_counter()
    while time.perf_counter() - t_ramp < RAMP_S:
        for _ in range(50):
            call(ramp_calls)
            ramp_calls += 1
        torch.cuda.synchronize()
    for i in range(warmup):
        call(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        call(i)
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(stop) / 1e3, wall, ramp_calls


RAMP_S = 0.05  # seconds of untimed feature calls before the W warm-up calls
COPY_BYTES = 1 << 30


def copy_calibration(torch, reps: int = 5) -> None:
    """Device-to-device copies of exactly COPY_BYTES: under rocprofv3 --pmc
    their FETCH_SIZE / WRITE_SIZE per dispatch calibrate the counters."""
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()


def summarize_pmc(fetch_csv: str, write_csv: str) -> dict:
    """HBM bytes per feature-kernel launch from two rocprofv3 --pmc runs of
    `bench.py --no-cpu --copy-calibration` (FETCH_SIZE, then WRITE_SIZE; KiB
    per dispatch), each scaled by what the counter reads for the 1 GiB copy."""
    import csv
    import statistics

    def per_kernel(path):
        out = {}
        for r in csv.DictReader(open(path)):
            out.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return out

    f, w = per_kernel(fetch_csv), per_kernel(write_csv)
    feat = next(k for k in f if "features_kernel" in k)
    copy = max((k for k in f if "copyBuffer" in k), key=lambda k: statistics.mean(f[k]))
    copy_kib = COPY_BYTES / 1024
    f_scale = copy_kib / max(f[copy])
    w_scale = copy_kib / max(w[copy])
    fetch_b = statistics.mean(f[feat]) * 1024 * f_scale
    write_b = statistics.mean(w[feat]) * 1024 * w_scale
    return {"kernel": feat, "dispatches": len(f[feat]),
            "fetch_kib_raw": statistics.mean(f[feat]), "write_kib_raw": statistics.mean(w[feat]),
            "fetch_scale": f_scale, "write_scale": w_scale,
            "copy_fetch_kib_raw": max(f[copy]), "copy_write_kib_raw": max(w[copy]),
            "hbm_bytes_per_launch": round(fetch_b + write_b),
            "algorithmic_bytes_per_launch": BYTES_PER_ENV * BATCH,
            "traffic_over_algorithmic": (fetch_b + write_b) / (BYTES_PER_ENV * BATCH)}


def verify_sample(torch, sets, host0) -> dict:
    """Checks the benchmarked set-0 outputs on 256 envs against the oracle."""
    import oracle
    from tests.conftest import assert_feature_parity
    idx = np.linspace(0, BATCH - 1, 256).astype(np.int64)
    got = sets[0][3].cpu().numpy()[idx]
    want = oracle.features(host0.obs[idx], host0.mission[idx], host0.cameras[idx])
    return assert_feature_parity(got, want, "bench-sample")


def _events_time(torch, launch, steps: int, warmup: int) -> float:
    """Seconds per call of `launch(i)` on the current stream (HIP events),
    after at least `warmup` untimed calls and at least SUITE_WARMUP_S of
    untimed calls (the first ~30 ms of a workload that follows host-side
    work run slower: the diagnostics kernel measured 117 -> 95 us per call
    over its first 250 calls)."""
    stream = torch.cuda.current_stream()
    i, t0 = 0, time.perf_counter()
    while i < warmup or time.perf_counter() - t0 < SUITE_WARMUP_S:
        for _ in range(max(warmup, 1)):
            launch(i, stream)
            i += 1
        torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(steps):
        launch(i, stream)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / 1e3 / steps


def _report(name: str, per_call: float, envs: int, bytes_per_env: int | None, **extra) -> dict:
    r = {"workload": name, "us_per_call": round(per_call * 1e6, 2),
         "envs_per_s": round(envs / per_call, 1)}
    if bytes_per_env:
        gbs = bytes_per_env * envs / per_call / 1e9
        r.update(bytes_per_env=bytes_per_env, achieved_GBs=round(gbs, 1),
                 frac_of_peak=round(gbs / HBM_PEAK_GBS, 4))
    r.update(extra)
    log("[suite] " + json.dumps(r))
    return r


SUITE_LEGS = ("depth", "diag", "onboard", "actor_prep", "sac_actor", "c5", "replay", "host")
# Untimed calls (and seconds of them) before each secondary workload.
SUITE_WARMUP = 20
SUITE_WARMUP_S = 0.1


def suite(torch, sets, threads: int, steps: int, legs=SUITE_LEGS) -> list:
    """Secondary workloads, printed to stderr (the stdout line is the headline).
    `legs` selects a subset of SUITE_LEGS."""
    out = []
    for leg in SUITE_LEGS:
        if leg not in legs:
            continue
        out += _suite_leg(leg, torch, sets, threads, steps)
    return out


def _suite_leg(leg: str, torch, sets, threads: int, steps: int) -> list:
    out = []
    if leg == "host":
        return host_legs(threads)
    tac = torch.empty((BATCH, 24), dtype=torch.float32, device="cuda")
    pri = torch.empty((BATCH, 15), dtype=torch.float32, device="cuda")
    if leg == "depth":
        _leg_depth(torch, sets, threads, steps, out)
    elif leg == "diag":
        _leg_diag(torch, sets, steps, out)
    elif leg == "onboard":
        _leg_onboard(torch, sets, steps, out, tac, pri)
    elif leg == "actor_prep":
        _leg_actor_prep(torch, sets, steps, out, tac, pri)
    elif leg == "sac_actor":
        _leg_sac_actor(torch, sets, steps, out)
    elif leg == "c5":
        _leg_c5(torch, threads, steps, out)
    elif leg == "replay":
        _leg_replay(torch, threads, steps, out)
    return out


def _leg_depth(torch, sets, threads, steps, out):
    from turbinator_c_amd import features, synth
    # fp32 depth cameras: the configurations' literal 4x64x64 fp32 cameras.
    dsets = []
    for k in range(3):
        b = synth.make_batch(BATCH, seed=142 + k, with_depth=True, threads=threads)
        dsets.append((torch.from_numpy(b.obs).cuda(), torch.from_numpy(b.mission).cuda(),
                      torch.from_numpy(b.depth).cuda(),
                      torch.empty((BATCH, 142), dtype=torch.float32, device="cuda")))
        del b

    def depth_call(i, s):
        o, m, d, f = dsets[i % 3]
        assert features.extract_features_depth_device(o, m, d, f, BATCH, s) == 1
    per = _events_time(torch, depth_call, steps, SUITE_WARMUP)
    stats = _depth_sample_parity(torch, dsets[0])
    out.append(_report("config 3 with fp32 depth cameras (16,384 envs, 3 rotating sets)",
                       per, BATCH, OBS_B + MISSION_B + 4 * CAMERA_B + OUT_B,
                       parity_sample=stats))
    del dsets


def _depth_sample_parity(torch, dset) -> dict:
    """256 environments of a depth set's features against the oracle of the
    luma bytes the depth maps to."""
    import oracle
    from tests.conftest import assert_feature_parity
    o, m, d, f = dset
    idx = torch.linspace(0, BATCH - 1, 256, device="cuda").long()
    obs, mis = o[idx].cpu().numpy(), m[idx].cpu().numpy()
    luma = oracle.depth_to_luma(d[idx].cpu().numpy())
    got = f[idx].cpu().numpy()
    return assert_feature_parity(got, oracle.features(obs, mis, luma), "bench-depth")


def _leg_diag(torch, sets, steps, out):
    from turbinator_c_amd import features
    diag_bytes = 432  # TB_HIP_DIAG_BYTES
    diag = torch.empty((BATCH, diag_bytes), dtype=torch.uint8, device="cuda")

    def diag_call(i, s):
        o, m, c, f = sets[i % len(sets)]
        assert features.extract_features_diagnostics_device(o, m, c, f, diag, BATCH, s) == 1
    out.append(_report(f"config 3 + diagnostics ({diag_bytes} B/env)",
                       _events_time(torch, diag_call, steps, SUITE_WARMUP), BATCH,
                       BYTES_PER_ENV + diag_bytes))


def onboard_scan_ray_bytes(mission: np.ndarray) -> np.ndarray:
    """Bytes of scan rays each environment's mission uses (onboard_features.cuh:
    107-109, 208-244): rows 0-3 of both heads (1,024 rays) for a dodge
    mission (m5 > 0.75), all 1,536 for a slalom mission (m4 > 0.75 and
    m5 <= 0.25), none otherwise; mission values map NaN -> 0, +-inf -> +-1
    first (onboard_features.cuh:13-15)."""
    mis = np.nan_to_num(np.asarray(mission, np.float32)[:, 4:6], nan=0.0, posinf=1.0,
                        neginf=-1.0)
    m4, m5 = mis[:, 0], mis[:, 1]
    slalom = (m4 > 0.75) & (m5 <= 0.25)
    dodge = m5 > 0.75
    return np.where(slalom, 4 * 1536, np.where(dodge, 4 * 1024, 0))


def _leg_onboard(torch, sets, steps, out, tac, pri):
    from turbinator_c_amd import features

    def onboard_call(i, s):
        o, m, _, _ = sets[i % len(sets)]
        assert features.onboard_tactical_prior_device(o, m, tac, pri, None, BATCH, s) == 1
    # H2 reads obs[0..47] and the mission row and writes 24 + 15 floats for
    # every environment; of the 1,536 scan rays (2 heads x 6 elevations x 128
    # azimuths) it reads those the mission uses: rows 0-3 (1,024 rays) for a
    # dodge mission (m5 > 0.75), all of them for a slalom mission (m4 > 0.75,
    # m5 <= 0.25), none otherwise (onboard_features.cuh:208-244).
    fixed = 4 * (48 + 10 + 24 + 15)
    full_scan = fixed + 4 * 1536
    ray_bytes = [float(onboard_scan_ray_bytes(m.cpu().numpy()).mean()) for _, m, _, _ in sets]
    onboard_bytes = int(round(fixed + sum(ray_bytes) / len(ray_bytes)))
    per_call = _events_time(torch, onboard_call, steps, SUITE_WARMUP)
    full_gbs = full_scan * BATCH / per_call / 1e9
    out.append(_report("onboard tactical+prior (16,384 envs)", per_call, BATCH,
                       onboard_bytes, full_scan_bytes_per_env=full_scan,
                       full_scan_GBs=round(full_gbs, 1),
                       full_scan_frac_of_peak=round(full_gbs / HBM_PEAK_GBS, 4),
                       note="bytes_per_env: proprio and mission read once, tactical and "
                            "prior written once, and the scan rays each environment's "
                            "mission uses (rows 0-3 for dodge, all for slalom, none "
                            "otherwise; this batch's average); full_scan_bytes_per_env "
                            "counts every scan ray, as the reference's loop reads them "
                            "(onboard_features.cuh:188-234), and full_scan_GBs is that "
                            "count over the measured time; latency-bound, not HBM-bound"))


def _leg_actor_prep(torch, sets, steps, out, tac, pri):
    from turbinator_c_amd import features
    # f3: the 618M actor's sensor preparation (network_gpu.cu:1446-1451) fused:
    # proprio 91 + mission 49 + tactical 24 + prior 15 + 6x16x128 LiDAR
    # channels + 4x64x64 luma per environment.
    a_pro = torch.empty((BATCH, 91), dtype=torch.float32, device="cuda")
    a_mis = torch.empty((BATCH, 49), dtype=torch.float32, device="cuda")
    a_lid = torch.empty((BATCH, 6, 16, 128), dtype=torch.float32, device="cuda")
    a_lum = torch.empty((BATCH, 4, 64, 64), dtype=torch.float32, device="cuda")

    def actor_call(i, s):
        o, m, c, _ = sets[i % len(sets)]
        assert features.actor_inputs_device(o, m, c, a_pro, a_mis, tac, pri, a_lid, a_lum,
                                            BATCH, s) == 1
    actor_bytes = OBS_B + MISSION_B + CAMERA_B + 4 * (91 + 49 + 24 + 15 + 6 * 2048 + 16384)
    out.append(_report("618M actor sensor preparation, fused (16,384 envs)",
                       _events_time(torch, actor_call, steps, SUITE_WARMUP), BATCH, actor_bytes,
                       note="bytes_per_env: inputs once + every output once"))
    del a_pro, a_mis, a_lid, a_lum


def _leg_sac_actor(torch, sets, steps, out):
    from turbinator_c_amd import features
    # f4: the compact SAC actor (hidden 128, the reference default) acting on
    # the device-resident features of the headline batch.
    from turbinator_c_amd import actor
    hidden = 128
    wrng = np.random.default_rng(3)
    ws = []
    for (o, i_), nb in actor.layer_shapes(hidden):
        ws.append(torch.from_numpy((wrng.standard_normal((o, i_)) * np.sqrt(2.0 / (o + i_)))
                                   .astype(np.float32)).cuda())
        ws.append(torch.zeros(nb, dtype=torch.float32, device="cuda"))
    packed = torch.empty(actor.packed_bytes(hidden) // 4, dtype=torch.float32, device="cuda")
    assert actor.pack_device(*ws, hidden, packed, torch.cuda.current_stream()) == 1
    normals = torch.randn((BATCH, 15), dtype=torch.float32, device="cuda")
    acts = torch.empty((BATCH, 15), dtype=torch.float32, device="cuda")
    logp = torch.empty((BATCH,), dtype=torch.float32, device="cuda")
    # The reference's fp32 flops per row, and the fp16 matrix-core flops the
    # kernel executes for them: three products per multiply-add (the
    # two-piece split), on 160 padded inputs and 32 padded outputs.
    flops_env = 2 * (142 * hidden + hidden * hidden + hidden * 30)
    mfma_flops_env = 3 * 2 * (160 * hidden + hidden * hidden + hidden * 32)

    def actor_only(i, s):
        feats = sets[i % len(sets)][3]
        assert actor.act_device(packed, hidden, feats, normals, acts, logp, None, BATCH, s) == 1
    per = _events_time(torch, actor_only, steps, SUITE_WARMUP)
    tf = flops_env * BATCH / per / 1e12
    tf16 = mfma_flops_env * BATCH / per / 1e12
    out.append(_report("compact SAC actor, hidden 128, stochastic (16,384 feature rows)",
                       per, BATCH, None, flops_per_env=flops_env, achieved_TFLOPs=round(tf, 2),
                       fp16_mfma_flops_per_env=mfma_flops_env,
                       frac_of_fp16_mfma_peak=round(tf16 / 2500.0, 4)))

    def features_then_actor(i, s):
        o, m, c, f = sets[i % len(sets)]
        assert features.extract_features_device(o, m, c, f, BATCH, s) == 1
        assert actor.act_device(packed, hidden, f, normals, acts, logp, None, BATCH, s) == 1
    out.append(_report("sensor features + compact actor, on device (16,384 envs)",
                       _events_time(torch, features_then_actor, steps, SUITE_WARMUP), BATCH, None))
    del packed, normals, acts, logp, ws


def _leg_c5(torch, threads, steps, out):
    from turbinator_c_amd import features, synth
    # Configuration 5: 65,536 replay records of 66,672 B, features in place.
    n5, rec = 65536, 66672
    buf = np.zeros(n5 * rec, np.uint8)
    synth.fill_records(buf, n5, rec, 0, 16592, 16632, seed=77, threads=threads)
    dbuf = torch.from_numpy(buf).cuda()
    del buf
    f5 = torch.empty((n5, 142), dtype=torch.float32, device="cuda")
    base = dbuf.data_ptr()

    def c5_call(i, s):
        assert features.extract_features_strided_device(base, rec, base + 16592, rec,
                                                        base + 16632, rec, f5, n5, s) == 1
    per = _events_time(torch, c5_call, max(steps // 4, 10), 5)
    stats = _c5_sample_parity(torch, dbuf, f5, rec)
    out.append(_report("config 5: 65,536 replay records x 66,672 B, in place",
                       per, n5, BYTES_PER_ENV, parity_sample=stats))
    del dbuf, f5


def _c5_sample_parity(torch, dbuf, f5, rec) -> dict:
    """256 records' features against the oracle on the same record bytes."""
    import oracle
    from tests.conftest import assert_feature_parity
    n5 = f5.shape[0]
    idx = np.linspace(0, n5 - 1, 256).astype(np.int64)
    rows = dbuf.view(n5, rec)[torch.from_numpy(idx).cuda()].cpu().numpy()
    want = oracle.features_strided(rows.reshape(-1), 256, rec, 0, 16592, 16632)
    return assert_feature_parity(f5[torch.from_numpy(idx).cuda()].cpu().numpy(), want,
                                 "bench-config5")


def _leg_replay(torch, threads, steps, out):
    from turbinator_c_amd import features, synth
    # Replay sampling (f1): 16,384 samples from a 65,536-slot SoA replay, fused
    # versus the reference's gather-into-a-batch followed by extraction.
    cap = 65536
    rep = synth.make_batch(cap, seed=5, threads=threads)
    r_obs = torch.from_numpy(rep.obs).cuda()
    r_mis = torch.from_numpy(rep.mission).cuda()
    r_cam = torch.from_numpy(rep.cameras).cuda()
    del rep
    idx = torch.randint(0, cap, (BATCH,), dtype=torch.int32, device="cuda")
    fo = torch.empty((BATCH, 142), dtype=torch.float32, device="cuda")

    def fused_call(i, s):
        assert features.extract_features_indexed_device(r_obs, OBS_B, r_mis, MISSION_B, r_cam,
                                                        CAMERA_B, cap, idx, fo, BATCH, s) == 1
    out.append(_report("replay sample 16,384 of 65,536 + features, fused",
                       _events_time(torch, fused_call, steps, SUITE_WARMUP), BATCH, BYTES_PER_ENV))
    g_obs = torch.empty((BATCH, 4148), dtype=torch.float32, device="cuda")
    g_mis = torch.empty((BATCH, 10), dtype=torch.float32, device="cuda")
    g_cam = torch.empty((BATCH, 16384), dtype=torch.uint8, device="cuda")
    lidx = idx.long()

    def gather_call(i, s):
        torch.index_select(r_obs, 0, lidx, out=g_obs)
        torch.index_select(r_mis, 0, lidx, out=g_mis)
        torch.index_select(r_cam, 0, lidx, out=g_cam)
        assert features.extract_features_device(g_obs, g_mis, g_cam, fo, BATCH, s) == 1
    out.append(_report("replay sample 16,384 of 65,536: gather batch, then features",
                       _events_time(torch, gather_call, steps, SUITE_WARMUP), BATCH, BYTES_PER_ENV,
                       note="bytes_per_env counts only the fused minimum"))
    del r_obs, r_mis, r_cam, g_obs, g_mis, g_cam


def host_legs(threads: int) -> list:
    """Host-side workloads, PCIe included: the reference's pageable host API
    and the pinned, double-buffered pipeline."""
    from turbinator_c_amd import features, synth
    out = []
    # Host API, PCIe included (pageable copies, as the reference): the
    # trainer's default batch 32 (latency) and the 1,024 cap (bandwidth).
    for n, reps in ((32, 200), (1024, 20)):
        hb = synth.make_batch(n, seed=9, threads=threads)
        outh = np.empty((n, 142), np.float32)
        fb = features.FeatureBatch.create(0, n)
        try:
            for _ in range(3):
                assert fb.extract_host(hb.obs, hb.mission, hb.cameras, n, outh) == 1
            t0 = time.perf_counter()
            for _ in range(reps):
                assert fb.extract_host(hb.obs, hb.mission, hb.cameras, n, outh) == 1
            per = (time.perf_counter() - t0) / reps
        finally:
            fb.destroy()
        out.append(_report(f"host API tb_cuda_extract_features_host, {n} envs (PCIe-inclusive)",
                           per, n, None, note="pageable host memory, synchronous",
                           host_GBs=round(n * (BYTES_PER_ENV - 0) / per / 1e9, 2)))

    # Pinned, double-buffered pipeline (tb_hip_feature_pipeline_*): the
    # producer's data already sits in the pinned slots; one slot measures
    # submit + wait latency, two slots the steady state with one batch in
    # flight while the other is collected and resubmitted.
    for n, slots, reps, direct in ((32, 1, 200, False), (32, 2, 200, False),
                                   (32, 1, 200, True), (32, 2, 200, True),
                                   (1024, 1, 20, False), (1024, 2, 20, False),
                                   (1024, 1, 20, True), (1024, 2, 20, True),
                                   (16384, 2, 6, False), (16384, 2, 6, True)):
        hb = synth.make_batch(n, seed=9, threads=threads)
        pipe = features.FeaturePipeline.create(0, n, slots)
        assert pipe is not None, "pipeline create failed"
        try:
            for s in range(slots):
                o, m, c = pipe.inputs(s)
                o[:] = hb.obs
                m[:] = hb.mission
                c[:] = hb.cameras
            submit = pipe.submit_direct if direct else pipe.submit
            for s in range(slots):
                assert submit(s, n) == 1, pipe.error()
                assert pipe.wait(s, n) is not None, pipe.error()
            t0 = time.perf_counter()
            if slots == 1:
                for _ in range(reps):
                    assert submit(0, n) == 1
                    assert pipe.wait(0, n) is not None
            else:
                for s in range(slots):
                    assert submit(s, n) == 1
                for r in range(reps):
                    s = r % slots
                    assert pipe.wait(s, n) is not None
                    assert submit(s, n) == 1
                for s in range(slots):
                    assert pipe.wait(s, n) is not None
                reps += slots
            per = (time.perf_counter() - t0) / reps
            got = pipe.wait(0, n).copy()
        finally:
            pipe.destroy()
        if n <= 1024:
            import oracle
            from tests.conftest import assert_feature_parity
            assert_feature_parity(got, oracle.features(hb.obs, hb.mission, hb.cameras),
                                  f"pipeline{n}")
        mode = "direct (kernel on pinned memory)" if direct else "copy engines"
        out.append(_report(f"pinned pipeline, {mode}, {n} envs, {slots} slot(s) "
                           "(PCIe-inclusive)",
                           per, n, None,
                           note="producer writes the pinned slots in place; "
                                + ("submit + wait" if slots == 1 else "steady state, "
                                   "one batch in flight while the other is collected"),
                           host_GBs=round(n * BYTES_PER_ENV / per / 1e9, 2)))
    return out


def cpu_baseline(host0, threads: int, budget_s: float) -> dict:
    """The reference's own CPU feature twin (src/training/training.c:102-142,
    compiled from its source into oracle/_ref with its Release flags, -O3
    -std=c11) over the first environments of the same batch, split over
    `threads` host threads, repeated until `budget_s` of wall time.  Where
    oracle/_ref was not built, the oracle's restatement of it is timed
    instead (kind "port")."""
    import oracle
    ref = oracle.ref_lib()
    sample = min(BATCH, 4096 * threads)
    out = np.empty((sample, 142), np.float32)
    if ref is not None:
        kind = "reference"
        run = lambda: ref.ref_features_batch(host0.obs.ctypes.data, host0.mission.ctypes.data,  # noqa: E731
                                             host0.cameras.ctypes.data, out.ctypes.data, sample,
                                             threads)
    else:
        kind = "port"
        lib = oracle.lib()
        args = (host0.obs.ctypes.data, OBS_B, host0.mission.ctypes.data, MISSION_B,
                host0.cameras.ctypes.data, CAMERA_B, out.ctypes.data, sample, threads)
        run = lambda: lib.orc_features_batch(*args)  # noqa: E731
    run()  # warm-up pass
    envs, t0, rates = 0, time.perf_counter(), []
    while True:
        tp = time.perf_counter()
        run()
        rates.append(sample / (time.perf_counter() - tp))
        envs += sample
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    rate = float(np.median(rates))  # median of the timed passes
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    what = ("the reference's tb_train_extract_features_cpu" if kind == "reference"
            else "the oracle restatement of tb_train_extract_features_cpu")
    return {"value": round(rate, 1), "unit": "envs/s", "cores": threads, "kind": kind,
            "sample": f"{what}: median of {len(rates)} timed passes over {sample}-env slices "
                      f"of the configuration-3 batch ({envs} envs, {el:.1f} s) on {threads} "
                      f"threads of {cpu}; {rate * BYTES_PER_ENV / 1e9:.2f} GB/s effective"}


def cpu_baselines(host0, threads: int, budget_s: float) -> dict:
    """All-cores figure (the host share: the affinity set, capped at
    CPU_THREAD_CAP threads) with the single-thread figure beside it."""
    allc = cpu_baseline(host0, threads, budget_s)
    one = cpu_baseline(host0, 1, budget_s)
    allc["affinity_cores"] = affinity_cores()
    allc["cores_cap"] = CPU_THREAD_CAP
    allc["single_thread"] = {"value": one["value"], "unit": "envs/s", "cores": 1,
                             "sample": one["sample"]}
    return allc


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--sets", type=int, default=3, help="rotating input buffer sets")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-threads", type=int, default=None,
                    help="host threads of the CPU baseline (default: the host share, at most 16)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the configuration-3 fp32-depth and configuration-5 lines")
    ap.add_argument("--suite", action="store_true",
                    help="also time the secondary workloads (stderr JSON lines)")
    ap.add_argument("--host-legs", action="store_true",
                    help="also time the host API and the pinned pipeline (stderr)")
    ap.add_argument("--legs", default=None,
                    help="comma-separated subset of the --suite workloads: " + ",".join(SUITE_LEGS))
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after timing, run 1 GiB device copies (PMC calibration)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write the traffic summary from two rocprofv3 --pmc CSVs and exit")
    args = ap.parse_args()
    if args.summarize_pmc:
        summary = summarize_pmc(*args.summarize_pmc)
        TRAFFIC_FILE.write_text(json.dumps(summary, indent=1) + "\n")
        print(json.dumps(summary, indent=1))
        return 0
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only. The feature path needs no "
              "inter-GPU exchange: a batch shards by contiguous environment ranges, one per "
              "GPU, each running the same kernel. Use --gpus 1.", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    from turbinator_c_amd import features
    features.hip_lib()
    threads = host_threads()
    log(f"[bench] generating {args.sets} x {BATCH} envs on {threads} threads")
    sets, host0 = make_sets(torch, args.sets, threads)
    log("[bench] timing")
    gpu_s, wall_s, ramp_calls = time_gpu(torch, sets, args.steps, args.warmup)
    per_call = gpu_s / args.steps
    stats = verify_sample(torch, sets, host0)
    log(f"[bench] parity sample ok: {stats}")
    if args.copy_calibration:
        copy_calibration(torch)
    if args.suite or args.legs:
        legs = SUITE_LEGS if not args.legs else tuple(args.legs.split(","))
        unknown = set(legs) - set(SUITE_LEGS)
        if unknown:
            print(f"bench.py: unknown legs {sorted(unknown)}", file=sys.stderr)
            return 2
        suite(torch, sets, threads, args.steps, legs)
    elif args.host_legs:
        host_legs(threads)
    secondary = None
    if not args.no_secondary:
        # BASELINE.json configurations 3 (literal fp32 depth cameras) and 5
        # (strided replay records), each with its own roofline fraction; then
        # the other rows of the path on the headline batch: the onboard
        # tactical + prior entry, the 618M actor's fused sensor preparation
        # and the compact actor (alone and behind the feature kernel).
        log("[bench] secondary: configuration 3 fp32 depth, configuration 5, onboard, "
            "actor preparation, compact actor")
        secondary = []
        _leg_depth(torch, sets, threads, max(args.steps // 5, 20), secondary)
        torch.cuda.empty_cache()
        _leg_c5(torch, threads, max(args.steps // 2, 40), secondary)
        torch.cuda.empty_cache()
        tac = torch.empty((BATCH, 24), dtype=torch.float32, device="cuda")
        pri = torch.empty((BATCH, 15), dtype=torch.float32, device="cuda")
        _leg_onboard(torch, sets, max(args.steps, 40), secondary, tac, pri)
        _leg_actor_prep(torch, sets, max(args.steps // 2, 40), secondary, tac, pri)
        _leg_sac_actor(torch, sets, max(args.steps, 40), secondary)
        del tac, pri
        torch.cuda.empty_cache()
    bytes_per_call = BYTES_PER_ENV * BATCH
    achieved = bytes_per_call / per_call / 1e9
    traffic, traffic_src = None, None
    if TRAFFIC_FILE.exists():
        tj = json.loads(TRAFFIC_FILE.read_text())
        traffic = tj.get("hbm_bytes_per_launch")
        traffic_src = (f"{TRAFFIC_FILE.relative_to(ROOT)}: stored rocprofv3 --pmc FETCH_SIZE "
                       f"and WRITE_SIZE runs of `bench.py --no-cpu --no-secondary "
                       f"--copy-calibration`, scaled by a 1 GiB copy; not measured in this run")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "traffic_source": traffic_src}
    cpu = None
    if not args.no_cpu:
        log(f"[bench] cpu baseline ({args.cpu_seconds:.0f} s budget, all cores then 1 thread)")
        cpu = cpu_baselines(host0, args.cpu_threads or threads, args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(BATCH / per_call, 1),
        "unit": "envs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(per_call * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "configuration 3: 16,384 envs/call, 4x64x64 u8 cameras + "
                               "4,148 f32 obs + 10 f32 mission -> 142 f32 features",
                   "global_batch": BATCH, "bytes_per_env": BYTES_PER_ENV,
                   "buffer_sets": args.sets, "entry": "tb_cuda_extract_features_device",
                   "wall_s_timed": round(wall_s, 4),
                   "device_ramp": {"seconds": RAMP_S, "calls": ramp_calls,
                                   "note": "untimed feature calls before the W warm-up calls"}},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
