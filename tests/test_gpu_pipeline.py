"""GPU parity of the pinned, double-buffered host pipeline
(tb_hip_feature_pipeline_*, include/turbinator/training/hip_features.h)
against the CPU oracle, through the C-ABI.

The pipeline replaces the pageable round trip of the reference host object
(src/cuda/features.cu:62-88) for producers that write into its pinned slots.
Cases: counts 1, 3, 32 and a full slot (the single-copy path), two slots in
flight with different data, ten ping-pong rounds with fresh data per round
(no slot sees another's rows), the no-camera submit, configuration 2
(1,024 envs) as one full slot, and the slot-state and argument errors.  The
direct submit (extraction on the pinned slot itself) gets the same parity
cases, alternating with copying submits on the same slots.
Tolerance classes are those of tests/conftest.py.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import oracle
from tests.conftest import assert_feature_parity
from turbinator_c_amd import synth

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def fill(pipe, slot: int, b) -> None:
    obs, mission, cams = pipe.inputs(slot)
    n = b.obs.shape[0]
    obs[:n] = b.obs
    mission[:n] = b.mission
    cams[:n] = b.cameras


@pytest.mark.parametrize("count", [1, 3, 32, 64])
def test_pipeline_parity(hip, count):
    note(f"pipeline max_batch 64, count {count}")
    pipe = hip.FeaturePipeline.create(0, 64, 2)
    assert pipe is not None
    try:
        b = synth.make_batch(count, seed=300 + count, variant=synth.ORDINARY)
        fill(pipe, 1, b)
        assert pipe.submit(1, count) == 1, pipe.error()
        got = pipe.wait(1, count)
        assert got is not None, pipe.error()
        assert pipe.error() == ""
        assert_feature_parity(got.copy(), oracle.features(b.obs, b.mission, b.cameras),
                              f"pipeline{count}")
    finally:
        pipe.destroy()


def test_pipeline_two_slots_in_flight(hip):
    note("pipeline: two slots in flight, then 10 ping-pong rounds")
    pipe = hip.FeaturePipeline.create(0, 256, 2)
    assert pipe is not None
    try:
        a = synth.make_batch(256, seed=7, variant=synth.ORDINARY)
        b = synth.make_batch(200, seed=8, variant=synth.EDGE_QUARTERS)
        fill(pipe, 0, a)
        fill(pipe, 1, b)
        assert pipe.submit(0, 256) == 1, pipe.error()
        assert pipe.submit(1, 200) == 1, pipe.error()
        got_b = pipe.wait(1, 200).copy()
        got_a = pipe.wait(0, 256).copy()
        assert_feature_parity(got_a, oracle.features(a.obs, a.mission, a.cameras), "slot0")
        assert_feature_parity(got_b, oracle.features(b.obs, b.mission, b.cameras), "slot1")
        # The trainer's pattern: produce into one slot while the other is in flight.
        pending = None
        for r in range(10):
            slot = r % 2
            n = 97 + 17 * r
            batch = synth.make_batch(n, seed=1000 + r, variant=synth.ORDINARY)
            fill(pipe, slot, batch)
            assert pipe.submit(slot, n) == 1, pipe.error()
            if pending is not None:
                pslot, pn, pb = pending
                got = pipe.wait(pslot, pn).copy()
                assert_feature_parity(got, oracle.features(pb.obs, pb.mission, pb.cameras),
                                      f"round{r - 1}")
            pending = (slot, n, batch)
        pslot, pn, pb = pending
        assert_feature_parity(pipe.wait(pslot, pn).copy(),
                              oracle.features(pb.obs, pb.mission, pb.cameras), "round9")
    finally:
        pipe.destroy()


def test_pipeline_without_cameras(hip):
    note("pipeline: no-camera submit")
    pipe = hip.FeaturePipeline.create(0, 48, 1)
    assert pipe is not None
    try:
        b = synth.make_batch(48, seed=21, variant=synth.ORDINARY)
        obs, mission, cams = pipe.inputs(0)
        obs[:] = b.obs
        mission[:] = b.mission
        cams[:] = 255  # must not be read
        assert pipe.submit(0, 48, with_cameras=False) == 1, pipe.error()
        got = pipe.wait(0, 48).copy()
        assert_feature_parity(got, oracle.features(b.obs, b.mission, None), "pipe-nocam")
        assert np.all(got[:, 126:142].view(np.uint32) == 0)
    finally:
        pipe.destroy()


def test_pipeline_config2_full_slot(hip):
    note("pipeline: configuration 2, 1024 envs as one full slot")
    pipe = hip.FeaturePipeline.create(0, 1024, 2)
    assert pipe is not None
    try:
        b = synth.make_batch(1024, seed=42)
        fill(pipe, 0, b)
        assert pipe.submit(0, 1024) == 1, pipe.error()
        got = pipe.wait(0, 1024).copy()
        stats = assert_feature_parity(got, oracle.features(b.obs, b.mission, b.cameras),
                                      "pipe-c2")
        note(f"pipe-c2 stats {stats}")
    finally:
        pipe.destroy()


def test_pipeline_state_and_argument_errors(hip):
    note("pipeline: slot-state and argument errors")
    pipe = hip.FeaturePipeline.create(0, 8, 2)
    assert pipe is not None
    try:
        b = synth.make_batch(8, seed=5)
        fill(pipe, 0, b)
        assert pipe.wait(1, 8) is None
        assert pipe.error() == "wait: slot 1 has nothing submitted"
        assert pipe.submit(0, 8) == 1
        assert pipe.error() == ""
        assert pipe.submit(0, 8) == 0
        assert pipe.error() == "submit: slot 0 is in flight"
        first = pipe.wait(0, 8)
        assert first is not None
        again = pipe.wait(0, 8)        # a completed slot returns the same rows
        assert again is not None and np.array_equal(first, again)
        want = oracle.features(b.obs, b.mission, b.cameras)
        assert_feature_parity(first.copy(), want, "errors")
        # Argument errors leave the text untouched.
        pipe.submit(0, 8)
        pipe.submit(0, 8)
        text = pipe.error()
        assert text == "submit: slot 0 is in flight"
        assert pipe.submit(0, 0) == 0 and pipe.error() == text
        assert pipe.submit(0, 9) == 0 and pipe.error() == text
        assert pipe.submit(2, 1) == 0 and pipe.error() == text
        assert pipe.submit(-1, 1) == 0 and pipe.error() == text
        with pytest.raises(ValueError):
            pipe.inputs(2)
        assert pipe.wait(0, 8) is not None
    finally:
        pipe.destroy()   # also drains anything still in flight


@pytest.mark.parametrize("count", [1, 32, 200, 256])
def test_direct_submit_parity(hip, count):
    note(f"pipeline direct submit, count {count}")
    pipe = hip.FeaturePipeline.create(0, 256, 2)
    assert pipe is not None
    try:
        b = synth.make_batch(count, seed=500 + count, variant=synth.EDGE_QUARTERS)
        fill(pipe, 0, b)
        assert pipe.submit_direct(0, count) == 1, pipe.error()
        got = pipe.wait(0, count)
        assert got is not None, pipe.error()
        assert_feature_parity(got.copy(), oracle.features(b.obs, b.mission, b.cameras),
                              f"direct{count}")
        # The same slot through the copying path, then direct again without
        # cameras: every submit sees only its own rows.
        c = synth.make_batch(count, seed=600 + count, variant=synth.ORDINARY)
        fill(pipe, 0, c)
        assert pipe.submit(0, count) == 1, pipe.error()
        assert_feature_parity(pipe.wait(0, count).copy(),
                              oracle.features(c.obs, c.mission, c.cameras), f"copy{count}")
        assert pipe.submit_direct(0, count, with_cameras=False) == 1, pipe.error()
        got = pipe.wait(0, count).copy()
        assert_feature_parity(got, oracle.features(c.obs, c.mission, None), f"direct-nocam{count}")
        assert pipe.submit_direct(0, count) == 1
        assert pipe.submit_direct(0, count) == 0
        assert pipe.error() == "submit: slot 0 is in flight"
        assert pipe.wait(0, count) is not None
    finally:
        pipe.destroy()


def test_direct_submit_two_slots_ping_pong(hip):
    note("pipeline direct submit: ten ping-pong rounds")
    pipe = hip.FeaturePipeline.create(0, 128, 2)
    assert pipe is not None
    try:
        pending = None
        for r in range(10):
            slot, n = r % 2, 64 + 6 * r
            batch = synth.make_batch(n, seed=2000 + r, variant=synth.ORDINARY)
            fill(pipe, slot, batch)
            assert pipe.submit_direct(slot, n) == 1, pipe.error()
            if pending is not None:
                pslot, pn, pb = pending
                assert_feature_parity(pipe.wait(pslot, pn).copy(),
                                      oracle.features(pb.obs, pb.mission, pb.cameras),
                                      f"direct-round{r - 1}")
            pending = (slot, n, batch)
        pslot, pn, pb = pending
        assert_feature_parity(pipe.wait(pslot, pn).copy(),
                              oracle.features(pb.obs, pb.mission, pb.cameras), "direct-round9")
    finally:
        pipe.destroy()
