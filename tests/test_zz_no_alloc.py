"""The allocation-free host entry (tb_hip_extract_features_host_static) against
the host object's tb_cuda_extract_features_host, through the C-ABI: bit-equal
features on two calls in a row, the second with a smaller batch, so that the
second call also shows that rows the first left in the static staging are not
read."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from turbinator_c_amd import synth

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def test_static_host_entry_matches_the_host_object(hip):
    batch = hip.FeatureBatch.create(0, hip.STATIC_MAX_BATCH)
    assert batch is not None
    try:
        for count, seed in ((hip.STATIC_MAX_BATCH, 71), (37, 72)):
            note(f"static host entry, {count} environments")
            b = synth.make_batch(count, seed=seed, variant=synth.SPECIAL if seed == 72 else
                                 synth.ORDINARY, threads=8)
            want = np.full((count, 142), np.nan, np.float32)
            got = np.full((count, 142), np.nan, np.float32)
            assert batch.extract_host(b.obs, b.mission, b.cameras, count, want) == 1, \
                batch.error()
            assert hip.extract_features_host_static(b.obs, b.mission, b.cameras, count, got) == 1
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
                f"{count}: {np.argwhere(got.view(np.uint32) != want.view(np.uint32))[:3]}"
    finally:
        batch.destroy()


def test_static_host_entry_rejects_more_than_its_staging(hip):
    count = hip.STATIC_MAX_BATCH + 1
    b = synth.make_batch(count, seed=73, threads=8)
    out = np.full((count, 142), np.nan, np.float32)
    assert hip.extract_features_host_static(b.obs, b.mission, b.cameras, count, out) == 0
    assert np.isnan(out).all()
