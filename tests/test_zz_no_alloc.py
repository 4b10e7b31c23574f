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


def test_static_host_entry_refuses_a_capturing_stream(torch_cuda, hip):
    """The entry is synchronous and copies pageable memory, which a stream
    under graph capture cannot take: it returns 0 with nothing enqueued, the
    capture ends normally and its graph replays, and afterwards the same
    stream serves the entry again."""
    import oracle
    from tests.conftest import assert_feature_parity

    torch = torch_cuda
    count = 8
    note("static host entry on a capturing stream")
    b = synth.make_batch(count, seed=74)
    out = np.full((count, 142), np.nan, np.float32)
    side = torch.cuda.Stream()
    probe = torch.zeros(64, device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        rc = hip.extract_features_host_static(b.obs, b.mission, b.cameras, count, out,
                                              torch.cuda.current_stream())
        probe.add_(1.0)
    assert rc == 0
    assert np.isnan(out).all()
    graph.replay()
    torch.cuda.synchronize()
    assert float(probe[0]) == 1.0
    assert hip.extract_features_host_static(b.obs, b.mission, b.cameras, count, out, side) == 1
    assert_feature_parity(out, oracle.features(b.obs, b.mission, b.cameras), "after capture")
