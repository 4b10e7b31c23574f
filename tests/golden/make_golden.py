"""Writes the 142-feature golden fixtures from the reference's own CPU twin.

Run in the build container (it needs oracle/_ref/libref_training.so, built by
`make -C oracle ref` from /root/reference/src/training/training.c):

    python tests/golden/make_golden.py

Fixtures (tests/golden/features_golden.npz + .json):
  ref3     the reference test's closed-form 3-env inputs
           (tests/test_cuda_features.c:17-25 of the reference)
  c1       configuration 1: 8 seeded ordinary envs (seed 42)
  c4       configuration 4: 4 envs from each quarter of the 4,096-env edge
           batch (envs 0-3, 1024-1027, 2048-2051, 3072-3075)
  special  8 envs of non-finite / signed-zero inputs (variant 5)
Inputs are not stored: the seeded generator recreates them and the JSON
holds their SHA-256 so a generator change is detected.  Outputs are stored
bit-for-bit as produced by the reference's tb_train_extract_features_cpu.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import platform
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from turbinator_c_amd import synth  # noqa: E402
from turbinator_c_amd.native import synth_lib  # noqa: E402

OUT_NPZ = Path(__file__).with_name("features_golden.npz")
OUT_JSON = Path(__file__).with_name("features_golden.json")

C4_ENVS = [0, 1, 2, 3, 1024, 1025, 1026, 1027, 2048, 2049, 2050, 2051, 3072, 3073, 3074, 3075]
C4_BATCH = 4096


def ref3_inputs():
    """The reference's tests/test_cuda_features.c:17-25 closed forms."""
    count = 3
    obs = np.zeros((count, 4148), np.float32)
    mission = np.zeros((count, 10), np.float32)
    cameras = np.zeros((count, 16384), np.uint8)
    for b in range(count):
        for i in range(4148):
            if 48 <= i < 4144:
                obs[b, i] = np.float32(0.5) + np.float32((i + 17 * b) % 119)
            else:
                obs[b, i] = np.float32((i * 11 + b * 7) % 81 - 40) * np.float32(0.125)
        for i in range(10):
            mission[b, i] = np.float32(i - 5 + b) * np.float32(0.2)
        i = np.arange(16384)
        cameras[b] = ((i * 13 + b * 29) & 255).astype(np.uint8)
    return obs, mission, cameras


def envs_inputs(seed: int, envs: list[int], variants: list[int]):
    n = len(envs)
    obs = np.empty((n, 4148), np.float32)
    mission = np.empty((n, 10), np.float32)
    cameras = np.empty((n, 16384), np.uint8)
    lib = synth_lib()
    for k, (e, v) in enumerate(zip(envs, variants)):
        lib.tb_synth_env(seed, e, v, obs[k].ctypes.data, mission[k].ctypes.data,
                         cameras[k].ctypes.data, None)
    return obs, mission, cameras


def c4_variant(env: int) -> int:
    return 1 + env * 4 // C4_BATCH


def fixture_sets():
    c1 = synth.make_batch(8, seed=42, variant=synth.ORDINARY)
    yield "ref3", ref3_inputs(), {"source": "reference tests/test_cuda_features.c:17-25"}
    yield "c1", (c1.obs, c1.mission, c1.cameras), {"seed": 42, "variant": 0, "envs": "0-7"}
    yield "c4", envs_inputs(42, C4_ENVS, [c4_variant(e) for e in C4_ENVS]), \
        {"seed": 42, "variant": "quarters of 4096", "envs": C4_ENVS}
    yield "special", envs_inputs(7, list(range(8)), [synth.SPECIAL] * 8), \
        {"seed": 7, "variant": 5, "envs": "0-7"}


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main() -> None:
    if oracle.ref_lib() is None:
        raise SystemExit("oracle/_ref/libref_training.so missing: run make -C oracle ref")
    arrays, meta = {}, {"generator": "turbinator_c_amd/csrc/synth.c",
                        "reference": "src/training/training.c tb_train_extract_features_cpu",
                        "libc": " ".join(platform.libc_ver()), "sets": {}}
    for name, (obs, mission, cameras), info in fixture_sets():
        out = oracle.reference_features(obs, mission, cameras)
        arrays[name] = out
        info = dict(info, inputs_sha256=digest(obs, mission, cameras), count=int(obs.shape[0]))
        meta["sets"][name] = info
    np.savez(OUT_NPZ, **arrays)
    OUT_JSON.write_text(json.dumps(meta, indent=1) + "\n")
    print("wrote", OUT_NPZ, OUT_JSON)


if __name__ == "__main__":
    main()
