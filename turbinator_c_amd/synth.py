"""Seeded synthetic sensor batches (numpy views over libturbinator_synth).

Variants: 0 ordinary, 1 all-LiDAR no-return, 2 constant-depth cameras,
3 tied sector minima, 4 clamp-limit values, 5 non-finite/signed-zero values,
-1 the four-quarter edge batch (variants 1..4 in order).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .native import CAMERA_BYTES, MISSION_DIM, OBS_DIM, synth_lib

DEFAULT_SEED = 42
ORDINARY, NO_RETURN, CONST_CAMERA, TIED_MINIMA, CLAMP_LIMITS, SPECIAL, EDGE_QUARTERS = \
    0, 1, 2, 3, 4, 5, -1


@dataclass
class Batch:
    obs: np.ndarray       # [B, 4148] float32
    mission: np.ndarray   # [B, 10] float32
    cameras: np.ndarray   # [B, 16384] uint8
    depth: np.ndarray | None = None  # [B, 16384] float32 metres

    @property
    def size(self) -> int:
        return self.obs.shape[0]


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


def make_batch(batch: int, seed: int = DEFAULT_SEED, variant: int = ORDINARY,
               with_depth: bool = False, threads: int = 8) -> Batch:
    obs = np.empty((batch, OBS_DIM), np.float32)
    mission = np.empty((batch, MISSION_DIM), np.float32)
    cameras = np.empty((batch, CAMERA_BYTES), np.uint8)
    depth = np.empty((batch, CAMERA_BYTES), np.float32) if with_depth else None
    synth_lib().tb_synth_batch(seed, variant, batch,
                               _ptr(obs), OBS_DIM * 4, _ptr(mission), MISSION_DIM * 4,
                               _ptr(cameras), CAMERA_BYTES, _ptr(depth), threads)
    return Batch(obs, mission, cameras, depth)


def fill_records(buf: np.ndarray, batch: int, record_bytes: int, obs_off: int,
                 mission_off: int, camera_off: int, seed: int = DEFAULT_SEED,
                 variant: int = ORDINARY, threads: int = 8) -> None:
    """Writes observations into array-of-structures records in place."""
    base = buf.ctypes.data
    if buf.nbytes < batch * record_bytes:
        raise ValueError("record buffer too small")
    synth_lib().tb_synth_batch(seed, variant, batch,
                               base + obs_off, record_bytes, base + mission_off, record_bytes,
                               base + camera_off, record_bytes, None, threads)
