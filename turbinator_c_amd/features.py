"""Python mirror of the sensor-feature boundary (include/turbinator/training/).

Names, argument meaning and return codes follow the reference C interface
include/turbinator/training/cuda_features.h:14-34 (src/cuda/features.cu):
functions return 1 on success and 0 on failure, exactly like the C entry
points they call.  Device arguments accept torch tensors on the GPU or raw
integer device addresses; `stream` accepts a torch.cuda.Stream, a raw
hipStream_t integer or None (null stream).
"""
from __future__ import annotations

import ctypes

import numpy as np

from .native import CAMERA_BYTES, FEATURE_DIM, MISSION_DIM, OBS_DIM, hip_lib  # noqa: F401


def _dev(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream(s) -> int | None:
    if s is None:
        return None
    if isinstance(s, int):
        return s
    return s.cuda_stream


def extract_features_device(obs, mission, cameras, features, batch_size: int,
                            stream=None) -> int:
    """tb_cuda_extract_features_device (cuda_features.h:14-19)."""
    return hip_lib().tb_cuda_extract_features_device(
        _dev(obs), _dev(mission), _dev(cameras), _dev(features), batch_size, _stream(stream))


def extract_features_strided_device(obs, obs_stride: int, mission, mission_stride: int,
                                    cameras, camera_stride: int, features, batch_size: int,
                                    stream=None) -> int:
    """tb_hip_extract_features_strided_device (hip_features.h)."""
    return hip_lib().tb_hip_extract_features_strided_device(
        _dev(obs), obs_stride, _dev(mission), mission_stride, _dev(cameras), camera_stride,
        _dev(features), batch_size, _stream(stream))


def extract_features_indexed_device(obs, obs_stride: int, mission, mission_stride: int,
                                    cameras, camera_stride: int, capacity: int, indices,
                                    features, batch_size: int, stream=None) -> int:
    """tb_hip_extract_features_indexed_device (hip_features.h)."""
    return hip_lib().tb_hip_extract_features_indexed_device(
        _dev(obs), obs_stride, _dev(mission), mission_stride, _dev(cameras), camera_stride,
        capacity, _dev(indices), _dev(features), batch_size, _stream(stream))


def extract_features_diagnostics_device(obs, mission, cameras, features, diagnostics,
                                        batch_size: int, stream=None) -> int:
    """tb_hip_extract_features_diagnostics_device (hip_features.h)."""
    return hip_lib().tb_hip_extract_features_diagnostics_device(
        _dev(obs), _dev(mission), _dev(cameras), _dev(features), _dev(diagnostics), batch_size,
        _stream(stream))


def extract_features_depth_device(obs, mission, depth, features, batch_size: int,
                                  stream=None) -> int:
    """tb_hip_extract_features_depth_device (hip_features.h)."""
    return hip_lib().tb_hip_extract_features_depth_device(
        _dev(obs), _dev(mission), _dev(depth), _dev(features), batch_size, _stream(stream))


def lidar_transform_device(ranges, out, count: int, stream=None) -> int:
    """tb_hip_lidar_transform_device (hip_features.h)."""
    return hip_lib().tb_hip_lidar_transform_device(_dev(ranges), _dev(out), count,
                                                   _stream(stream))


def onboard_tactical_prior_device(obs, mission, tactical, prior, diag, batch_size: int,
                                  stream=None) -> int:
    """tb_hip_onboard_tactical_prior_device (hip_features.h)."""
    return hip_lib().tb_hip_onboard_tactical_prior_device(
        _dev(obs), _dev(mission), _dev(tactical), _dev(prior), _dev(diag), batch_size,
        _stream(stream))


def actor_inputs_device(obs, mission, cameras, proprio, mission_vec, tactical, prior,
                        lidar_channels, camera_luma, batch_size: int, stream=None) -> int:
    """tb_hip_actor_inputs_device (hip_features.h)."""
    return hip_lib().tb_hip_actor_inputs_device(
        _dev(obs), _dev(mission), _dev(cameras), _dev(proprio), _dev(mission_vec),
        _dev(tactical), _dev(prior), _dev(lidar_channels), _dev(camera_luma), batch_size,
        _stream(stream))


def synchronize(stream=None) -> int:
    """tb_cuda_synchronize (cuda_features.h:20)."""
    return hip_lib().tb_cuda_synchronize(_stream(stream))


class FeatureBatch:
    """tb_cuda_feature_batch handle (cuda_features.h:22-34)."""

    def __init__(self, handle: int):
        self._handle = handle

    @classmethod
    def create(cls, device_id: int, max_batch: int) -> "FeatureBatch | None":
        h = hip_lib().tb_cuda_feature_batch_create(device_id, max_batch)
        return cls(h) if h else None

    @property
    def handle(self) -> int | None:
        return self._handle

    def error(self) -> str:
        return hip_lib().tb_cuda_feature_batch_error(self._handle).decode()

    def extract_host(self, obs: np.ndarray, mission: np.ndarray, cameras: np.ndarray,
                     count: int, out: np.ndarray) -> int:
        for a, dt, width in ((obs, np.float32, OBS_DIM), (mission, np.float32, MISSION_DIM),
                             (cameras, np.uint8, CAMERA_BYTES), (out, np.float32, FEATURE_DIM)):
            if a.dtype != dt or not a.flags.c_contiguous or a.size < count * width:
                raise ValueError("host arrays must be C-contiguous with count rows of the "
                                 "reference layout")
        return hip_lib().tb_cuda_extract_features_host(
            self._handle, obs.ctypes.data, mission.ctypes.data, cameras.ctypes.data, count,
            out.ctypes.data)

    def destroy(self) -> None:
        if self._handle:
            hip_lib().tb_cuda_feature_batch_destroy(self._handle)
            self._handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()


STATIC_MAX_BATCH = 256  # TB_HIP_STATIC_MAX_BATCH in hip_features.h


def extract_features_host_static(obs: np.ndarray, mission: np.ndarray, cameras: np.ndarray,
                                 count: int, out: np.ndarray, stream=None) -> int:
    """tb_hip_extract_features_host_static: the host entry without a handle,
    staged in the library's static device array (count <= STATIC_MAX_BATCH)."""
    for a, dt, width in ((obs, np.float32, OBS_DIM), (mission, np.float32, MISSION_DIM),
                         (cameras, np.uint8, CAMERA_BYTES), (out, np.float32, FEATURE_DIM)):
        if a.dtype != dt or not a.flags.c_contiguous or a.size < count * width:
            raise ValueError("host arrays must be C-contiguous with count rows of the "
                             "reference layout")
    return hip_lib().tb_hip_extract_features_host_static(
        obs.ctypes.data, mission.ctypes.data, cameras.ctypes.data, count, out.ctypes.data,
        _stream(stream))


def feature_batch_error(handle) -> str:
    """tb_cuda_feature_batch_error for a raw handle (None -> NULL)."""
    return hip_lib().tb_cuda_feature_batch_error(handle).decode()


class FeaturePipeline:
    """tb_hip_feature_pipeline handle (hip_features.h): pinned staging slots
    the producer writes in place, asynchronous submit, blocking wait."""

    def __init__(self, handle: int, max_batch: int, slots: int):
        self._handle = handle
        self.max_batch = max_batch
        self.slots = slots

    @classmethod
    def create(cls, device_id: int, max_batch: int, slots: int = 2) -> "FeaturePipeline | None":
        h = hip_lib().tb_hip_feature_pipeline_create(device_id, max_batch, slots)
        return cls(h, max_batch, slots) if h else None

    @property
    def handle(self) -> int | None:
        return self._handle

    def error(self) -> str:
        return hip_lib().tb_hip_feature_pipeline_error(self._handle).decode()

    def inputs(self, slot: int):
        """(obs, mission, cameras) numpy views of the slot's pinned arrays."""
        o, m, c = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        if hip_lib().tb_hip_feature_pipeline_inputs(self._handle, slot, ctypes.byref(o),
                                                    ctypes.byref(m), ctypes.byref(c)) != 1:
            raise ValueError(f"slot {slot} out of range")
        n = self.max_batch

        def view(addr, ctype, shape):
            return np.ctypeslib.as_array(ctypes.cast(addr, ctypes.POINTER(ctype)), shape=shape)

        return (view(o.value, ctypes.c_float, (n, OBS_DIM)),
                view(m.value, ctypes.c_float, (n, MISSION_DIM)),
                view(c.value, ctypes.c_ubyte, (n, CAMERA_BYTES)))

    def submit(self, slot: int, count: int, with_cameras: bool = True) -> int:
        return hip_lib().tb_hip_feature_pipeline_submit(self._handle, slot, count,
                                                        1 if with_cameras else 0)

    def submit_direct(self, slot: int, count: int, with_cameras: bool = True) -> int:
        """Extraction on the pinned slot itself (no copy-engine transfers)."""
        return hip_lib().tb_hip_feature_pipeline_submit_direct(self._handle, slot, count,
                                                               1 if with_cameras else 0)

    def wait(self, slot: int, count: int) -> np.ndarray | None:
        """The slot's [count,142] pinned feature rows (a view), or None."""
        addr = hip_lib().tb_hip_feature_pipeline_wait(self._handle, slot)
        if not addr:
            return None
        return np.ctypeslib.as_array(ctypes.cast(addr, ctypes.POINTER(ctypes.c_float)),
                                     shape=(count, FEATURE_DIM))

    def destroy(self) -> None:
        if self._handle:
            hip_lib().tb_hip_feature_pipeline_destroy(self._handle)
            self._handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()


__all__ = ["extract_features_device", "extract_features_strided_device",
           "extract_features_diagnostics_device", "extract_features_indexed_device",
           "extract_features_depth_device", "lidar_transform_device",
           "onboard_tactical_prior_device", "actor_inputs_device", "synchronize", "FeatureBatch",
           "feature_batch_error", "FeaturePipeline", "extract_features_host_static",
           "STATIC_MAX_BATCH"]
