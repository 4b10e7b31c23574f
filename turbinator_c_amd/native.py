"""ctypes bindings of libturbinator_hip.so and libturbinator_synth.so.

The product path is the C-ABI library; this module only declares its
signatures (include/turbinator/training/cuda_features.h and hip_features.h)
so Python callers, the tests and the benchmark call exactly what a C caller
links.  Loading fails loudly when the library has not been built: there is no
fallback implementation.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_size_t, c_ubyte, c_uint64, c_void_p
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_HIP_PATH = PKG / "libturbinator_hip.so"
LIB_SYNTH_PATH = PKG / "libturbinator_synth.so"

OBS_DIM = 4148
MISSION_DIM = 10
CAMERA_BYTES = 16384
FEATURE_DIM = 142
DIAG_BYTES = 432
TACTICAL_DIM = 24
PRIOR_DIM = 15

# Every symbol include/turbinator/training/*.h declares, with its signature.
HIP_SIGNATURES = {
    "tb_cuda_extract_features_device":
        (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "tb_cuda_synchronize": (c_int, [c_void_p]),
    "tb_cuda_feature_batch_create": (c_void_p, [c_int, c_size_t]),
    "tb_cuda_feature_batch_destroy": (None, [c_void_p]),
    "tb_cuda_feature_batch_error": (c_char_p, [c_void_p]),
    "tb_cuda_extract_features_host":
        (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "tb_hip_extract_features_strided_device":
        (c_int, [c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t, c_void_p,
                 c_size_t, c_void_p]),
    "tb_hip_extract_features_indexed_device":
        (c_int, [c_void_p, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t, c_size_t, c_void_p,
                 c_void_p, c_size_t, c_void_p]),
    "tb_hip_extract_features_diagnostics_device":
        (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "tb_hip_extract_features_depth_device":
        (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "tb_hip_extract_features_host_static":
        (c_int, [c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "tb_hip_lidar_transform_device": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "tb_hip_actor_inputs_device": (c_int, [c_void_p] * 9 + [c_size_t, c_void_p]),
    "tb_hip_sac_actor_packed_bytes": (c_size_t, [c_int]),
    "tb_hip_sac_actor_pack_device": (c_int, [c_void_p] * 6 + [c_int, c_void_p, c_void_p]),
    "tb_hip_sac_actor_act_device":
        (c_int, [c_void_p, c_int] + [c_void_p] * 5 + [c_size_t, c_void_p]),
    "tb_hip_sac_read_actor": (c_size_t, [c_char_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "tb_hip_sac_normals": (None, [c_void_p, c_void_p, c_size_t]),
    "tb_hip_onboard_tactical_prior_device":
        (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "tb_hip_feature_pipeline_create": (c_void_p, [c_int, c_size_t, c_int]),
    "tb_hip_feature_pipeline_destroy": (None, [c_void_p]),
    "tb_hip_feature_pipeline_error": (c_char_p, [c_void_p]),
    "tb_hip_feature_pipeline_inputs": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
    "tb_hip_feature_pipeline_submit": (c_int, [c_void_p, c_int, c_size_t, c_int]),
    "tb_hip_feature_pipeline_submit_direct": (c_int, [c_void_p, c_int, c_size_t, c_int]),
    "tb_hip_feature_pipeline_wait": (c_void_p, [c_void_p, c_int]),
}

SYNTH_SIGNATURES = {
    "tb_synth_env": (None, [c_uint64, c_uint64, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "tb_synth_batch": (None, [c_uint64, c_int, c_size_t, c_void_p, c_size_t, c_void_p, c_size_t,
                              c_void_p, c_size_t, c_void_p, c_int]),
}

_hip = None
_synth = None


class LibraryMissing(RuntimeError):
    pass


def _load(path: Path, signatures: dict) -> ctypes.CDLL:
    if not path.exists():
        raise LibraryMissing(
            f"{path.name} is not built; run `python -m turbinator_c_amd.build` "
            "(there is no non-HIP fallback)")
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in signatures.items():
        fn = getattr(lib, name)  # AttributeError names a missing export
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


def hip_lib() -> ctypes.CDLL:
    global _hip
    if _hip is None:
        _hip = _load(LIB_HIP_PATH, HIP_SIGNATURES)
    return _hip


def synth_lib() -> ctypes.CDLL:
    global _synth
    if _synth is None:
        _synth = _load(LIB_SYNTH_PATH, SYNTH_SIGNATURES)
    return _synth
