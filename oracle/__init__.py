"""TEST INFRASTRUCTURE ONLY: Python handle on the CPU checker.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg;
never by turbinator_c_amd.  Wraps oracle/liboracle.so (restatement of the
reference algorithms) and, when built, oracle/_ref/libref_training.so (the
reference's own src/training/training.c).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_size_t, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# TB_ORACLE_LIB names another build of the restatement: the mutation test
# (tests/test_onboard_oracle_mutants.py) runs the pin tests against copies with
# a planted mistake.
LIB_ORACLE = Path(os.environ.get("TB_ORACLE_LIB") or HERE / "liboracle.so")
LIB_REF = HERE / "_ref" / "libref_training.so"

OBS, MISSION, CAMERA, FEATURES, DIAG_BYTES = 4148, 10, 16384, 142, 432
# min_r, argmin ray, min_dx_c, cluster_count, cluster_y_sum
ONBOARD_DIAG = 5

_orc = None
_ref = None


def lib() -> ctypes.CDLL:
    global _orc
    if _orc is None:
        if not LIB_ORACLE.exists():
            raise RuntimeError(f"{LIB_ORACLE} not built (make -C oracle)")
        l = ctypes.CDLL(str(LIB_ORACLE))
        l.orc_features_env.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p]
        l.orc_features_env.restype = None
        l.orc_features_batch.argtypes = [c_void_p, c_size_t, c_void_p, c_size_t, c_void_p,
                                         c_size_t, c_void_p, c_size_t, c_int]
        l.orc_features_batch.restype = None
        l.orc_lidar_feature.argtypes = [c_float]
        l.orc_lidar_feature.restype = c_float
        l.orc_lidar_feature_array.argtypes = [c_void_p, c_void_p, c_size_t, c_int]
        l.orc_lidar_feature_array.restype = None
        l.orc_depth_to_luma.argtypes = [c_float]
        l.orc_depth_to_luma.restype = ctypes.c_uint8
        l.orc_depth_to_luma_array.argtypes = [c_void_p, c_void_p, c_size_t]
        l.orc_depth_to_luma_array.restype = None
        l.orc_diagnostics_env.argtypes = [c_void_p, c_void_p, c_void_p]
        l.orc_diagnostics_env.restype = None
        l.orc_onboard_env.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]
        l.orc_onboard_env.restype = None
        l.orc_actor_inputs_env.argtypes = [c_void_p] * 9
        l.orc_actor_inputs_env.restype = None
        l.orc_sac_normals.argtypes = [c_void_p, c_void_p, c_size_t]
        l.orc_sac_normals.restype = None
        l.orc_sac_actor_env.argtypes = [c_void_p] * 6 + [c_int] + [c_void_p] * 5
        l.orc_sac_actor_env.restype = None
        l.orc_onboard_ray_dir.argtypes = [c_int, c_void_p]
        l.orc_onboard_ray_dir.restype = None
        _orc = l
    return _orc


def ref_lib() -> ctypes.CDLL | None:
    """The reference's own training.c, or None when it was not built."""
    global _ref
    if _ref is None and LIB_REF.exists():
        l = ctypes.CDLL(str(LIB_REF))
        l.tb_train_extract_features_cpu.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p]
        l.tb_train_extract_features_cpu.restype = None
        l.tb_train_config_default.argtypes = [c_void_p]
        l.tb_train_config_default.restype = None
        l.tb_sac_create.argtypes = [c_void_p]
        l.tb_sac_create.restype = c_void_p
        l.tb_sac_destroy.argtypes = [c_void_p]
        l.tb_sac_destroy.restype = None
        l.tb_sac_save.argtypes = [c_void_p, ctypes.c_char_p]
        l.tb_sac_save.restype = c_int
        l.tb_sac_act_features.argtypes = [c_void_p, c_void_p, c_int, c_void_p, c_void_p]
        l.tb_sac_act_features.restype = c_int
        l.ref_features_batch.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_int]
        l.ref_features_batch.restype = None
        _ref = l
    return _ref


def _p(a):
    return None if a is None else a.ctypes.data


def features(obs: np.ndarray, mission: np.ndarray, cameras: np.ndarray | None,
             threads: int = 8) -> np.ndarray:
    """[B,142] features of dense [B,4148]/[B,10]/[B,16384] host arrays."""
    obs = np.ascontiguousarray(obs, np.float32)
    mission = np.ascontiguousarray(mission, np.float32)
    if cameras is not None:
        cameras = np.ascontiguousarray(cameras, np.uint8)
    b = obs.shape[0]
    out = np.empty((b, FEATURES), np.float32)
    lib().orc_features_batch(_p(obs), OBS * 4, _p(mission), MISSION * 4, _p(cameras), CAMERA,
                             _p(out), b, threads)
    return out


def features_strided(buf: np.ndarray, batch: int, record: int, obs_off: int, mission_off: int,
                     camera_off: int | None, threads: int = 8) -> np.ndarray:
    out = np.empty((batch, FEATURES), np.float32)
    base = buf.ctypes.data
    lib().orc_features_batch(base + obs_off, record, base + mission_off, record,
                             None if camera_off is None else base + camera_off, record,
                             _p(out), batch, threads)
    return out


def reference_features(obs: np.ndarray, mission: np.ndarray,
                       cameras: np.ndarray | None) -> np.ndarray:
    """[B,142] from the reference's compiled tb_train_extract_features_cpu."""
    r = ref_lib()
    if r is None:
        raise RuntimeError("oracle/_ref not built")
    obs = np.ascontiguousarray(obs, np.float32)
    mission = np.ascontiguousarray(mission, np.float32)
    out = np.empty((obs.shape[0], FEATURES), np.float32)
    for e in range(obs.shape[0]):
        cam = None if cameras is None else cameras[e].ctypes.data
        r.tb_train_extract_features_cpu(obs[e].ctypes.data, mission[e].ctypes.data, cam,
                                        out[e].ctypes.data)
    return out


def lidar_feature(values: np.ndarray, threads: int = 8) -> np.ndarray:
    v = np.ascontiguousarray(values, np.float32)
    out = np.empty_like(v)
    lib().orc_lidar_feature_array(_p(v), _p(out), v.size, threads)
    return out


def onboard(obs: np.ndarray, mission: np.ndarray):
    """(tactical [B,24], prior [B,15], diag [B,ONBOARD_DIAG]) per environment."""
    b = obs.shape[0]
    tac = np.empty((b, 24), np.float32)
    pri = np.empty((b, 15), np.float32)
    diag = np.empty((b, ONBOARD_DIAG), np.float32)
    for e in range(b):
        lib().orc_onboard_env(np.ascontiguousarray(obs[e], np.float32).ctypes.data,
                              np.ascontiguousarray(mission[e], np.float32).ctypes.data,
                              tac[e].ctypes.data, pri[e].ctypes.data, diag[e].ctypes.data)
    return tac, pri, diag


def actor_inputs(obs: np.ndarray, mission: np.ndarray, cameras: np.ndarray | None) -> dict:
    """The 618M actor's prepared inputs per environment (dict of arrays)."""
    b = obs.shape[0]
    out = {"proprio": np.empty((b, 91), np.float32), "mission": np.empty((b, 49), np.float32),
           "tactical": np.empty((b, 24), np.float32), "prior": np.empty((b, 15), np.float32),
           "lidar": np.empty((b, 6, 16, 128), np.float32),
           "luma": None if cameras is None else np.empty((b, 4, 64, 64), np.float32)}
    for e in range(b):
        cam = None if cameras is None else np.ascontiguousarray(cameras[e]).ctypes.data
        lib().orc_actor_inputs_env(
            np.ascontiguousarray(obs[e], np.float32).ctypes.data,
            np.ascontiguousarray(mission[e], np.float32).ctypes.data, cam,
            out["proprio"][e].ctypes.data, out["mission"][e].ctypes.data,
            out["tactical"][e].ctypes.data, out["prior"][e].ctypes.data,
            out["lidar"][e].ctypes.data,
            None if out["luma"] is None else out["luma"][e].ctypes.data)
    return out


def onboard_ray_table() -> np.ndarray:
    out = np.empty((1536, 3), np.float32)
    for ray in range(1536):
        lib().orc_onboard_ray_dir(ray, out[ray].ctypes.data)
    return out


def depth_to_luma(depth: np.ndarray) -> np.ndarray:
    d = np.ascontiguousarray(depth, np.float32)
    out = np.empty(d.shape, np.uint8)
    lib().orc_depth_to_luma_array(_p(d), _p(out), d.size)
    return out


def diagnostics(obs: np.ndarray, cameras: np.ndarray | None) -> np.ndarray:
    b = obs.shape[0]
    out = np.empty((b, DIAG_BYTES), np.uint8)
    for e in range(b):
        cam = None if cameras is None else np.ascontiguousarray(cameras[e]).ctypes.data
        lib().orc_diagnostics_env(np.ascontiguousarray(obs[e], np.float32).ctypes.data, cam,
                                  out[e].ctypes.data)
    return out


class SacActorWeights:
    """Actor weights in the reference's tb_dense layout (training.c:13-16)."""

    def __init__(self, w0, b0, w1, b1, w2, b2):
        self.w0, self.b0, self.w1, self.b1, self.w2, self.b2 = (
            np.ascontiguousarray(a, np.float32) for a in (w0, b0, w1, b1, w2, b2))
        self.hidden = self.b0.shape[0]

    def arrays(self):
        return self.w0, self.b0, self.w1, self.b1, self.w2, self.b2


def sac_normals(state: int, count: int) -> tuple[np.ndarray, int]:
    """`count` draws of the agent's tb_normal stream from rng state `state`;
    returns (draws, state afterwards)."""
    st = np.array([state], np.uint64)
    out = np.empty(count, np.float32)
    lib().orc_sac_normals(st.ctypes.data, _p(out), count)
    return out, int(st[0])


def sac_actor(weights: SacActorWeights, features: np.ndarray, normals: np.ndarray | None):
    """(action [B,15], log_prob [B], raw [B,30]) of the compact actor per row."""
    f = np.ascontiguousarray(features, np.float32)
    b = f.shape[0]
    act = np.empty((b, 15), np.float32)
    lp = np.empty(b, np.float32)
    raw = np.empty((b, 30), np.float32)
    nrm = None if normals is None else np.ascontiguousarray(normals, np.float32).reshape(b, 15)
    w = weights.arrays()
    for e in range(b):
        lib().orc_sac_actor_env(*(a.ctypes.data for a in w), weights.hidden, f[e].ctypes.data,
                                None if nrm is None else nrm[e].ctypes.data,
                                act[e].ctypes.data, lp[e:].ctypes.data, raw[e].ctypes.data)
    return act, lp, raw
