"""Python mirror of the batched compact SAC actor entries (hip_features.h).

The reference acts one environment per call, tb_sac_act_features
(src/training/training.c:382-392).  Here a whole batch of device-resident
feature rows is acted on at once: pack the actor's weights after each update,
then call act_device per batch.  Every function goes through the C ABI of
libturbinator_hip.so; there is no host fallback.
"""
from __future__ import annotations

import ctypes

import numpy as np

from .features import _dev, _stream
from .native import hip_lib

FEATURES, RAW, ACTIONS = 142, 30, 15


def layer_shapes(hidden: int) -> list[tuple[tuple[int, int], int]]:
    """((outputs, inputs), bias) per layer, the reference's tb_net_init order."""
    return [((hidden, FEATURES), hidden), ((hidden, hidden), hidden), ((RAW, hidden), RAW)]


def split_actor(flat: np.ndarray, hidden: int) -> list[np.ndarray]:
    """[w0, b0, w1, b1, w2, b2] views of the concatenated actor weights."""
    out, pos = [], 0
    for (o, i), b in layer_shapes(hidden):
        out.append(flat[pos:pos + o * i].reshape(o, i))
        pos += o * i
        out.append(flat[pos:pos + b])
        pos += b
    if pos != flat.size:
        raise ValueError(f"expected {pos} floats for hidden {hidden}, got {flat.size}")
    return out


def read_checkpoint_actor(path: str) -> tuple[list[np.ndarray], int, int]:
    """Actor weights of a tb_sac_save checkpoint, its hidden width and the
    agent's rng state (tb_hip_sac_read_actor)."""
    lib = hip_lib()
    hidden = ctypes.c_int(0)
    rng = ctypes.c_uint64(0)
    need = lib.tb_hip_sac_read_actor(path.encode(), None, 0, ctypes.byref(hidden),
                                     ctypes.byref(rng))
    if need == 0:
        raise ValueError(f"{path}: not a readable TBSAC01 checkpoint")
    flat = np.empty(need, np.float32)
    got = lib.tb_hip_sac_read_actor(path.encode(), flat.ctypes.data, need, None, None)
    if got != need:
        raise ValueError(f"{path}: short read")
    return split_actor(flat, hidden.value), hidden.value, rng.value


def normals(state: int, count: int) -> tuple[np.ndarray, int]:
    """`count` draws of the agent's normal stream; returns (draws, new state)."""
    st = ctypes.c_uint64(state)
    out = np.empty(count, np.float32)
    hip_lib().tb_hip_sac_normals(ctypes.byref(st), out.ctypes.data, count)
    return out, st.value


def packed_bytes(hidden: int) -> int:
    return hip_lib().tb_hip_sac_actor_packed_bytes(hidden)


def pack_device(w0, b0, w1, b1, w2, b2, hidden: int, packed, stream=None) -> int:
    return hip_lib().tb_hip_sac_actor_pack_device(
        _dev(w0), _dev(b0), _dev(w1), _dev(b1), _dev(w2), _dev(b2), hidden, _dev(packed),
        _stream(stream))


def act_device(packed, hidden: int, features, normals_dev, actions, log_prob, raw,
               batch_size: int, stream=None) -> int:
    return hip_lib().tb_hip_sac_actor_act_device(
        _dev(packed), hidden, _dev(features), _dev(normals_dev), _dev(actions),
        _dev(log_prob), _dev(raw), batch_size, _stream(stream))


__all__ = ["layer_shapes", "split_actor", "read_checkpoint_actor", "normals", "packed_bytes",
           "pack_device", "act_device"]
