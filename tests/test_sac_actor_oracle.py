"""Pins the CPU oracle of the compact SAC actor (oracle/sac_actor_oracle.c)
and the host helpers of the batched actor (checkpoint reader, normal stream).

Where the reference was compiled (oracle/_ref), an agent is created with
tb_sac_create, written with tb_sac_save, and read back through
tb_hip_sac_read_actor.  The oracle, given those weights and the normals that
tb_hip_sac_normals draws from the checkpoint's rng state, must reproduce
consecutive tb_sac_act_features calls bit for bit, deterministic and
stochastic.  That one check pins the weight layout (a transposed layer
fails), the sampling formulas and the random stream together.

Without the compiled reference, a float64 numpy forward pass checks the
network orientation and the sampling on random weights.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest

import oracle
from turbinator_c_amd import actor


class TrainConfig(ctypes.Structure):
    """training.h:23-37."""
    _fields_ = [("seed", ctypes.c_uint64), ("replay_capacity", ctypes.c_size_t),
                ("hidden_dim", ctypes.c_int)] + [
        (n, ctypes.c_float) for n in ("gamma", "tau", "actor_lr", "critic_lr", "alpha_lr",
                                      "initial_alpha", "target_entropy", "reference_weight",
                                      "max_grad_norm", "reward_scale")]


def reference_agent(tmp_path: Path, hidden: int, seed: int):
    ref = oracle.ref_lib()
    cfg = TrainConfig()
    ref.tb_train_config_default(ctypes.byref(cfg))
    cfg.hidden_dim, cfg.seed, cfg.replay_capacity = hidden, seed, 16
    agent = ref.tb_sac_create(ctypes.byref(cfg))
    assert agent
    path = tmp_path / f"agent_{hidden}.bin"
    assert ref.tb_sac_save(agent, str(path).encode()) == 1
    return ref, agent, path


def random_features(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    f = rng.uniform(-1, 1, (n, 142)).astype(np.float32)
    f[0] = 0.0
    f[1] = 1.0
    f[2] = -1.0
    return f


@pytest.mark.parametrize("hidden", [16, 37, 128, 256])
def test_oracle_matches_reference_agent(tmp_path, hidden):
    if oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    ref, agent, path = reference_agent(tmp_path, hidden, seed=1000 + hidden)
    try:
        weights, h, rng = actor.read_checkpoint_actor(str(path))
        assert h == hidden
        w = oracle.SacActorWeights(*weights)
        feats = random_features(24, hidden)
        # deterministic: no draws
        want_a = np.empty((24, 15), np.float32)
        want_lp = np.empty(24, np.float32)
        for e in range(24):
            assert ref.tb_sac_act_features(agent, feats[e].ctypes.data, 1,
                                           want_a[e].ctypes.data, want_lp[e:].ctypes.data) == 1
        got_a, got_lp, _ = oracle.sac_actor(w, feats, None)
        assert np.array_equal(got_a.view(np.uint32), want_a.view(np.uint32))
        assert np.all(got_lp == 0) and np.all(want_lp == 0)
        # stochastic: 15 draws per call from the agent's stream
        for e in range(24):
            assert ref.tb_sac_act_features(agent, feats[e].ctypes.data, 0,
                                           want_a[e].ctypes.data, want_lp[e:].ctypes.data) == 1
        draws, _ = actor.normals(rng, 24 * 15)
        got_a, got_lp, _ = oracle.sac_actor(w, feats, draws.reshape(24, 15))
        assert np.array_equal(got_a.view(np.uint32), want_a.view(np.uint32))
        assert np.array_equal(got_lp.view(np.uint32), want_lp.view(np.uint32))
    finally:
        ref.tb_sac_destroy(agent)


def test_product_normals_match_oracle_stream():
    got, s1 = actor.normals(0x9E3779B97F4A7C15, 1000)
    want, s2 = oracle.sac_normals(0x9E3779B97F4A7C15, 1000)
    assert s1 == s2 and np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # A standard normal sample: mean ~0, variance ~1 (n = 1000: 5 sigma bounds).
    assert abs(float(got.mean())) < 0.16 and abs(float(got.var()) - 1) < 0.25


def numpy_actor(w, feats, draws):
    w0, b0, w1, b1, w2, b2 = (a.astype(np.float64) for a in w)
    h0 = np.tanh(feats @ w0.T + b0)
    h1 = np.tanh(h0 @ w1.T + b1)
    raw = h1 @ w2.T + b2
    log_std = np.clip(raw[:, 15:], -3.5, -1.6)
    scale = np.ones(15)
    scale[14] = 0.15
    eps = np.zeros((feats.shape[0], 15)) if draws is None else draws * scale
    z = np.clip(raw[:, :15] + np.exp(log_std) * eps, -8, 8)
    a = np.tanh(z)
    lp = (-0.5 * eps * eps - log_std - 0.5 * np.log(2 * np.pi) - np.log(1 - a * a + 1e-6)).sum(1)
    return a, (lp if draws is not None else np.zeros(feats.shape[0])), raw


@pytest.mark.parametrize("hidden", [16, 100])
def test_oracle_against_float64_numpy(hidden):
    rng = np.random.default_rng(hidden)
    w = []
    for (o, i), b in actor.layer_shapes(hidden):
        w.append((rng.standard_normal((o, i)) * np.sqrt(2.0 / (o + i))).astype(np.float32))
        w.append((rng.standard_normal(b) * 0.1).astype(np.float32))
    feats = random_features(16, hidden + 1)
    draws = rng.standard_normal((16, 15)).astype(np.float32)
    for d in (None, draws):
        a, lp, raw = oracle.sac_actor(oracle.SacActorWeights(*w), feats, d)
        wa, wlp, wraw = numpy_actor(w, feats.astype(np.float64), d)
        assert np.abs(raw - wraw).max() < 1e-5
        assert np.abs(a - wa).max() < 1e-5
        assert np.abs(lp - wlp).max() < 1e-3 * (1 + np.abs(wlp).max())


def test_checkpoint_reader_rejects_bad_files(tmp_path):
    lib = actor.hip_lib()
    assert lib.tb_hip_sac_read_actor(str(tmp_path / "missing.bin").encode(), None, 0, None,
                                     None) == 0
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"TBSAC02\0" + bytes(200))
    assert lib.tb_hip_sac_read_actor(str(bad).encode(), None, 0, None, None) == 0
    short = tmp_path / "short.bin"
    cfg = TrainConfig()
    cfg.hidden_dim = 128
    short.write_bytes(b"TBSAC01\0" + bytes(cfg) + bytes(64))
    assert lib.tb_hip_sac_read_actor(str(short).encode(), None, 0, None, None) == 0
    assert lib.tb_hip_sac_read_actor(None, None, 0, None, None) == 0


def test_packed_sizes():
    assert actor.packed_bytes(15) == 0 and actor.packed_bytes(257) == 0
    # hidden 128: 8 tiles of 16 outputs, 4 chunks of 32 inputs (5 for the 142
    # features).  Per layer, 2 KiB of fp16 weight pieces per (tile, chunk) and
    # 128 bytes of fp32 biases and int exponents per tile; then the fp32
    # first-layer weights; every section rounded up to 256 bytes.
    def up(x):
        return (x + 255) // 256 * 256

    def layout(ht, hc, hidden):
        return [ht * 5 * 2048, ht * 128, ht * hc * 2048, ht * 128, 2 * hc * 2048, 2 * 128,
                hidden * 142 * 4]
    assert actor.packed_bytes(128) == sum(up(x) for x in layout(8, 4, 128)) == 238848
    assert actor.packed_bytes(37) == sum(up(x) for x in layout(3, 2, 37))
    assert actor.packed_bytes(256) == sum(up(x) for x in layout(16, 8, 256))
