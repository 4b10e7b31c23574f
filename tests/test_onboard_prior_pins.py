"""Pins of the onboard tactical / prior oracle (oracle/onboard_oracle.c) on
the mission modes and outputs the reference's four fixture rows do not reach.

The reference restated is tb_onboard_prior (src/network/onboard_features.cuh:
88-513); its own test holds 40 goldens on four rows (hover, slalom, BWB
cruise, BWB arena; tests/test_onboard_features.cu:19-39,55-73).  The checks
below are closed forms the control law takes at chosen states, and
invariants of the law, picked so that a plausible restatement mistake (a
swapped constant, a wrong sign, a transposed arm, a branch taken on the
wrong condition) fails at least one of them:

* Level flight (identity attitude, equal spools, gimbals at zero): yaw, tilt
  and tilt error vanish and the mixer (:312-393) reduces to `level_mixer`
  below, a few lines per arm.  Each mission mode then only changes the
  commanded accelerations and a handful of limits, and every test states
  those in closed form for one regime: hover / climb / descent caps, the
  horizontal gains and force cap, yaw and roll damping, the mass model, the
  landing law (:254-283) in each of its vertical regimes (mid, touch, align,
  transit, with their clamps), its horizontal caps, land-idle (:375,386),
  heavy and light cargo, turbine-out, lateral, inversion-mission limits,
  arena stand-off target, yaw and cannon (:158-183,341-348,407-431),
  slalom without and with obstacles (lane choice and speed limits,
  :235-252), and the dodge vector (:208-212).
* Inversion recovery (:394-405) at 150 degree roll / pitch: the arm-moment
  sign rule, its 12 N m threshold with the 52 x rate term, the outer
  gimbal law, zero inner gimbals and the cannon flag.
* BWB modes (:432-503) at level cruise: throttle pairs u_coll +- diff_u,
  the pitch / yaw gimbal laws, endurance speed, climb, slow-flight pitch cap,
  turn saturation and the BWB cannon solution.
* Mirror symmetry: reflecting the world in the x-z plane maps the state
  (py, vy, qx, qz, wx, wz, outer gimbals, the y goal offset, arms 1 <-> 3)
  and must map the multicopter outputs (throttles and inner gimbals swap
  arms 1 and 3, outer gimbals also change sign) and the BWB outputs
  (throttle pairs swap, yaw gimbal and arena cannon azimuth change sign),
  on random states of every non-arena mode.  Any sign slip in a y term of
  the law breaks it.
* Tactical features (:25-86): all 24 against a second formulation with
  rotation matrices (heading and body frames as matrix products) on random
  attitudes, arms, goals and cannon states.

tests/test_onboard_oracle_mutants.py plants single mistakes in copies of the
oracle (swapped or altered constants, flipped signs, transposed rows or arms,
moved thresholds) and requires this file or the reference goldens to fail
for every one that an input can reach.

Expected values are evaluated in float64 from the float32 inputs; the oracle
runs in float32, so the comparisons carry a 2e-5 bar (the kernel's own bar
against the oracle is 5e-5).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle

MAX_INST = 294.2 * 0.85           # max_installed, :91
MIN_T = MAX_INST * 0.08           # min_thrust, :93
G = 9.80665
PI = float(np.float32(math.pi))
TOL = 2e-5
BASE = 43.0                       # mass without fuel, ammo, payload; 40 in arena (:135)


def clamp(x, lo, hi):
    return min(hi, max(lo, x))


def thrust(s):
    return MAX_INST * (0.08 + 0.92 * s)


def az_actual(s, mass):
    """(total_fz * ct - weight) / mass at level attitude: every arm lifts."""
    return (4.0 * thrust(s) - mass * G) / mass


def run_prior(obs, mission):
    _, pri, _ = oracle.onboard(obs[None].astype(np.float32), mission[None].astype(np.float32))
    return pri[0].astype(np.float64)


def level_obs(s, px=0.0, py=0.0, pz=8.0, vx=0.0, vy=0.0, vz=0.0, ox=0.0, oy=0.0, oz=0.0,
              fuel=0.0, ammo=0.0, payload=0.0, lidar=()):
    """obs[4148] at identity attitude, spools s, gimbals at zero, no LiDAR
    return except the (ray, range) pairs given (ray = head*768+el*128+azi)."""
    o = np.zeros(4148, np.float32)
    o[0:6] = (px, py, pz, vx, vy, vz)
    o[6] = 1.0
    o[10:13] = (ox, oy, oz)
    o[16:20] = s
    o[24:28] = 1.0
    o[40], o[41], o[47] = fuel, payload, ammo
    o[48:4144] = -1.0
    for ray, r in lidar:
        h, el, a = ray // 768, (ray % 768) // 128, ray % 128
        o[48 + (16 * h + el) * 128 + a] = r
    return o


def level_mixer(s, mass, des_ax, des_ay, des_az, vx=0.0, vy=0.0, ox=0.0, oy=0.0, oz=0.0,
                spool_gain=2.4, max_fh=80.0, max_sin=0.32, parasite=1.0, max_txy=260.0,
                damp_v=0.4, idle_target=None, headroom=False):
    """prior[15] at identity attitude with every spool at s and gimbals at 0,
    for commanded world accelerations (onboard_features.cuh:312-393, 505-512
    with yaw = tilt = tilt error = 0, jammed yaw force 0, desired yaw 0)."""
    T = thrust(s)
    weight = mass * G
    # with headroom the collective cap shrinks with the body rate (:314-316)
    max_coll = clamp(3.95 - 0.90 * math.sqrt(ox * ox + oy * oy + oz * oz), 2.55, 3.95) \
        if headroom else 3.95
    fz_des = clamp(weight + mass * des_az, 0.1 * weight, max_coll * MAX_INST)
    fx = clamp(mass * des_ax + damp_v * vx, -max_fh, max_fh)
    fy = clamp(mass * des_ay + damp_v * vy, -max_fh, max_fh)
    tx_par = -0.1625 * fy * parasite
    ty_par = 0.1625 * fx * parasite
    tau_x = clamp(-64.0 * ox - 0.9 * tx_par - tx_par, -max_txy, max_txy)
    tau_y = clamp(-64.0 * oy - 0.9 * ty_par - ty_par, -max_txy, max_txy)
    tau_z = clamp(-18.0 * oz, -70.0, 70.0)
    fz_cmd = [0.25 * fz_des - 0.5 * tau_y, 0.25 * fz_des + 0.5 * tau_x,
              0.25 * fz_des + 0.5 * tau_y, 0.25 * fz_des - 0.5 * tau_x]
    radial = [0.5 * fx, 0.5 * fy, -0.5 * fx, -0.5 * fy]  # arms at +x, +y, -x, -y
    n = np.zeros(15)
    u_raw = []
    for i in range(4):
        alpha = math.asin(clamp(0.25 * tau_z / max(T, 30.0), -0.35, 0.35))
        outer = clamp(6.5 * alpha, -2.0, 2.0)
        inner = clamp(math.asin(clamp(radial[i] / max(T, 40.0), -max_sin, max_sin)),
                      -0.9 * PI / 4, 0.9 * PI / 4)
        nominal = max(math.cos(alpha) * math.cos(inner), 0.70)
        target = max(fz_cmd[i], 0.0) / nominal if idle_target is None else idle_target
        u = clamp((target - MIN_T) / (MAX_INST - MIN_T), 0.0, 1.0)
        u_raw.append(u + spool_gain * (u - s))
        n[4 + i] = outer / 2.0
        n[8 + i] = inner / (PI / 4)
    excess = clamp(max(u_raw) - 1.0, 0.0, 0.45) if headroom else 0.0
    for i in range(4):
        n[i] = 2.0 * clamp(u_raw[i] - excess, 0.0, 1.0) - 1.0
    n[12], n[13], n[14] = 0.0, 0.0, -0.8
    return n


def pick_spool(model):
    """The first spool on a 0.01 grid whose throttles all stay inside
    (-0.9, 0.9): the throttle then carries the commanded force instead of a
    clamp."""
    for s in np.arange(0.02, 0.99, 0.01):
        s = float(np.float32(round(s, 2)))
        if np.all(np.abs(model(s)[:4]) < 0.9):
            return s
    raise AssertionError("no spool keeps the throttles unsaturated")


def check_level(law, obs_kw=None, mission=None, mixer_kw=None, mass=BASE, s=None,
                expect_unsaturated=True):
    """Oracle prior == level_mixer(law(s, mass)) for the state obs_kw at a
    spool where the throttles are unsaturated (or the given s)."""
    obs_kw = dict(obs_kw or {})
    mixer_kw = dict(mixer_kw or {})
    m = np.zeros(10, np.float32)
    for k, v in (mission or {}).items():
        m[k] = v
    kin = {k: obs_kw[k] for k in ("vx", "vy", "ox", "oy", "oz") if k in obs_kw}

    def model(sp):
        ax, ay, az = law(sp, mass)
        return level_mixer(sp, mass, ax, ay, az, **kin, **mixer_kw)

    if s is None:
        s = pick_spool(model)
    want = model(s)
    if expect_unsaturated:
        assert np.all(np.abs(want[:4]) < 1.0)
    got = run_prior(level_obs(s, **obs_kw), m)
    err = np.abs(got - want)
    assert err.max() <= TOL, f"spool {s}: got {got}\nwant {want}\nerr {err}"
    return got


# ---------------------------------------------------------------- standard law
# Standard target (:156-166, 285-310): hover point (0, 0, 8); gains 0.9 (x, y),
# 1.25 (z); velocity caps 3.0 / 2.6; acceleration gains 2.4 (x), 2.6 (y), 3.8
# (z) with 0.8 az_actual damping, caps 3.8 and [-4, 6.5].

def test_hover_hold():
    check_level(lambda s, m: (0.0, 0.0, clamp(-0.8 * az_actual(s, m), -4.0, 6.5)))


def test_climb_within_caps():
    # upz = 0.5 -> des_vz = 0.625; vz = 0.2
    check_level(lambda s, m: (0.0, 0.0, clamp(3.8 * (0.625 - 0.2) - 0.8 * az_actual(s, m),
                                              -4.0, 6.5)),
                dict(pz=7.5, vz=0.2))


def test_climb_velocity_cap():
    # upz = 6 -> des_vz = 2.6 (cap); 3.8 * 2.6 - 0.8 az > 6.5 -> 6.5
    law = lambda s, m: (0.0, 0.0, clamp(3.8 * 2.6 - 0.8 * az_actual(s, m), -4.0, 6.5))
    assert law(0.5, BASE)[2] == 6.5
    check_level(law, dict(pz=2.0))


def test_descent_acceleration_floor():
    # upz = -6 -> des_vz = -2.6 -> 3.8 * -2.6 - 0.8 az < -4 at spool 0.15 -> -4
    law = lambda s, m: (0.0, 0.0, clamp(3.8 * -2.6 - 0.8 * az_actual(s, m), -4.0, 6.5))
    assert law(0.15, BASE)[2] == -4.0
    check_level(law, dict(pz=14.0), s=0.15)


def test_sinking_fast_raises_caps_and_hits_collective_cap():
    # vz < -2: velocity cap 6.5, vz < -1.8: acceleration cap 14; upz = 6 ->
    # des_vz 6.5 -> des_az 14 -> fz_des = min(weight + 14 m, 3.95 max_installed)
    law = lambda s, m: (0.0, 0.0, clamp(3.8 * (6.5 + 2.5) - 0.8 * az_actual(s, m), -4.0, 14.0))
    assert BASE * G + BASE * 14.0 > 3.95 * MAX_INST
    check_level(law, dict(pz=2.0, vz=-2.5), s=0.99)


def test_horizontal_gains():
    # up = (-0.3, 0.2): des_v = (-0.27, 0.18); des_a = (2.4 * -0.27, 2.6 * (0.18 - 0.1))
    check_level(lambda s, m: (2.4 * -0.27, 2.6 * (0.18 - 0.1), -0.8 * az_actual(s, m)),
                dict(px=0.3, py=-0.2, vy=0.1))


def test_horizontal_velocity_cap():
    # upx = -5 -> des_vx = -3 (cap); vx = -2.5 -> des_ax = 2.4 * -0.5
    check_level(lambda s, m: (2.4 * (-3.0 + 2.5), 0.0, -0.8 * az_actual(s, m)),
                dict(px=5.0, vx=-2.5))


def test_horizontal_force_cap():
    # des_a = (3.8, -3.8) (caps) -> forces 163 N, capped at 80 N
    check_level(lambda s, m: (3.8, -3.8, -0.8 * az_actual(s, m)), dict(px=-3.0, py=3.0))


@pytest.mark.parametrize("oz", [0.8, -0.5, 5.0])
def test_yaw_rate_damping(oz):
    # tau_z = clamp(-18 oz, +-70): outer gimbals 6.5 asin(tau_z / 4 / thrust)
    check_level(lambda s, m: (0.0, 0.0, -0.8 * az_actual(s, m)), dict(oz=oz))


@pytest.mark.parametrize("ox,oy", [(0.5, 0.0), (0.0, -0.4), (0.3, 0.2)])
def test_roll_pitch_rate_damping(ox, oy):
    # tau_x = -64 ox, tau_y = -64 oy: arms 1/3 and 2/0 split the collective
    check_level(lambda s, m: (0.0, 0.0, -0.8 * az_actual(s, m)), dict(ox=ox, oy=oy))


@pytest.mark.parametrize("fuel,ammo,payload,mass", [
    (0.5, 2.0, 0.0, BASE + 4.5 + 12.0), (1.0, 5.0, 0.0, BASE + 9.0 + 24.0),
    (-1.0, -1.0, 0.6, BASE + 30.0)])
def test_mass_model(fuel, ammo, payload, mass):
    # mass = 43 + 9 clamp(fuel, 0, 1) + 6 clamp(ammo, 0, 4) + 30 [payload > 0.5]
    check_level(lambda s, m: (0.0, 0.0, -0.8 * az_actual(s, m)),
                dict(fuel=fuel, ammo=ammo, payload=payload), mass=mass)


# ---------------------------------------------------------------- landing law
# Landing (m[1] > 0.75, :254-283): pad at z = 0.6 under the origin; acceleration
# x/y = clamp(2.4 (des_v - v), +-2.6), z = clamp(4.5 (des_vz - vz) - 0.8 az,
# -2.8, 5.5); des_v x/y = clamp(1.05 up, +-cap), cap 3.4 beyond 1.8 m, else
# 0.55 below 1.2 m above the pad, else 1.6.

LAND = {1: 1.0}


def land_az(des_vz, vz=0.0):
    return lambda s, m: clamp(4.5 * (des_vz - vz) - 0.8 * az_actual(s, m), -2.8, 5.5)


@pytest.mark.parametrize("pz,des_vz", [(2.0, -0.70 * 1.4), (3.0, -1.4)])
def test_landing_mid_descent(pz, des_vz):
    # above pad > 1.05 m: des_vz = clamp(-0.70 above_pad, -1.4, -0.25)
    az = land_az(des_vz)
    check_level(lambda s, m: (0.0, 0.0, az(s, m)), dict(pz=pz), LAND)


def test_landing_touchdown():
    # above pad <= 1.05, over the pad, slow: des_vz = -0.16 above 0.635 m
    az = land_az(-0.16)
    check_level(lambda s, m: (0.0, 0.0, az(s, m)), dict(pz=1.0), LAND)


def test_landing_touchdown_below_0635():
    # des_vz = 0 at or below 0.635 m; vz = 0.25 keeps land-idle off
    az = land_az(0.0, vz=0.25)
    check_level(lambda s, m: (0.0, 0.0, az(s, m)), dict(pz=0.63, vz=0.25), LAND)


def test_landing_align_off_pad():
    # 1 m off the pad (0.85 < d <= 1.8), 0.6 m above it: des_vz =
    # clamp(1.2 (0.6 + 0.9 - 1.2), -0.3, 0.6) = 0.36; des_vx = clamp(-1.05, +-0.55)
    az = land_az(1.2 * 0.3)
    check_level(lambda s, m: (2.4 * -0.55, 0.0, az(s, m)), dict(px=1.0, pz=1.2), LAND)


def test_landing_align_when_moving():
    # over the pad but horizontal speed 0.8 > 0.65: align regime; des_vx = 0
    az = land_az(1.2 * 0.3)
    check_level(lambda s, m: (2.4 * (0.0 - 0.8), 0.0, az(s, m)), dict(vx=0.8, pz=1.2), LAND)


def test_landing_align_cap():
    # 1.2 (0.6 + 0.9 - 0.7) = 0.96 -> 0.6
    az = land_az(0.6)
    check_level(lambda s, m: (2.4 * -0.55, 0.0, az(s, m)), dict(px=1.0, pz=0.7), LAND)


@pytest.mark.parametrize("px,pz,vx,des_vz,des_ax", [
    (3.0, 1.5, -2.6, 1.3 * 0.5, 2.4 * (-3.15 + 2.6)),   # des_vx = -3.15 (1.05 up)
    (3.0, 5.0, 0.0, -1.6, -2.6),                         # 1.3 (2 - 5) -> -1.6
    (-3.0, 0.8, 2.5, 1.4, 2.4 * (3.15 - 2.5)),           # 1.3 (2 - 0.8) -> 1.4
    (3.5, 1.5, -2.8, 1.3 * 0.5, 2.4 * (-3.4 + 2.8)),     # -3.675 -> cap 3.4
    (1.7, 2.2, -1.0, -0.70 * 1.6, 2.4 * (-1.6 + 1.0))])  # mid height: cap 1.6
def test_landing_transit_and_caps(px, pz, vx, des_vz, des_ax):
    # beyond 1.8 m: des_vz = clamp(1.3 (2.0 - pz), -1.6, 1.4), cap 3.4; the
    # accelerations stay below the 80 N force cap where x is pinned
    az = land_az(des_vz)
    check_level(lambda s, m: (clamp(des_ax, -2.6, 2.6), 0.0, az(s, m)),
                dict(px=px, pz=pz, vx=vx), LAND)


@pytest.mark.parametrize("pz", [0.6, 0.635])
def test_land_idle(pz):
    # at most 0.638 m, over the pad, slow: every arm targets 0.15 weight / 4
    # (:375,386)
    mass = BASE + 9.0 + 6.0 + 30.0
    heavy = dict(fuel=1.0, ammo=1.0, payload=1.0)
    n = check_level(lambda s, m: (0.0, 0.0, 0.0), dict(pz=pz, vz=0.1, **heavy),
                    LAND, dict(idle_target=0.15 * mass * G * 0.25), mass=mass, s=0.04)
    assert np.all(n[:4] == n[0]) and n[0] > -1.0
    # 0.2 m/s of sink ends idle: the law's own target applies again
    busy = run_prior(level_obs(0.04, pz=pz, vz=0.2, **heavy), np.array(
        [0, 1, 0, 0, 0, 0, 0, 0, 0, 0], np.float32))
    assert abs(busy[0] - n[0]) > 1e-3


def test_no_land_idle_above_0638():
    # 0.64 m: touchdown law, des_vz = -0.16
    mass = BASE + 9.0 + 6.0 + 30.0
    az = land_az(-0.16, vz=0.1)
    check_level(lambda s, m: (0.0, 0.0, az(s, m)),
                dict(pz=0.64, vz=0.1, fuel=1.0, ammo=1.0, payload=1.0), LAND, mass=mass)


# ---------------------------------------------------------------- cargo
# Heavy cargo (cargo mission m[2] > 0.75 and payload): the landing law with
# gains 0.75 / 5.0 / 1.0, caps 2.65 (transit), 2.2 (acceleration), -1.8 (z),
# the cargo descent clamp(1.6 (0.64 - pz), -0.3, 0.18), transit height
# max(1.2 + 0.28 d, 2), sink limit -1.05; force cap 52 N, inner limit 0.22,
# spool gain 4.5, torque cap 120.  The pad is (15, 0) at the current height.

HEAVY = dict(max_fh=52.0, max_sin=0.22, spool_gain=4.5, max_txy=120.0)
HEAVY_MASS = BASE + 30.0


def heavy_az(des_vz, vz=0.0):
    return lambda s, m: clamp(5.0 * (des_vz - vz) - 1.0 * az_actual(s, m), -1.8, 5.5)


@pytest.mark.parametrize("px,pz,vx,des_vz,des_ax", [
    (12.0, 3.0, 1.5, -1.05, 2.4 * (0.75 * 3.0 - 1.5)),       # transit z 2.04, sink cap
    (5.0, 3.0, 0.0, 1.3 * (1.2 + 0.28 * 10.0 - 3.0), 2.2),   # transit z 4.0; cap 2.65, 2.2
    (14.5, 0.7, 0.0, 1.6 * (0.64 - 0.7), 2.4 * 0.75 * 0.5),  # low: cargo descent
    (14.5, 1.0, 0.0, -0.3, 2.4 * 0.75 * 0.5),                # cargo descent clamp
    (14.0, 1.0, 0.0, 0.6, 2.4 * 0.55)])                      # align: 1.08 -> 0.6; cap 0.55
def test_heavy_cargo(px, pz, vx, des_vz, des_ax):
    az = heavy_az(des_vz)
    check_level(lambda s, m: (clamp(des_ax, -2.2, 2.2), 0.0, az(s, m)),
                dict(px=px, pz=pz, vx=vx, payload=1.0), {2: 1.0}, HEAVY, mass=HEAVY_MASS)


# The heavy-cargo limits below are hidden at the states above by a clamp
# further down the law: 52 N of force is only 0.71 m/s^2 at 73 kg, so every
# horizontal acceleration above that is clipped, and a steep vertical command
# meets the -1.8 floor.  Each state here makes the named limit the binding one
# and keeps everything after it unclipped (asserted at the spool used).

def check_heavy_binding(des_ax, des_vz, obs_kw):
    """check_level for heavy cargo, with the force and the vertical
    acceleration asserted inside their caps at the spool the check uses."""
    vx, vz = obs_kw.get("vx", 0.0), obs_kw.get("vz", 0.0)
    assert abs(HEAVY_MASS * des_ax + 0.4 * vx) < 52.0
    raw_az = lambda s: 5.0 * (des_vz - vz) - az_actual(s, HEAVY_MASS)
    law = lambda s, m: (des_ax, 0.0, clamp(raw_az(s), -1.8, 5.5))
    s = pick_spool(lambda sp: level_mixer(sp, HEAVY_MASS, *law(sp, HEAVY_MASS), vx=vx,
                                          **HEAVY))
    assert -1.8 < raw_az(s) < 5.5
    check_level(law, dict(obs_kw, payload=1.0), {2: 1.0}, HEAVY, mass=HEAVY_MASS, s=s)


def test_heavy_cargo_transit_speed_cap():
    # 10 m from the pad: des_vx = clamp(0.75 * 10, +-2.65) = 2.65 (:257); at
    # vx = 2.45 that asks 2.4 * 0.2 m/s^2, 36 N; transit height 1.2 + 0.28 * 10
    check_heavy_binding(2.4 * (2.65 - 2.45), 1.3 * (1.2 + 0.28 * 10.0 - 3.5),
                        dict(px=5.0, pz=3.5, vx=2.45))


def test_heavy_cargo_climb_clamp():
    # 0.4 m up, 0.1 m short of the pad, no landing flag (so no land-idle):
    # cargo descent law clamp(1.6 (0.64 - 0.4), -0.3, 0.18) = 0.18 (:264)
    assert 1.6 * (0.64 - 0.4) > 0.18
    check_heavy_binding(2.4 * 0.75 * 0.1, 0.18, dict(px=14.9, pz=0.4))


def test_heavy_cargo_transit_sink_cap():
    # 3 m out, 1.46 m above the 2.04 m transit height: 1.3 * -1.46 -> -1.05
    # (:270); sinking at 1 m/s already, so the command stays above -1.8
    assert 1.3 * (1.2 + 0.28 * 3.0 - 3.5) < -1.05
    check_heavy_binding(2.4 * (0.75 * 3.0 - 2.0), -1.05, dict(px=12.0, pz=3.5, vx=2.0, vz=-1.0))


def test_heavy_cargo_acceleration_cap():
    # 2.4 (2.25 + 280) -> 2.2 (:276); the 0.4 vx damping (-112 N) brings
    # 73 * 2.2 = 160.6 N under the 52 N force cap, which a 2.6 cap would not
    check_heavy_binding(2.2, 1.3 * (1.2 + 0.28 * 3.0 - 2.0), dict(px=12.0, pz=2.0, vx=-280.0))


def test_light_cargo_uses_standard_law():
    # no payload: standard law towards (15, 0, pz)
    check_level(lambda s, m: (2.4 * 0.9, 0.0, -0.8 * az_actual(s, m)),
                dict(px=14.0, pz=5.0), {2: 1.0})


# ---------------------------------------------------------------- faults, lateral
def test_turbine_out_gain_and_parasite_torque():
    # m[3] > 0.75 with m[2] < -0.25: spool gain 10.5, parasite torques x 0.35
    check_level(lambda s, m: (2.4 * -0.27, 2.6 * (0.18 - 0.1), -0.8 * az_actual(s, m)),
                dict(px=0.3, py=-0.2, vy=0.1), {3: 1.0, 2: -0.5},
                dict(spool_gain=10.5, parasite=0.35))


def rel(v, lim=0.9995):
    return math.atanh(clamp(float(np.float32(v)), -lim, lim)) * 20.0


@pytest.mark.parametrize("m7,m8,vx,vy", [(0.05, 0.02, 0.5, 0.1), (0.1, 0.1, 0.8, 1.0),
                                         (0.1, 0.02, 1.5, 0.1), (0.02, 0.1, 0.2, 1.5),
                                         (math.tanh(0.15), math.tanh(0.07), 1.0, 1.0),
                                         (math.tanh(0.15), math.tanh(0.0665), 1.0, 1.0)])
def test_lateral(m7, m8, vx, vy):
    # m[4] > 0.75, m[5] > 0.25: goal = position + 20 atanh(m[7..8]); gains
    # 0.95 / 1.05; y cap 3.4, x cap 1.45 when |up_y| > 1.35 else 3.8 (:287);
    # force cap 125 N, inner limit 0.44.  The last two states put |up_y| at
    # 1.40 and 1.33, either side of the threshold, with 0.95 up_x = 2.85 above
    # the 1.45 cap
    ux, uy = rel(m7), rel(m8)
    cap_x = 1.45 if abs(uy) > 1.35 else 3.8
    dvx = clamp(0.95 * ux, -cap_x, cap_x)
    dvy = clamp(1.05 * uy, -3.4, 3.4)
    check_level(lambda s, m: (clamp(2.4 * (dvx - vx), -3.8, 3.8),
                              clamp(2.6 * (dvy - vy), -3.8, 3.8), -0.8 * az_actual(s, m)),
                dict(px=2.0, py=-1.0, vx=vx, vy=vy), {4: 1.0, 5: 0.5, 7: m7, 8: m8},
                dict(max_fh=125.0, max_sin=0.44))


# ---------------------------------------------------------------- inversion mission
# m[3] > 0.75, m[0] < -0.25: hover point (0, 0, 14), gain 0.85, x/y cap 4.2
# (6.2 when far, level and near height), z cap 6.5, acceleration cap 14,
# climb floor 0.8 when sinking; the headroom logic is active (no tilt here).
INV = {3: 1.0, 0: -0.5}


@pytest.mark.parametrize("px,pz,vx,vz,dvx,dvz", [
    (1.0, 12.0, 0.0, 0.0, -0.85, 1.25 * 2.0),
    (-12.0, 13.0, 5.8, 0.0, 6.2, 1.25 * 1.0),      # far, level, near height: 6.2
    (0.5, 16.0, 0.0, -1.5, -0.425, 0.8)])          # sinking: climb floor 0.8
def test_inversion_mission_limits(px, pz, vx, vz, dvx, dvz):
    max_az = 14.0
    check_level(lambda s, m: (clamp(2.4 * (dvx - vx), -3.8, 3.8), 0.0,
                              clamp(3.8 * (dvz - vz) - 0.8 * az_actual(s, m), -4.0, max_az)),
                dict(px=px, pz=pz, vx=vx, vz=vz), INV, dict(headroom=True))


@pytest.mark.parametrize("ox,s", [(-2.5, 0.45), (-3.5, 0.45)])
def test_headroom_excess(ox, s):
    """With headroom (inversion mission), a raw throttle above 1 lowers every
    arm by the excess, at most 0.45 (:395-397)."""
    law = lambda sp, m: (0.0, 0.0, clamp(3.8 * 1.25 * 2.0 - 0.8 * az_actual(sp, m), -4.0, 14.0))
    ax, ay, az = law(s, BASE)
    probe = level_mixer(s, BASE, ax, ay, az, ox=ox)      # no headroom: raw throttles
    assert probe[1] == 1.0                              # arm 1 saturates without it
    # (the collective cap is 2.55 max_installed at these rates)
    assert 0.9 * abs(ox) > 3.95 - 2.55
    check_level(law, dict(pz=12.0, ox=ox), INV, dict(headroom=True), s=s,
                expect_unsaturated=False)


@pytest.mark.parametrize("tilt,px,mission", [
    (0.60, 1.0, {}),            # standard law: headroom from cos(tilt) = 0.825 < 0.88
    (0.60, -2.0, {}),
    (0.30, 1.0, INV),           # inversion mission: headroom at any tilt
    (0.17, -1.5, INV),
    (0.10, 1.0, INV)])          # below 0.15 rad: no reduction
def test_headroom_tilt_scales_horizontal_force(tilt, px, mission):
    """Pitched hover with headroom (:318-324): the world horizontal force is
    scaled by clamp(1 - 1.5 max(tilt - 0.15, 0), 0, 1).  At a pure pitch the
    yaw is 0, so the body force equals the world force, and with the outer
    gimbals at zero the inner gimbals carry it alone: arm 0 takes
    asin(0.5 fx / thrust), arm 2 the negative, arms 1 and 3 nothing
    (:380-384).  Outer gimbals, cannon and fire flag are at rest."""
    s = 0.5
    o = level_obs(s, px=px, pz=14.0 if mission else 8.0)
    o[6], o[8] = math.cos(tilt / 2.0), math.sin(tilt / 2.0)
    mis = np.zeros(10, np.float32)
    for k, v in mission.items():
        mis[k] = v
    got = run_prior(o, mis)
    kp, cap = (0.85, 4.2) if mission else (0.90, 3.0)
    des_ax = clamp(2.4 * clamp(kp * -px, -cap, cap), -3.8, 3.8)
    scale = clamp(1.0 - 1.5 * max(tilt - 0.15, 0.0), 0.0, 1.0)
    fx = clamp(BASE * des_ax * scale, -80.0, 80.0)
    sin_in = 0.5 * fx / thrust(s)
    assert abs(sin_in) < 0.32                    # the inner limit does not clip
    want = np.zeros(15)
    want[8], want[10] = math.asin(sin_in) / (PI / 4), -math.asin(sin_in) / (PI / 4)
    want[14] = -0.8
    err = np.abs(got - want)[4:]
    assert err.max() <= TOL, f"got {got[4:]}\nwant {want[4:]}"


# ---------------------------------------------------------------- arena
def arena_point(px, py, relx, rely):
    """Arena stand-off point (:170-181): 12.5 m short of the goal on the line
    from the goal to the vehicle, scaled into a 16 m disc about the origin,
    then pulled towards the origin beyond a 21 m radius."""
    tx, ty = px + relx, py + rely
    d = math.hypot(relx, rely)
    ax, ay = tx - relx / d * 12.5, ty - rely / d * 12.5
    scale = min(16.0 / max(math.hypot(ax, ay), 1e-3), 1.0)
    pull = clamp((math.hypot(px, py) - 21.0) / 10.0, 0.0, 1.0)
    return ax * scale * (1.0 - pull), ay * scale * (1.0 - pull)


def pick_arena_position(relx, rely, scaled):
    """A float32 position whose stand-off point is 1..3.5 m away in y (so the
    y command is not capped); with `scaled`, one beyond the 21 m ring whose
    stand-off point needed the 16 m disc."""
    for x in np.arange(-30.0, 30.0, 0.5):
        for y in np.arange(-30.0, 30.0, 0.5):
            px, py = float(np.float32(x)), float(np.float32(y))
            tx, ty = px + relx, py + rely
            d = math.hypot(relx, rely)
            pre = math.hypot(tx - relx / d * 12.5, ty - rely / d * 12.5)
            if scaled != (math.hypot(px, py) > 21.0 and pre > 16.0):
                continue
            ex, ey = arena_point(px, py, relx, rely)
            if 1.0 < abs(ey - py) < 3.5 and 1.0 < math.hypot(ex - px, ey - py) < 3.5 * (
                    4.0 if scaled else 1.0):
                return px, py
    raise AssertionError("no position found")


@pytest.mark.parametrize("m7,m8,scaled,cannon_free", [
    (0.55, 0.3, False, True), (-0.3, -0.55, True, False),
    (0.75, 0.3, False, True),                             # goal 20.4 m away: fire
    (0.95, 0.3, False, False)])                           # 37 m: beyond 34 m, no fire
def test_arena_standoff_yaw_and_cannon(m7, m8, scaled, cannon_free):
    """Arena, level at 9 m: velocity toward the stand-off point (:170-181),
    yaw to the goal bearing minus the cannon's 45 degree offset (:343-348),
    cannon aim at the ballistic lead and fire inside 0.28 rad (:407-431)."""
    relx, rely = rel(m7), rel(m8)
    px, py = pick_arena_position(relx, rely, scaled)
    ex, ey = arena_point(px, py, relx, rely)
    dvx, dvy = clamp(0.9 * (ex - px), -3.2, 3.2), clamp(0.9 * (ey - py), -3.2, 3.2)
    pz = 9.0
    vx, vy = float(np.float32(dvx - 0.4)), float(np.float32(dvy + 0.3))
    mass = 40.0 + 6.0                    # arena frame + one ammo unit
    assert abs(dvy) < 3.2
    des_ax, des_ay = clamp(2.4 * (dvx - vx), -3.8, 3.8), clamp(2.6 * (dvy - vy), -3.8, 3.8)
    tx, ty, tz = px + relx, py + rely, pz
    yaw_err = math.atan2(ty - py, tx - px) - PI / 4
    to = (tx - px, ty - py, tz - pz)
    dist = max(math.sqrt(sum(c * c for c in to)), 1.0)
    fl = dist / 20.0
    aim = (to[0] - vx * 0.65 * fl, to[1] - vy * 0.65 * fl, to[2] + 0.53 * G * fl * fl)
    caz = clamp(math.atan2(aim[1], aim[0]), PI / 4 - PI / 6, PI / 4 + PI / 6)
    cel = clamp(math.atan2(aim[2], max(math.hypot(aim[0], aim[1]), 0.2)), -PI / 6, PI / 6)
    o44, o45 = float(np.float32(caz + 0.05)), float(np.float32(cel - 0.05))

    def model(s):
        az = clamp(-0.8 * az_actual(s, mass), -4.0, 6.5)
        n = level_mixer(s, mass, des_ax, des_ay, az, vx=vx, vy=vy, headroom=True)
        # the yaw error adds a yaw torque: outer gimbals and nominal cosines
        T = thrust(s)
        alpha = math.asin(clamp(0.25 * clamp(22.0 * yaw_err, -70.0, 70.0) / max(T, 30.0),
                                -0.35, 0.35))
        n[4:8] = clamp(6.5 * alpha, -2.0, 2.0) / 2.0
        weight = mass * G
        fz_des = clamp(weight + mass * az, 0.1 * weight, 3.95 * MAX_INST)
        fx = clamp(mass * des_ax + 0.4 * vx, -80.0, 80.0)
        fy = clamp(mass * des_ay + 0.4 * vy, -80.0, 80.0)
        tau_x, tau_y = -1.9 * (-0.1625 * fy), -1.9 * (0.1625 * fx)
        fz_cmd = [0.25 * fz_des - 0.5 * tau_y, 0.25 * fz_des + 0.5 * tau_x,
                  0.25 * fz_des + 0.5 * tau_y, 0.25 * fz_des - 0.5 * tau_x]
        u_raw = []
        for i in range(4):
            nominal = max(math.cos(alpha) * math.cos(n[8 + i] * PI / 4), 0.7)
            u = clamp((max(fz_cmd[i], 0.0) / nominal - MIN_T) / (MAX_INST - MIN_T), 0.0, 1.0)
            u_raw.append(u + 2.4 * (u - s))
        excess = clamp(max(u_raw) - 1.0, 0.0, 0.45)
        for i in range(4):
            n[i] = 2.0 * clamp(u_raw[i] - excess, 0.0, 1.0) - 1.0
        n[12] = clamp((caz - PI / 4) / (PI / 6), -1.0, 1.0)
        n[13] = clamp(cel / (PI / 6), -1.0, 1.0)
        n[14] = 0.8 if (math.hypot(caz - o44, cel - o45) < 0.28 and dist < 34.0) else -0.8
        return n

    s = pick_spool(model)
    want = model(s)
    assert (want[14] == 0.8) == (dist < 34.0) and abs(want[4]) > 0.01
    assert (abs(want[12]) < 1.0) == cannon_free
    obs = level_obs(s, px=px, py=py, pz=pz, vx=vx, vy=vy, ammo=1.0)
    obs[44], obs[45] = o44, o45
    mis = np.zeros(10, np.float32)
    mis[6], mis[7], mis[8] = 1.0, m7, m8
    got = run_prior(obs, mis)
    assert np.abs(got - want).max() <= TOL, f"got {got}\nwant {want}"
    # out of cannon cooldown (o[46] > 0.02): no fire
    obs[46] = 0.05
    assert run_prior(obs, mis)[14] == np.float32(-0.8)


# ---------------------------------------------------------------- slalom
# Slalom (m[4] > 0.75, not lateral): goal x = 36, height 8 + 2.5 sin(pi hill)
# with hill = clamp((px - 6) / 30, 0, 1).  With a corridor obstacle ahead the
# lane target is -1.85 m when the cluster's mean y >= 0, else +1.85 m, the
# speed limit 1.55 / 2.75 / 4.10 by lane error (3.10 when the obstacle is at
# least 6.6 m ahead and px > 4), gains 1.25 / 1.45 / 3.0, y cap 3.2, damping
# 0.8, force cap 105 N, inner limit 0.42.
SLALOM = {4: 1.0}
AHEAD, RIGHT_22 = 112, 120          # head 0, el 0: azimuth 2 pi, 22.5 degrees


def test_slalom_open_course():
    # px = 21: hill 0.5 -> height 10.5; upz 0.5; x cap 3.5, y cap 3.0
    check_level(lambda s, m: (2.4 * (3.5 - 3.0), 2.6 * (0.9 * -0.4), clamp(
        3.8 * 1.25 * 0.5 - 0.8 * az_actual(s, m), -4.0, 6.5)),
                dict(px=21.0, py=0.4, pz=10.0, vx=3.0), SLALOM)


@pytest.mark.parametrize("px,py,ray,rng,vx,vy,lane,limit", [
    (6.0, 0.3, AHEAD, 4.0, 1.0, -2.0, -1.85, 1.55),     # obstacle right of lane: -1.85
    (6.0, -0.3, AHEAD, 4.0, 1.0, 2.0, 1.85, 1.55),      # mirror
    (6.0, -1.85, RIGHT_22, 4.0, 3.5, 0.5, -1.85, 4.10),  # in lane
    (6.0, -1.0, RIGHT_22, 4.0, 2.2, 0.5, -1.85, 2.75),  # lane error 0.85
    (6.0, 0.3, AHEAD, 6.0, 2.5, -2.0, -1.85, 3.10),     # obstacle 7.1 m ahead, px > 4
    (4.5, 0.3, AHEAD, 6.0, 2.5, -2.0, -1.85, 3.10),
    (3.5, 0.3, AHEAD, 6.0, 1.0, -2.0, -1.85, 1.55)])    # px <= 4: lane limit stays
def test_slalom_obstacle_lane_and_speed(px, py, ray, rng, vx, vy, lane, limit):
    dvx = clamp(1.25 * (36.0 - px), -limit, limit)
    dvy = clamp(1.45 * (lane - py), -3.2, 3.2)
    check_level(lambda s, m: (clamp(3.0 * (dvx - vx), -3.8, 3.8),
                              clamp(3.0 * (dvy - vy), -3.8, 3.8), -0.8 * az_actual(s, m)),
                dict(px=px, py=py, vx=vx, vy=vy, lidar=[(ray, rng)]), SLALOM,
                dict(max_fh=105.0, max_sin=0.42, damp_v=0.8))


# ---------------------------------------------------------------- dodge
DODGE = {5: 1.0}


@pytest.mark.parametrize("rays,nearest", [
    ([(116, 5.0)], 0), ([(20, 5.0)], 0), ([(116, 6.0), (20, 5.0)], 1),
    ([(128 * 3 + 116, 5.0)], 0), ([(768 + 20, 4.0)], 0)])
def test_dodge_vector(rays, nearest):
    """dodge (m[5] > 0.75) with a return closer than 7.5 m on elevation rows
    0..3: velocity offset (-sin, cos) * 2.2 of the return's bearing."""
    table = oracle.onboard_ray_table().astype(np.float64)
    ray, r = rays[nearest]
    bearing = math.atan2(table[ray, 1] * r, table[ray, 0] * r)
    avx, avy = -math.sin(bearing) * 2.2, math.cos(bearing) * 2.2
    check_level(lambda s, m: (clamp(2.4 * clamp(avx, -3, 3), -3.8, 3.8),
                              clamp(2.6 * clamp(avy, -3, 3), -3.8, 3.8), -0.8 * az_actual(s, m)),
                dict(lidar=rays), DODGE)


@pytest.mark.parametrize("rays", [[(116, 8.0)], [(128 * 4 + 116, 5.0)], [(116, 0.3)]])
def test_no_dodge(rays):
    # 7.5 m or farther, elevation rows 4..5, or outside the 0.35 m window
    check_level(lambda s, m: (0.0, 0.0, -0.8 * az_actual(s, m)), dict(lidar=rays), DODGE)


# ---------------------------------------------------------------- inversion recovery
def tilted_obs(axis, deg, ox=0.0, oy=0.0, outer=(0.0, 0.0, 0.0, 0.0), s=0.5):
    o = level_obs(s, ox=ox, oy=oy)
    h = math.radians(deg) / 2.0
    o[6] = math.cos(h)
    o[7 + axis] = math.sin(h)
    for i, a in enumerate(outer):
        o[20 + i], o[24 + i] = math.sin(a), math.cos(a)
    return o


@pytest.mark.parametrize("axis,deg,ox,oy,fires", [
    (0, 150.0, 0.0, 0.0, (3,)),           # roll right: e_rx = -tilt -> arm 3
    (0, -150.0, 0.0, 0.0, (1,)),          # roll left -> arm 1
    (1, 150.0, 0.0, 0.0, (0,)),           # pitch: e_ry = -tilt -> arm 0
    (1, -150.0, 0.0, 0.0, (2,)),
    (0, 150.0, 0.0, 0.25, (3, 0)),        # -52 oy = -13: arm 0 moment 13 > 12
    (0, 150.0, 0.0, 0.20, (3,)),          # 10.4 < 12
    (0, 150.0, -6.3, 0.0, (3,)),          # 130 tilt - 52 * 6.3 = 12.7 > 12
    (0, 150.0, -6.4, 0.0, ())])           # 7.5
def test_inversion_recovery_arm_rule(axis, deg, ox, oy, fires):
    """ct < 0.2 (:394-405): arm moments {-ty, tx, ty, -tx} with
    tx = 130 e_rx - 52 ox, ty = 130 e_ry - 52 oy; an arm above 12 runs at
    0.58 throttle (n = 0.16), the rest at 0 (n = -1); inner gimbals 0; outer
    gimbals clamp(-6 outer, +-2); cannon azimuth flag -1, elevation 0."""
    outer = (0.1, -0.2, 0.5, -0.05)
    got = run_prior(tilted_obs(axis, deg, ox, oy, outer), np.zeros(10, np.float32))
    want_thr = [0.16 if i in fires else -1.0 for i in range(4)]
    assert np.allclose(got[:4], want_thr, atol=TOL), got[:4]
    assert np.allclose(got[4:8], [clamp(-6.0 * a, -2.0, 2.0) / 2.0 for a in outer], atol=TOL)
    assert np.all(got[8:12] == 0.0)
    assert got[12] == -1.0 and got[13] == 0.0 and got[14] == np.float32(-0.8)


def test_inversion_threshold_is_ct_020():
    # cos(tilt) = 0.19 -> recovery law (n[12] = -1); 0.21 -> normal law
    for ct, inv in ((0.19, True), (0.21, False)):
        got = run_prior(tilted_obs(0, math.degrees(math.acos(ct))), np.zeros(10, np.float32))
        assert (got[12] == -1.0) == inv and (got[12] == 0.0) != inv
        recovery = np.allclose(got[:4], [-1.0, -1.0, -1.0, 0.16], atol=TOL)
        assert recovery == inv, got[:4]


# ---------------------------------------------------------------- BWB
def bwb_obs(vx, pz=60.0, ox=0.0, oy=0.0, oz=0.0, o44=0.0, o45=0.0, ammo=0.0, bank=0.0):
    o = level_obs(0.5, pz=pz, vx=vx, ox=ox, oy=oy, oz=oz, ammo=ammo)
    o[44], o[45] = o44, o45
    if bank:
        o[6], o[7] = math.cos(bank / 2.0), math.sin(bank / 2.0)
    return o


def bwb_expect(vx, m, ox=0.0, oy=0.0, oz=0.0, arena=False, speed=22.4, base=0.44, bank=0.0):
    """:432-503 at position (0, 0), speed vx along x, attitude level or
    rolled right by `bank` radians about the body x axis (pitch and yaw 0,
    so the body speed is vx and the sideslip 0)."""
    brx, bry, brz = (rel(m.get(k, 0.0), 0.9999) for k in (7, 8, 9))
    gx, gy, gz = brx, bry, brz
    course_err = math.atan2(gy, gx)          # ground track along x: course yaw 0
    u_coll = clamp(base + 0.065 * (speed - vx) + 0.018 * gz, 0.12, 0.90)
    diff_u = clamp(0.90 * (clamp(-1.35 * course_err, -0.55, 0.55) - bank) - 0.34 * ox,
                   -0.45, 0.45)
    u0, u1 = clamp(u_coll + diff_u, 0.05, 1.0), clamp(u_coll - diff_u, 0.05, 1.0)
    climb = clamp(0.42 * gz, -5.0, 5.0)
    gamma = math.atan2(climb, max(vx, 14.0))
    cb, sb = math.cos(bank), math.sin(bank)
    pitch = clamp(0.062831853 + 0.75 * gamma + 0.035 * climb + 0.09 * (1.0 - max(cb, 0.5)),
                  -0.15, 0.25)
    if vx < 15.5:
        pitch = min(pitch, 0.02)
    theta_dot = 2.20 * pitch
    # coordinated-turn yaw rate g / max(speed, 12) * tan(-bank), bank within 0.75
    psi_dot = G / max(vx, 12.0) * math.tan(clamp(-bank, -0.75, 0.75)) + 0.35 * course_err
    q_up = cb * theta_dot - sb * psi_dot
    r_left = sb * theta_dot + cb * psi_dot
    gimbal = PI / 6
    i0 = clamp(0.85 * (q_up + oy) + 0.03, -gimbal, gimbal)
    i1 = clamp(-0.65 * (r_left - oz), -gimbal, gimbal)
    n = np.zeros(15)
    n[0] = n[2] = 2 * u0 - 1
    n[1] = n[3] = 2 * u1 - 1
    n[8], n[9] = i0 / (PI / 4), i1 / (PI / 4)
    n[14] = -0.8
    return n


@pytest.mark.parametrize("vx,m,ox,oy,oz,kw", [
    (22.4, {4: 1.0, 2: 0.5, 7: 0.2}, 0.5, 0.0, 0.0, {}),               # level cruise
    (20.0, {4: 1.0, 2: 0.5, 0: 0.5, 7: 0.2}, 0.0, 0.0, 0.0,
     dict(speed=18.5, base=0.36)),                                       # endurance
    (22.4, {4: 1.0, 2: 0.5, 7: 0.2, 9: 0.1}, 0.0, 0.1, 0.0, {}),       # climb
    (14.0, {4: 1.0, 2: 0.5, 7: 0.2}, 0.0, 0.0, 0.3, {}),               # slow: pitch cap
    (22.4, {4: 1.0, 2: 0.5, 7: 0.2, 8: 0.1}, 0.0, 0.0, 0.0, {}),       # turn: roll cap
    (22.4, {4: 1.0, 2: 0.5, 7: 0.2, 8: -0.1}, 0.2, 0.0, 0.0, {})])     # other way
def test_bwb_cruise(vx, m, ox, oy, oz, kw):
    mis = np.zeros(10, np.float32)
    for k, v in m.items():
        mis[k] = v
    got = run_prior(bwb_obs(vx, ox=ox, oy=oy, oz=oz), mis)
    want = bwb_expect(vx, m, ox, oy, oz, **kw)
    assert np.abs(got - want).max() <= TOL, f"got {got}\nwant {want}"


@pytest.mark.parametrize("vx,bank", [(8.0, 0.3), (8.0, -0.5), (11.0, 0.9), (20.0, 0.3),
                                     (20.0, -0.2)])
def test_bwb_banked_turn_rate(vx, bank):
    """Banked BWB cruise, goal straight ahead (:455-478): the roll enters the
    differential throttle (0.9 (0 - roll)) and the pitch target; the yaw rate
    is the coordinated turn g / max(body speed, 12) tan(-roll), roll clamped
    to 0.75, split into the two gimbal rates by the bank.  Below 12 m/s the
    12 m/s floor sets it, above it the body speed does."""
    m = {4: 1.0, 2: 0.5, 7: 0.2}
    mis = np.zeros(10, np.float32)
    for k, v in m.items():
        mis[k] = v
    got = run_prior(bwb_obs(vx, bank=bank), mis)
    want = bwb_expect(vx, m, bank=bank)
    assert np.abs(got - want).max() <= TOL, f"got {got}\nwant {want}"


@pytest.mark.parametrize("o44,fire", [(0.48, True), (0.40, False)])
def test_bwb_arena_cannon(o44, fire):
    """BWB arena (m[6] > 0.75, m[4] < -0.25): opponent lead with closing speed
    75 m/s, gravity drop, azimuth limit pi/6, fire inside 0.045 rad."""
    vx = 24.0
    m = {6: 1.0, 4: -1.0, 7: 0.3, 8: 0.1}
    mis = np.zeros(10, np.float32)
    for k, v in m.items():
        mis[k] = v
    got = run_prior(bwb_obs(vx, o44=o44, ammo=1.0), mis)
    want = bwb_expect(vx, m, speed=24.0)            # goal closer than 38 m: 24 m/s
    brx, bry = rel(0.3, 0.9999), rel(0.1, 0.9999)
    opp = (brx - vx * 0.10, bry, 0.0)
    bdist = max(math.sqrt(sum(c * c for c in opp)), 1.0)
    fl = bdist / 75.0
    b = (opp[0], opp[1], opp[2] + 0.5 * G * fl * fl)
    baz = clamp(math.atan2(b[1], max(b[0], 0.2)), -PI / 6, PI / 6)
    bel = clamp(math.atan2(b[2], max(math.hypot(b[0], b[1]), 0.2)), -PI / 6, PI / 6)
    want[12], want[13] = baz / (PI / 6), bel / (PI / 6)
    want[14] = 0.8 if fire else -0.8
    assert (math.hypot(baz - o44, bel) < 0.045) == fire
    assert np.abs(got - want).max() <= TOL, f"got {got}\nwant {want}"


# ---------------------------------------------------------------- mirror symmetry
ARMS = [0, 3, 2, 1]                    # y -> -y swaps the arms at +y and -y


def mirror(obs, mission):
    o, m = obs.copy(), mission.copy()
    for k in (1, 4, 7, 9, 10, 12, 14):    # py, vy, qx, qz, wx, wz, specific force y
        o[k] = -o[k]
    for base, sign in ((16, 1), (20, -1), (24, 1), (28, 1), (32, -1), (36, 1)):
        vals = obs[base:base + 4].copy()
        for i in range(4):
            o[base + ARMS[i]] = sign * vals[i]
    lid = obs[48:4144].reshape(2, 16, 128)
    az = (96 - np.arange(128)) % 128    # azimuth pi (0.25 + a / 64) -> its mirror
    o[48:4144] = lid[:, :, az].reshape(-1)
    m[8] = -m[8]
    return o, m


def random_states(n, seed, modes):
    rng = np.random.default_rng(seed)
    obs = np.zeros((n, 4148), np.float32)
    mis = np.zeros((n, 10), np.float32)
    for e in range(n):
        o = obs[e]
        o[0:3] = rng.uniform(-4, 4), rng.uniform(-4, 4), rng.uniform(1, 14)
        o[3:6] = rng.uniform(-3, 3, 3)
        q = np.r_[1.0, rng.normal(0, 0.25, 3)]
        o[6:10] = q / np.linalg.norm(q)
        o[10:13] = rng.uniform(-1, 1, 3)
        o[16:20] = rng.uniform(0.2, 0.8, 4)
        outer = rng.uniform(-0.3, 0.3, 4)
        o[20:24], o[24:28] = np.sin(outer), np.cos(outer)
        o[28:32] = rng.uniform(-0.2, 0.2, 4)
        o[40], o[41], o[47] = rng.uniform(0, 1), rng.integers(0, 2), rng.uniform(0, 3)
        o[48:4144] = -1.0
        mis[e] = modes[e % len(modes)]
        mis[e, 7:10] = rng.uniform(-0.5, 0.5, 3)
    return obs, mis


MULTICOPTER_MODES = [
    [0, 0, 0, 0, 0, 0, 0, 0, 0, 0],         # hover
    [0, 1, 0, 0, 0, 0, 0, 0, 0, 0],         # landing
    [0, 0, 1, 0, 0, 0, 0, 0, 0, 0],         # cargo
    [-1, 0, 0, 1, 0, 0, 0, 0, 0, 0],        # inversion
    [0, 0, -1, 1, 0, 0, 0, 0, 0, 0],        # turbine out
    [0, 0, 0, 0, 1, 0.5, 0, 0, 0, 0],       # lateral
    [0, 0, 0, 0, 1, 0, 0, 0, 0, 0],         # slalom
    [0, 0, 0, 0, 0, 1, 0, 0, 0, 0]]         # dodge
BWB_MODES = [
    [0, 0, 0.5, 0, 1, 0, 0, 0, 0, 0],       # BWB cruise
    [0.5, 0, 0.5, 0, 1, 0, 0, 0, 0, 0],     # BWB endurance
    [0, 0, 0, 0, -1, 0, 1, 0, 0, 0],        # BWB arena
    [0, 0, 0, 0, 0, 0.8, 1, 0, 0, 0]]       # BWB intercept


def test_mirror_symmetry_multicopter_modes():
    obs, mis = random_states(256, 11, MULTICOPTER_MODES)
    # tilted states past the recovery threshold too
    obs[::8, 6:10] = np.array([0.2588, 0.9659, 0.0, 0.0], np.float32)
    mo, mm = zip(*(mirror(o, m) for o, m in zip(obs, mis)))
    _, p, _ = oracle.onboard(obs, mis)
    _, q, _ = oracle.onboard(np.array(mo), np.array(mm))
    want = np.empty_like(p)
    for i in range(4):
        want[:, ARMS[i]] = p[:, i]
        want[:, 4 + ARMS[i]] = -p[:, 4 + i]
        want[:, 8 + ARMS[i]] = p[:, 8 + i]
    want[:, 12:] = p[:, 12:]
    err = np.abs(q - want).max(axis=1)
    assert np.all(err <= 1e-4), f"envs {np.argwhere(err > 1e-4).ravel()[:5]} err {err.max()}"
    # the states span the laws: some throttles, gimbals and torques non-trivial
    assert np.std(p[:, 0]) > 0.1 and np.std(p[:, 8]) > 0.05 and np.std(p[:, 4]) > 0.05


def test_mirror_symmetry_bwb_modes():
    obs, mis = random_states(128, 12, BWB_MODES)
    obs[:, 3] = np.abs(obs[:, 3]) * 5 + 14     # flying forward at 14..29 m/s
    obs[:, 44] = np.random.default_rng(3).uniform(-0.4, 0.4, 128)
    mo, mm = zip(*(mirror(o, m) for o, m in zip(obs, mis)))
    mo = np.array(mo)
    mo[:, 44] = -obs[:, 44]                    # cannon azimuth is a y-odd angle here
    _, p, _ = oracle.onboard(obs, mis)
    _, q, _ = oracle.onboard(mo, np.array(mm))
    want = p.copy()
    want[:, [0, 2]] = p[:, [1, 3]]
    want[:, [1, 3]] = p[:, [0, 2]]
    want[:, 9] = -p[:, 9]
    want[:, 12] = -p[:, 12]
    err = np.abs(q - want).max(axis=1)
    assert np.all(err <= 1e-4), f"envs {np.argwhere(err > 1e-4).ravel()[:5]} err {err.max()}"
    assert np.all(p[:, 4:8] == 0.0) and np.all(p[:, 10:12] == 0.0)
    assert np.all(p[:, 0] == p[:, 2]) and np.all(p[:, 1] == p[:, 3])
    assert np.std(p[:, 0] - p[:, 1]) > 0.05


# ---------------------------------------------------------------- tactical
def rotation(q):
    """Rotation matrix (body -> world) of the unit quaternion (w, x, y, z)."""
    w, x, y, z = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def tactical_by_matrices(o, m):
    """tb_onboard_tactical (onboard_features.cuh:25-86) in another
    formulation: frames as rotation matrices, the goal and the cannon aim
    expressed in the heading and body frames by matrix products, the arm
    terms as vector sums."""
    o = o.astype(np.float64)
    m = m.astype(np.float64)
    s = np.clip(o[16:20], 0.0, 1.0)
    thrust = 0.036 + 0.964 * s
    lift = thrust * o[24:28] * np.cos(o[28:32])     # cos(outer) cos(inner)
    side = thrust * o[20:24] * np.cos(o[28:32])     # sin(outer) cos(inner)
    t = np.zeros(24)
    t[0], t[1] = lift[1] - lift[3], lift[2] - lift[0]
    t[2], t[3] = 0.5 * side.sum(), lift.mean() - 0.5
    t[4:8] = 2.0 * (s - s.mean())
    R = rotation(o[6:10])
    yaw = math.atan2(R[1, 0], R[0, 0])
    heading = np.array([[math.cos(yaw), math.sin(yaw)], [-math.sin(yaw), math.cos(yaw)]])
    bz = heading @ R[:2, 2]                         # body z in the heading frame
    t[8], t[9] = bz[1], -bz[0]
    ct = clamp(R[2, 2], -1.0, 1.0)
    t[10], t[11] = ct, float(ct < 0.20)
    r = np.arctanh(np.clip(m[7:10], -0.995, 0.995)) * 20.0
    rh, vh = heading @ r[:2], heading @ o[3:5]
    t[12], t[13] = math.tanh(rh[0] * 0.08), math.tanh(rh[1] * 0.08)
    t[14], t[15] = math.tanh(r[2] * 0.12), math.tanh(math.hypot(r[0], r[1]) * 0.05)
    t[16], t[17] = math.tanh(vh[0] * 0.15), math.tanh(vh[1] * 0.15)
    t[18] = math.exp(-max(o[2] - 0.62, 0.0))
    dist = max(float(np.linalg.norm(r)), 1.0)
    fl = dist / 20.0
    w = r - o[3:6] * 0.5 * fl + np.array([0.0, 0.0, 0.5 * G * fl * fl])
    b = R.T @ w                                    # world -> body
    az = clamp(math.atan2(b[1], b[0]), PI / 12, 5 * PI / 12)
    el = clamp(math.atan2(b[2], max(math.hypot(b[0], b[1]), 0.2)), -PI / 6, PI / 6)
    err = math.hypot(az - o[44], el - o[45])
    t[19], t[20], t[21] = (az - PI / 4) / (PI / 6), el / (PI / 6), math.tanh(2.0 * err)
    t[22] = 1.0 if (o[46] <= 0.02 and o[47] > 0.01 and err < 0.26 and dist < 34.0) else -1.0
    t[23] = math.sin(math.atan2(r[1], r[0]) - PI / 4 - yaw)
    margins = (abs(ct - 0.20), abs(err - 0.26), abs(dist - 34.0))
    return t, (az, el), min(margins)


def test_tactical_matches_rotation_matrix_formulation():
    rng = np.random.default_rng(23)
    n = 512
    obs = np.zeros((n, 4148), np.float32)
    mis = np.zeros((n, 10), np.float32)
    for e in range(n):
        o = obs[e]
        o[0:6] = rng.uniform(-5, 5, 6)
        o[2] = rng.uniform(0.0, 3.0)                 # ground proximity term active
        q = rng.normal(0, 1, 4) if e % 2 else np.r_[1.0, rng.normal(0, 0.3, 3)]
        o[6:10] = q / np.linalg.norm(q)
        o[16:20] = rng.uniform(-0.2, 1.2, 4)
        outer = rng.uniform(-1.0, 1.0, 4)
        o[20:24], o[24:28] = np.sin(outer), np.cos(outer)
        o[28:32] = rng.uniform(-0.6, 0.6, 4)
        o[46], o[47] = rng.choice([0.0, 0.05]), rng.choice([0.0, 1.0])
        mis[e, 7:10] = rng.uniform(-1.0, 1.0, 3)    # past the 0.995 clamp at times
        _, (az, el), _ = tactical_by_matrices(o, mis[e])
        o[44], o[45] = az + rng.uniform(-0.3, 0.3), el + rng.uniform(-0.3, 0.3)
    tac, _, _ = oracle.onboard(obs, mis)
    fired = 0
    for e in range(n):
        want, _, margin = tactical_by_matrices(obs[e], mis[e])
        if margin < 1e-4:
            continue                                  # a threshold within rounding
        err = np.abs(tac[e] - want)
        assert err.max() <= TOL, f"env {e}: index {err.argmax()} got {tac[e][err.argmax()]} " \
                                 f"want {want[err.argmax()]}"
        fired += want[22] > 0
    assert fired > 20 and (tac[:, 11] == 1.0).sum() > 20
