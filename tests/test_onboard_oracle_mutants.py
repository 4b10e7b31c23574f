"""Mutation check of the onboard tactical / prior oracle's pins (CPU only).

The oracle (oracle/onboard_oracle.c) restates tb_onboard_tactical and
tb_onboard_prior (src/network/onboard_features.cuh:25-513 of the reference),
and the GPU kernels are compared with it.  Its pins are the reference's 40
goldens and the closed forms, invariants and second formulations of
tests/test_onboard_prior_pins.py and tests/test_onboard_oracle.py.  This test
shows that those pins would catch a restatement mistake: each entry of
MUTANTS plants one plausible mistake (an altered or swapped constant, a
flipped sign, a transposed row or arm, a moved threshold) in a copy of the
source, builds it into a library of its own, and runs both pin files against
it (oracle/__init__.py loads the library TB_ORACLE_LIB names).  Every mutant
must make them fail, except those listed in UNREACHABLE with the reason no
input reaches the changed code.

The constants of the second group sit behind a clamp further down the law at
ordinary states (the 52 N heavy-cargo force cap, the -1.8 vertical floor, a
level attitude where the tilt term vanishes); the pins hold them at states
where each one binds.
"""
from __future__ import annotations

import math
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
ORACLE = ROOT / "oracle"
SOURCE = ORACLE / "onboard_oracle.c"
PIN_FILES = ["tests/test_onboard_prior_pins.py", "tests/test_onboard_oracle.py"]

# (name, text in onboard_oracle.c, replacement); the line cited is the
# reference line the text restates (src/network/onboard_features.cuh).
MUTANTS = [
    # tactical features (:25-86)
    ("t1 arms swapped", "t[1] = fz[2] - fz[0];", "t[1] = fz[0] - fz[2];"),
    ("t2 half torque", "t[2] = 0.5f * tau_z;", "t[2] = 0.25f * tau_z;"),
    ("t4 spool mean", "t[4 + i] = 2.0f * (spool[i] - spool_mean);",
     "t[4 + i] = 2.0f * (spool[i] - 0.5f);"),
    ("tactical thrust law", "const float thrust = 0.036f + 0.964f * spool[i];",
     "const float thrust = 0.04f + 0.96f * spool[i];"),
    ("t9 sign", "t[9] = -sy * bz_y - cy * bz_x;", "t[9] = -sy * bz_y + cy * bz_x;"),
    ("t11 threshold", "t[11] = ct < 0.20f ? 1.0f : 0.0f;", "t[11] = ct < 0.25f ? 1.0f : 0.0f;"),
    ("t14 gain", "t[14] = tanhf(rz * 0.12f);", "t[14] = tanhf(rz * 0.10f);"),
    ("t17 sign", "t[17] = tanhf((-sy * o[3] + cy * o[4]) * 0.15f);",
     "t[17] = tanhf((sy * o[3] + cy * o[4]) * 0.15f);"),
    ("t18 ground height", "t[18] = expf(-fmaxf(o[2] - 0.62f, 0.0f));",
     "t[18] = expf(-fmaxf(o[2] - 0.60f, 0.0f));"),
    ("t22 aim error", "err < 0.26f && dist < 34.0f) ? 1.0f : -1.0f;",
     "err < 0.30f && dist < 34.0f) ? 1.0f : -1.0f;"),
    ("tactical gravity drop", "+ 0.5f * 9.80665f * flight * flight;",
     "+ 0.53f * 9.80665f * flight * flight;"),
    ("tactical azimuth clamp", "ob_clamp(atan2f(by, bx), pi / 12.0f, pi * 5.0f / 12.0f);",
     "ob_clamp(atan2f(by, bx), pi / 12.0f, pi * 4.0f / 12.0f);"),
    ("tactical atanh clamp", "const float rx = atanhf(ob_clamp(m[7], -0.995f, 0.995f)) * 20.0f;",
     "const float rx = atanhf(ob_clamp(m[7], -0.9995f, 0.9995f)) * 20.0f;"),
    # attitude, mass, targets (:105-183)
    ("rotation r12 sign", "1.0f - 2.0f * (qx * qx + qz * qz), 2.0f * (qy * qz - qw * qx),",
     "1.0f - 2.0f * (qx * qx + qz * qz), 2.0f * (qy * qz + qw * qx),"),
    ("ammo mass clamp", "const float ammo_mass = ob_clamp(o[47], 0.0f, 4.0f) * 6.0f;",
     "const float ammo_mass = ob_clamp(o[47], 0.0f, 5.0f) * 6.0f;"),
    ("arena stand-off range", "const float desired_range = intercept ? 8.5f : 12.5f;",
     "const float desired_range = intercept ? 8.5f : 12.0f;"),
    # LiDAR-driven targets (:208-252)
    ("dodge magnitude", "avoid_x = -sinf(min_az) * 2.2f;", "avoid_x = -sinf(min_az) * 2.0f;"),
    ("dodge sign", "avoid_y = cosf(min_az) * 2.2f;", "avoid_y = -cosf(min_az) * 2.2f;"),
    ("dodge range", "if (dodge && scan.min_r < 7.5f) {", "if (dodge && scan.min_r < 8.5f) {"),
    ("slalom lane side", "ey = cluster_y >= 0.0f ? -1.85f : 1.85f;",
     "ey = cluster_y >= 0.0f ? 1.85f : -1.85f;"),
    ("slalom speed 2.75", "float speed_limit = lane_err > 0.55f ? 2.75f : 4.10f;",
     "float speed_limit = lane_err > 0.55f ? 2.5f : 4.10f;"),
    ("slalom open-course x", "if (min_dx_c >= 6.6f && px > 4.0f) speed_limit = 3.10f;",
     "if (min_dx_c >= 6.6f && px > 5.0f) speed_limit = 3.10f;"),
    ("slalom hill height", "ez = 2.5f * sinf(pi * hill) + 8.0f;",
     "ez = 2.5f * sinf(pi * hill) + 8.5f;"),
    # landing and cargo law (:254-283)
    ("landing gains swapped", "const float kp_land = heavy_cargo ? 0.75f : 1.05f;",
     "const float kp_land = heavy_cargo ? 1.05f : 0.75f;"),
    ("landing mid-height cap", "const float low_cap = above_pad < 1.2f ? 0.55f : "
     "(heavy_cargo ? 1.25f : 1.6f);",
     "const float low_cap = above_pad < 1.2f ? 0.55f : (heavy_cargo ? 1.25f : 1.5f);"),
    ("cargo descent pad height", "ob_clamp(1.6f * (0.64f - pz), -0.30f, 0.18f);",
     "ob_clamp(1.6f * (0.66f - pz), -0.30f, 0.18f);"),
    ("landing descent cap", "const float max_desc = cargo ? -0.82f : -1.4f;",
     "const float max_desc = cargo ? -0.82f : -1.5f;"),
    ("landing align cap", "ob_clamp(1.2f * (pad_z + 0.90f - pz), -0.30f, 0.60f);",
     "ob_clamp(1.2f * (pad_z + 0.90f - pz), -0.30f, 0.65f);"),
    ("cargo transit height", "fmaxf(1.2f + 0.28f * up_horiz, 2.0f) : 2.0f;",
     "fmaxf(1.2f + 0.26f * up_horiz, 2.0f) : 2.0f;"),
    ("transit sink caps swapped", "const float max_desc_trans = heavy_cargo ? -1.05f : -1.6f;",
     "const float max_desc_trans = heavy_cargo ? -1.6f : -1.05f;"),
    ("landing vertical gain", "const float kp_az_land = heavy_cargo ? 5.0f : 4.5f;",
     "const float kp_az_land = heavy_cargo ? 5.0f : 4.0f;"),
    ("land-idle thrust", "target_thrust = 0.15f * weight * 0.25f;",
     "target_thrust = 0.16f * weight * 0.25f;"),
    ("land-idle height", "pz <= 0.638f", "pz <= 0.6f"),
    # standard law, collective and torques (:285-393)
    ("lateral threshold on x", "const float lat_vx = fabsf(upy) > 1.35f ? 1.45f : 3.8f;",
     "const float lat_vx = fabsf(upx) > 1.35f ? 1.45f : 3.8f;"),
    ("lateral y gain", "(lateral ? 1.05f : kp_xy);", "(lateral ? 0.95f : kp_xy);"),
    ("inversion far cap", "&& ct > 0.90f ? 6.2f : 4.2f;", "&& ct > 0.90f ? 6.0f : 4.2f;"),
    ("parasite torque sign", "const float tau_y_par = 0.1625f * fx_body * parasite_scale;",
     "const float tau_y_par = -0.1625f * fx_body * parasite_scale;"),
    ("turbine-out parasite", "const float parasite_scale = turbine_out ? 0.35f : 1.0f;",
     "const float parasite_scale = turbine_out ? 0.45f : 1.0f;"),
    ("yaw rate gain", "ob_clamp(22.0f * yaw_err - 18.0f * oz, -70.0f, 70.0f);",
     "ob_clamp(22.0f * yaw_err - 16.0f * oz, -70.0f, 70.0f);"),
    ("arm 1 torque sign", "        0.25f * fz_des + tau_x_cmd * 0.5f,\n",
     "        0.25f * fz_des - tau_x_cmd * 0.5f,\n"),
    ("arm y unit swapped", "const float ury = i == 1 ? 1.0f : (i == 3 ? -1.0f : 0.0f);",
     "const float ury = i == 3 ? 1.0f : (i == 1 ? -1.0f : 0.0f);"),
    ("turbine-out spool gain", "const float spool_gain = turbine_out ? 10.5f :",
     "const float spool_gain = turbine_out ? 10.0f :"),
    ("headroom excess cap", "urgent_climb ? 0.10f : 0.45f);", "urgent_climb ? 0.10f : 0.35f);"),
    ("inner gimbal lower clamp", "-inner_limit * 0.90f, inner_limit * 0.90f);",
     "-inner_limit * 0.80f, inner_limit * 0.90f);"),
    # inverted recovery (:394-405)
    ("recovery arm moments", "const float arm_mom[4] = {-ty_inv, tx_inv, ty_inv, -tx_inv};",
     "const float arm_mom[4] = {ty_inv, tx_inv, -ty_inv, -tx_inv};"),
    ("recovery rate gain", "const float tx_inv = 130.0f * inv_rx - 52.0f * ox;",
     "const float tx_inv = 130.0f * inv_rx - 50.0f * ox;"),
    ("recovery threshold", "throttle[i] = arm_mom[i] > 12.0f ? 0.58f : 0.0f;",
     "throttle[i] = arm_mom[i] > 10.0f ? 0.58f : 0.0f;"),
    ("recovery outer sign", "outer_cmd[i] = ob_clamp(-outer[i] * 6.0f, -outer_limit, outer_limit);",
     "outer_cmd[i] = ob_clamp(outer[i] * 6.0f, -outer_limit, outer_limit);"),
    # cannon (:407-431)
    ("cannon fire range", "aim_err < 0.28f && dist < 34.0f;", "aim_err < 0.28f && dist < 20.0f;"),
    # BWB (:432-503)
    ("BWB body sideslip row", "const float vb_y = r01 * vx + r11 * vy + r21 * vz;",
     "const float vb_y = r10 * vx + r11 * vy + r21 * vz;"),
    ("BWB endurance speed", "const float desired_speed = bwb_endurance ? 18.5f :",
     "const float desired_speed = bwb_endurance ? 19.5f :"),
    ("BWB speed gain", "0.065f * speed_err", "0.06f * speed_err"),
    ("BWB roll-rate sign", "0.90f * (desired_roll - roll_right) - 0.34f * ox,",
     "0.90f * (desired_roll - roll_right) + 0.34f * ox,"),
    ("BWB slow pitch cap", "desired_pitch = fminf(desired_pitch, 0.02f);",
     "desired_pitch = fminf(desired_pitch, 0.03f);"),
    ("BWB yaw gimbal rate sign", "ob_clamp(-0.65f * (r_left - oz) - 0.025f * vb_y,",
     "ob_clamp(-0.65f * (r_left + oz) - 0.025f * vb_y,"),
    ("BWB fire error", "b_err < 0.045f", "b_err < 0.09f"),
    # constants behind downstream clamps at ordinary states
    ("heavy transit speed cap (:257)", "const float transit_cap = heavy_cargo ? 2.65f : 3.4f;",
     "const float transit_cap = heavy_cargo ? 3.4f : 3.4f;"),
    ("cargo climb clamp (:264)", "ob_clamp(1.6f * (0.64f - pz), -0.30f, 0.18f);",
     "ob_clamp(1.6f * (0.64f - pz), -0.30f, 0.28f);"),
    ("heavy transit sink cap (:270)", "heavy_cargo ? -1.05f : -1.6f;",
     "heavy_cargo ? -1.6f : -1.6f;"),
    ("heavy acceleration cap (:276)", "const float max_axy_land = heavy_cargo ? 2.2f : 2.6f;",
     "const float max_axy_land = heavy_cargo ? 2.6f : 2.6f;"),
    ("lateral threshold (:287)", "fabsf(upy) > 1.35f ? 1.45f : 3.8f;",
     "fabsf(upy) > 1.45f ? 1.45f : 3.8f;"),
    ("headroom tilt threshold (:320)", "1.5f * fmaxf(tilt - 0.15f, 0.0f)",
     "1.5f * fmaxf(tilt - 0.20f, 0.0f)"),
    ("BWB turn-rate speed floor (:475)", "(gravity / fmaxf(vb_x, 12.0f))",
     "(gravity / fmaxf(vb_x, 10.0f))"),
]

# Mutants no input reaches, with the reason.
UNREACHABLE = {
    # sin_in is clamped to at most 0.44 in magnitude before the asin, and
    # asin(0.44) = 0.456 < 0.8 * pi/4 = 0.628: neither clamp bound can bind.
    "inner gimbal lower clamp",
}


def _build(src_text: str, out_dir: Path) -> Path:
    (out_dir / "onboard_oracle.c").write_text(src_text)
    others = [str(p) for p in sorted(ORACLE.glob("*_oracle.c")) if p.name != SOURCE.name]
    lib = out_dir / "liboracle.so"
    subprocess.run(["gcc", "-O3", "-std=c11", "-fPIC", "-shared", "-D_POSIX_C_SOURCE=200809L",
                    f"-I{ORACLE}", "-o", str(lib), str(out_dir / "onboard_oracle.c"), *others,
                    "-lm", "-lpthread"], check=True, capture_output=True)
    return lib


def _pins_fail(lib: Path) -> tuple[int, str]:
    env = dict(os.environ, TB_ORACLE_LIB=str(lib))
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        *PIN_FILES], cwd=ROOT, env=env, capture_output=True, text=True)
    failed = next((l for l in r.stdout.splitlines() if l.startswith("FAILED")), "")
    return r.returncode, failed


def _run(text: str) -> tuple[int, str]:
    with tempfile.TemporaryDirectory(prefix="tb_mutant_") as d:
        return _pins_fail(_build(text, Path(d)))


@pytest.fixture(scope="module")
def source() -> str:
    if shutil.which("gcc") is None:
        pytest.skip("gcc is needed to build the mutants")
    return SOURCE.read_text()


def test_every_mutant_applies_once(source):
    for name, old, new in MUTANTS:
        assert source.count(old) == 1, f"{name}: text found {source.count(old)} times"
        assert old != new, name
    assert len({m[0] for m in MUTANTS}) == len(MUTANTS)
    assert UNREACHABLE <= {m[0] for m in MUTANTS}


def test_unreachable_reason_holds():
    assert math.asin(0.44) < 0.8 * math.pi / 4


def test_pins_catch_every_reachable_mutant(source):
    # the unmodified source, built the same way, passes the pins
    rc, failed = _run(source)
    assert rc == 0, f"faithful oracle fails its pins: {failed}"
    jobs = [(name, source.replace(old, new, 1)) for name, old, new in MUTANTS]
    with ThreadPoolExecutor(max_workers=max(1, min(8, os.cpu_count() or 1))) as pool:
        results = list(pool.map(lambda job: (job[0], *_run(job[1])), jobs))
    missed = [name for name, rc, _ in results if rc == 0 and name not in UNREACHABLE]
    broken = [(name, rc) for name, rc, _ in results if rc not in (0, 1)]
    assert not broken, f"pin run errored instead of failing: {broken}"
    assert not missed, f"mutants no pin catches: {missed}"
