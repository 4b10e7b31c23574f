"""The onboard kernels round atan2 near +-pi correctly (ob_atan2 in
turbinator_c_amd/csrc/onboard.hip): there the result's side of pi decides the
controller's angle wraps, and the single-precision device routine can be one
ulp off.  tests/csrc/check_atan2_near_pi.c (~5 s) checks the closed form
sign(y) (pi - |y / x|) against the double-precision atan2 and the host atan2f
that the oracle uses."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent


def test_near_pi_closed_form(tmp_path):
    exe = tmp_path / "check_atan2"
    subprocess.run(["gcc", "-O2", "-std=c11", "-o", str(exe),
                    str(HERE / "csrc" / "check_atan2_near_pi.c"), "-lm"], check=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout
    # "<n> checked, <a> differ from double atan2, <b> from atan2f"
    words = proc.stdout.split()
    assert int(words[0]) > 100_000_000, proc.stdout
    assert words[2] == "0" and words[7] == "0", proc.stdout
