"""Device-library identities the kernels rely on, checked on the GPU.

* sincosf(x) returns the same bits as sinf(x) and cosf(x) for every float
  (tests/csrc/check_sincos.hip, all 2^32 inputs): the onboard controller
  evaluates each sine/cosine pair of one angle through sincosf, so its
  results equal those of the separate calls the reference makes
  (onboard_features.cuh:18,49,119-120,210-211,325,469).
"""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parent / "csrc" / "bin"


@pytest.mark.gpu
def test_sincos_matches_separate_calls_for_every_float():
    exe = BIN / "check_sincos"
    if not exe.exists():
        pytest.fail(f"{exe} is not built (run __graft_entry__.build())")
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.startswith("0 mismatches"), proc.stdout
