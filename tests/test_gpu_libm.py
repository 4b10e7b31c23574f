"""Device-library identities the kernels rely on, checked on the GPU.

* sincosf(x) returns the same bits as sinf(x) and cosf(x) for every float
  (tests/csrc/check_sincos.hip, all 2^32 inputs): the onboard controller
  evaluates each sine/cosine pair of one angle through sincosf, so its
  results equal those of the separate calls the reference makes
  (onboard_features.cuh:18,49,119-120,210-211,325,469).
* (float)atan2((double)y, (double)x), the controller's atan2 for the angles
  that reach its angle wraps, is correctly rounded on 8.4e6 arguments, and
  equals the host libm's atan2f (the oracle's) on the arguments that reach
  the wraps' discontinuity exactly: equal, opposite and zero components and
  results near +-pi (tests/csrc/check_atan2.hip).
* One v_mfma_f32_16x16x32_f16 instruction drops the bits of a product that
  lie more than 2^-24 below the largest product of its group (one lane's
  eight k values) before it rounds the sum, and over random blocks its error
  stays within a few u sum|p| (tests/csrc/check_mfma_sum.hip): the compact
  actor's error analysis and its conditioned parity bound rest on this.
* recip_range(y), the hardware reciprocal refined by one Newton step, is
  the IEEE quotient 1.0f / y for every float y in [0.2, 30]
  (tests/csrc/check_recip.hip, all 61,027,124 of them): the 618M actor's
  inverse-range channel (network_gpu.cu:467-479) divides by a value in that
  range, so its bits equal the reference's correctly rounded division.
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


@pytest.mark.gpu
def test_wrap_angles_match_the_host_atan2f():
    exe = BIN / "check_atan2"
    if not exe.exists():
        pytest.fail(f"{exe} is not built (run __graft_entry__.build())")
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    # "<n> checked, <a> differ from double atan2, <m> exact-angle arguments,
    #  <b> differ from atan2f, <c> other arguments differ from atan2f"
    words = proc.stdout.split("\n")[-2].split()
    assert int(words[0]) > 8_000_000 and words[2] == "0", proc.stdout
    assert int(words[7]) > 2_000_000 and words[10] == "0", proc.stdout


@pytest.mark.gpu
def test_mfma_block_sum_drops_low_product_bits():
    exe = BIN / "check_mfma_sum"
    if not exe.exists():
        pytest.fail(f"{exe} is not built (run __graft_entry__.build())")
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    w = proc.stdout.split()
    smallest, across, half = int(w[0]), int(w[2]), int(w[4])
    truncated, above, outputs = int(w[6]), int(w[8]), int(w[10])
    worst, mean = float(w[13]), float(w[15])
    # beside +2^20 - 2^20 in one group 2^-4 = 2^(20 - 24) survives, 2^-5 does not
    assert smallest == -4, proc.stdout
    # in other lanes' k values the small product always survives; in the other
    # half of the same lane's eight it is dropped like in the first half
    assert across == 16 and half == 13, proc.stdout
    # not the correctly rounded sum: some results lie below the nearest float
    assert truncated > 0 and above > 0, proc.stdout
    assert outputs == 262144 and worst <= 6.0 and mean <= 1.0, proc.stdout


@pytest.mark.gpu
def test_range_reciprocal_is_the_ieee_quotient():
    exe = BIN / "check_recip"
    if not exe.exists():
        pytest.fail(f"{exe} is not built (run __graft_entry__.build())")
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    w = proc.stdout.split()
    assert int(w[0]) == 0x41F00000 - 0x3E4CCCCD + 1, proc.stdout
    assert w[2] == "0" and w[8] == "0", proc.stdout
