"""Builds the gfx950 feature library and the host helpers in-tree.

Outputs (git-ignored, shipped with the working tree):
  turbinator_c_amd/libturbinator_hip.so    HIP kernels + the C-ABI boundary
  turbinator_c_amd/libturbinator_synth.so  seeded synthetic batch generator
  oracle/liboracle.so, oracle/_ref/...     CPU checker (test infrastructure)

Run as ``python -m turbinator_c_amd.build``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = ROOT / "_build"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    f"-I{INCLUDE}",
]
C_FLAGS = ["-O2", "-std=c11", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROCM / 'include'}", f"-I{INCLUDE}"]

HIP_SOURCES = ["features.hip", "onboard.hip", "sac_actor.hip"]
HOST_C_SOURCES = ["feature_batch.c", "feature_pipeline.c", "sac_host.c"]

LIB_HIP = PKG / "libturbinator_hip.so"
LIB_SYNTH = PKG / "libturbinator_synth.so"


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def hipcc() -> str:
    exe = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the gfx950 library cannot be built")
    return exe


def generate_ray_table() -> Path:
    """onboard_rays.inc: ray directions evaluated with the host libm (no
    optimisation, so no compile-time folding replaces the libm calls)."""
    BUILD.mkdir(exist_ok=True)
    exe = BUILD / "gen_ray_table"
    _run(["gcc", "-O0", "-std=c11", "-fno-builtin", "-ffp-contract=off", "-o", str(exe),
          str(CSRC / "gen_ray_table.c"), "-lm"])
    inc = BUILD / "onboard_rays.inc"
    text = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    inc.write_text(text)
    return inc


def build_hip_library() -> Path:
    BUILD.mkdir(exist_ok=True)
    generate_ray_table()
    objs = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".hip.o")
        _run([hipcc(), *HIP_FLAGS, f"-I{BUILD}", "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    for src in HOST_C_SOURCES:
        obj = BUILD / (Path(src).stem + ".c.o")
        _run(["gcc", *C_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(obj)
    tmp = LIB_HIP.with_suffix(".so.tmp")
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs), f"-L{ROCM / 'lib'}", "-lamdhip64",
          f"-Wl,-rpath,{ROCM / 'lib'}"])
    os.replace(tmp, LIB_HIP)
    return LIB_HIP


def build_synth_library() -> Path:
    tmp = LIB_SYNTH.with_suffix(".so.tmp")
    _run(["gcc", "-O3", "-std=c11", "-fPIC", "-shared", "-Wall", "-Wextra",
          "-D_POSIX_C_SOURCE=200809L", "-o", str(tmp), str(CSRC / "synth.c"), "-lm", "-lpthread"])
    os.replace(tmp, LIB_SYNTH)
    return LIB_SYNTH


def build_oracle() -> None:
    _run(["make", "-s", "-C", str(ROOT / "oracle"), "all"])


GPU_CHECKS = ROOT / "tests" / "csrc"
GPU_CHECK_BIN = GPU_CHECKS / "bin"


def build_gpu_checks() -> None:
    """Stand-alone gfx950 probes the GPU tests run (tests/csrc/*.hip)."""
    GPU_CHECK_BIN.mkdir(exist_ok=True)
    for src in sorted(GPU_CHECKS.glob("*.hip")):
        exe = GPU_CHECK_BIN / src.stem
        _run([hipcc(), *HIP_FLAGS, "-o", str(exe), str(src)])


def build_all() -> None:
    build_synth_library()
    build_oracle()
    build_hip_library()
    build_gpu_checks()


if __name__ == "__main__":
    build_all()
    print("built", LIB_HIP, LIB_SYNTH, file=sys.stderr)
