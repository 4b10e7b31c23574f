"""The CMake integration a maintainer adds to the reference tree builds.

A throwaway CMake project (written to a temp dir) adds turbinator_c_amd/ with
add_subdirectory, as a maintainer would add it to the reference's
CMakeLists.txt, and links the reference's own tests/test_cuda_features.c and
src/training/training.c (compiled from /root/reference, which exists only in
the build container) against the turbinator_hip target.  Nothing is run: the
GPU run of the same sources is tests/test_gpu_features.py's drop-in test.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF = Path("/root/reference")

PROJECT = """
cmake_minimum_required(VERSION 3.21)
project(turbinator_dropin LANGUAGES C)
option(TURBINATOR_ENABLE_HIP "Build the gfx950 HIP feature kernels" ON)
if(TURBINATOR_ENABLE_HIP)
  add_subdirectory({pkg} turbinator_hip)
endif()
add_executable(cuda_feature_batch_dropin {ref}/tests/test_cuda_features.c
                                         {ref}/src/training/training.c)
set_target_properties(cuda_feature_batch_dropin PROPERTIES C_STANDARD 11 C_EXTENSIONS OFF)
target_include_directories(cuda_feature_batch_dropin PRIVATE {ref}/include)
target_link_libraries(cuda_feature_batch_dropin PRIVATE turbinator_hip m)
"""


@pytest.mark.skipif(not (REF / "tests" / "test_cuda_features.c").exists(),
                    reason="reference tree absent (GPU box)")
@pytest.mark.skipif(shutil.which("cmake") is None, reason="cmake not installed")
def test_reference_test_links_through_cmake(tmp_path):
    src = tmp_path / "src"
    src.mkdir()
    (src / "CMakeLists.txt").write_text(PROJECT.format(pkg=ROOT / "turbinator_c_amd", ref=REF))
    build = tmp_path / "build"
    cfg = subprocess.run(["cmake", "-S", str(src), "-B", str(build),
                          "-DCMAKE_HIP_COMPILER=/opt/rocm/llvm/bin/clang++",
                          "-DCMAKE_PREFIX_PATH=/opt/rocm"],
                         capture_output=True, text=True, timeout=300)
    assert cfg.returncode == 0, cfg.stdout + cfg.stderr
    bld = subprocess.run(["cmake", "--build", str(build), "-j8"], capture_output=True,
                         text=True, timeout=900)
    assert bld.returncode == 0, bld.stdout[-4000:] + bld.stderr[-4000:]
    exe = build / "cuda_feature_batch_dropin"
    assert exe.exists()
    syms = subprocess.run(["nm", str(exe)], capture_output=True, text=True).stdout
    for name in ("tb_cuda_feature_batch_create", "tb_cuda_extract_features_host",
                 "tb_cuda_extract_features_device", "tb_train_extract_features_cpu"):
        assert f" T {name}" in syms, name
