"""The CMake integration a maintainer adds to the reference tree builds.

A throwaway CMake project (written to a temp dir) adds turbinator_c_amd/ with
add_subdirectory, as a maintainer would add it to the reference's
CMakeLists.txt, and builds two reference targets from /root/reference (which
exists only in the build container) against the turbinator_hip target in
place of turbinator_cuda:

* the reference's own parity test, tests/test_cuda_features.c with
  src/training/training.c (the GPU run of the same sources is
  tests/test_gpu_features.py's drop-in test);
* the production caller, turbinator_trainer, laid out as the reference's
  CMakeLists.txt:46-138 lays it out: the turbinator_sim shared library
  (src/sim/physics.c, sensors.c, c_api.c and src/trainer/tui.c), the
  turbinator_training and turbinator_network static libraries, and
  src/trainer/main.c + http.c.  Its CUDA feature engine (main.c:483-713)
  compiles only when TURBINATOR_HAS_CUDA is defined, and here that
  definition reaches main.c from turbinator_hip's PUBLIC compile
  definitions alone, as it reaches it from turbinator_cuda in the reference
  (CMakeLists.txt:66).

Nothing is run.
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
set(CMAKE_C_STANDARD 11)
set(CMAKE_C_STANDARD_REQUIRED ON)
set(CMAKE_C_EXTENSIONS OFF)
set(CMAKE_POSITION_INDEPENDENT_CODE ON)
option(TURBINATOR_ENABLE_HIP "Build the gfx950 HIP feature kernels" ON)
if(TURBINATOR_ENABLE_HIP)
  add_subdirectory({pkg} turbinator_hip)
endif()

add_executable(cuda_feature_batch_dropin {ref}/tests/test_cuda_features.c
                                         {ref}/src/training/training.c)
target_include_directories(cuda_feature_batch_dropin PRIVATE {ref}/include)
target_link_libraries(cuda_feature_batch_dropin PRIVATE turbinator_hip m)

add_library(turbinator_sim SHARED {ref}/src/sim/physics.c {ref}/src/sim/sensors.c
                                  {ref}/src/sim/c_api.c {ref}/src/trainer/tui.c)
target_include_directories(turbinator_sim PUBLIC {ref}/include)
target_compile_definitions(turbinator_sim PRIVATE TURBINATOR_SIM_BUILD)
target_link_libraries(turbinator_sim PRIVATE m)
add_library(turbinator_training STATIC {ref}/src/training/training.c)
target_include_directories(turbinator_training PUBLIC {ref}/include)
target_link_libraries(turbinator_training PUBLIC m)
add_library(turbinator_network STATIC {ref}/src/network/network.c)
target_include_directories(turbinator_network PUBLIC {ref}/include)
target_link_libraries(turbinator_network PUBLIC m)
add_executable(turbinator_trainer {ref}/src/trainer/main.c {ref}/src/trainer/http.c)
target_include_directories(turbinator_trainer PRIVATE {ref}/include)
target_link_libraries(turbinator_trainer PRIVATE turbinator_sim turbinator_training
                      turbinator_network)
if(TURBINATOR_ENABLE_HIP)
  target_link_libraries(turbinator_trainer PRIVATE turbinator_hip)
endif()
"""

# The host-object entry points the trainer's CUDA feature engine calls
# (main.c:513,526,528,566,568,618,620,673,676,706,712).
TRAINER_IMPORTS = ("tb_cuda_feature_batch_create", "tb_cuda_extract_features_host",
                   "tb_cuda_feature_batch_error", "tb_cuda_feature_batch_destroy")

needs_reference = pytest.mark.skipif(
    not (REF / "tests" / "test_cuda_features.c").exists()
    or not (REF / "src" / "trainer" / "main.c").exists(),
    reason="reference tree absent (GPU box)")
needs_cmake = pytest.mark.skipif(shutil.which("cmake") is None, reason="cmake not installed")


def _symbols(path: Path, *flags: str) -> str:
    return subprocess.run(["nm", *flags, str(path)], capture_output=True, text=True,
                          check=True).stdout


@pytest.fixture(scope="module")
def build(tmp_path_factory) -> Path:
    tmp = tmp_path_factory.mktemp("cmake_dropin")
    src = tmp / "src"
    src.mkdir()
    (src / "CMakeLists.txt").write_text(PROJECT.format(pkg=ROOT / "turbinator_c_amd", ref=REF))
    out = tmp / "build"
    cfg = subprocess.run(["cmake", "-S", str(src), "-B", str(out),
                          "-DCMAKE_HIP_COMPILER=/opt/rocm/llvm/bin/clang++",
                          "-DCMAKE_PREFIX_PATH=/opt/rocm"],
                         capture_output=True, text=True, timeout=300)
    assert cfg.returncode == 0, cfg.stdout + cfg.stderr
    bld = subprocess.run(["cmake", "--build", str(out), "-j8"], capture_output=True,
                         text=True, timeout=900)
    assert bld.returncode == 0, bld.stdout[-4000:] + bld.stderr[-4000:]
    return out


@needs_reference
@needs_cmake
def test_reference_test_links_through_cmake(build):
    exe = build / "cuda_feature_batch_dropin"
    assert exe.exists()
    syms = _symbols(exe)
    for name in ("tb_cuda_feature_batch_create", "tb_cuda_extract_features_host",
                 "tb_cuda_extract_features_device", "tb_train_extract_features_cpu"):
        assert f" T {name}" in syms, name


@needs_reference
@needs_cmake
def test_reference_trainer_links_through_cmake(build):
    """turbinator_trainer builds unchanged with turbinator_hip linked in: its
    main.c object imports the host-object entries (so TURBINATOR_HAS_CUDA
    reached it from the target), the HIP library defines them, and the
    executable carries those definitions and needs the HIP runtime."""
    exe = build / "turbinator_trainer"
    assert exe.exists()
    main_obj = next(build.rglob("main.c.o"))
    undefined = _symbols(main_obj, "--undefined-only")
    hip_archive = next(build.rglob("libturbinator_hip.a"))
    archive = _symbols(hip_archive, "--defined-only")
    linked = _symbols(exe, "--defined-only")
    for name in TRAINER_IMPORTS:
        assert f" U {name}" in undefined, f"main.c does not call {name}: engine not compiled"
        assert f" T {name}" in archive, f"libturbinator_hip.a does not define {name}"
        assert f" T {name}" in linked, f"trainer does not carry {name}"
    needed = subprocess.run(["readelf", "-d", str(exe)], capture_output=True, text=True,
                            check=True).stdout
    assert "libamdhip64.so" in needed
    assert "libturbinator_sim.so" in needed
