"""Host-side checks of the C-ABI library that need no GPU.

* every function declared in include/turbinator/training/*.h is exported by
  libturbinator_hip.so;
* argument validation that returns before any HIP call behaves like the
  reference (src/cuda/features.cu:29,58-60,66-67,164-165);
* the Python bindings fail loudly when the library is absent.
"""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from turbinator_c_amd import native

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").rglob("*.h"))


def declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(tb_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def exported_symbols(lib: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True,
                         text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_headers_declare_the_reference_abi():
    names = declared_functions()
    reference_abi = {"tb_cuda_extract_features_device", "tb_cuda_synchronize",
                     "tb_cuda_feature_batch_create", "tb_cuda_feature_batch_destroy",
                     "tb_cuda_feature_batch_error", "tb_cuda_extract_features_host"}
    assert reference_abi <= names


def test_library_exports_every_declared_symbol():
    exported = exported_symbols(native.LIB_HIP_PATH)
    missing = declared_functions() - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    assert set(native.HIP_SIGNATURES) <= exported
    assert set(native.HIP_SIGNATURES) == declared_functions(), \
        "bindings and headers disagree"


def test_argument_validation_without_gpu():
    lib = native.hip_lib()
    dummy = ctypes.c_void_p(16)
    # Device entry: NULL obs/mission/features, batch 0 and > 0x7fffffff.
    assert lib.tb_cuda_extract_features_device(None, dummy, None, dummy, 1, None) == 0
    assert lib.tb_cuda_extract_features_device(dummy, None, None, dummy, 1, None) == 0
    assert lib.tb_cuda_extract_features_device(dummy, dummy, None, None, 1, None) == 0
    assert lib.tb_cuda_extract_features_device(dummy, dummy, None, dummy, 0, None) == 0
    assert lib.tb_cuda_extract_features_device(dummy, dummy, None, dummy, 0x80000000,
                                               None) == 0
    # Allocation-free host entry: NULL pointers, count 0 and count above its
    # static staging (TB_HIP_STATIC_MAX_BATCH = 256), before any runtime call.
    assert lib.tb_hip_extract_features_host_static(None, dummy, dummy, 1, dummy, None) == 0
    assert lib.tb_hip_extract_features_host_static(dummy, dummy, None, 1, dummy, None) == 0
    assert lib.tb_hip_extract_features_host_static(dummy, dummy, dummy, 1, None, None) == 0
    assert lib.tb_hip_extract_features_host_static(dummy, dummy, dummy, 0, dummy, None) == 0
    assert lib.tb_hip_extract_features_host_static(dummy, dummy, dummy, 257, dummy, None) == 0
    # Diagnostics rows are written with 16-byte stores: a pointer that is
    # only 4-byte aligned is refused.
    assert lib.tb_hip_extract_features_diagnostics_device(dummy, dummy, None, dummy,
                                                          ctypes.c_void_p(20), 1, None) == 0
    # Strided entry additionally rejects misaligned float rows.
    assert lib.tb_hip_extract_features_strided_device(dummy, 4148 * 4 + 2, dummy, 40, None, 0,
                                                      dummy, 1, None) == 0
    assert lib.tb_hip_extract_features_strided_device(ctypes.c_void_p(18), 16592, dummy, 40,
                                                      None, 0, dummy, 1, None) == 0
    assert lib.tb_hip_extract_features_indexed_device(dummy, 16592, dummy, 40, None, 0, 8, None,
                                                      dummy, 1, None) == 0
    assert lib.tb_hip_extract_features_indexed_device(dummy, 16592, dummy, 40, None, 0, 0, dummy,
                                                      dummy, 1, None) == 0
    odd = ctypes.c_void_p(20)
    assert lib.tb_hip_actor_inputs_device(None, dummy, dummy, dummy, dummy, dummy, dummy, dummy,
                                          dummy, 1, None) == 0
    assert lib.tb_hip_actor_inputs_device(dummy, dummy, None, dummy, dummy, dummy, dummy, dummy,
                                          dummy, 1, None) == 0
    assert lib.tb_hip_actor_inputs_device(odd, dummy, dummy, dummy, dummy, dummy, dummy, dummy,
                                          dummy, 1, None) == 0
    assert lib.tb_hip_lidar_transform_device(None, dummy, 1, None) == 0
    assert lib.tb_hip_lidar_transform_device(dummy, dummy, 0, None) == 0
    # Host object: max_batch 0 or above 1024 -> NULL before any device call.
    assert not lib.tb_cuda_feature_batch_create(0, 0)
    assert not lib.tb_cuda_feature_batch_create(0, 1025)
    # NULL handle error text and NULL-safe destroy.
    assert lib.tb_cuda_feature_batch_error(None) == b"CUDA feature batch unavailable"
    lib.tb_cuda_feature_batch_destroy(None)
    assert lib.tb_cuda_extract_features_host(None, dummy, dummy, dummy, 1, dummy) == 0
    # Pipeline: invalid create arguments -> NULL before any device call;
    # NULL handles are rejected.
    assert not lib.tb_hip_feature_pipeline_create(0, 0, 2)
    assert not lib.tb_hip_feature_pipeline_create(0, 0x80000000, 2)
    assert not lib.tb_hip_feature_pipeline_create(0, 4, 0)
    assert not lib.tb_hip_feature_pipeline_create(0, 4, 9)
    assert lib.tb_hip_feature_pipeline_error(None) == b"HIP feature pipeline unavailable"
    lib.tb_hip_feature_pipeline_destroy(None)
    assert lib.tb_hip_feature_pipeline_inputs(None, 0, None, None, None) == 0
    assert lib.tb_hip_feature_pipeline_submit(None, 0, 1, 1) == 0
    assert lib.tb_hip_feature_pipeline_submit_direct(None, 0, 1, 1) == 0
    assert not lib.tb_hip_feature_pipeline_wait(None, 0)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    with pytest.raises(native.LibraryMissing):
        native._load(tmp_path / "libturbinator_hip.so", native.HIP_SIGNATURES)
