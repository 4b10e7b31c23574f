"""MI355X (gfx950) batched onboard sensor-feature path of Turbinator_C.

The product is the C-ABI library libturbinator_hip.so (HIP kernels for
gfx950 behind include/turbinator/training/cuda_features.h); this package
holds its sources (csrc/), the build driver and thin Python bindings.
"""
from .native import (CAMERA_BYTES, FEATURE_DIM, MISSION_DIM, OBS_DIM, LibraryMissing,
                     hip_lib, synth_lib)

__all__ = ["CAMERA_BYTES", "FEATURE_DIM", "MISSION_DIM", "OBS_DIM", "LibraryMissing",
           "hip_lib", "synth_lib"]
