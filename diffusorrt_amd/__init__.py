"""diffusorrt_amd: an MI355X (gfx950) ``rocm`` backend for DiffusorRT's
diffusion-LM denoise step (BD3LM block diffusion, Dream full-canvas diffusion).

Layers:
  * ``libdrt_rocm.so`` (``csrc/``): HIP kernels + C++ runtime/session + C-ABI
    (``include/drt_rocm.h``);
  * :mod:`.runtime`  -- ``Runtime`` / ``DeviceSession`` (the device-session contract);
  * :mod:`.decode`   -- host control plane of the fixed-quota strategies;
  * :mod:`.kernels`  -- per-op kernel table (rms_norm / linear / rope / swiglu / attention);
  * :mod:`.synthetic` -- seeded synthetic models and inputs for the workloads.
"""
from __future__ import annotations

BACKEND_ID = "rocm"

__all__ = ["BACKEND_ID"]
