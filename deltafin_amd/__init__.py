"""MI355X-native routed-expert MXFP4 path (gfx950 HIP kernels behind a C ABI).

Submodules:
  deltafin_amd.build  -- compiles lib/libk3hipmoe.so for gfx950
  deltafin_amd._lib   -- ctypes binding of include/k3_hip_moe_abi.h
  deltafin_amd.moe    -- torch-tensor operators over the C ABI
  deltafin_amd.synth  -- host-side synthetic inputs (same counter RNG as the kernels)
"""
from ._lib import LIB_PATH, K3HipError, load  # noqa: F401

__all__ = ["LIB_PATH", "K3HipError", "load"]
