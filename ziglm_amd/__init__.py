"""ziglm fused per-layer ops on AMD Instinct MI355X (gfx950).

The product is the C-ABI library libhip_bridge.so (include/hip_bridge.h). This package
holds its HIP sources (csrc/), the build recipe (build.py), the ctypes binding
(bridge.py), the host operator interface mirroring ziglm's CudaDevice (device.py) and the
seeded synthetic-data generator shared by tests and bench (synth.py).
"""
__all__ = ["bridge", "device", "synth", "build"]
