"""msplat_amd — MI355X (gfx950) implementation of msplat's per-step splatting hot path.

The compute runs in libmsplat_hip.so (hand-written HIP kernels behind the C ABI
of include/msplat_hip.h).  Python modules:
  _abi       ctypes binding of the C ABI
  device     device-memory driver (PyTorch tensors as buffers)
  camera     prepareCam (view / projection matrices)
  synthetic  deterministic scenes of the benchmark configurations
"""
__version__ = "0.1.0"
