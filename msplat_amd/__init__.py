"""msplat_amd — MI355X (gfx950) implementation of msplat's per-step splatting hot path.

The compute runs in libmsplat_hip.so (hand-written HIP kernels behind the C ABI
of include/msplat_hip.h).  Python modules:
  _abi       ctypes binding of the C ABI
  device     device-memory driver (PyTorch tensors as buffers)
  camera     prepareCam (view / projection matrices)
  synthetic  deterministic scenes of the benchmark configurations
"""
__version__ = "0.1.0"

# The reference module's top-level names (python/msplat/__init__.py), loaded
# on first use so that importing the package needs neither torch nor a GPU.
__all__ = ["TrainingConfig", "TrainingStats", "Dataset", "GaussianTrainer", "sync", "cleanup",
           "load_dataset"]


def __getattr__(name):
    if name in ("GaussianTrainer", "TrainingConfig", "TrainingStats"):
        from . import trainer
        return getattr(trainer, name)
    if name == "Dataset":
        from .dataset import Dataset
        return Dataset
    raise AttributeError(f"module 'msplat_amd' has no attribute {name!r}")


def load_dataset(path: str, downscale_factor: float = 1.0, eval_mode: bool = False,
                 test_every: int = 8):
    """Load a COLMAP dataset (the reference's load_dataset; Nerfstudio and
    Polycam layouts are not read here)."""
    from .dataset import Dataset
    return Dataset(path, downscale_factor=downscale_factor, eval_mode=eval_mode, test_every=test_every)


def sync() -> None:
    """Wait for all queued GPU work (msplat.sync)."""
    from . import device
    device.sync()


def cleanup() -> None:
    """Release the library's cached GPU buffers (msplat.cleanup); the next
    call re-initialises on demand."""
    from . import _abi, device
    if getattr(device, "_initialised", False):
        _abi.check(_abi.load().msplat_hip_shutdown())
        device._initialised = False
