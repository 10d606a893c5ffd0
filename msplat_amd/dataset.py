"""COLMAP datasets through the library (include/msplat_trainer.h
msplat_dataset_*): cameras with OpenGL camera-to-world poses sorted by image
name, the normalised sparse point cloud, its normalisation, the reference's
train / test split and the initial gaussians of the cloud (nearest-neighbour
scales on the GPU).  Each camera carries its image path; load_image decodes
it and prepares it on the GPU like the reference's Camera::loadImage.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Tuple

import numpy as np

from . import _abi
from .camera import Camera


class Dataset:
    """A COLMAP dataset.  downscale_factor is the load-time image downscale
    of load_image; with eval_mode every test_every-th camera is held out
    (num_train / num_test as the reference's Dataset, python/bindings.cpp)."""

    def __init__(self, path: str, image_dir: Optional[str] = None, downscale_factor: float = 1.0,
                 eval_mode: bool = False, test_every: int = 8):
        self.downscale_factor = float(downscale_factor)
        self.eval_mode = bool(eval_mode)
        self.test_every = int(test_every)
        self._lib = _abi.load()
        self._h = self._lib.msplat_dataset_open_colmap(str(path).encode(),
                                                  str(image_dir).encode() if image_dir else None)
        if not self._h:
            raise _abi.MsplatError(self._lib.msplat_trainer_last_error().decode())
        self.cameras: List[Camera] = []
        self.distortion: List[np.ndarray] = []
        self.image_paths: List[str] = []
        for i in range(self._lib.msplat_dataset_num_cameras(self._h)):
            c = _abi.TrainerCamera()
            d = (ctypes.c_float * 4)()
            p = ctypes.c_char_p()
            _abi.check(self._lib.msplat_dataset_camera(self._h, i, ctypes.byref(c), d, ctypes.byref(p)))
            cam = Camera(width=c.width, height=c.height, fx=c.fx, fy=c.fy, cx=c.cx, cy=c.cy,
                         cam_to_world=np.array(c.camToWorld[:], np.float32).reshape(4, 4))
            self.cameras.append(cam)
            self.distortion.append(np.array(d[:], np.float32))
            self.image_paths.append(p.value.decode())

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.msplat_dataset_destroy(h)
            self._h = None

    def points(self) -> Tuple[np.ndarray, np.ndarray]:
        n = int(self._lib.msplat_dataset_num_points(self._h))
        xyz = np.empty((n, 3), np.float32)
        rgb = np.empty((n, 3), np.uint8)
        _abi.check(self._lib.msplat_dataset_points(self._h, xyz.ctypes.data, rgb.ctypes.data))
        return xyz, rgb

    def normalisation(self) -> Tuple[float, np.ndarray]:
        s = ctypes.c_float()
        t = (ctypes.c_float * 3)()
        _abi.check(self._lib.msplat_dataset_normalisation(self._h, ctypes.byref(s), t))
        return float(s.value), np.array(t[:], np.float32)

    def load_image(self, i: int, downscale: Optional[float] = None):
        """Camera i's image decoded, downscaled (default: the dataset's
        downscale_factor) and undistorted on the GPU (Camera::loadImage):
        (updated camera, CUDA (H, W, 3) float32)."""
        from .image_io import load_camera_image
        ds = self.downscale_factor if downscale is None else downscale
        return load_camera_image(self.image_paths[i], self.cameras[i], self.distortion[i], ds)

    @property
    def num_test(self) -> int:
        return len(self.split_train_test(self.test_every)[1]) if self.eval_mode else 0

    @property
    def num_train(self) -> int:
        return len(self.cameras) - self.num_test

    def split_train_test(self, test_every: int = 8):
        """InputData::splitTrainTest (input_data.cpp:148-158): every test_every-th camera is a test camera."""
        train = [c for i, c in enumerate(self.cameras) if i % test_every != 0]
        test = [c for i, c in enumerate(self.cameras) if i % test_every == 0]
        return train, test

    def init_gaussians(self, sh_degree: int = 3) -> List[np.ndarray]:
        """[means, log-scales, quats, f_dc, f_rest, opacities (N,1)] of the point cloud (GPU KNN)."""
        from . import device
        device.init()
        n = int(self._lib.msplat_dataset_num_points(self._h))
        nb = (sh_degree + 1) ** 2 - 1
        out = [np.empty((n, 3), np.float32), np.empty((n, 3), np.float32), np.empty((n, 4), np.float32),
               np.empty((n, 3), np.float32), np.empty((n, nb, 3), np.float32), np.empty((n, 1), np.float32)]
        pp = (ctypes.c_void_p * 6)(*[a.ctypes.data for a in out])
        rc = self._lib.msplat_dataset_init_gaussians(self._h, sh_degree, pp)
        if rc != 0:
            raise _abi.MsplatError(self._lib.msplat_trainer_last_error().decode())
        return out
