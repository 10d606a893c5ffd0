"""Camera set-up: OpenGL camera-to-world pose -> view / projection matrices.

Model::prepareCam (core/src/model.cpp:490-534) lives in the C++ host layer
(msplat_amd/host/model.cpp): the OpenGL -> OpenCV column flip, viewmat =
[R^T | -R^T T], projection with near 0.001 / far 1000 and FOV from W / (2 fx),
projmat = P V accumulated in fp32, tile bounds ceil(W/16) x ceil(H/16).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

BLOCK = 16


@dataclass
class Camera:
    """A pinhole camera (input_data.hpp:20-38); cam_to_world is 4x4 row-major OpenGL."""

    width: int
    height: int
    fx: float
    fy: float
    cx: float
    cy: float
    cam_to_world: np.ndarray = field(default_factory=lambda: np.eye(4, dtype=np.float32))


@dataclass
class CamSetup:
    """Model::CamSetup (model.hpp:33-38) plus the matrices prepareCam caches."""

    fx: float
    fy: float
    cx: float
    cy: float
    height: int
    width: int
    viewmat: np.ndarray   # (4,4) float32 row-major
    projmat: np.ndarray   # (4,4) float32 row-major, P @ V
    cam_pos: np.ndarray   # (3,) float32
    tile_bounds: tuple

    @property
    def num_tiles(self) -> int:
        return self.tile_bounds[0] * self.tile_bounds[1]


def prepare_cam(cam: Camera, downscale: int = 1) -> CamSetup:
    """Model::prepareCam through the host library (msplat_prepare_cam in
    include/msplat_trainer.h), so that every caller gets the matrices the C++
    trainer uses, bit for bit.  Host-only: no device is touched."""
    import ctypes

    from . import _abi
    lib = _abi.load()
    k = _abi.TrainerCamera()
    k.width, k.height = int(cam.width), int(cam.height)
    k.fx, k.fy, k.cx, k.cy = float(cam.fx), float(cam.fy), float(cam.cx), float(cam.cy)
    k.camToWorld[:] = [float(v) for v in np.asarray(cam.cam_to_world, np.float32).reshape(16)]
    out = _abi.CamSetupC()
    if lib.msplat_prepare_cam(ctypes.byref(k), int(downscale), ctypes.byref(out)) != 0:
        raise ValueError("prepare_cam: bad camera or downscale factor")
    vm = np.array(out.viewmat[:], np.float32).reshape(4, 4)
    pm = np.array(out.projmat[:], np.float32).reshape(4, 4)
    return CamSetup(out.fx, out.fy, out.cx, out.cy, out.height, out.width, vm, pm,
                    np.array(out.cam_pos[:], np.float32), tuple(out.tile_bounds[:]))


def look_at(position, target=(0.0, 0.0, 0.0), up=(0.0, 1.0, 0.0)) -> np.ndarray:
    """OpenGL camera-to-world (camera looks down -Z, +Y up) placed at position."""
    p = np.asarray(position, dtype=np.float64)
    f = np.asarray(target, dtype=np.float64) - p
    f /= np.linalg.norm(f)
    u = np.asarray(up, dtype=np.float64)
    if abs(float(np.dot(f, u))) > 0.99:
        u = np.array([0.0, 0.0, 1.0])
    r = np.cross(f, u)
    r /= np.linalg.norm(r)
    u2 = np.cross(r, f)
    m = np.eye(4)
    m[:3, 0], m[:3, 1], m[:3, 2], m[:3, 3] = r, u2, -f, p
    return m.astype(np.float32)


def pinhole(width: int, height: int, fov_x_deg: float, cam_to_world: np.ndarray) -> Camera:
    """Square-pixel pinhole with horizontal FOV fov_x_deg, principal point at the centre."""
    fx = width / (2.0 * math.tan(math.radians(fov_x_deg) / 2.0))
    return Camera(width, height, fx, fx, width / 2.0, height / 2.0, np.asarray(cam_to_world, np.float32))
