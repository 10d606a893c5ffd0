"""Camera set-up: OpenGL camera-to-world pose -> view / projection matrices.

Mirrors Model::prepareCam (/root/reference/core/src/model.cpp:490-534): the
OpenGL -> OpenCV column flip, viewmat = [R^T | -R^T T], projection with near
0.001 / far 1000 and FOV from W / (2 fx), projmat = P @ V accumulated in fp32,
tile bounds ceil(W/16) x ceil(H/16).
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
    f32 = np.float32
    sf = f32(downscale)
    fx, fy, cx, cy = f32(cam.fx) / sf, f32(cam.fy) / sf, f32(cam.cx) / sf, f32(cam.cy) / sf
    height, width = int(cam.height / float(sf)), int(cam.width / float(sf))
    fov_x = f32(2.0) * f32(math.atan(float(f32(width) / (f32(2.0) * fx))))
    fov_y = f32(2.0) * f32(math.atan(float(f32(height) / (f32(2.0) * fy))))
    d = np.asarray(cam.cam_to_world, dtype=f32).reshape(16)
    R = np.empty((3, 3), f32)
    T = np.empty(3, f32)
    for i in range(3):
        R[i, 0], R[i, 1], R[i, 2], T[i] = d[i * 4 + 0], -d[i * 4 + 1], -d[i * 4 + 2], d[i * 4 + 3]
    Rinv = R.T.copy()
    Tinv = np.empty(3, f32)
    for i in range(3):
        Tinv[i] = -(Rinv[i, 0] * T[0] + Rinv[i, 1] * T[1] + Rinv[i, 2] * T[2])
    vm = np.array([Rinv[0, 0], Rinv[0, 1], Rinv[0, 2], Tinv[0],
                   Rinv[1, 0], Rinv[1, 1], Rinv[1, 2], Tinv[1],
                   Rinv[2, 0], Rinv[2, 1], Rinv[2, 2], Tinv[2],
                   0, 0, 0, 1], dtype=f32)
    t_p = f32(0.001) * f32(math.tan(float(f32(0.5) * fov_y)))
    r_p = f32(0.001) * f32(math.tan(float(f32(0.5) * fov_x)))
    n, fa = f32(0.001), f32(1000.0)
    pm = np.array([n / r_p, 0, 0, 0,
                   0, n / t_p, 0, 0,
                   0, 0, (fa + n) / (fa - n), -fa * n / (fa - n),
                   0, 0, 1, 0], dtype=f32)
    pvm = np.zeros(16, dtype=f32)
    for i in range(4):
        for j in range(4):
            acc = f32(0.0)
            for k in range(4):
                acc = f32(acc + f32(pm[i * 4 + k] * vm[k * 4 + j]))
            pvm[i * 4 + j] = acc
    tb = ((width + BLOCK - 1) // BLOCK, (height + BLOCK - 1) // BLOCK, 1)
    return CamSetup(float(fx), float(fy), float(cx), float(cy), height, width,
                    vm.reshape(4, 4), pvm.reshape(4, 4), T.copy(), tb)


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
