"""Deterministic synthetic scenes for the five benchmark configurations.

The reference trains on COLMAP scenes (datasets/ holds only Git-LFS pointers),
so every configuration here is synthetic, generated from a counter-based
SplitMix64 stream (one stream per field, drawn in a fixed order) with
Box–Muller normals.  Base seed of configuration c: 0x6D73706C00 + c.
Parameter layouts are the reference's (model.cpp:59-109): means [N,3],
log-scales [N,3], quats [N,4] (w,x,y,z), f_dc [N,3], f_rest [N,K-1,3],
opacity logits [N,1].
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable, List, Optional

import numpy as np

from .camera import Camera, look_at, pinhole

BASE_SEED = 0x6D73706C00
_U64 = np.uint64


def _splitmix(x: np.ndarray) -> np.ndarray:
    x = x + _U64(0x9E3779B97F4A7C15)
    x = (x ^ (x >> _U64(30))) * _U64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> _U64(27))) * _U64(0x94D049BB133111EB)
    return x ^ (x >> _U64(31))


class Stream:
    """Counter-based generator: value i of stream s is splitmix64(key_s + i)."""

    def __init__(self, seed: int):
        self.seed = seed & 0xFFFFFFFFFFFFFFFF
        self.next_stream = 0

    def _key(self) -> np.uint64:
        with np.errstate(over="ignore"):
            k = _splitmix(np.array([self.seed ^ (self.next_stream * 0xD1B54A32D192ED03 & 0xFFFFFFFFFFFFFFFF)],
                                   dtype=_U64))[0]
        self.next_stream += 1
        return k

    def uniform(self, n: int) -> np.ndarray:
        """float64 in [0, 1)."""
        key = self._key()
        out = np.empty(n, dtype=np.float64)
        step = 1 << 23
        with np.errstate(over="ignore"):
            for s in range(0, n, step):
                idx = np.arange(s, min(n, s + step), dtype=_U64) + key
                out[s:s + len(idx)] = (_splitmix(idx) >> _U64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
        return out

    def normal(self, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
        u1 = 1.0 - self.uniform(n)   # (0, 1]
        u2 = self.uniform(n)
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * math.pi * u2)
        return (mean + std * z)


@dataclass
class Scene:
    """Gaussian parameters plus cameras (and targets once made)."""

    means: np.ndarray
    scales: np.ndarray
    quats: np.ndarray
    opacities: np.ndarray
    f_dc: np.ndarray
    f_rest: np.ndarray
    sh_degree: int
    cameras: List[Camera]
    background: np.ndarray = field(default_factory=lambda: np.array([0.6130, 0.0101, 0.3984], np.float32))
    targets: Optional[List[np.ndarray]] = None
    name: str = ""

    @property
    def n(self) -> int:
        return int(self.means.shape[0])

    def params(self):
        return [self.means, self.scales, self.quats, self.f_dc, self.f_rest, self.opacities]


def _quats(st: Stream, n: int) -> np.ndarray:
    q = st.normal(4 * n).reshape(n, 4)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    return q.astype(np.float32)


def _sphere_dirs(st: Stream, n: int) -> np.ndarray:
    v = st.normal(3 * n).reshape(n, 3)
    return v / np.linalg.norm(v, axis=1, keepdims=True)


def _gaussians(st: Stream, n: int, degree: int, means: np.ndarray, dc_std: float, rest_std: float) -> dict:
    nb = (degree + 1) ** 2 - 1
    scales = st.normal(3 * n, -4.5, 0.5).reshape(n, 3).astype(np.float32)
    quats = _quats(st, n)
    opac = st.normal(n).reshape(n, 1).astype(np.float32)
    f_dc = st.normal(3 * n, 0.0, dc_std).reshape(n, 3).astype(np.float32)
    f_rest = (st.normal(nb * 3 * n, 0.0, rest_std).reshape(n, nb, 3).astype(np.float32)
              if nb else np.zeros((n, 0, 3), np.float32))
    return dict(means=means.astype(np.float32), scales=scales, quats=quats, opacities=opac, f_dc=f_dc,
                f_rest=f_rest)


def config1(n: int = 10_000, width: int = 256, height: int = 256) -> Scene:
    """Config 1: 10k SH0 gaussians, U[-1,1]^3, camera at (0,0,-4) looking at the origin, FOV 60."""
    st = Stream(BASE_SEED + 1)
    means = st.uniform(3 * n).reshape(n, 3) * 2.0 - 1.0
    g = _gaussians(st, n, 0, means, 0.3, 0.0)
    c2w = np.diag([1.0, -1.0, -1.0, 1.0]).astype(np.float32)   # viewmat = [I | (0,0,4)]
    c2w[2, 3] = -4.0
    cam = pinhole(width, height, 60.0, c2w)
    sc = Scene(sh_degree=0, cameras=[cam], name="config1", **g)
    sc.targets = [st.uniform(height * width * 3).reshape(height, width, 3).astype(np.float32)]
    return sc


def _clipped_normal_means(st: Stream, n: int) -> np.ndarray:
    return np.clip(st.normal(3 * n, 0.0, 1.5).reshape(n, 3), -4.0, 4.0)


def config2(n: int = 500_000, width: int = 1297, height: int = 840, n_cams: int = 1, seed_off: int = 2) -> Scene:
    """Config 2: SH3 cloud N(0,1.5^2) clipped to +-4, FOV 70, poses on a radius-5 sphere."""
    st = Stream(BASE_SEED + seed_off)
    means = _clipped_normal_means(st, n)
    g = _gaussians(st, n, 3, means, 0.3, 0.05)
    dirs = _sphere_dirs(st, n_cams)
    cams = [pinhole(width, height, 70.0, look_at(5.0 * d)) for d in dirs]
    return Scene(sh_degree=3, cameras=cams, name="config2", **g)


def config3(n: int = 1_500_000, width: int = 1297, height: int = 840, n_cams: int = 32) -> Scene:
    """Config 3: as config 2 at 1.5M, 32 cameras at radius U[4,6] in uniform directions."""
    st = Stream(BASE_SEED + 3)
    means = _clipped_normal_means(st, n)
    g = _gaussians(st, n, 3, means, 0.3, 0.05)
    dirs = _sphere_dirs(st, n_cams)
    radii = 4.0 + 2.0 * st.uniform(n_cams)
    cams = [pinhole(width, height, 70.0, look_at(r * d)) for r, d in zip(radii, dirs)]
    return Scene(sh_degree=3, cameras=cams, name="config3", **g)


def config4(n: int = 1_000_000, width: int = 2594, height: int = 1680) -> Scene:
    """Config 4: 70% tight blob 1.5 units in front of the camera, 30% uniform background."""
    st = Stream(BASE_SEED + 4)
    cam_pos = np.array([0.0, 0.0, 5.0])
    c2w = look_at(cam_pos)
    fwd = -c2w[:3, 2].astype(np.float64)
    nb = int(0.7 * n)
    blob = cam_pos + 1.5 * fwd + st.normal(3 * nb, 0.0, 0.05).reshape(nb, 3)
    bg = st.uniform(3 * (n - nb)).reshape(n - nb, 3) * 8.0 - 4.0
    means = np.concatenate([blob, bg], axis=0)
    g = _gaussians(st, n, 3, means, 0.3, 0.05)
    cam = pinhole(width, height, 70.0, c2w)
    return Scene(sh_degree=3, cameras=[cam], name="config4", **g)


def config5(n: int = 6_000_000, width: int = 4946, height: int = 3286, n_poses: int = 100) -> Scene:
    """Config 5: render-only, 6M SH3 gaussians as config 2, 100 poses on a radius-5 sphere."""
    st = Stream(BASE_SEED + 5)
    means = _clipped_normal_means(st, n)
    g = _gaussians(st, n, 3, means, 0.3, 0.05)
    dirs = _sphere_dirs(st, n_poses)
    cams = [pinhole(width, height, 70.0, look_at(5.0 * d)) for d in dirs]
    return Scene(sh_degree=3, cameras=cams, name="config5", **g)


def make_targets(scene: Scene, render: Callable[[Scene, Camera], np.ndarray], seed_off: int = 100,
                 jitter: float = 0.02, noise: float = 0.01) -> List[np.ndarray]:
    """Targets of configs 2/3: a render of the cloud with means jittered by
    N(0, jitter) plus N(0, noise) pixel noise (not clamped).  `render` draws
    one image of a scene from a camera."""
    st = Stream(BASE_SEED + seed_off)
    jit = Scene(**{**scene.__dict__})
    jit.means = (scene.means + st.normal(scene.means.size, 0.0, jitter).reshape(scene.means.shape)).astype(np.float32)
    out = []
    for cam in scene.cameras:
        img = render(jit, cam)
        out.append((img + st.normal(img.size, 0.0, noise).reshape(img.shape)).astype(np.float32))
    return out


def device_randn(n: int, seed: int, mean: float = 0.0, std: float = 1.0):
    """n normals on cuda:0 from the library's counter-based generator."""
    from . import _abi, device
    T = device.torch()
    x = T.empty(n, dtype=T.float32, device="cuda")
    if n:
        _abi.check(device.init().msplat_hip_randn(device.ptr(x), n, seed & 0xFFFFFFFFFFFFFFFF))
    return x.mul_(std).add_(mean)


def device_cloud(n: int, degree: int, seed: int):
    """Config-2/3/5 gaussians generated on the GPU: means N(0,1.5^2) clipped to
    +-4, log-scales N(-4.5,0.5), quats normalize(N(0,1)^4), opacity logits
    N(0,1), DC N(0,0.3), higher bands N(0,0.05).  Returns 6 device tensors."""
    nb = (degree + 1) ** 2 - 1
    k = lambda i: (seed << 8) + i
    means = device_randn(3 * n, k(0), 0.0, 1.5).clamp_(-4.0, 4.0).view(n, 3)
    scales = device_randn(3 * n, k(1), -4.5, 0.5).view(n, 3)
    quats = device_randn(4 * n, k(2)).view(n, 4)
    quats /= quats.norm(dim=1, keepdim=True)
    opac = device_randn(n, k(3)).view(n, 1)
    f_dc = device_randn(3 * n, k(4), 0.0, 0.3).view(n, 3)
    f_rest = device_randn(nb * 3 * n, k(5), 0.0, 0.05).view(n, nb, 3)
    return [means, scales, quats.contiguous(), f_dc, f_rest, opac]


# Poses and targets of the benchmark workloads whose gaussians are generated
# on the GPU (device_cloud).  Each pose set has a stream of its own, so it
# does not depend on how the gaussians were drawn.

def config2_cameras(n_cams: int = 1, width: int = 1297, height: int = 840) -> List[Camera]:
    """Config-2 poses: uniform directions on a radius-5 sphere, FOV 70."""
    st = Stream(BASE_SEED + 2 + 1000)
    dirs = _sphere_dirs(st, n_cams)
    return [pinhole(width, height, 70.0, look_at(5.0 * d)) for d in dirs]


def config3_cameras(n_cams: int = 32, width: int = 1297, height: int = 840) -> List[Camera]:
    """Config-3 poses: 32 cameras at radius U[4,6] in uniform directions, FOV 70."""
    st = Stream(BASE_SEED + 3 + 1000)
    dirs = _sphere_dirs(st, n_cams)
    radii = 4.0 + 2.0 * st.uniform(n_cams)
    return [pinhole(width, height, 70.0, look_at(r * d)) for r, d in zip(radii, dirs)]


def config5_cameras(n_poses: int = 100, width: int = 4946, height: int = 3286) -> List[Camera]:
    """Config-5 poses: uniform directions on a radius-5 sphere, FOV 70."""
    st = Stream(BASE_SEED + 5 + 1000)
    dirs = _sphere_dirs(st, n_poses)
    return [pinhole(width, height, 70.0, look_at(5.0 * d)) for d in dirs]


def device_targets(params, cams, degree: int, background, seed: int):
    """Targets of configs 2/3 on the GPU: a render of the cloud (six device
    tensors) with means jittered by N(0, 0.02), plus N(0, 0.01) pixel noise
    (not clamped), one (H, W, 3) device tensor per camera."""
    from . import camera, device
    jit = list(params)
    jit[0] = params[0] + device_randn(params[0].numel(), seed * 7 + 11, 0.0, 0.02).view_as(params[0])
    g = device.DeviceGaussians.from_tensors(jit, degree)
    out = []
    for i, c in enumerate(cams):
        img = device.render(g, camera.prepare_cam(c), degree, background).clone()
        img += device_randn(img.numel(), seed * 13 + i, 0.0, 0.01).view_as(img)
        out.append(img)
    del g
    return out
