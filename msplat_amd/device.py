"""Device-side driver of the C ABI for Python callers (tests, bench, trainer).

PyTorch provides device memory and the copies; every computation runs in
libmsplat_hip.so.  The library works on its own blocking HIP stream, which is
ordered with PyTorch's default stream.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from . import _abi

_initialised = False


def init(device: int = 0):
    global _initialised
    lib = _abi.load()
    if not _initialised:
        _abi.check(lib.msplat_hip_init(device))
        _initialised = True
    return lib


def torch():
    import torch as _t
    return _t


def ptr(t) -> Optional[int]:
    return None if t is None else int(t.data_ptr())


def to_dev(a: np.ndarray, dtype=None):
    T = torch()
    t = T.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to("cuda")


def sync():
    _abi.check(init().msplat_hip_sync())
    torch().cuda.synchronize()


@dataclass
class DeviceGaussians:
    """Six parameter groups (means, scales, quats, f_dc, f_rest, opacities) with
    Adam moments and densify statistics, in buffers of `capacity` rows whose
    first `n` rows are active (the reference's *_buf + view(n), model.cpp:184-195)."""

    bufs: List
    m: List
    v: List
    vis: object
    gnorm: object
    max2d: object
    n: int
    capacity: int
    sh_degree: int

    @staticmethod
    def from_arrays(params, sh_degree: int, capacity: Optional[int] = None) -> "DeviceGaussians":
        T = torch()
        init()
        n = int(params[0].shape[0])
        cap = max(capacity or n, n, 1)
        bufs, ms, vs = [], [], []
        for a in params:
            a = np.ascontiguousarray(a, np.float32)
            shape = (cap,) + tuple(a.shape[1:])
            b = T.zeros(shape, dtype=T.float32, device="cuda")
            if n:
                b[:n].copy_(T.from_numpy(a))
            bufs.append(b)
            ms.append(T.zeros(shape, dtype=T.float32, device="cuda"))
            vs.append(T.zeros(shape, dtype=T.float32, device="cuda"))
        z = lambda: T.zeros(cap, dtype=T.float32, device="cuda")
        return DeviceGaussians(bufs, ms, vs, z(), z(), z(), n, cap, sh_degree)

    @staticmethod
    def from_tensors(params, sh_degree: int, capacity: Optional[int] = None) -> "DeviceGaussians":
        """Same as from_arrays for tensors already on the device."""
        T = torch()
        init()
        n = int(params[0].shape[0])
        cap = max(capacity or n, n, 1)
        bufs, ms, vs = [], [], []
        for a in params:
            shape = (cap,) + tuple(a.shape[1:])
            b = T.zeros(shape, dtype=T.float32, device="cuda")
            if n:
                b[:n].copy_(a)
            bufs.append(b)
            ms.append(T.zeros(shape, dtype=T.float32, device="cuda"))
            vs.append(T.zeros(shape, dtype=T.float32, device="cuda"))
        z = lambda: T.zeros(cap, dtype=T.float32, device="cuda")
        return DeviceGaussians(bufs, ms, vs, z(), z(), z(), n, cap, sh_degree)

    def view(self, i: int):
        return self.bufs[i][: self.n]

    def rest_bases(self) -> int:
        return int(self.bufs[4].shape[1]) if self.bufs[4].dim() == 3 else 0

    def numpy(self):
        return [b[: self.n].cpu().numpy().copy() for b in self.bufs]

    def reset_stats(self):
        self.vis.zero_(); self.gnorm.zero_(); self.max2d.zero_()


def render_args(g: DeviceGaussians, setup, degrees_to_use: int, background, clip=0.01,
                glob_scale=1.0) -> _abi.RenderArgs:
    a = _abi.RenderArgs()
    a.num_points = g.n
    a.means3d, a.scales, a.quats = ptr(g.bufs[0]), ptr(g.bufs[1]), ptr(g.bufs[2])
    a.features_dc, a.features_rest, a.opacities = ptr(g.bufs[3]), ptr(g.bufs[4]), ptr(g.bufs[5])
    a.glob_scale = glob_scale
    a.viewmat[:] = [float(x) for x in np.asarray(setup.viewmat, np.float32).reshape(16)]
    a.projmat[:] = [float(x) for x in np.asarray(setup.projmat, np.float32).reshape(16)]
    a.fx, a.fy, a.cx, a.cy = setup.fx, setup.fy, setup.cx, setup.cy
    a.img_height, a.img_width = setup.height, setup.width
    a.tile_bounds[:] = list(setup.tile_bounds)
    a.clip_thresh = clip
    a.degree = g.sh_degree
    a.degrees_to_use = min(degrees_to_use, g.sh_degree)
    a.cam_pos[:] = [float(x) for x in setup.cam_pos]
    a.background[:] = [float(x) for x in background]
    return a


def render(g: DeviceGaussians, setup, degrees_to_use: int, background, out=None, clip=0.01):
    """msplat_render: returns a (H, W, 3) float32 device tensor."""
    T = torch()
    lib = init()
    if out is None:
        out = T.empty((setup.height, setup.width, 3), dtype=T.float32, device="cuda")
    a = render_args(g, setup, degrees_to_use, background, clip=clip)
    _abi.check(lib.msplat_hip_render(ctypes.byref(a), ptr(out)))
    return out


def image_metrics(img, gt, window_size: int = 11, sigma: float = 1.5) -> dict:
    """PSNR / SSIM / L1 of two (H, W, 3) float32 CUDA images (msplat_hip_image_metrics)."""
    lib = init()
    torch().cuda.synchronize()
    H, W = int(img.shape[0]), int(img.shape[1])
    m = _abi.ImageMetrics()
    _abi.check(lib.msplat_hip_image_metrics(ptr(img.contiguous()), ptr(gt.contiguous()), H, W,
                                            window_size, sigma, ctypes.byref(m)))
    return {"psnr": m.psnr, "ssim": m.ssim, "l1": m.l1}


def image_to_rgba8(img):
    """(H, W, 4) uint8 CUDA tensor of a (H, W, 3) float32 CUDA image (msplat_hip_image_to_rgba8)."""
    T = torch()
    lib = init()
    T.cuda.synchronize()
    out = T.empty(img.shape[:-1] + (4,), dtype=T.uint8, device="cuda")
    n = int(img.numel() // 3)
    _abi.check(lib.msplat_hip_image_to_rgba8(ptr(img.contiguous()), n, ptr(out)))
    sync()
    return out


def adam_constants(lrs, step: int, beta1=0.9, beta2=0.999):
    """Bias corrections of fullIteration (model.cpp:558-571), in fp32."""
    f = np.float32
    bc1 = f(1.0) - f(beta1) ** f(step)
    bc2 = f(1.0) - f(beta2) ** f(step)
    return [float(f(lr) / bc1) for lr in lrs], [float(np.sqrt(bc2))] * 6


def train_args(g: DeviceGaussians, setup, degrees_to_use: int, background, gt, ssim_weight: float,
               lrs, step: int, beta1=0.9, beta2=0.999, eps=1e-8, grads_out=None) -> _abi.TrainArgs:
    t = _abi.TrainArgs()
    t.r = render_args(g, setup, degrees_to_use, background)
    t.gt = ptr(gt)
    t.ssim_weight = ssim_weight
    t.loss_inv_n = float(np.float32(1.0) / np.float32(setup.height * setup.width * 3))
    t.features_rest_bases = g.rest_bases()
    t.num_adam_groups = 6
    for i in range(6):
        t.adam_params[i] = ptr(g.bufs[i])
        t.adam_exp_avg[i] = ptr(g.m[i])
        t.adam_exp_avg_sq[i] = ptr(g.v[i])
    ss, bc = adam_constants(lrs, step, beta1, beta2)
    t.adam_step_sizes[:] = ss
    t.adam_bc2_sqrts[:] = bc
    t.adam_beta1, t.adam_beta2, t.adam_eps = beta1, beta2, eps
    t.vis_counts, t.xys_grad_norm, t.max_2d_size = ptr(g.vis), ptr(g.gnorm), ptr(g.max2d)
    t.inv_max_dim = float(np.float32(1.0) / np.float32(max(setup.height, setup.width)))
    if grads_out is not None:
        t.v_mean3d_out, t.v_scale_out, t.v_quat_out = (ptr(grads_out[k]) for k in ("v_mean3d", "v_scale", "v_quat"))
    return t


def train_step(g: DeviceGaussians, setup, degrees_to_use: int, background, gt, ssim_weight: float, lrs,
               step: int, want_loss: bool = True, radii_out=None, grads_out=None):
    lib = init()
    t = train_args(g, setup, degrees_to_use, background, gt, ssim_weight, lrs, step, grads_out=grads_out)
    loss = ctypes.c_float(0.0)
    _abi.check(lib.msplat_hip_train_step(ctypes.byref(t), ptr(radii_out), ctypes.byref(loss) if want_loss else None))
    return float(loss.value) if want_loss else None


def intermediate(name: str, dtype=np.float32, shape=None) -> np.ndarray:
    lib = init()
    nb = ctypes.c_size_t(0)
    _abi.check(lib.msplat_hip_copy_intermediate(name.encode(), None, ctypes.byref(nb)))
    out = np.empty(nb.value // np.dtype(dtype).itemsize, dtype=dtype)
    if nb.value:
        _abi.check(lib.msplat_hip_copy_intermediate(name.encode(), out.ctypes.data_as(ctypes.c_void_p),
                                                    ctypes.byref(nb)))
    return out.reshape(shape) if shape is not None else out


RASTER_WORK_KEYS = ("fwd_tested", "fwd_in_range", "fwd_composited",
                    "bwd_tested", "bwd_in_range", "bwd_with_grad")


def raster_work() -> dict:
    """(pixel, entry) pair counts of the last render / train step's rasteriser
    (msplat_hip_raster_work): the algorithmic work behind its flop count."""
    lib = init()
    out = (ctypes.c_int64 * 6)()
    _abi.check(lib.msplat_hip_raster_work(out))
    return dict(zip(RASTER_WORK_KEYS, (int(v) for v in out)))


def drain_raster_counters() -> tuple:
    """(forward pairs composited, backward pairs with gradient, forward wave
    steps, backward wave steps) summed over the calls made while stage timing
    was on; restarts the sums."""
    lib = init()
    out = (ctypes.c_int64 * 4)()
    _abi.check(lib.msplat_hip_drain_raster_counters(out))
    return tuple(int(v) for v in out)


def meta() -> dict:
    raw = intermediate("meta", np.uint8)
    total = int(np.frombuffer(raw[:8].tobytes(), np.int64)[0])
    rest = np.frombuffer(raw[8:8 + 24].tobytes(), np.int32)
    return dict(total_isect=total, max_count=int(rest[0]), n_items=int(rest[1]), n_chunked_tiles=int(rest[2]),
                n_large=int(rest[3]), n_huge=int(rest[4]))


def densify_args(g: DeviceGaussians, grad_thresh, size_thresh, screen_thresh, check_screen, cull_alpha,
                 cull_scale, cull_screen, check_huge, half_max_dim, random_samples=None, seed=0):
    a = _abi.DensifyArgs()
    a.N = g.n
    a.buf_capacity = g.capacity
    a.grad_thresh, a.size_thresh, a.screen_thresh = grad_thresh, size_thresh, screen_thresh
    a.check_screen = int(check_screen)
    a.cull_alpha_thresh, a.cull_scale_thresh, a.cull_screen_size = cull_alpha, cull_scale, cull_screen
    a.check_huge = int(check_huge)
    a.xys_grad_norm, a.vis_counts, a.max_2d_size = ptr(g.gnorm), ptr(g.vis), ptr(g.max2d)
    a.half_max_dim = half_max_dim
    for i in range(6):
        a.bufs[i] = ptr(g.bufs[i])
        a.adam_exp_avg_buf[i] = ptr(g.m[i])
        a.adam_exp_avg_sq_buf[i] = ptr(g.v[i])
    a.fr_stride = g.rest_bases() * 3
    a.random_samples = ptr(random_samples)
    a.seed = seed
    return a


def densify(g: DeviceGaussians, **kw) -> int:
    lib = init()
    a = densify_args(g, **kw)
    out = ctypes.c_int32(0)
    _abi.check(lib.msplat_hip_densify(ctypes.byref(a), ctypes.byref(out)))
    g.n = int(out.value)
    return g.n
