"""Model / GaussianTrainer over the HIP hot path.

Mirrors the reference's host orchestration:
  Model::setupOptimizers      model.cpp:119-164  (4x capacity buffers, LR table)
  Model::schedulersStep       model.cpp:179-182  (means LR log-lerp, applied after the step)
  Model::prepareCam           model.cpp:490-534  (camera.prepare_cam)
  Model::fullIteration        model.cpp:546-597  (Adam step count, bias corrections)
  Model::afterTrain           model.cpp:236-296  (densify / opacity-reset policy)
  GaussianTrainer::step       python/bindings.cpp:144-167
  GaussianTrainer::render_from_pose  python/bindings.cpp:236-259
Every computation is a call into libmsplat_hip.so.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from . import _abi, device
from .camera import Camera, prepare_cam

LR_INIT = [0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05]   # model.cpp:138
MEANS_LR_FINAL = 0.0000016                                    # model.cpp:149
RESET_LOGIT = -1.3862943611198906                             # logit(0.2), model.cpp:282


@dataclass
class TrainingConfig:
    """TrainingConfig (python/bindings.cpp:25-46); cull thresholds exposed
    (model.cpp:263 hard-codes 0.1 / 0.5 / 0.15)."""

    iterations: int = 30000
    sh_degree: int = 3
    sh_degree_interval: int = 1000        # 0: use sh_degree from the first step
    ssim_weight: float = 0.2
    num_downscales: int = 2
    resolution_schedule: int = 3000
    refine_every: int = 100
    warmup_length: int = 500
    reset_alpha_every: int = 30
    densify_grad_thresh: float = 0.0002
    densify_size_thresh: float = 0.01
    stop_screen_size_at: int = 4000
    split_screen_size: float = 0.05
    cull_alpha_thresh: float = 0.1
    cull_scale_thresh: float = 0.5
    cull_screen_size: float = 0.15
    bg_color: List[float] = field(default_factory=lambda: [0.6130, 0.0101, 0.3984])
    shuffle_cameras: bool = True


@dataclass
class TrainingStats:
    iteration: int
    splat_count: int
    ms_per_step: float


class Model:
    def __init__(self, params, cfg: TrainingConfig, num_cameras: int):
        self.cfg = cfg
        self.num_cameras = num_cameras
        n = int(params[0].shape[0])
        if hasattr(params[0], "data_ptr"):
            self.g = device.DeviceGaussians.from_tensors(params, cfg.sh_degree, capacity=4 * n)
        else:
            self.g = device.DeviceGaussians.from_arrays(params, cfg.sh_degree, capacity=4 * n)
        self.adam_lr = list(LR_INIT)
        self.adam_step_count = 0
        self.stop_split_at = cfg.iterations // 2
        self.last_hw = (0, 0)
        self.background = np.asarray(cfg.bg_color, np.float32)
        self._setups = {}

    @property
    def num_active(self) -> int:
        return self.g.n

    def downscale_factor(self, step: int) -> int:
        return 1 << max(self.cfg.num_downscales - step // self.cfg.resolution_schedule, 0)

    def degrees_to_use(self, step: int) -> int:
        if self.cfg.sh_degree_interval <= 0:
            return self.cfg.sh_degree
        return min(step // self.cfg.sh_degree_interval, self.cfg.sh_degree)

    def setup(self, cam: Camera, step: int):
        ds = self.downscale_factor(step)
        key = (id(cam), ds)
        s = self._setups.get(key)
        if s is None:
            s = prepare_cam(cam, ds)
            self._setups[key] = s
        return s

    def schedulers_step(self, step: int):
        t = min(max(step / self.cfg.iterations, 0.0), 1.0)
        f = np.float32
        self.adam_lr[0] = float(np.exp(f(np.log(f(LR_INIT[0]))) * f(1 - t) + f(np.log(f(MEANS_LR_FINAL))) * f(t)))

    def full_iteration(self, cam: Camera, step: int, gt, want_loss: bool = False):
        s = self.setup(cam, step)
        self.last_hw = (s.height, s.width)
        self.adam_step_count += 1
        return device.train_step(self.g, s, self.degrees_to_use(step), self.background, gt,
                                 self.cfg.ssim_weight, self.adam_lr, self.adam_step_count, want_loss=want_loss)

    def ensure_capacity(self, needed: int):
        g = self.g
        if needed <= g.capacity:
            return
        T = device.torch()
        new_cap = max(needed, 2 * g.capacity)

        def grow(b):
            nb = T.zeros((new_cap,) + tuple(b.shape[1:]), dtype=b.dtype, device=b.device)
            nb[: g.n].copy_(b[: g.n])
            return nb

        g.bufs = [grow(b) for b in g.bufs]
        g.m = [grow(b) for b in g.m]
        g.v = [grow(b) for b in g.v]
        g.vis, g.gnorm, g.max2d = grow(g.vis), grow(g.gnorm), grow(g.max2d)
        g.capacity = new_cap

    def after_train(self, step: int) -> Optional[int]:
        """Model::afterTrain: densify / opacity reset at refine steps.  Returns the new count when densified."""
        cfg = self.cfg
        res = None
        if step % cfg.refine_every == 0 and step > cfg.warmup_length:
            reset_interval = cfg.reset_alpha_every * cfg.refine_every
            do_densify = step < self.stop_split_at and step % reset_interval > self.num_cameras + cfg.refine_every
            if do_densify:
                self.ensure_capacity(3 * self.g.n)
                H, W = self.last_hw
                res = device.densify(
                    self.g, grad_thresh=cfg.densify_grad_thresh, size_thresh=cfg.densify_size_thresh,
                    screen_thresh=cfg.split_screen_size, check_screen=step < cfg.stop_screen_size_at,
                    cull_alpha=cfg.cull_alpha_thresh, cull_scale=cfg.cull_scale_thresh,
                    cull_screen=cfg.cull_screen_size, check_huge=step > cfg.refine_every * cfg.reset_alpha_every,
                    half_max_dim=0.5 * max(W, H), random_samples=None, seed=step)
            if step < self.stop_split_at and step % reset_interval == cfg.refine_every:
                op = self.g.bufs[5][: self.g.n]
                op.clamp_(max=RESET_LOGIT)
                self.g.m[5][: self.g.n].zero_()
                self.g.v[5][: self.g.n].zero_()
            self.g.reset_stats()
        return res

    def render(self, cam: Camera, step: int):
        s = self.setup(cam, step)
        return device.render(self.g, s, self.degrees_to_use(step), self.background)


class GaussianTrainer:
    """GaussianTrainer (python/bindings.cpp:101-280) over an in-memory dataset
    of cameras and target images (device tensors)."""

    def __init__(self, params, cameras: List[Camera], targets, cfg: TrainingConfig = None, seed: int = 42):
        self.config = cfg or TrainingConfig()
        self.cameras = cameras
        self.targets = targets
        self.model = Model(params, self.config, len(cameras))
        self.current_step = 0
        self._rng = np.random.default_rng(seed)
        self._order = list(range(len(cameras)))
        self._pos = len(cameras)

    def _next_camera(self) -> int:
        if self._pos >= len(self._order):
            if self.config.shuffle_cameras:
                self._rng.shuffle(self._order)
            self._pos = 0
        i = self._order[self._pos]
        self._pos += 1
        return i

    def step(self, timed: bool = False) -> TrainingStats:
        self.current_step += 1
        ci = self._next_camera()
        t0 = time.perf_counter()
        self.model.full_iteration(self.cameras[ci], self.current_step, self.targets[ci])
        self.model.schedulers_step(self.current_step)
        self.model.after_train(self.current_step)
        if timed:
            device.sync()
        ms = (time.perf_counter() - t0) * 1e3
        return TrainingStats(self.current_step, self.model.num_active, ms)

    def splat_count(self) -> int:
        return self.model.num_active

    def render_from_pose(self, cam_to_world, ref_cam_idx: int = 0):
        """Render a pose with the intrinsics of reference camera ref_cam_idx -> (H, W, 3) numpy."""
        cw = np.asarray(cam_to_world, np.float32)
        if cw.size != 16:
            raise ValueError("cam_to_world must have 16 elements (4x4 matrix)")
        if not 0 <= ref_cam_idx < len(self.cameras):
            raise IndexError("ref_cam_idx out of range")
        ref = self.cameras[ref_cam_idx]
        cam = Camera(ref.width, ref.height, ref.fx, ref.fy, ref.cx, ref.cy, cw.reshape(4, 4))
        s = prepare_cam(cam, self.model.downscale_factor(self.current_step))
        img = device.render(self.model.g, s, self.model.degrees_to_use(self.current_step), self.model.background)
        return img.cpu().numpy()
