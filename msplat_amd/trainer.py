"""GaussianTrainer: Python face of the C++ trainer (include/msplat_trainer.h).

The model, its optimiser state, camera set-up and refinement policy live in
C++ (msplat_amd/host/model.cpp, trainer.cpp), mirroring the reference's
Model (core/src/model.cpp) and GaussianTrainer (python/bindings.cpp:101-280);
this module only marshals arguments through ctypes, as the reference's
nanobind module does for its C++ trainer.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from . import _abi, device
from .camera import Camera

LR_INIT = [0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05]   # model.cpp:138


@dataclass
class TrainingConfig:
    """TrainingConfig (python/bindings.cpp:25-46) plus the cull thresholds that
    model.cpp:263 hard-codes, the camera order and its seed."""

    iterations: int = 30000
    sh_degree: int = 3
    sh_degree_interval: int = 1000        # <= 0: all bands from the first step
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
    seed: int = 42

    def to_c(self) -> _abi.TrainerConfig:
        c = _abi.TrainerConfig()
        c.iterations, c.shDegree, c.shDegreeInterval = self.iterations, self.sh_degree, self.sh_degree_interval
        c.ssimWeight, c.numDownscales, c.resolutionSchedule = self.ssim_weight, self.num_downscales, \
            self.resolution_schedule
        c.refineEvery, c.warmupLength, c.resetAlphaEvery = self.refine_every, self.warmup_length, \
            self.reset_alpha_every
        c.densifyGradThresh, c.densifySizeThresh = self.densify_grad_thresh, self.densify_size_thresh
        c.stopScreenSizeAt, c.splitScreenSize = self.stop_screen_size_at, self.split_screen_size
        c.bgColor[:] = [float(v) for v in self.bg_color]
        c.cullAlphaThresh, c.cullScaleThresh, c.cullScreenSize = self.cull_alpha_thresh, \
            self.cull_scale_thresh, self.cull_screen_size
        c.shuffleCameras, c.seed = int(self.shuffle_cameras), self.seed
        return c


@dataclass
class TrainingStats:
    iteration: int
    splat_count: int
    ms_per_step: float


def _c_camera(cam: Camera) -> _abi.TrainerCamera:
    k = _abi.TrainerCamera()
    k.width, k.height = cam.width, cam.height
    k.fx, k.fy, k.cx, k.cy = cam.fx, cam.fy, cam.cx, cam.cy
    k.camToWorld[:] = [float(v) for v in np.asarray(cam.cam_to_world, np.float32).reshape(16)]
    return k


def _pose(cam_to_world):
    cw = np.ascontiguousarray(cam_to_world, np.float32)
    if cw.size != 16:
        raise ValueError("cam_to_world must have 16 elements (4x4 matrix)")
    return cw.reshape(16), cw.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class GaussianTrainer:
    """Trains gaussians against target images of given cameras.

    params: [means (N,3), scales (N,3) log, quats (N,4) wxyz, f_dc (N,3),
    f_rest (N,K-1,3), opacities (N,) or (N,1) logits] as numpy arrays or CUDA
    tensors; targets: one (H,W,3) float32 image per camera (numpy or CUDA).
    """

    def __init__(self, params, cameras=None, targets=None, cfg: Optional[TrainingConfig] = None):
        self._dataset = None
        if hasattr(params, "init_gaussians") and hasattr(params, "load_image"):
            # GaussianTrainer(dataset, config) as in the reference module
            # (python/bindings.cpp:113-167): the training cameras' images are
            # decoded and prepared on the GPU, the gaussians start from the
            # point cloud.
            ds = params
            cfg = cameras if isinstance(cameras, TrainingConfig) else cfg
            cfg = cfg or TrainingConfig()
            test = set(range(0, len(ds.cameras), ds.test_every)) if ds.eval_mode else set()
            loaded = [ds.load_image(i) for i in range(len(ds.cameras)) if i not in test]
            cameras, targets = [c for c, _ in loaded], [im for _, im in loaded]
            params = [device.to_dev(a) for a in ds.init_gaussians(cfg.sh_degree)]
            self._dataset = ds
        if cameras is None or targets is None:
            raise ValueError("cameras and targets are needed (or a Dataset)")
        self.config = cfg or TrainingConfig()
        self.cameras = list(cameras)
        lib = device.init()
        self._lib = lib
        on_dev = hasattr(params[0], "data_ptr")
        n = int(params[0].shape[0])
        keep = []
        if on_dev:
            device.torch().cuda.synchronize()   # the inputs come from torch's stream
            ps = [p.contiguous().float() for p in params]
            keep += ps
            pp = (ctypes.c_void_p * 6)(*[p.data_ptr() for p in ps])
            ts = [t.contiguous().float() for t in targets]
            keep += ts
            tp = (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])
        else:
            ps = [np.ascontiguousarray(p, np.float32) for p in params]
            keep += ps
            pp = (ctypes.c_void_p * 6)(*[p.ctypes.data for p in ps])
            ts = [np.ascontiguousarray(t, np.float32) for t in targets]
            keep += ts
            tp = (ctypes.c_void_p * len(ts))(*[t.ctypes.data for t in ts])
        for cam, t in zip(self.cameras, ts):
            if tuple(t.shape) != (cam.height, cam.width, 3):
                raise ValueError(f"target shape {tuple(t.shape)} does not match camera {cam.height}x{cam.width}")
        cams = (_abi.TrainerCamera * len(self.cameras))(*[_c_camera(c) for c in self.cameras])
        cfg_c = self.config.to_c()
        self._h = lib.msplat_trainer_create_from_arrays(ctypes.byref(cfg_c), n, pp, len(self.cameras), cams,
                                                        ctypes.cast(tp, ctypes.POINTER(ctypes.c_void_p)),
                                                        int(on_dev))
        if not self._h:
            raise _abi.MsplatError(lib.msplat_trainer_last_error().decode())
        if on_dev:
            device.sync()   # the copies above read the caller's tensors

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.msplat_trainer_destroy(h)
            self._h = None

    def step(self) -> TrainingStats:
        s = self._lib.msplat_trainer_step(self._h)
        if s.iteration < 0:
            raise _abi.MsplatError(self._lib.msplat_trainer_last_error().decode())
        return TrainingStats(s.iteration, s.splatCount, s.msPerStep)

    def splat_count(self) -> int:
        return int(self._lib.msplat_trainer_splat_count(self._h))

    @property
    def current_step(self) -> int:
        return int(self._lib.msplat_trainer_iteration(self._h))

    @property
    def iteration(self) -> int:
        return self.current_step

    def train(self, callback=None, callback_every: int = 0) -> None:
        """Steps until config.iterations, calling callback(stats) every
        callback_every steps (GaussianTrainer::train, python/bindings.cpp:169-177)."""
        while self.current_step < self.config.iterations:
            st = self.step()
            if callback is not None and callback_every > 0 and st.iteration % callback_every == 0:
                callback(st)

    def last_loss(self, wait: bool = False) -> float:
        return float(self._lib.msplat_trainer_last_loss(self._h, int(wait)))

    def _to_numpy(self, buf: _abi.PixelBuffer) -> np.ndarray:
        if not buf.data:
            raise _abi.MsplatError(self._lib.msplat_trainer_last_error().decode())
        try:
            return np.ctypeslib.as_array(buf.data, shape=(buf.height, buf.width, 3)).copy()
        finally:
            ctypes.CDLL(None).free(ctypes.cast(buf.data, ctypes.c_void_p))

    def render(self, camera_index: int) -> np.ndarray:
        if not 0 <= camera_index < len(self.cameras):
            raise IndexError("camera index out of range")
        return self._to_numpy(self._lib.msplat_trainer_render(self._h, camera_index, False))

    def render_from_pose(self, cam_to_world, ref_cam_idx: int = 0) -> np.ndarray:
        """Render a pose with the intrinsics of camera ref_cam_idx -> (H, W, 3) numpy."""
        if not 0 <= ref_cam_idx < len(self.cameras):
            raise IndexError("ref_cam_idx out of range")
        _, p = _pose(cam_to_world)
        return self._to_numpy(self._lib.msplat_trainer_render_pose(self._h, p, ref_cam_idx))

    def render_pose_device(self, cam_to_world, ref_cam_idx: int, out) -> None:
        """Render into a (H, W, 3) float32 CUDA tensor without a host copy or sync."""
        _, p = _pose(cam_to_world)
        w, h = ctypes.c_int32(0), ctypes.c_int32(0)
        rc = self._lib.msplat_trainer_render_pose_device(self._h, p, ref_cam_idx, out.data_ptr(),
                                                         ctypes.byref(w), ctypes.byref(h))
        if rc != 0:
            raise _abi.MsplatError(self._lib.msplat_trainer_last_error().decode())

    def render_from_pose_rgba8(self, cam_to_world, ref_cam_idx: int = 0) -> np.ndarray:
        """renderFromPoseToBuffer: (H, W, 4) uint8 display image (converted on the GPU)."""
        if not 0 <= ref_cam_idx < len(self.cameras):
            raise IndexError("ref_cam_idx out of range")
        _, p = _pose(cam_to_world)
        w, h = ctypes.c_int(0), ctypes.c_int(0)
        self._lib.msplat_trainer_render_pose_to_buffer(self._h, p, ref_cam_idx, None, ctypes.byref(w),
                                                       ctypes.byref(h))
        self._raise_on_error()
        out = np.empty((h.value, w.value, 4), np.uint8)
        self._lib.msplat_trainer_render_pose_to_buffer(self._h, p, ref_cam_idx, out.ctypes.data,
                                                       ctypes.byref(w), ctypes.byref(h))
        self._raise_on_error()
        return out

    def _raise_on_error(self) -> None:
        """Raise the message of the latest failed call (the reference's void
        calls report failures only through msplat_trainer_last_error)."""
        msg = self._lib.msplat_trainer_last_error()
        if msg:
            raise _abi.MsplatError(msg.decode())

    def evaluate(self, cameras: Optional[List[Camera]] = None, images=None) -> dict:
        """Metrics on held-out cameras (GaussianTrainer.evaluate, python/bindings.cpp:180-205):
        dict with psnr, ssim, l1, num_test, num_gaussians.  images: one
        full-resolution (H, W, 3) float32 target per camera (numpy).  Without
        arguments, a trainer made from a Dataset in eval mode uses its
        held-out cameras."""
        if cameras is None and images is None:
            ds = self._dataset
            if ds is None or not ds.eval_mode:
                raise ValueError("No test cameras. Load dataset with eval_mode=True.")
            loaded = [ds.load_image(i) for i in range(0, len(ds.cameras), ds.test_every)]
            cameras = [c for c, _ in loaded]
            images = [im.cpu().numpy() for _, im in loaded]
        if cameras is None or images is None or len(cameras) != len(images) or not cameras:
            raise ValueError("one image per test camera is needed")
        ims = [np.ascontiguousarray(im, np.float32) for im in images]
        for cam, im in zip(cameras, ims):
            if im.shape != (cam.height, cam.width, 3):
                raise ValueError("test image shape does not match its camera")
        cams = (_abi.TrainerCamera * len(cameras))(*[_c_camera(c) for c in cameras])
        ptrs = (ctypes.c_void_p * len(ims))(*[im.ctypes.data for im in ims])
        m = self._lib.msplat_trainer_evaluate_images(self._h, len(cameras), cams,
                                                     ctypes.cast(ptrs, ctypes.POINTER(ctypes.c_void_p)), 0)
        if m.numTest == 0:
            raise _abi.MsplatError(self._lib.msplat_trainer_last_error().decode())
        return {"psnr": m.psnr, "ssim": m.ssim, "l1": m.l1, "num_test": m.numTest,
                "num_gaussians": m.numGaussians}

    def _path_call(self, fn, path: str) -> int:
        rc = fn(self._h, str(path).encode())
        if rc < 0:
            raise _abi.MsplatError(self._lib.msplat_trainer_last_error().decode())
        return int(rc)

    def _void_path_call(self, fn, path: str) -> None:
        fn(self._h, str(path).encode())
        self._raise_on_error()

    def export_ply(self, path: str) -> None:
        self._void_path_call(self._lib.msplat_trainer_export_ply, path)

    def export_splat(self, path: str) -> None:
        self._void_path_call(self._lib.msplat_trainer_export_splat, path)

    def save_checkpoint(self, path: str) -> None:
        self._void_path_call(self._lib.msplat_trainer_save_checkpoint, path)

    def load_checkpoint(self, path: str) -> int:
        """Restore a checkpoint; returns its step (training continues after it)."""
        return self._path_call(self._lib.msplat_trainer_load_checkpoint, path)

    def load_ply(self, path: str) -> int:
        """Replace the gaussians by an exported PLY (restarting the optimiser);
        returns the step recorded in the file."""
        return self._path_call(self._lib.msplat_trainer_load_ply, path)

    def set_crs(self, scale: float, translation, keep: bool = True) -> None:
        t = (ctypes.c_float * 3)(*[float(v) for v in translation])
        if self._lib.msplat_trainer_set_crs(self._h, float(scale), t, int(keep)) != 0:
            raise ValueError("bad coordinate normalisation")

    def group(self, g: int, which: int = 0) -> np.ndarray:
        """Host copy of the active rows of parameter group g (which=0) or of its
        Adam moments (1, 2)."""
        ptr, rows, per = ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_int64()
        rc = self._lib.msplat_trainer_group(self._h, g, which, ctypes.byref(ptr), ctypes.byref(rows),
                                            ctypes.byref(per))
        if rc != 0:
            raise _abi.MsplatError(self._lib.msplat_trainer_last_error().decode())
        out = np.empty((rows.value, per.value), np.float32)
        if out.size:
            _abi.check(self._lib.msplat_hip_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), ptr, out.nbytes))
        return out

    def params(self) -> list:
        return [self.group(g) for g in range(6)]
