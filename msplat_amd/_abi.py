"""ctypes binding of the C ABI in include/msplat_hip.h (libmsplat_hip.so).

The library is built in-tree by ``make -C msplat_amd`` (see __graft_entry__.build).
There is no fallback: if the shared object is missing or fails to load, every
entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_bool, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_uint64, c_void_p

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmsplat_hip.so")


class RenderArgs(ctypes.Structure):
    """MsplatRenderArgs — everything msplat_render takes (bindings.h:37-46)."""

    _fields_ = [
        ("num_points", c_int32),
        ("means3d", c_void_p),
        ("scales", c_void_p),
        ("glob_scale", c_float),
        ("quats", c_void_p),
        ("viewmat", c_float * 16),
        ("projmat", c_float * 16),
        ("fx", c_float), ("fy", c_float), ("cx", c_float), ("cy", c_float),
        ("img_height", c_uint32), ("img_width", c_uint32),
        ("tile_bounds", c_int32 * 3),
        ("clip_thresh", c_float),
        ("degree", c_uint32),
        ("degrees_to_use", c_uint32),
        ("cam_pos", c_float * 3),
        ("features_dc", c_void_p),
        ("features_rest", c_void_p),
        ("opacities", c_void_p),
        ("background", c_float * 3),
    ]


class TrainArgs(ctypes.Structure):
    """MsplatTrainArgs — everything msplat_train_step takes (bindings.h:50-67)."""

    _fields_ = [
        ("r", RenderArgs),
        ("gt", c_void_p),
        ("ssim_weight", c_float),
        ("loss_inv_n", c_float),
        ("features_rest_bases", c_int32),
        ("num_adam_groups", c_int32),
        ("adam_params", c_void_p * 6),
        ("adam_exp_avg", c_void_p * 6),
        ("adam_exp_avg_sq", c_void_p * 6),
        ("adam_step_sizes", c_float * 6),
        ("adam_bc2_sqrts", c_float * 6),
        ("adam_beta1", c_float), ("adam_beta2", c_float), ("adam_eps", c_float),
        ("vis_counts", c_void_p),
        ("xys_grad_norm", c_void_p),
        ("max_2d_size", c_void_p),
        ("inv_max_dim", c_float),
        ("v_mean3d_out", c_void_p),
        ("v_scale_out", c_void_p),
        ("v_quat_out", c_void_p),
    ]


class DensifyArgs(ctypes.Structure):
    """MsplatDensifyArgs — msplat_densify's arguments (bindings.h:69-84)."""

    _fields_ = [
        ("N", c_int32),
        ("buf_capacity", c_int32),
        ("grad_thresh", c_float), ("size_thresh", c_float), ("screen_thresh", c_float),
        ("check_screen", c_int32),
        ("cull_alpha_thresh", c_float), ("cull_scale_thresh", c_float), ("cull_screen_size", c_float),
        ("check_huge", c_int32),
        ("xys_grad_norm", c_void_p),
        ("vis_counts", c_void_p),
        ("max_2d_size", c_void_p),
        ("half_max_dim", c_float),
        ("bufs", c_void_p * 6),
        ("fr_stride", c_int32),
        ("adam_exp_avg_buf", c_void_p * 6),
        ("adam_exp_avg_sq_buf", c_void_p * 6),
        ("random_samples", c_void_p),
        ("seed", c_uint64),
    ]


class TrainerConfig(ctypes.Structure):
    """MsplatTrainerConfig (include/msplat_trainer.h)."""

    _fields_ = [
        ("iterations", c_int32), ("shDegree", c_int32), ("shDegreeInterval", c_int32),
        ("ssimWeight", c_float), ("numDownscales", c_int32), ("resolutionSchedule", c_int32),
        ("refineEvery", c_int32), ("warmupLength", c_int32), ("resetAlphaEvery", c_int32),
        ("densifyGradThresh", c_float), ("densifySizeThresh", c_float), ("stopScreenSizeAt", c_int32),
        ("splitScreenSize", c_float), ("bgColor", c_float * 3),
        ("cullAlphaThresh", c_float), ("cullScaleThresh", c_float), ("cullScreenSize", c_float),
        ("shuffleCameras", c_int32), ("seed", c_uint32),
    ]


class Config(ctypes.Structure):
    """MsplatConfig (include/msplat_c_api.h, the reference's layout)."""

    _fields_ = [
        ("iterations", c_int), ("shDegree", c_int), ("shDegreeInterval", c_int),
        ("ssimWeight", c_float), ("numDownscales", c_int), ("resolutionSchedule", c_int),
        ("refineEvery", c_int), ("warmupLength", c_int), ("resetAlphaEvery", c_int),
        ("densifyGradThresh", c_float), ("densifySizeThresh", c_float), ("stopScreenSizeAt", c_int),
        ("splitScreenSize", c_float), ("keepCrs", c_bool), ("downscaleFactor", c_float),
        ("bgColor", c_float * 3),
    ]


def default_config() -> Config:
    """msplat_default_config() (a static inline function of the header)."""
    c = Config()
    c.iterations, c.shDegree, c.shDegreeInterval, c.ssimWeight = 30000, 3, 1000, 0.2
    c.numDownscales, c.resolutionSchedule, c.refineEvery, c.warmupLength = 2, 3000, 100, 500
    c.resetAlphaEvery, c.densifyGradThresh, c.densifySizeThresh = 30, 0.0002, 0.01
    c.stopScreenSizeAt, c.splitScreenSize, c.keepCrs, c.downscaleFactor = 4000, 0.05, False, 1.0
    c.bgColor[:] = [0.6130, 0.0101, 0.3984]
    return c


# int (*)(const char* path, float** rgb, int* width, int* height)
ImageDecoder = ctypes.CFUNCTYPE(c_int, c_char_p, POINTER(POINTER(c_float)), POINTER(c_int), POINTER(c_int))


class TrainerCamera(ctypes.Structure):
    """MsplatTrainerCamera (include/msplat_trainer.h)."""

    _fields_ = [("width", c_int32), ("height", c_int32), ("fx", c_float), ("fy", c_float),
                ("cx", c_float), ("cy", c_float), ("camToWorld", c_float * 16)]


class CamSetupC(ctypes.Structure):
    """MsplatCamSetup (include/msplat_trainer.h)."""

    _fields_ = [("fx", c_float), ("fy", c_float), ("cx", c_float), ("cy", c_float),
                ("width", c_int32), ("height", c_int32), ("viewmat", c_float * 16), ("projmat", c_float * 16),
                ("cam_pos", c_float * 3), ("tile_bounds", c_int32 * 3)]


class Stats(ctypes.Structure):
    """MsplatStats (include/msplat_c_api.h)."""

    _fields_ = [("iteration", c_int32), ("splatCount", c_int32), ("msPerStep", c_float)]


class PixelBuffer(ctypes.Structure):
    """MsplatPixelBuffer (include/msplat_c_api.h)."""

    _fields_ = [("data", POINTER(c_float)), ("width", c_int32), ("height", c_int32)]


class ImageMetrics(ctypes.Structure):
    """MsplatImageMetrics (include/msplat_hip.h)."""

    _fields_ = [("psnr", c_float), ("ssim", c_float), ("l1", c_float)]


class EvalMetrics(ctypes.Structure):
    """MsplatEvalMetrics (include/msplat_c_api.h)."""

    _fields_ = [("psnr", c_float), ("ssim", c_float), ("l1", c_float), ("numTest", c_int32),
                ("numGaussians", c_int32)]


# (name, restype, argtypes) for every symbol declared in include/msplat_hip.h,
# include/msplat_c_api.h and include/msplat_trainer.h
SIGNATURES = [
    ("msplat_hip_init", c_int, [c_int]),
    ("msplat_hip_shutdown", c_int, []),
    ("msplat_hip_last_error", c_char_p, []),
    ("msplat_hip_set_stream", c_int, [c_void_p]),
    ("msplat_hip_get_stream", c_void_p, []),
    ("msplat_hip_alloc", c_int, [POINTER(c_void_p), c_size_t]),
    ("msplat_hip_free", c_int, [c_void_p]),
    ("msplat_hip_memset", c_int, [c_void_p, c_int, c_size_t]),
    ("msplat_hip_memcpy_h2d", c_int, [c_void_p, c_void_p, c_size_t]),
    ("msplat_hip_memcpy_d2h", c_int, [c_void_p, c_void_p, c_size_t]),
    ("msplat_hip_memcpy_d2d", c_int, [c_void_p, c_void_p, c_size_t]),
    ("msplat_hip_alloc_mapped", c_int, [POINTER(c_void_p), c_size_t]),
    ("msplat_hip_free_mapped", c_int, [c_void_p]),
    ("msplat_hip_commit", c_int, []),
    ("msplat_hip_sync", c_int, []),
    ("msplat_hip_render", c_int, [POINTER(RenderArgs), c_void_p]),
    ("msplat_hip_train_step", c_int, [POINTER(TrainArgs), c_void_p, POINTER(c_float)]),
    ("msplat_hip_last_loss", c_int, [POINTER(c_float), c_int]),
    ("msplat_hip_densify", c_int, [POINTER(DensifyArgs), POINTER(c_int32)]),
    ("msplat_hip_randn", c_int, [c_void_p, c_int64, c_uint64]),
    ("msplat_hip_clamp_max", c_int, [c_void_p, c_int64, c_float]),
    ("msplat_hip_enable_stage_timing", c_int, [c_int]),
    ("msplat_hip_set_stage_timing_mask", c_int, [c_uint32]),
    ("msplat_hip_drain_stage_times", c_int,
     [POINTER(c_double), POINTER(c_int64), POINTER(c_char_p), c_int, POINTER(c_int), POINTER(c_int64)]),
    ("msplat_hip_copy_intermediate", c_int, [c_char_p, c_void_p, POINTER(c_size_t)]),
    ("msplat_hip_raster_work", c_int, [POINTER(c_int64)]),
    ("msplat_hip_drain_call_times", c_int, [POINTER(c_double), c_int, POINTER(c_int)]),
    ("msplat_hip_drain_raster_counters", c_int, [POINTER(c_int64)]),
    ("msplat_hip_image_to_rgba8", c_int, [c_void_p, c_int64, c_void_p]),
    ("msplat_hip_knn_mean_dist", c_int, [c_void_p, c_int64, c_void_p]),
    ("msplat_hip_resize_area", c_int, [c_void_p, c_int32, c_int32, c_void_p, c_int32, c_int32]),
    ("msplat_undistort_roi", c_int, [c_int32, c_int32, POINTER(c_float), POINTER(c_float), POINTER(c_int32)]),
    ("msplat_hip_undistort", c_int,
     [c_void_p, c_int32, c_int32, POINTER(c_float), POINTER(c_float), POINTER(c_int32), c_void_p]),
    ("msplat_hip_image_metrics", c_int,
     [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_float, POINTER(ImageMetrics)]),
    ("msplat_hip_image_metrics_noalloc", c_int,
     [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_float, POINTER(ImageMetrics)]),
    # include/msplat_c_api.h (the reference's C API)
    ("msplat_dataset_create", c_void_p, [c_char_p, c_float, c_bool, c_int]),
    ("msplat_dataset_destroy", None, [c_void_p]),
    ("msplat_dataset_num_train", c_int, [c_void_p]),
    ("msplat_dataset_num_test", c_int, [c_void_p]),
    ("msplat_trainer_create", c_void_p, [c_void_p, Config]),
    ("msplat_trainer_destroy", None, [c_void_p]),
    ("msplat_trainer_step", Stats, [c_void_p]),
    ("msplat_trainer_train", None, [c_void_p]),
    ("msplat_trainer_evaluate", EvalMetrics, [c_void_p]),
    ("msplat_trainer_render", PixelBuffer, [c_void_p, c_int, c_bool]),
    ("msplat_trainer_render_pose", PixelBuffer, [c_void_p, POINTER(c_float), c_int]),
    ("msplat_trainer_render_pose_to_buffer", None,
     [c_void_p, POINTER(c_float), c_int, c_void_p, POINTER(c_int), POINTER(c_int)]),
    ("msplat_trainer_export_ply", None, [c_void_p, c_char_p]),
    ("msplat_trainer_export_splat", None, [c_void_p, c_char_p]),
    ("msplat_trainer_save_checkpoint", None, [c_void_p, c_char_p]),
    ("msplat_trainer_load_checkpoint", c_int, [c_void_p, c_char_p]),
    ("msplat_trainer_splat_count", c_int, [c_void_p]),
    ("msplat_trainer_iteration", c_int, [c_void_p]),
    ("msplat_dataset_camera_pose", None, [c_void_p, c_int, POINTER(c_float)]),
    ("msplat_set_metallib_path", None, [c_char_p]),
    ("msplat_sync", None, []),
    ("msplat_cleanup", None, []),
    # include/msplat_trainer.h
    ("msplat_trainer_create_from_arrays", c_void_p,
     [POINTER(TrainerConfig), c_int64, c_void_p * 6, c_int32, POINTER(TrainerCamera), POINTER(c_void_p), c_int32]),
    ("msplat_trainer_last_error", c_char_p, []),
    ("msplat_trainer_last_loss", c_float, [c_void_p, c_int32]),
    ("msplat_trainer_render_pose_device", c_int32,
     [c_void_p, POINTER(c_float), c_int32, c_void_p, POINTER(c_int32), POINTER(c_int32)]),
    ("msplat_prepare_cam", c_int32, [POINTER(TrainerCamera), c_int32, POINTER(CamSetupC)]),
    ("msplat_trainer_evaluate_images", EvalMetrics,
     [c_void_p, c_int32, POINTER(TrainerCamera), POINTER(c_void_p), c_int32]),
    ("msplat_trainer_load_ply", c_int32, [c_void_p, c_char_p]),
    ("msplat_trainer_set_crs", c_int32, [c_void_p, c_float, POINTER(c_float), c_int32]),
    ("msplat_scene_write_ply", c_int32,
     [c_char_p, c_int64, c_int32, c_void_p * 6, c_float, POINTER(c_float), c_int32, c_int32]),
    ("msplat_scene_write_splat", c_int32,
     [c_char_p, c_int64, c_int32, c_void_p * 6, c_float, POINTER(c_float), c_int32]),
    ("msplat_scene_read_ply", c_int32,
     [c_char_p, c_float, POINTER(c_float), c_int32, POINTER(c_int64), POINTER(c_int32),
      POINTER(c_int32), POINTER(c_void_p)]),
    ("msplat_dataset_open_colmap", c_void_p, [c_char_p, c_char_p]),
    ("msplat_dataset_num_cameras", c_int32, [c_void_p]),
    ("msplat_dataset_camera", c_int32,
     [c_void_p, c_int32, POINTER(TrainerCamera), POINTER(c_float), POINTER(c_char_p)]),
    ("msplat_dataset_num_points", c_int64, [c_void_p]),
    ("msplat_dataset_points", c_int32, [c_void_p, c_void_p, c_void_p]),
    ("msplat_dataset_normalisation", c_int32, [c_void_p, POINTER(c_float), POINTER(c_float)]),
    ("msplat_dataset_init_gaussians", c_int32, [c_void_p, c_int32, c_void_p * 6]),
    ("msplat_trainer_group", c_int32,
     [c_void_p, c_int32, c_int32, POINTER(c_void_p), POINTER(c_int64), POINTER(c_int64)]),
    ("msplat_set_image_decoder", None, [ImageDecoder]),
    ("msplat_image_read", c_int32, [c_char_p, POINTER(POINTER(c_float)), POINTER(c_int32), POINTER(c_int32)]),
]

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libmsplat_hip.so (once) and declare its signatures.  Raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build the HIP extension first (python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(path)
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class MsplatError(RuntimeError):
    pass


def check(rc: int) -> None:
    if rc != 0:
        msg = load().msplat_hip_last_error()
        raise MsplatError(f"msplat_hip error {rc}: {msg.decode() if msg else ''}")
