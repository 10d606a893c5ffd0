"""Camera images: decode / encode and the load-time preparation of a target
image (Camera::loadImage, input_data.cpp:17-52).

* imread_rgb (imreadRGB, image_io.cpp:12-50): float32 RGB in [0, 1], each
  byte / 255, transparent pixels drawn over black as the reference's
  CoreGraphics context without alpha draws them.  PNG and JPEG are decoded
  by the library itself (msplat_image_read: the same samples as libjpeg's
  default decoding for JPEG; the reference's closed decoder may differ in
  the last bit of a JPEG sample); other formats by Pillow.
* imwrite_rgb (imwriteRGB, image_io.cpp:54-89): PNG, each channel
  clamp(v * 255, 0, 255) + 0.5 truncated to a byte.
* load_camera_image: the decoded image on the GPU, the camera's intrinsics
  rescaled when the file's size differs from the camera's, then the optional
  load-time downscale by an area resize and the undistortion of Brown-Conrady
  cameras (msplat_hip_resize_area, msplat_undistort_roi,
  msplat_hip_undistort), with the camera updated as the reference updates
  it.  Intrinsics arithmetic is fp32, as in the reference.
"""
from __future__ import annotations

import ctypes
from dataclasses import replace
from typing import Optional, Sequence, Tuple

import numpy as np

from . import _abi
from .camera import Camera

F32 = np.float32


def imread_rgb(path: str) -> np.ndarray:
    with open(path, "rb") as f:
        sig = f.read(8)
    if sig.startswith(b"\x89PNG\r\n\x1a\n") or sig.startswith(b"\xff\xd8\xff"):
        lib = _abi.load()
        rgb = ctypes.POINTER(ctypes.c_float)()
        w, h = ctypes.c_int32(0), ctypes.c_int32(0)
        if lib.msplat_image_read(path.encode(), ctypes.byref(rgb), ctypes.byref(w), ctypes.byref(h)) != 0:
            raise RuntimeError(lib.msplat_trainer_last_error().decode())
        try:
            return np.ctypeslib.as_array(rgb, shape=(h.value, w.value, 3)).copy()
        finally:
            ctypes.CDLL(None).free(ctypes.cast(rgb, ctypes.c_void_p))
    from PIL import Image
    with Image.open(path) as im:
        rgba = np.asarray(im.convert("RGBA"), dtype=np.uint32)
    rgb = (rgba[..., :3] * rgba[..., 3:] + 127) // 255   # over black
    return rgb.astype(np.float32) / np.float32(255.0)


def imwrite_rgb(path: str, img: np.ndarray) -> None:
    from PIL import Image
    v = np.clip(np.asarray(img, np.float32) * F32(255.0), F32(0.0), F32(255.0))
    Image.fromarray((v + F32(0.5)).astype(np.uint8), "RGB").save(path, format="PNG")


def _f32p(a) -> Tuple[np.ndarray, ctypes.POINTER(ctypes.c_float)]:
    a = np.ascontiguousarray(a, np.float32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def resize_area(img, width: int, height: int):
    """Area resize of a CUDA (H, W, 3) float32 tensor to (height, width, 3)."""
    from . import device
    lib = device.init()
    torch = device.torch()
    src = img.contiguous()
    out = torch.empty((height, width, 3), dtype=torch.float32, device=src.device)
    _abi.check(lib.msplat_hip_resize_area(device.ptr(src), src.shape[1], src.shape[0],
                                          device.ptr(out), width, height))
    return out


def undistort(img, cam: Camera, distortion: Sequence[float]):
    """(cropped undistorted image, roi {x, y, w, h}) of a CUDA (H, W, 3)
    image; distortion = k1 k2 p1 p2 [k3]."""
    from . import device
    lib = device.init()
    torch = device.torch()
    d = list(distortion) + [0.0] * (5 - len(distortion))
    ia, ip = _f32p([cam.fx, cam.fy, cam.cx, cam.cy])
    da, dp = _f32p(d)
    h, w = img.shape[:2]
    roi = (ctypes.c_int32 * 4)()
    _abi.check(lib.msplat_undistort_roi(w, h, ip, dp, roi))
    src = img.contiguous()
    out = torch.empty((roi[3], roi[2], 3), dtype=torch.float32, device=src.device)
    _abi.check(lib.msplat_hip_undistort(device.ptr(src), w, h, ip, dp, roi, device.ptr(out)))
    return out, tuple(roi)


def load_camera_image(path: str, cam: Camera, distortion: Optional[Sequence[float]] = None,
                      downscale: float = 1.0):
    """Camera::loadImage: (updated camera, CUDA (H, W, 3) float32 image)."""
    from . import device
    raw = imread_rgb(path)
    img = device.to_dev(raw)
    h, w = raw.shape[:2]
    fx, fy, cx, cy = F32(cam.fx), F32(cam.fy), F32(cam.cx), F32(cam.cy)
    width, height = cam.width, cam.height
    if width > 0 and height > 0 and (w != width or h != height):
        sx, sy = F32(w) / F32(width), F32(h) / F32(height)
        fx, fy, cx, cy = fx * sx, fy * sy, cx * sx, cy * sy
        width, height = w, h
    elif width == 0 or height == 0:
        width, height = w, h
    ds = F32(downscale)
    if ds > F32(1.0):
        nw, nh = int(F32(width) / ds), int(F32(height) / ds)
        img = resize_area(img, nw, nh)
        s = F32(1.0) / ds
        fx, fy, cx, cy = fx * s, fy * s, cx * s, cy * s
        width, height = nw, nh
    d = [float(v) for v in (distortion if distortion is not None else [])]
    if any(v != 0.0 for v in d):
        cur = replace(cam, width=width, height=height, fx=float(fx), fy=float(fy), cx=float(cx), cy=float(cy))
        img, (rx, ry, rw, rh) = undistort(img, cur, d)
        cx, cy = cx - F32(rx), cy - F32(ry)
        width, height = rw, rh
    out = replace(cam, width=int(width), height=int(height), fx=float(fx), fy=float(fy),
                  cx=float(cx), cy=float(cy))
    return out, img
