"""Target-image steps on the GPU against the oracle, bit for bit: the area
resize (msplat_hip_resize_area; resizeArea, image_io.cpp:91-138) at the
training pyramid's integer factors, at a load-time fractional factor, on
non-divisible sizes, upscaling and 1x1; the undistortion
(msplat_undistort_roi + msplat_hip_undistort; undistortImage,
image_io.cpp:140-330) for barrel, pincushion with tangential terms and zero
distortion, plus argument checks.  The oracle's functions are pinned in
tests/test_image_cpu.py.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import orc
from helpers import assert_bits_equal

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from msplat_amd import _abi, device
    device.init(0)
    return torch, device, _abi


RESIZES = [(1297, 840, 648, 420), (1297, 840, 324, 210), (1297, 840, 864, 560), (97, 61, 48, 30),
           (10, 7, 23, 15), (1, 1, 1, 1), (4946, 3286, 1236, 821)]


@pytest.mark.parametrize("sw,sh,dw,dh", RESIZES)
def test_resize_area_matches_oracle(mods, sw, sh, dw, dh):
    torch, device, _abi = mods
    print(f"resize {sw}x{sh} -> {dw}x{dh}", flush=True)
    img = np.random.default_rng(sw + dh).random((sh, sw, 3), dtype=np.float32)
    src = torch.from_numpy(img).cuda()
    dst = torch.empty((dh, dw, 3), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    _abi.check(device.init().msplat_hip_resize_area(device.ptr(src), sw, sh, device.ptr(dst), dw, dh))
    device.sync()
    assert_bits_equal(dst.cpu().numpy(), orc.resize_area(img, dw, dh), f"resize {sw}x{sh}->{dw}x{dh}")


CAMS = [
    (160, 120, [150.0, 152.0, 80.5, 59.5], [-0.12, 0.03, 1e-3, -5e-4, 0.0]),
    (160, 120, [140.0, 140.0, 78.0, 61.0], [0.08, -0.01, -2e-3, 1e-3, 0.002]),
    (97, 61, [90.0, 90.0, 48.0, 30.0], [0.0, 0.0, 0.0, 0.0, 0.0]),
    (1297, 840, [1150.0, 1148.0, 648.3, 419.7], [-0.051, 0.012, 2e-4, -1e-4, 0.0]),
]


def _f(a):
    a = np.ascontiguousarray(a, np.float32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


@pytest.mark.parametrize("cam", range(len(CAMS)))
def test_undistort_matches_oracle(mods, cam):
    torch, device, _abi = mods
    w, h, intr, dist = CAMS[cam]
    print(f"undistort {w}x{h} dist={dist}", flush=True)
    img = np.random.default_rng(cam).random((h, w, 3), dtype=np.float32)
    want, want_roi = orc.undistort(img, intr, dist)
    lib = device.init()
    ia, ip = _f(intr)
    da, dp = _f(dist)
    roi = (ctypes.c_int32 * 4)()
    _abi.check(lib.msplat_undistort_roi(w, h, ip, dp, roi))
    assert list(roi) == list(want_roi)
    src = torch.from_numpy(img).cuda()
    dst = torch.empty((roi[3], roi[2], 3), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    _abi.check(lib.msplat_hip_undistort(device.ptr(src), w, h, ip, dp, roi, device.ptr(dst)))
    device.sync()
    assert_bits_equal(dst.cpu().numpy(), want, f"undistort cam {cam}")


def test_image_arguments_rejected(mods):
    torch, device, _abi = mods
    lib = device.init()
    x = torch.zeros((8, 8, 3), dtype=torch.float32, device="cuda")
    y = torch.zeros((8, 8, 3), dtype=torch.float32, device="cuda")
    assert lib.msplat_hip_resize_area(device.ptr(x), 8, 8, device.ptr(y), 0, 8) == -1
    assert lib.msplat_hip_resize_area(None, 8, 8, device.ptr(y), 4, 4) == -1
    ia, ip = _f([0.0, 10.0, 4.0, 4.0])
    da, dp = _f([0.1, 0, 0, 0, 0])
    roi = (ctypes.c_int32 * 4)()
    assert lib.msplat_undistort_roi(8, 8, ip, dp, roi) == -1          # fx = 0
    ia, ip = _f([10.0, 10.0, 4.0, 4.0])
    bad = (ctypes.c_int32 * 4)(2, 2, 7, 3)                             # x + w > width
    assert lib.msplat_hip_undistort(device.ptr(x), 8, 8, ip, dp, bad, device.ptr(y)) == -1
    assert b"outside" in lib.msplat_hip_last_error()


def test_load_camera_image(mods, tmp_path):
    """Camera::loadImage (input_data.cpp:17-52): file smaller than the
    camera's metadata (intrinsics rescaled), load-time downscale 1.5 by area
    resize, then undistortion; camera and pixels against the oracle chain."""
    torch, device, _abi = mods
    from PIL import Image
    from msplat_amd import image_io
    from msplat_amd.camera import Camera
    b = np.random.default_rng(11).integers(0, 256, (121, 161, 3), dtype=np.uint8)
    Image.fromarray(b, "RGB").save(tmp_path / "im.png")
    cam = Camera(width=322, height=242, fx=300.0, fy=301.0, cx=160.7, cy=120.2)
    dist = [-0.08, 0.01, 5e-4, -3e-4]
    got_cam, got = image_io.load_camera_image(str(tmp_path / "im.png"), cam, dist, downscale=1.5)
    f = np.float32
    sx, sy = f(161) / f(322), f(121) / f(242)
    fx, fy, cx, cy = f(300.0) * sx, f(301.0) * sy, f(160.7) * sx, f(120.2) * sy
    nw, nh = int(f(161) / f(1.5)), int(f(121) / f(1.5))
    s = f(1.0) / f(1.5)
    fx, fy, cx, cy = fx * s, fy * s, cx * s, cy * s
    small = orc.resize_area(b.astype(np.float32) / f(255), nw, nh)
    want, roi = orc.undistort(small, [fx, fy, cx, cy], dist + [0.0])
    assert (got_cam.width, got_cam.height) == (int(roi[2]), int(roi[3]))
    assert [f(got_cam.fx), f(got_cam.fy), f(got_cam.cx), f(got_cam.cy)] == \
        [fx, fy, cx - f(roi[0]), cy - f(roi[1])]
    device.sync()
    assert_bits_equal(got.cpu().numpy(), want, "loadImage chain")
