"""msplat_hip_image_metrics_noalloc against msplat_hip_image_metrics.

The allocation-free variant runs the same metric kernels with its partial
sums in the library's fixed per-GPU workspace, so its PSNR / SSIM / L1 must
equal the allocating entry point's bit for bit.  Two calls in a row, the
second on a smaller image (the workspace keeps the first call's partials,
which must not leak into the second), plus an image beyond the workspace,
which is rejected before any kernel runs.  Both entry points are called
through the C ABI.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from msplat_amd import device
    return device.init(0)


def _images(h, w, seed):
    import torch
    g = torch.Generator().manual_seed(seed)
    img = torch.rand((h, w, 3), generator=g, dtype=torch.float32)
    gt = (img + 0.1 * torch.randn((h, w, 3), generator=g, dtype=torch.float32)).clamp_(0, 1)
    return img.cuda().contiguous(), gt.cuda().contiguous()


def _call(lib, fn, img, gt, ws=11, sigma=1.5):
    from msplat_amd import _abi
    h, w = int(img.shape[0]), int(img.shape[1])
    m = _abi.ImageMetrics()
    rc = getattr(lib, fn)(ctypes.c_void_p(img.data_ptr()), ctypes.c_void_p(gt.data_ptr()), h, w, ws,
                          ctypes.c_float(sigma), ctypes.byref(m))
    return rc, (m.psnr, m.ssim, m.l1)


def _bits(t):
    return np.array(t, np.float32).view(np.uint32).tolist()


def test_noalloc_metrics_match_allocating_entry_point(lib):
    import torch
    cases = [(1680, 2594, 11, 1.5, 7), (93, 167, 11, 1.5, 8), (93, 167, 7, 1.0, 9)]
    for h, w, ws, sigma, seed in cases:
        print(f"noalloc metrics: {w}x{h} window {ws}", flush=True)
        img, gt = _images(h, w, seed)
        rc_n, got = _call(lib, "msplat_hip_image_metrics_noalloc", img, gt, ws, sigma)
        assert rc_n == 0, lib.msplat_hip_last_error()
        rc_a, want = _call(lib, "msplat_hip_image_metrics", img, gt, ws, sigma)
        assert rc_a == 0, lib.msplat_hip_last_error()
        assert _bits(got) == _bits(want), (w, h, got, want)
        assert 0.0 < got[1] < 1.0 and got[2] > 0.0
        torch.cuda.synchronize()


def test_noalloc_metrics_rejects_images_beyond_the_workspace(lib):
    img, gt = _images(16, 16, 3)
    from msplat_amd import _abi
    m = _abi.ImageMetrics()
    # 8256 x 8192 needs 129 x 512 = 66048 tiles of 64 x 16 pixels (> 65536);
    # rejected on the host before any kernel reads the (small) images
    rc = lib.msplat_hip_image_metrics_noalloc(ctypes.c_void_p(img.data_ptr()), ctypes.c_void_p(gt.data_ptr()),
                                              8192, 8256, 11, ctypes.c_float(1.5), ctypes.byref(m))
    assert rc == -1
    assert b"allocation-free workspace" in lib.msplat_hip_last_error()
    # the workspace still serves a call after the rejection
    rc, got = _call(lib, "msplat_hip_image_metrics_noalloc", img, gt)
    assert rc == 0
    _, want = _call(lib, "msplat_hip_image_metrics", img, gt)
    assert _bits(got) == _bits(want)
