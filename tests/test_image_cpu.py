"""Pins of the oracle's target-image steps (CPU): area resize
(resizeArea, image_io.cpp:91-138) and Brown-Conrady undistortion
(undistortImage, image_io.cpp:140-330).

The reference's image_io.cpp includes CoreGraphics, so it does not build
here; the oracle's restatement is pinned by methods that share none of its
code:
* resize: a float64 matrix form (exact overlap weights of every output row /
  column, between cell edges rounded to fp32 like the reference's, as two
  dense matrices, out = Wy . img . Wx^T normalised by the weight sums;
  equal up to the fp32 accumulation) on non-square, non-divisible sizes, so a swapped axis, a
  dropped edge fraction or an off-by-one footprint fails; identity sizes copy
  exactly; a 2x box mean of known values; constant images stay constant;
* undistortion: the remap checked against a float64 numpy bilinear sampler at
  the forward-distorted coordinates; a linear ramp is reproduced at the
  sample positions (catches x/y transposition); zero distortion is the
  identity; the crop rectangle agrees within one pixel with one found from a
  float64 Newton inverse of the distortion on the image borders, and lies in
  the image.
"""
from __future__ import annotations

import numpy as np
import pytest

import orc


def _weights(n_src: int, n_dst: int) -> np.ndarray:
    """Exact overlap of destination cell [d*s, (d+1)*s) with source pixel [i, i+1),
    the cell edges rounded to fp32 as the reference forms them."""
    s = np.float32(n_src) / np.float32(n_dst)
    w = np.zeros((n_dst, n_src))
    for d in range(n_dst):
        a, b = float(np.float32(d) * s), float(np.float32(d + 1) * s)
        for i in range(int(np.floor(a)), min(int(np.ceil(b)), n_src)):
            w[d, i] = max(0.0, min(i + 1, b) - max(i, a))
    return w


@pytest.mark.parametrize("sw,sh,dw,dh", [(97, 61, 48, 30), (97, 61, 24, 15), (1297, 840, 648, 420),
                                         (50, 37, 33, 24), (10, 7, 23, 15), (64, 64, 64, 32)])
def test_resize_matches_float64_matrix_form(sw, sh, dw, dh):
    rng = np.random.default_rng(sw * 7 + dh)
    img = rng.random((sh, sw, 3), dtype=np.float32)
    got = orc.resize_area(img, dw, dh)
    wy, wx = _weights(sh, dh), _weights(sw, dw)
    rows = np.tensordot(wy, img.astype(np.float64), axes=(1, 0))          # (dh, sw, 3)
    want = np.tensordot(rows, wx, axes=(1, 1)).transpose(0, 2, 1)         # (dh, dw, 3)
    want /= (wy.sum(1)[:, None] * wx.sum(1)[None, :])[..., None]
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-7)


def test_resize_identity_and_box_mean():
    rng = np.random.default_rng(3)
    img = rng.random((13, 17, 3), dtype=np.float32)
    assert np.array_equal(orc.resize_area(img, 17, 13), img)
    v = np.arange(4 * 4 * 3, dtype=np.float32).reshape(4, 4, 3)
    want = v.reshape(2, 2, 2, 2, 3).mean(axis=(1, 3))
    assert np.array_equal(orc.resize_area(v, 2, 2), want.astype(np.float32))


def test_resize_constant_image():
    img = np.full((61, 97, 3), 0.3712, np.float32)
    got = orc.resize_area(img, 41, 26)
    np.testing.assert_allclose(got, 0.3712, rtol=4e-7)


def _distort64(x, y, k1, k2, p1, p2, k3):
    r2 = x * x + y * y
    radial = 1 + k1 * r2 + k2 * r2 ** 2 + k3 * r2 ** 3
    return (x * radial + 2 * p1 * x * y + p2 * (r2 + 2 * x * x),
            y * radial + p1 * (r2 + 2 * y * y) + 2 * p2 * x * y)


def _bilinear64(img, sx, sy):
    h, w = img.shape[:2]
    x0 = np.floor(sx).astype(np.int64)
    y0 = np.floor(sy).astype(np.int64)
    fx, fy = (sx - np.floor(sx))[..., None], (sy - np.floor(sy))[..., None]
    cx0, cx1 = np.clip(x0, 0, w - 1), np.clip(x0 + 1, 0, w - 1)
    cy0, cy1 = np.clip(y0, 0, h - 1), np.clip(y0 + 1, 0, h - 1)
    im = img.astype(np.float64)
    top = im[cy0, cx0] * (1 - fx) + im[cy0, cx1] * fx
    bot = im[cy1, cx0] * (1 - fx) + im[cy1, cx1] * fx
    return top * (1 - fy) + bot * fy


CAMS = [  # (w, h, intr, dist k1 k2 p1 p2 k3)
    (160, 120, [150.0, 152.0, 80.5, 59.5], [-0.12, 0.03, 1e-3, -5e-4, 0.0]),
    (160, 120, [140.0, 140.0, 78.0, 61.0], [0.08, -0.01, -2e-3, 1e-3, 0.002]),
    (97, 61, [90.0, 90.0, 48.0, 30.0], [0.0, 0.0, 0.0, 0.0, 0.0]),
]


def _smooth(h, w, seed):
    yy, xx = np.mgrid[0:h, 0:w].astype(np.float64)
    rng = np.random.default_rng(seed)
    ph = rng.random(3) * 6
    img = np.stack([0.5 + 0.4 * np.sin(xx / 13.0 + ph[c]) * np.cos(yy / 17.0 - ph[c]) for c in range(3)], -1)
    return img.astype(np.float32)


@pytest.mark.parametrize("cam", range(len(CAMS)))
def test_undistort_matches_float64_remap(cam):
    w, h, intr, dist = CAMS[cam]
    img = _smooth(h, w, cam)
    got, roi = orc.undistort(img, intr, dist)
    x0, y0, rw, rh = roi
    assert 0 <= x0 and 0 <= y0 and rw > 0 and rh > 0 and x0 + rw <= w and y0 + rh <= h
    fx, fy, cx, cy = intr
    oy, ox = np.mgrid[y0:y0 + rh, x0:x0 + rw].astype(np.float64)
    xd, yd = _distort64((ox - cx) / fx, (oy - cy) / fy, *dist)
    want = _bilinear64(img, xd * fx + cx, yd * fy + cy)
    np.testing.assert_allclose(got, want, atol=2e-5)


def test_undistort_reproduces_linear_ramp():
    w, h, intr, dist = CAMS[0]
    yy, xx = np.mgrid[0:h, 0:w].astype(np.float32)
    img = np.stack([xx / w, yy / h, (xx + 2 * yy) / (w + 2 * h)], -1).astype(np.float32)
    got, (x0, y0, rw, rh) = orc.undistort(img, intr, dist)
    fx, fy, cx, cy = intr
    oy, ox = np.mgrid[y0:y0 + rh, x0:x0 + rw].astype(np.float64)
    xd, yd = _distort64((ox - cx) / fx, (oy - cy) / fy, *dist)
    sx, sy = np.clip(xd * fx + cx, 0, w - 1), np.clip(yd * fy + cy, 0, h - 1)
    np.testing.assert_allclose(got[..., 0], sx / w, atol=3e-5)
    np.testing.assert_allclose(got[..., 1], sy / h, atol=3e-5)


def test_zero_distortion_is_identity():
    w, h, intr, dist = CAMS[2]
    img = np.random.default_rng(5).random((h, w, 3), dtype=np.float32)
    got, (x0, y0, rw, rh) = orc.undistort(img, intr, dist)
    assert x0 <= 1 and y0 <= 1 and x0 + rw >= w - 1 and y0 + rh >= h - 1
    np.testing.assert_allclose(got, img[y0:y0 + rh, x0:x0 + rw], atol=1e-5)


def _newton_inverse(xd, yd, dist):
    x, y = xd.copy(), yd.copy()
    for _ in range(50):
        fx_, fy_ = _distort64(x, y, *dist)
        e = 1e-7
        jxx = (_distort64(x + e, y, *dist)[0] - fx_) / e
        jxy = (_distort64(x, y + e, *dist)[0] - fx_) / e
        jyx = (_distort64(x + e, y, *dist)[1] - fy_) / e
        jyy = (_distort64(x, y + e, *dist)[1] - fy_) / e
        det = jxx * jyy - jxy * jyx
        rx, ry = fx_ - xd, fy_ - yd
        x = x - (jyy * rx - jxy * ry) / det
        y = y - (-jyx * rx + jxx * ry) / det
    return x, y


@pytest.mark.parametrize("cam", [0, 1])
def test_roi_agrees_with_newton_inverse(cam):
    w, h, intr, dist = CAMS[cam]
    fx, fy, cx, cy = intr
    t = np.arange(200) / 199.0
    def edge(px, py):
        xu, yu = _newton_inverse((px - cx) / fx, (py - cy) / fy, dist)
        return xu * fx + cx, yu * fy + cy
    top = edge(t * w, np.zeros(200))[1].max()
    bottom = edge(t * w, np.full(200, h - 1.0))[1].min()
    left = edge(np.zeros(200), t * h)[0].max()
    right = edge(np.full(200, w - 1.0), t * h)[0].min()
    rx, ry = max(0, int(np.ceil(left))), max(0, int(np.ceil(top)))
    want = [rx, ry, min(w, int(np.floor(right))) - rx, min(h, int(np.floor(bottom))) - ry]
    got = orc.undistort_roi(w, h, intr, dist)
    assert np.abs(got - np.array(want)).max() <= 1, (got, want)


def test_png_read_write_bytes(tmp_path):
    """imreadRGB gives byte / 255 (image_io.cpp:44-48); imwriteRGB writes
    clamp(v * 255, 0, 255) + 0.5 truncated (image_io.cpp:62-66)."""
    pytest.importorskip("PIL")
    from PIL import Image
    from msplat_amd import image_io
    b = np.random.default_rng(1).integers(0, 256, (7, 9, 3), dtype=np.uint8)
    Image.fromarray(b, "RGB").save(tmp_path / "a.png")
    got = image_io.imread_rgb(str(tmp_path / "a.png"))
    assert got.dtype == np.float32 and np.array_equal(got, b.astype(np.float32) / np.float32(255))
    image_io.imwrite_rgb(str(tmp_path / "b.png"), got)
    assert np.array_equal(np.asarray(Image.open(tmp_path / "b.png")), b)
    v = np.array([[[-0.2, 1.7, 0.5 / 255]], [[1.49 / 255, 1.51 / 255, 0.999]]], np.float32)
    image_io.imwrite_rgb(str(tmp_path / "c.png"), v)
    assert np.asarray(Image.open(tmp_path / "c.png")).tolist() == [[[0, 255, 1]], [[1, 2, 255]]]
    Image.fromarray(b[..., 0], "L").save(tmp_path / "g.png")      # grey: replicated channels
    g = image_io.imread_rgb(str(tmp_path / "g.png"))
    assert np.array_equal(g, np.repeat(b[..., :1], 3, axis=2).astype(np.float32) / np.float32(255))
