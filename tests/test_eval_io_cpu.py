"""Evaluation metrics, RGBA8 conversion and scene files on the CPU.

* The oracle's ssim_eval restatement is pinned against the reference's own
  ssim_eval (core/src/ssim.cpp:61-123) compiled from its source into
  oracle/_ref/ssim_eval (bit for bit), against a float64 brute-force SSIM with
  edge-clamped borders, and against SSIM(x, x) = 1; PSNR / L1
  (model.cpp:25-40) against float64 sums; RGBA8 (msplat_api.mm:230-238)
  against numpy's clamp-scale-truncate.
* PLY / .splat files written by the library's host-only writers
  (msplat_scene_write_*) are parsed here by a restatement of
  save_gaussians.cpp's layouts: header lines, row layout with f_rest
  transposed to [3, K-1], keepCrs transforms, .splat order and
  quantisation; the reader round-trips and rejects malformed files.
"""
from __future__ import annotations

import math
import os
import struct
import subprocess

import numpy as np
import pytest

import orc
from msplat_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SSIM = os.path.join(ROOT, "oracle", "_ref", "ssim_eval")
SH_C0 = 0.28209479177387814
# The writers call the C library's expf / logf (std::exp / std::log on
# floats); numpy's float32 exp / log may differ from them in the last bit, so
# the expected values use libm itself.
_LIBM = __import__("ctypes").CDLL("libm.so.6")
_LIBM.expf.restype = _LIBM.logf.restype = __import__("ctypes").c_float
_LIBM.expf.argtypes = _LIBM.logf.argtypes = [__import__("ctypes").c_float]
expf = np.vectorize(lambda x: np.float32(_LIBM.expf(float(x))), otypes=[np.float32])
logf = np.vectorize(lambda x: np.float32(_LIBM.logf(float(x))), otypes=[np.float32])


def _images(h, w, seed, lo=0.0, hi=1.0):
    rng = np.random.default_rng(seed)
    a = rng.uniform(lo, hi, (h, w, 3)).astype(np.float32)
    b = np.clip(a + rng.normal(0, 0.1, a.shape), lo, hi).astype(np.float32)
    return a, b


def _ref_ssim(img, gt, ws, sigma, tmp_path):
    f = tmp_path / "pair.bin"
    with open(f, "wb") as fh:
        fh.write(struct.pack("<iiif", img.shape[0], img.shape[1], ws, sigma))
        fh.write(np.ascontiguousarray(img, np.float32).tobytes())
        fh.write(np.ascontiguousarray(gt, np.float32).tobytes())
    out = subprocess.check_output([REF_SSIM, str(f)], text=True).strip()
    return np.float32(float.fromhex(out))


@pytest.mark.parametrize("shape,ws,sigma", [((840 // 8, 1297 // 8), 11, 1.5), ((7, 5), 11, 1.5),
                                            ((33, 70), 11, 1.5), ((40, 41), 7, 1.0)])
def test_oracle_ssim_matches_reference_build(shape, ws, sigma, tmp_path):
    if not os.path.exists(REF_SSIM):
        pytest.skip("oracle/_ref/ssim_eval not built (needs /root/reference)")
    img, gt = _images(*shape, seed=shape[0] * 7 + ws)
    got = orc.image_metrics(img, gt, ws, sigma)["ssim"]
    assert np.float32(got) == _ref_ssim(img, gt, ws, sigma, tmp_path)


def _ssim_f64(img, gt, ws=11, sigma=1.5):
    """Brute-force SSIM in float64: separable Gaussian with edge-clamped borders."""
    x = np.arange(ws) - ws // 2
    k = np.exp(-(x * x) / (2 * sigma * sigma))
    k /= k.sum()
    H, W = img.shape[:2]
    pad = ws // 2

    def blur(a):
        ap = np.pad(a, pad, mode="edge")
        h = sum(k[i] * ap[:, i:i + W] for i in range(ws))
        return sum(k[i] * h[i:i + H, :] for i in range(ws))

    vals = []
    for c in range(3):
        r, g = img[..., c].astype(np.float64), gt[..., c].astype(np.float64)
        m1, m2 = blur(r), blur(g)
        s11, s22, s12 = blur(r * r) - m1 * m1, blur(g * g) - m2 * m2, blur(r * g) - m1 * m2
        C1, C2 = 0.01 ** 2, 0.03 ** 2
        vals.append((2 * m1 * m2 + C1) * (2 * s12 + C2) / ((m1 * m1 + m2 * m2 + C1) * (s11 + s22 + C2)))
    return float(np.mean(vals))


def test_oracle_ssim_closed_forms():
    img, gt = _images(45, 61, 3)
    assert abs(orc.image_metrics(img, gt)["ssim"] - _ssim_f64(img, gt)) < 2e-5
    assert orc.image_metrics(img, img)["ssim"] == 1.0
    # the clamped border: a constant image blurs to itself everywhere
    flat = np.full((9, 12, 3), 0.25, np.float32)
    assert orc.image_metrics(flat, flat)["ssim"] == 1.0


def test_oracle_psnr_l1_closed_forms():
    img, gt = _images(50, 60, 5)
    m = orc.image_metrics(img, gt)
    d = (img - gt).astype(np.float64).ravel()   # float32 differences, fp64 sums
    mse = math.fsum(d * d) / d.size
    assert abs(m["psnr"] - 10.0 * math.log10(1.0 / mse)) < 1e-4
    assert abs(m["l1"] - math.fsum(np.abs(d)) / d.size) < 1e-7
    same = orc.image_metrics(img, img)
    assert same["psnr"] == float("inf") and same["l1"] == 0.0


def test_oracle_rgba8_truncates():
    vals = np.array([-1.0, 0.0, 1 / 255, 0.5, 0.99999, 1.0, 2.0, np.nan, np.inf, -np.inf, 0.003921],
                    np.float32)
    img = np.stack([vals, vals[::-1], np.roll(vals, 3)], axis=-1)[None]
    got = orc.image_to_rgba8(img)
    with np.errstate(invalid="ignore"):
        c = np.where(np.isnan(img), 0.0, np.clip(img, 0.0, 1.0)).astype(np.float32)
    want = (c * np.float32(255.0)).astype(np.uint8)
    assert np.array_equal(got[..., :3], want)
    assert (got[..., 3] == 255).all()
    assert got[0, 3, 0] == 127 and got[0, 5, 0] == 255   # 0.5 * 255 = 127.5 truncates


# ---- scene files ----

def _lib_or_skip():
    if not os.path.exists(_abi.LIB_PATH):
        pytest.skip("libmsplat_hip.so not built")
    from msplat_amd import scene_io
    return scene_io


def _cloud(n, degree, seed):
    rng = np.random.default_rng(seed)
    nb = (degree + 1) ** 2 - 1
    q = rng.normal(size=(n, 4)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    return [rng.normal(0, 1.5, (n, 3)).astype(np.float32),
            rng.normal(-4.5, 0.5, (n, 3)).astype(np.float32), q,
            rng.normal(0, 0.3, (n, 3)).astype(np.float32),
            rng.normal(0, 0.05, (n, nb, 3)).astype(np.float32),
            rng.normal(0, 1, (n, 1)).astype(np.float32)]


def _parse_ply(path):
    raw = open(path, "rb").read()
    end = raw.index(b"end_header\n") + len(b"end_header\n")
    header = raw[:end].decode().splitlines()
    return header, raw[end:]


@pytest.mark.parametrize("degree", [0, 1, 3])
def test_ply_layout_and_round_trip(degree, tmp_path):
    sio = _lib_or_skip()
    p = _cloud(257, degree, degree + 1)
    nb = (degree + 1) ** 2 - 1
    path = tmp_path / "g.ply"
    sio.write_ply(path, p, step=1234)
    header, body = _parse_ply(path)
    want = (["ply", "format binary_little_endian 1.0", "comment msplat v1234", "element vertex 257",
             "property float x", "property float y", "property float z",
             "property float nx", "property float ny", "property float nz"]
            + [f"property float f_dc_{i}" for i in range(3)]
            + [f"property float f_rest_{i}" for i in range(3 * nb)]
            + ["property float opacity"] + [f"property float scale_{i}" for i in range(3)]
            + [f"property float rot_{i}" for i in range(4)] + ["end_header"])
    assert header == want
    rows = np.frombuffer(body, np.float32).reshape(257, -1)
    expect = np.concatenate([p[0], np.zeros((257, 3), np.float32), p[3],
                             p[4].transpose(0, 2, 1).reshape(257, -1), p[5], p[1], p[2]], axis=1)
    assert np.array_equal(rows, expect)
    back, step = sio.read_ply(path)
    assert step == 0          # the writer's comment is not the reader's iteration comment
    for a, b in zip(back, p):
        assert np.array_equal(a.reshape(b.shape), b)


def test_ply_keep_crs(tmp_path):
    sio = _lib_or_skip()
    p = _cloud(64, 1, 9)
    scale, t = 0.37, (1.5, -2.0, 0.25)
    path = tmp_path / "crs.ply"
    sio.write_ply(path, p, crs=(scale, t))
    rows = np.frombuffer(_parse_ply(path)[1], np.float32).reshape(64, -1)
    f = np.float32
    assert np.array_equal(rows[:, :3], p[0] / f(scale) + np.array(t, np.float32))
    assert np.array_equal(rows[:, -7:-4], logf(expf(p[1]) / f(scale)))
    back, _ = sio.read_ply(path, crs=(scale, t))
    assert np.allclose(back[0], p[0], atol=1e-5)
    assert np.allclose(back[1], p[1], atol=1e-5)


def test_ply_iteration_comment_and_errors(tmp_path):
    sio = _lib_or_skip()
    p = _cloud(5, 0, 2)
    path = tmp_path / "a.ply"
    sio.write_ply(path, p)
    header, body = _parse_ply(path)
    header[2] = "comment Generated by msplat at iteration 777"
    with open(tmp_path / "b.ply", "wb") as fh:
        fh.write(("\n".join(header) + "\n").encode() + body)
    assert sio.read_ply(tmp_path / "b.ply")[1] == 777
    with open(tmp_path / "trunc.ply", "wb") as fh:
        fh.write(("\n".join(header) + "\n").encode() + body[:-8])
    with pytest.raises(_abi.MsplatError, match="truncated"):
        sio.read_ply(tmp_path / "trunc.ply")
    (tmp_path / "bad.ply").write_text("solid mesh\n")
    with pytest.raises(_abi.MsplatError, match="Not a PLY"):
        sio.read_ply(tmp_path / "bad.ply")
    with pytest.raises(_abi.MsplatError, match="Cannot open"):
        sio.read_ply(tmp_path / "missing.ply")


def test_splat_order_and_quantisation(tmp_path):
    sio = _lib_or_skip()
    p = _cloud(300, 2, 4)
    p[5][:10] = 0.0
    p[1][:10] = -4.0          # ten equal sort keys: ties keep index order
    path = tmp_path / "g.splat"
    sio.write_splat(path, p)
    raw = np.frombuffer(open(path, "rb").read(), np.uint8).reshape(300, 32)
    f = np.float32
    e = expf(p[1])
    s = e[:, 0] + e[:, 1] + e[:, 2]
    key = s / (f(1) + expf(-p[5][:, 0]))
    order = sorted(range(300), key=lambda i: (-key[i], i))
    pos = raw[:, :12].copy().view(np.float32)
    sc = raw[:, 12:24].copy().view(np.float32)
    assert np.array_equal(pos, p[0][order])
    assert np.array_equal(sc, e[order])
    rgb = np.clip((p[3][order].astype(np.float64) * SH_C0 + 0.5) * 255.0, 0, 255).astype(np.uint8)
    assert np.array_equal(raw[:, 24:27], rgb)
    sig = f(1) / (f(1) + expf(-p[5][order, 0]))
    assert np.array_equal(raw[:, 27], np.clip(sig * f(255), 0, 255).astype(np.uint8))
    q = np.clip(p[2][order] * f(128) + f(128), 0, 255).astype(np.uint8)
    assert np.array_equal(raw[:, 28:32], q)
