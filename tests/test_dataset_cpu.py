"""COLMAP dataset ingest on the CPU (msplat_dataset_*, host code only).

A small COLMAP model is written here in COLMAP's binary format (cameras.bin,
images.bin with 2D points, points3D.bin with tracks) and read back through
the library.  The expected cameras restate load_colmap.cpp's conversion
(quaternion to rotation in float64, transpose, -R^T t in fp32, OpenGL flip of
columns 1 and 2), the sort by image name and the skip of images whose camera
is missing; the normalisation restates autoScaleAndCenter
(input_data.cpp:79-125) in fp32 in the same order, so every value is
compared bit for bit.  The points3D.ply fallback is read in binary and ascii
form, and the train / test split follows splitTrainTest.
"""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

from msplat_amd import _abi

f32 = np.float32


def _lib_or_skip():
    if not os.path.exists(_abi.LIB_PATH):
        pytest.skip("libmsplat_hip.so not built")
    from msplat_amd import dataset
    return dataset


CAMS = {  # id: (model, w, h, params)
    1: (1, 640, 480, [500.0, 510.0, 320.5, 239.5]),            # PINHOLE
    2: (4, 800, 600, [600.0, 601.0, 400.0, 300.0, 0.01, -0.002, 0.001, 0.0005]),   # OPENCV
    3: (2, 320, 240, [250.0, 160.0, 120.0, 0.05]),             # SIMPLE_RADIAL
}
IMAGES = [  # (image id, qvec wxyz, tvec, camera id, name, n 2D points)
    (5, [0.9, 0.1, -0.2, 0.3], [0.5, -1.0, 4.0], 1, "c.jpg", 3),
    (2, [0.2, 0.7, 0.1, -0.6], [-2.0, 0.3, 1.5], 2, "a.jpg", 0),
    (9, [1.0, 0.0, 0.0, 0.0], [0.0, 0.0, 3.0], 3, "b.jpg", 5),
    (4, [0.5, 0.5, 0.5, 0.5], [1.0, 1.0, 1.0], 7, "d.jpg", 1),   # camera 7 is missing: skipped
]


def _write_model(d, n_points=50, seed=0):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "cameras.bin"), "wb") as f:
        f.write(struct.pack("<Q", len(CAMS)))
        for cid, (model, w, h, p) in CAMS.items():
            f.write(struct.pack("<IIQQ", cid, model, w, h))
            f.write(struct.pack(f"<{len(p)}d", *p))
    with open(os.path.join(d, "images.bin"), "wb") as f:
        f.write(struct.pack("<Q", len(IMAGES)))
        for iid, q, t, cid, name, n2 in IMAGES:
            f.write(struct.pack("<I4d3dI", iid, *q, *t, cid))
            f.write(name.encode() + b"\0")
            f.write(struct.pack("<Q", n2))
            for k in range(n2):
                f.write(struct.pack("<ddq", 1.5 * k, 2.5 * k, k))
    rng = np.random.default_rng(seed)
    xyz = rng.normal(0, 2, (n_points, 3))
    rgb = rng.integers(0, 256, (n_points, 3)).astype(np.uint8)
    with open(os.path.join(d, "points3D.bin"), "wb") as f:
        f.write(struct.pack("<Q", n_points))
        for i in range(n_points):
            f.write(struct.pack("<Q3d3Bd", 100 + i, *xyz[i], *rgb[i], 0.5))
            track = i % 4
            f.write(struct.pack("<Q", track))
            f.write(b"\x01\0\0\0\x02\0\0\0" * track)
    return xyz, rgb


def _expected_cameras():
    out = []
    for iid, q, t, cid, name, _ in sorted(IMAGES, key=lambda r: r[4]):
        if cid not in CAMS:
            continue
        w, x, y, z = (float(v) for v in q)
        n = (w * w + x * x + y * y + z * z) ** 0.5
        w, x, y, z = w / n, x / n, y / n, z / n
        R = [f32(1 - 2 * (y * y + z * z)), f32(2 * (x * y - w * z)), f32(2 * (x * z + w * y)),
             f32(2 * (x * y + w * z)), f32(1 - 2 * (x * x + z * z)), f32(2 * (y * z - w * x)),
             f32(2 * (x * z - w * y)), f32(2 * (y * z + w * x)), f32(1 - 2 * (x * x + y * y))]
        Ri = [R[0], R[3], R[6], R[1], R[4], R[7], R[2], R[5], R[8]]
        tf = [f32(v) for v in t]
        Ti = [-(Ri[3 * r] * tf[0] + Ri[3 * r + 1] * tf[1] + Ri[3 * r + 2] * tf[2]) for r in range(3)]
        m = [Ri[0], -Ri[1], -Ri[2], Ti[0], Ri[3], -Ri[4], -Ri[5], Ti[1],
             Ri[6], -Ri[7], -Ri[8], Ti[2], f32(0), f32(0), f32(0), f32(1)]
        out.append((cid, name, np.array(m, np.float32)))
    return out


def _normalise(cams, xyz):
    mean = [f32(0), f32(0), f32(0)]
    for _, _, m in cams:
        for k, idx in enumerate((3, 7, 11)):
            mean[k] = f32(mean[k] + m[idx])
    mean = [f32(v / f32(len(cams))) for v in mean]
    for _, _, m in cams:
        for k, idx in enumerate((3, 7, 11)):
            m[idx] = f32(m[idx] - mean[k])
    mx = f32(0)
    for _, _, m in cams:
        for idx in (3, 7, 11):
            mx = max(mx, abs(m[idx]))
    scale = f32(f32(1) / mx)
    for _, _, m in cams:
        for idx in (3, 7, 11):
            m[idx] = f32(m[idx] * scale)
    pts = (xyz.astype(np.float32) - np.array(mean, np.float32)) * scale
    return scale, np.array(mean, np.float32), pts


@pytest.mark.parametrize("layout", ["flat", "sparse"])
def test_colmap_cameras_points_and_normalisation(layout, tmp_path):
    ds_mod = _lib_or_skip()
    root = str(tmp_path)
    model_dir = root if layout == "flat" else os.path.join(root, "sparse", "0")
    xyz, rgb = _write_model(model_dir)
    if layout == "sparse":
        os.makedirs(os.path.join(root, "images"))
    ds = ds_mod.Dataset(root)
    want = _expected_cameras()
    scale, mean, pts = _normalise(want, xyz)
    assert len(ds.cameras) == len(want) == 3
    img_dir = root if layout == "flat" else os.path.join(root, "images")
    for cam, path, dist, (cid, name, m) in zip(ds.cameras, ds.image_paths, ds.distortion, want):
        model, w, h, p = CAMS[cid]
        assert (cam.width, cam.height) == (w, h)
        fx, fy, cx, cy = ((p[0], p[0], p[1], p[2]) if model in (0, 2, 3) else tuple(p[:4]))
        assert (cam.fx, cam.fy, cam.cx, cam.cy) == tuple(float(f32(v)) for v in (fx, fy, cx, cy))
        assert np.array_equal(cam.cam_to_world.reshape(16), m), name
        assert path == img_dir + "/" + name
        if model == 4:
            assert np.array_equal(dist, np.array(p[4:8], np.float32))
    s, t = ds.normalisation()
    assert s == scale and np.array_equal(t, mean)
    got_xyz, got_rgb = ds.points()
    assert np.array_equal(got_xyz, pts) and np.array_equal(got_rgb, rgb)
    train, test = ds.split_train_test(2)
    assert [c.width for c in test] == [ds.cameras[0].width, ds.cameras[2].width]
    assert [c.width for c in train] == [ds.cameras[1].width]


def _ply_points(path, xyz, rgb, ascii):
    hdr = ["ply", "format ascii 1.0" if ascii else "format binary_little_endian 1.0",
           f"element vertex {len(xyz)}", "property double x", "property double y", "property double z",
           "property uchar red", "property uchar green", "property uchar blue", "end_header"]
    with open(path, "wb") as f:
        f.write(("\n".join(hdr) + "\n").encode())
        for p, c in zip(xyz, rgb):
            if ascii:
                f.write(f"{float(p[0])!r} {float(p[1])!r} {float(p[2])!r} {c[0]} {c[1]} {c[2]}\n".encode())
            else:
                f.write(struct.pack("<3d3B", *p, *c))


@pytest.mark.parametrize("ascii", [False, True])
def test_points_ply_fallback(ascii, tmp_path):
    ds_mod = _lib_or_skip()
    xyz, rgb = _write_model(str(tmp_path))
    # fp32-representable coordinates: the ascii reader rounds the text to fp32
    # directly, the binary one the double
    xyz = xyz.astype(np.float32).astype(np.float64)
    os.remove(tmp_path / "points3D.bin")
    _ply_points(tmp_path / "points3D.ply", xyz, rgb, ascii)
    ds = ds_mod.Dataset(str(tmp_path))
    _, _, pts = _normalise(_expected_cameras(), xyz)
    got_xyz, got_rgb = ds.points()
    assert np.array_equal(got_xyz, pts) and np.array_equal(got_rgb, rgb)


def test_missing_model_raises(tmp_path):
    ds_mod = _lib_or_skip()
    with pytest.raises(_abi.MsplatError, match="Cannot open"):
        ds_mod.Dataset(str(tmp_path))


def test_package_names_and_config_defaults(tmp_path):
    """The reference module's top-level names and TrainingConfig defaults
    (tests/test_msplat.py:15-52 of the reference), and load_dataset's
    train / test split (num_test 0 unless eval_mode)."""
    import msplat_amd as msplat
    for name in ("GaussianTrainer", "TrainingConfig", "TrainingStats", "Dataset", "load_dataset",
                 "sync", "cleanup"):
        assert hasattr(msplat, name), name
    cfg = msplat.TrainingConfig()
    assert cfg.iterations == 30000 and cfg.sh_degree == 3 and cfg.refine_every == 100
    assert cfg.warmup_length == 500 and abs(cfg.ssim_weight - 0.2) < 1e-9
    cfg = msplat.TrainingConfig(iterations=100, sh_degree=1, ssim_weight=0.0)
    assert (cfg.iterations, cfg.sh_degree, cfg.ssim_weight) == (100, 1, 0.0)
    cfg.iterations = 500
    assert cfg.iterations == 500
    _write_model(str(tmp_path), n_points=200, seed=5)
    ds = msplat.load_dataset(str(tmp_path))
    assert ds.num_test == 0 and ds.num_train == len(ds.cameras)
    ds = msplat.load_dataset(str(tmp_path), eval_mode=True, test_every=2)
    assert ds.num_test == len(ds.cameras[::2]) and ds.num_train + ds.num_test == len(ds.cameras)
