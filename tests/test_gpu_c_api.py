"""The reference-shaped C API (include/msplat_c_api.h) end to end on a GPU.

A small COLMAP dataset with PNG images is trained through the C calls a
Swift or C caller of the reference makes (msplat_dataset_create,
msplat_trainer_create / train / evaluate / render / render_pose_to_buffer /
export_ply / save_checkpoint / load_checkpoint ...).  The same dataset
trained by the Python GaussianTrainer(dataset, config) (images decoded by
Pillow, prepared on the GPU by the same kernels, the same C++ trainer) must
start from the same gaussians bit for bit and end within rounding of the
same state and evaluation (the raster backward's float atomics sum in an
order that varies from run to run, so two trainings differ in the last
bits).  A JPEG
dataset loads through a decoder registered with msplat_set_image_decoder.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from helpers import grad_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    pytest.importorskip("PIL")
    from msplat_amd import device
    return device.init(0)


def _dataset(tmp_path, fmt="PNG", n_points=3000):
    from PIL import Image
    from test_dataset_cpu import _write_model
    import msplat_amd as msplat
    _write_model(str(tmp_path), n_points=n_points, seed=9)
    probe = msplat.load_dataset(str(tmp_path))
    rng = np.random.default_rng(41)
    for cam, path in zip(probe.cameras, probe.image_paths):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        # the file names end in .jpg; the bytes are in `fmt`
        img = rng.integers(0, 256, (cam.height, cam.width, 3), dtype=np.uint8)
        Image.fromarray(img, "RGB").save(path, format=fmt)
    return probe


def _config(iterations=6):
    from msplat_amd import _abi
    c = _abi.default_config()
    c.iterations, c.numDownscales, c.shDegreeInterval = iterations, 0, 0
    return c


def _group(lib, t, g, which=0):
    from msplat_amd import _abi
    p, rows, per = ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_int64()
    assert lib.msplat_trainer_group(t, g, which, ctypes.byref(p), ctypes.byref(rows), ctypes.byref(per)) == 0
    out = np.empty((rows.value, per.value), np.float32)
    _abi.check(lib.msplat_hip_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), p, out.nbytes))
    return out


def _take(buf):
    assert buf.data, "empty pixel buffer"
    try:
        return np.ctypeslib.as_array(buf.data, shape=(buf.height, buf.width, 3)).copy()
    finally:
        ctypes.CDLL(None).free(ctypes.cast(buf.data, ctypes.c_void_p))


def test_c_api_trains_like_the_python_trainer(lib, tmp_path):
    import msplat_amd as msplat
    probe = _dataset(tmp_path)
    ds = lib.msplat_dataset_create(str(tmp_path).encode(), 1.0, True, 2)
    assert ds, lib.msplat_trainer_last_error()
    try:
        n_cams = len(probe.cameras)
        assert lib.msplat_dataset_num_test(ds) == (n_cams + 1) // 2
        assert lib.msplat_dataset_num_train(ds) == n_cams // 2
        pose = (ctypes.c_float * 16)()
        lib.msplat_dataset_camera_pose(ds, 0, pose)
        assert np.array_equal(np.array(pose, np.float32), np.asarray(probe.cameras[1].cam_to_world,
                                                                     np.float32).reshape(16))
        t = lib.msplat_trainer_create(ds, _config())
        assert t, lib.msplat_trainer_last_error()
        try:
            lib.msplat_trainer_train(t)
            assert lib.msplat_trainer_last_error() == b""
            assert lib.msplat_trainer_iteration(t) == 6 and lib.msplat_trainer_splat_count(t) == 3000
            m_c = lib.msplat_trainer_evaluate(t)
            assert m_c.numTest == lib.msplat_dataset_num_test(ds) and m_c.numGaussians == 3000

            # the Python trainer on the same dataset
            pds = msplat.load_dataset(str(tmp_path), eval_mode=True, test_every=2)
            tr = msplat.GaussianTrainer(pds, msplat.TrainingConfig(iterations=6, num_downscales=0,
                                                                   sh_degree_interval=0))
            tr.train()
            for g in range(6):
                for which in range(3):
                    a, b = _group(lib, t, g, which), tr.group(g, which)
                    # the parity tests' tolerance (D5)
                    grad_close(a, b, rtol=2e-3 if which == 2 else 1e-3, what=f"group {g} state {which}")
            m_p = tr.evaluate()
            for k, v in (("psnr", m_c.psnr), ("ssim", m_c.ssim), ("l1", m_c.l1)):
                assert abs(v - m_p[k]) <= 1e-4 * max(1.0, abs(m_p[k])), (k, v, m_p[k])

            # renders of a training and a held-out camera; out of range -> empty
            tr_img = _take(lib.msplat_trainer_render(t, 0, False))
            # last-bit differences in the parameters can flip a pair across the
            # 1/255 or stop threshold at a handful of pixels
            diff = np.abs(tr_img - tr.render(0))
            assert (diff > 1e-5).mean() < 1e-3 and diff.max() < 1e-2, ((diff > 1e-5).sum(), diff.max())
            te_img = _take(lib.msplat_trainer_render(t, 0, True))
            assert te_img.shape[2] == 3 and np.isfinite(te_img).all()
            bad = lib.msplat_trainer_render(t, 99, False)
            assert not bad.data and bad.width == 0
            # RGBA8 display buffer: size query, then the pixels
            c2w = np.asarray(probe.cameras[1].cam_to_world, np.float32).reshape(16)
            cp = (ctypes.c_float * 16)(*c2w)
            w, h = ctypes.c_int(0), ctypes.c_int(0)
            lib.msplat_trainer_render_pose_to_buffer(t, cp, 0, None, ctypes.byref(w), ctypes.byref(h))
            assert (h.value, w.value) == tr_img.shape[:2]
            rgba = np.zeros((h.value, w.value, 4), np.uint8)
            lib.msplat_trainer_render_pose_to_buffer(t, cp, 0, rgba.ctypes.data, ctypes.byref(w), ctypes.byref(h))
            # bytes may differ where a value sits on a rounding boundary or a
            # threshold flips
            ref = tr.render_from_pose_rgba8(c2w.reshape(4, 4), 0)
            bd = np.abs(rgba.astype(np.int16) - ref.astype(np.int16))
            assert (bd > 1).mean() < 1e-3 and bd.max() <= 3, ((bd > 1).sum(), bd.max())
            # scene files and checkpoints
            lib.msplat_trainer_export_ply(t, str(tmp_path / "out.ply").encode())
            lib.msplat_trainer_export_splat(t, str(tmp_path / "out.splat").encode())
            lib.msplat_trainer_save_checkpoint(t, str(tmp_path / "ck.msplat").encode())
            assert lib.msplat_trainer_last_error() == b""
            assert os.path.getsize(tmp_path / "out.ply") > 3000 * 62 * 4
            assert os.path.getsize(tmp_path / "out.splat") == 3000 * 32
            assert lib.msplat_trainer_load_checkpoint(t, str(tmp_path / "ck.msplat").encode()) == 6
            lib.msplat_trainer_save_checkpoint(t, str(tmp_path / "missing_dir" / "ck.msplat").encode())
            assert lib.msplat_trainer_last_error() != b""
            lib.msplat_sync()
        finally:
            lib.msplat_trainer_destroy(t)
    finally:
        lib.msplat_dataset_destroy(ds)


def test_c_api_jpeg_dataset_native_and_registered_decoder(lib, tmp_path):
    """A COLMAP scene with JPEG images loads and trains with no decoder
    registered (the library's own JPEG decoder, as the reference decodes its
    JPEG datasets itself).  A decoder the application registers (Pillow
    through a ctypes callback) takes precedence; both decode the same
    samples, so the first train step's loss is the same bit for bit."""
    from PIL import Image
    from msplat_amd import _abi
    _dataset(tmp_path, fmt="JPEG", n_points=500)

    def first_loss():
        ds = lib.msplat_dataset_create(str(tmp_path).encode(), 2.0, False, 8)
        assert ds, lib.msplat_trainer_last_error()
        try:
            assert lib.msplat_dataset_num_test(ds) == 0
            t = lib.msplat_trainer_create(ds, _config(iterations=2))
            assert t, lib.msplat_trainer_last_error()
            try:
                s = lib.msplat_trainer_step(t)
                assert s.iteration == 1 and s.splatCount == 500
                img = _take(lib.msplat_trainer_render(t, 0, False))
                assert np.isfinite(img).all()
                return lib.msplat_trainer_last_loss(t, 1), lib.msplat_dataset_num_train(ds)
            finally:
                lib.msplat_trainer_destroy(t)
        finally:
            lib.msplat_dataset_destroy(ds)

    native, n_train = first_loss()
    libc = ctypes.CDLL(None)
    libc.malloc.restype = ctypes.c_void_p
    libc.malloc.argtypes = [ctypes.c_size_t]
    calls = []

    def decode(path, rgb, width, height):
        with Image.open(path.decode()) as im:
            a = np.ascontiguousarray(np.asarray(im.convert("RGB"), np.float32) / np.float32(255.0))
        p = libc.malloc(a.nbytes)
        ctypes.memmove(p, a.ctypes.data, a.nbytes)
        rgb[0] = ctypes.cast(p, ctypes.POINTER(ctypes.c_float))
        width[0], height[0] = a.shape[1], a.shape[0]
        calls.append(path)
        return 0

    cb = _abi.ImageDecoder(decode)
    lib.msplat_set_image_decoder(cb)
    try:
        registered, _ = first_loss()
        assert len(calls) == n_train
        assert np.isfinite(native) and native == registered, (native, registered)
    finally:
        lib.msplat_set_image_decoder(_abi.ImageDecoder(0))
