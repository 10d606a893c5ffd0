"""The steps either side of the render on the GPU: evaluation metrics, the
RGBA8 display image, scene files and checkpoints through the trainer.

* msplat_hip_image_metrics against the oracle's psnr / ssim_eval / l1_loss
  (itself pinned bit for bit to the reference's compiled ssim_eval): the
  per-pixel terms are formed in the same float operations, only the fp64
  sums over pixels run in a different order, hence the 1e-6 tolerance.
* msplat_hip_image_to_rgba8 bit-exact against the oracle, special values
  included; the trainer's render_pose_to_buffer is the RGBA8 of its float
  render.
* Trainer evaluate = mean of the oracle's metrics of its renders.
* export_ply / export_splat write the bytes of the host writers for the
  trainer's parameters; load_ply restores them with a fresh optimiser.
* Checkpoints: the file parses with the reference's layout (model.cpp:361-399)
  and holds the trainer's parameters and moments; loading it into another
  trainer restores them bit for bit, with the step, Adam step count and
  learning rates, and training continues from there.
"""
from __future__ import annotations

import os
import struct

import numpy as np
import pytest

import orc
from helpers import BG, assert_bits_equal, grad_close, small_scene, target_for
from msplat_amd import camera, scene_io

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from msplat_amd import device, trainer
    device.init(0)
    return torch, device, trainer


def _pair(h, w, seed):
    rng = np.random.default_rng(seed)
    a = rng.uniform(0, 1, (h, w, 3)).astype(np.float32)
    b = np.clip(a + rng.normal(0, 0.08, a.shape), 0, 1).astype(np.float32)
    return a, b


@pytest.mark.parametrize("shape,ws,sigma", [((840, 1297), 11, 1.5), ((5, 7), 11, 1.5),
                                            ((17, 200), 11, 1.5), ((64, 65), 7, 1.0)])
def test_image_metrics_match_oracle(mods, shape, ws, sigma):
    torch, device, _ = mods
    print(f"image metrics {shape} ws={ws}", flush=True)
    a, b = _pair(*shape, seed=shape[1])
    got = device.image_metrics(torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda(), ws, sigma)
    want = orc.image_metrics(a, b, ws, sigma)
    for k in ("psnr", "ssim", "l1"):
        assert abs(got[k] - want[k]) <= 1e-6 * max(1.0, abs(want[k])), (k, got[k], want[k])


def test_image_metrics_identical_images(mods):
    torch, device, _ = mods
    a, _ = _pair(48, 80, 3)
    t = torch.from_numpy(a).cuda()
    m = device.image_metrics(t, t)
    assert m["ssim"] == 1.0 and m["l1"] == 0.0 and m["psnr"] == float("inf")


def test_rgba8_matches_oracle(mods):
    torch, device, _ = mods
    vals = np.array([-1.0, 0.0, 1 / 255, 0.5, 0.99999, 1.0, 2.0, np.nan, np.inf, -np.inf, 0.003921, 0.25],
                    np.float32)
    rng = np.random.default_rng(0)
    img = np.concatenate([np.stack([vals, vals[::-1], np.roll(vals, 5)], axis=-1)[None],
                          rng.uniform(-0.2, 1.2, (1, 12, 3)).astype(np.float32)], axis=0)
    got = device.image_to_rgba8(torch.from_numpy(img).cuda()).cpu().numpy()
    assert_bits_equal(got, orc.image_to_rgba8(img), "rgba8")


def _trainer(trainer, n=2000, seed=610, cams=1):
    sc = small_scene(n=n, seed_off=seed)
    if cams > 1:
        sc.cameras.append(camera.pinhole(sc.cameras[0].width, sc.cameras[0].height, 70.0,
                                         camera.look_at(np.array([3.5, 1.0, -3.0]))))
    tg = [target_for(sc, (c.height, c.width), seed_off=seed + 1 + i) for i, c in enumerate(sc.cameras)]
    cfg = trainer.TrainingConfig(iterations=1000, sh_degree=3, sh_degree_interval=0, num_downscales=0,
                                 warmup_length=10_000, shuffle_cameras=False)
    return sc, tg, trainer.GaussianTrainer(sc.params(), sc.cameras, tg, cfg)


def test_render_to_rgba8_buffer(mods):
    _, _, trainer = mods
    sc, _, tr = _trainer(trainer)
    tr.step()
    pose = np.asarray(sc.cameras[0].cam_to_world, np.float32)
    rgba = tr.render_from_pose_rgba8(pose, 0)
    img = tr.render_from_pose(pose, 0)
    assert rgba.shape == img.shape[:2] + (4,)
    assert_bits_equal(rgba, orc.image_to_rgba8(img), "render_pose_to_buffer")


def test_trainer_evaluate(mods):
    _, _, trainer = mods
    sc, tg, tr = _trainer(trainer, cams=2)
    for _ in range(3):
        tr.step()
    m = tr.evaluate(sc.cameras, tg)
    want = [orc.image_metrics(tr.render(i), tg[i]) for i in range(2)]
    for k in ("psnr", "ssim", "l1"):
        ref = float(np.mean([w[k] for w in want]))
        assert abs(m[k] - ref) <= 1e-5 * max(1.0, abs(ref)), (k, m[k], ref)
    assert m["num_test"] == 2 and m["num_gaussians"] == tr.splat_count()


def test_export_and_load_ply(mods, tmp_path):
    _, _, trainer = mods
    sc, tg, tr = _trainer(trainer)
    for _ in range(2):
        tr.step()
    params = tr.params()
    tr.export_ply(tmp_path / "t.ply")
    scene_io.write_ply(tmp_path / "h.ply", params, step=tr.current_step)
    assert open(tmp_path / "t.ply", "rb").read() == open(tmp_path / "h.ply", "rb").read()
    tr.export_splat(tmp_path / "t.splat")
    scene_io.write_splat(tmp_path / "h.splat", params)
    assert open(tmp_path / "t.splat", "rb").read() == open(tmp_path / "h.splat", "rb").read()
    # resume a second trainer from the PLY: same parameters, fresh moments
    _, _, tr2 = _trainer(trainer, seed=611)
    assert tr2.load_ply(tmp_path / "t.ply") == 0
    assert tr2.splat_count() == tr.splat_count()
    for g in range(6):
        assert_bits_equal(tr2.group(g), params[g], f"group {g}")
        assert not tr2.group(g, 1).any() and not tr2.group(g, 2).any()


def _parse_checkpoint(path):
    raw = open(path, "rb").read()
    magic, ver, step, n, deg, adam_steps = struct.unpack_from("<6I", raw, 0)
    lr = struct.unpack_from("<6f", raw, 24)
    lr_init, lr_final = struct.unpack_from("<2f", raw, 48)
    off, tensors = 56, []
    for _ in range(18):
        (ndim,) = struct.unpack_from("<I", raw, off)
        shape = struct.unpack_from(f"<{ndim}q", raw, off + 4)
        (nbytes,) = struct.unpack_from("<Q", raw, off + 4 + 8 * ndim)
        off += 4 + 8 * ndim + 8
        tensors.append(np.frombuffer(raw, np.float32, nbytes // 4, off).reshape(shape))
        off += nbytes
    assert off == len(raw)
    return dict(magic=magic, version=ver, step=step, n=n, degree=deg, adam_steps=adam_steps, lr=lr,
                lr_init=lr_init, lr_final=lr_final, tensors=tensors)


def test_checkpoint_round_trip(mods, tmp_path):
    _, _, trainer = mods
    sc, tg, tr = _trainer(trainer)
    for _ in range(3):
        tr.step()
    path = tmp_path / "c.msplat"
    tr.save_checkpoint(path)
    ck = _parse_checkpoint(path)
    assert ck["magic"] == 0x4C50534D and ck["version"] == 1
    assert ck["step"] == 3 and ck["n"] == tr.splat_count() and ck["degree"] == 3 and ck["adam_steps"] == 3
    assert ck["lr_init"] == np.float32(0.00016) and ck["lr_final"] == np.float32(0.0000016)
    assert ck["lr"][1:] == tuple(np.float32(x) for x in (0.005, 0.001, 0.0025, 0.000125, 0.05))
    shapes = [(3,), (3,), (4,), (3,), (15, 3), (1,)]
    for k in range(18):
        g, which = k % 6, k // 6
        assert ck["tensors"][k].shape == (ck["n"],) + shapes[g]
        assert_bits_equal(ck["tensors"][k].reshape(ck["n"], -1), tr.group(g, which), f"tensor {k}")
    # a trainer on other gaussians (same camera and target) takes over the
    # state and continues
    other = small_scene(n=1500, seed_off=612)
    cfg = trainer.TrainingConfig(iterations=1000, sh_degree=3, sh_degree_interval=0, num_downscales=0,
                                 warmup_length=10_000, shuffle_cameras=False)
    tr2 = trainer.GaussianTrainer(other.params(), sc.cameras, tg, cfg)
    assert tr2.load_checkpoint(path) == 3
    assert tr2.current_step == 3 and tr2.splat_count() == tr.splat_count()
    for g in range(6):
        for which in range(3):
            assert_bits_equal(tr2.group(g, which), tr.group(g, which), f"group {g}/{which}")
    s1, s2 = tr.step(), tr2.step()
    assert s1.iteration == s2.iteration == 4
    for g in range(6):
        grad_close(tr2.group(g), tr.group(g), what=f"after resume, group {g}")
    with pytest.raises(Exception, match="Not a valid msplat checkpoint"):
        bad = tmp_path / "bad.msplat"
        bad.write_bytes(b"\0" * 64)
        tr2.load_checkpoint(bad)


def test_evaluate_at_downscaled_resolution(mods):
    """num_downscales = 2 before the first resolution step: training and
    evaluation use the target at 1/4 by the reference's area resize
    (Camera::getImage, input_data.cpp:54-65), here on a 163x117 image that 4
    does not divide (40x29 cells of 4.075 x 4.034 source pixels)."""
    _, _, trainer = mods
    sc = small_scene(n=2000, width=163, height=117, seed_off=613)
    tg = [target_for(sc, (117, 163), seed_off=614)]
    cfg = trainer.TrainingConfig(iterations=10, sh_degree=3, sh_degree_interval=0, num_downscales=2,
                                 warmup_length=10_000, shuffle_cameras=False)
    tr = trainer.GaussianTrainer(sc.params(), sc.cameras, tg, cfg)
    tr.step()
    small = orc.resize_area(tg[0], 163 // 4, 117 // 4)
    r = tr.render(0)
    assert r.shape == small.shape
    m = tr.evaluate(sc.cameras, tg)
    want = orc.image_metrics(r, small)
    for k in ("psnr", "ssim", "l1"):
        assert abs(m[k] - want[k]) <= 1e-5 * max(1.0, abs(want[k])), (k, m[k], want[k])


def test_trainer_from_dataset(mods, tmp_path):
    """GaussianTrainer(dataset, config) and train(callback, callback_every)
    as the reference module's tests use them (tests/test_msplat.py:77-91):
    images decoded from disk and prepared on the GPU, gaussians from the
    point cloud, held-out cameras evaluated without arguments."""
    from PIL import Image
    from test_dataset_cpu import _write_model
    import msplat_amd as msplat
    _write_model(str(tmp_path), n_points=3000, seed=9)
    probe = msplat.load_dataset(str(tmp_path))
    rng = np.random.default_rng(4)
    for cam, path in zip(probe.cameras, probe.image_paths):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        Image.fromarray(rng.integers(0, 256, (cam.height, cam.width, 3), dtype=np.uint8), "RGB").save(path)
    ds = msplat.load_dataset(str(tmp_path), eval_mode=True, test_every=2)
    cfg = msplat.TrainingConfig(iterations=6, num_downscales=0, sh_degree_interval=0)
    tr = msplat.GaussianTrainer(ds, cfg)
    seen = []
    tr.train(lambda s: seen.append(s.iteration), callback_every=2)
    assert seen == [2, 4, 6] and tr.iteration == 6 and tr.splat_count() == 3000
    m = tr.evaluate()
    assert m["num_test"] == ds.num_test and np.isfinite(m["psnr"]) and 0.0 <= m["l1"] <= 1.0
