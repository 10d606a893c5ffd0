"""The C++ host trainer (include/msplat_trainer.h) on the GPU.

Checks GaussianTrainer::step against the oracle's train step sequence (the
trainer's Model builds the same camera set-up, bias corrections and Adam
arguments as model.cpp:546-597), the afterTrain policy (opacity reset at
step % (resetAlphaEvery * refineEvery) == refineEvery, densification after
the camera epoch, model.cpp:236-296) and render_from_pose.
"""
from __future__ import annotations

import numpy as np
import pytest

import orc
from helpers import BG, LRS, assert_bits_equal, grad_close, small_scene, target_for
from msplat_amd import camera, synthetic

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from msplat_amd import device, trainer
    device.init(0)
    return device, trainer


def _scene_two_cams(n=2500, seed=400):
    sc = small_scene(n=n, seed_off=seed)
    cam2 = camera.pinhole(sc.cameras[0].width, sc.cameras[0].height, 70.0,
                          camera.look_at(np.array([4.0, 1.0, -2.5])))
    sc.cameras.append(cam2)
    tg = [target_for(sc, (c.height, c.width), seed_off=seed + 1 + i) for i, c in enumerate(sc.cameras)]
    return sc, tg


def test_trainer_steps_match_oracle(mods):
    device, trainer = mods
    sc, tg = _scene_two_cams()
    cfg = trainer.TrainingConfig(iterations=1000, sh_degree=3, sh_degree_interval=0, num_downscales=0,
                                 warmup_length=10_000, shuffle_cameras=False)
    tr = trainer.GaussianTrainer(sc.params(), sc.cameras, tg, cfg)
    params = [np.ascontiguousarray(a, np.float32).copy() for a in sc.params()]
    m = [np.zeros_like(a) for a in params]
    v = [np.zeros_like(a) for a in params]
    n = sc.n
    vis, gn, mx = (np.zeros(n, np.float32) for _ in range(3))
    lrs = list(LRS)
    for step in range(1, 4):
        ci = (step - 1) % 2
        st = tr.step()
        assert st.iteration == step and st.splat_count == n
        su = camera.prepare_cam(sc.cameras[ci])
        cam = orc.camera(su, 3, 3, BG)
        orc.train_step(cam, params, m, v, orc.adam_hparams(lrs, step), tg[ci], 0.2, vis, gn, mx)
        # schedulersStep (model.cpp:179-182) after the step
        t = min(max(step / 1000, 0.0), 1.0)
        lrs[0] = float(np.exp(np.log(np.float32(0.00016)) * (1 - t) + np.log(np.float32(0.0000016)) * t))
    loss = tr.last_loss(wait=True)
    assert np.isfinite(loss) and 0 < loss < 1
    got = tr.params()
    for g in range(6):
        grad_close(got[g].reshape(params[g].shape), params[g], rtol=1e-3, floor=1e-6, what=f"param {g}")
        grad_close(tr.group(g, 1).reshape(m[g].shape), m[g], what=f"exp_avg {g}")


def test_trainer_refinement_policy(mods):
    """refineEvery 2, resetAlphaEvery 5 (reset interval 10), two cameras:
    step 2 resets opacities to <= logit(0.2) and zeroes their moments; steps
    6 and 8 (step % 10 > 2 + 2) densify; step 10 does neither."""
    device, trainer = mods
    sc, tg = _scene_two_cams(n=3000, seed=410)
    cfg = trainer.TrainingConfig(iterations=100, sh_degree=3, sh_degree_interval=0, num_downscales=0,
                                 warmup_length=0, refine_every=2, reset_alpha_every=5,
                                 densify_grad_thresh=1e-7, cull_alpha_thresh=0.005, shuffle_cameras=False)
    tr = trainer.GaussianTrainer(sc.params(), sc.cameras, tg, cfg)
    counts = []
    for step in range(1, 11):
        tr.step()
        counts.append(tr.splat_count())
        if step == 2:
            op = tr.group(5)
            assert op.max() <= np.float32(-1.3862943611198906)
            assert not tr.group(5, 1).any() and not tr.group(5, 2).any()
    assert counts[0] == counts[1] == counts[2] == counts[3] == counts[4] == 3000
    assert counts[5] > 3000, counts          # densified at step 6
    assert counts[7] > counts[6], counts     # and at step 8
    assert counts[9] == counts[8], counts    # step 10: 10 % 10 = 0, no densify


def test_trainer_render_from_pose(mods):
    device, trainer = mods
    sc, tg = _scene_two_cams(n=1500, seed=420)
    cfg = trainer.TrainingConfig(iterations=100, sh_degree_interval=0, num_downscales=0)
    tr = trainer.GaussianTrainer(sc.params(), sc.cameras, tg, cfg)
    pose = np.asarray(sc.cameras[1].cam_to_world, np.float32)
    img = tr.render_from_pose(pose, 1)
    su = camera.prepare_cam(sc.cameras[1])
    ref, _, _ = orc.render(orc.camera(su, 3, 3, BG), sc.means, sc.scales, sc.quats, sc.f_dc, sc.f_rest,
                           sc.opacities)
    assert_bits_equal(img, ref, "render_from_pose")
    with pytest.raises(IndexError):
        tr.render_from_pose(pose, 5)
    with pytest.raises(ValueError):
        tr.render_from_pose(np.eye(3), 0)
