"""smoke(): one small render + train step on cuda:0, checked against the CPU oracle."""
from __future__ import annotations

import numpy as np


def run_smoke() -> None:
    import torch

    import orc
    from helpers import BG, LRS, assert_bits_equal, grad_close, small_scene, target_for
    from msplat_amd import camera, device

    if not torch.cuda.is_available():
        raise RuntimeError("smoke() needs cuda:0")
    device.init(0)
    sc = small_scene(n=2000, seed_off=90)
    su = camera.prepare_cam(sc.cameras[0])
    H, W = su.height, su.width
    gt = target_for(sc, (H, W))
    g = device.DeviceGaussians.from_arrays(sc.params(), 3)
    img = device.render(g, su, 3, BG).cpu().numpy()
    cam = orc.camera(su, 3, 3, BG)
    ref_img, _, _ = orc.render(cam, sc.means, sc.scales, sc.quats, sc.f_dc, sc.f_rest, sc.opacities)
    assert_bits_equal(img, ref_img, "smoke render")
    loss = device.train_step(g, su, 3, BG, device.to_dev(gt), 0.2, LRS, 1)
    params = [np.ascontiguousarray(a, np.float32).copy() for a in sc.params()]
    m = [np.zeros_like(a) for a in params]
    v = [np.zeros_like(a) for a in params]
    z = [np.zeros(sc.n, np.float32) for _ in range(3)]
    loss_o, _ = orc.train_step(cam, params, m, v, orc.adam_hparams(LRS, 1), gt, 0.2, *z)
    assert abs(loss - loss_o) <= 1e-5 * abs(loss_o), (loss, loss_o)
    for i, p in enumerate(g.numpy()):
        grad_close(p, params[i], rtol=1e-3, floor=1e-6, what=f"smoke param {i}")
    print(f"smoke ok: loss {loss:.6f} (oracle {loss_o:.6f}), render bit-exact")
