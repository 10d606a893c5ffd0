"""Writes the golden fixtures of the splatting path (tests/golden/*.npz).

The reference holds no golden vectors for this path (its tests are
end-to-end smoke tests on Apple hardware), so the fixtures are produced by
the CPU oracle, whose functions are pinned by tests/test_oracle_pins.py.
Each fixture holds one small seeded scene, its camera and target, and the
oracle's outputs of every stage: projection, tile bins and sorted ids, the
forward image / final T / final index, the SSIM loss and its image gradient,
the raster and projection gradients with the oracle's bounds on a GPU's
rounding difference, the gradient of each Adam group, and the parameters
and moments after one Adam step.

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import orc  # noqa: E402
from helpers import BG, LRS, small_scene, target_for  # noqa: E402
from msplat_amd import camera  # noqa: E402

CASES = {
    # name: (n, width, height, seed, spread, degree)  -- 2x3 and 3x2 tiles: chunked mode
    "sh3_small": (256, 48, 32, 301, 1.5, 3),
    "sh1_dense": (1000, 32, 32, 302, 0.4, 1),
}


def make(name, n, width, height, seed, spread, degree):
    sc = small_scene(n=n, width=width, height=height, degree=degree, seed_off=seed, spread=spread)
    su = camera.prepare_cam(sc.cameras[0])
    cam = orc.camera(su, degree, degree, BG)
    gt = target_for(sc, (su.height, su.width), seed_off=seed + 1)
    p = orc.project(cam, sc.means, sc.scales, sc.quats, sc.f_dc, sc.f_rest)
    counts, tile_bins, ids = orc.bin_sort(cam, p)
    r = orc.rasterize(cam, p, sc.opacities, tile_bins, ids)
    params = [np.ascontiguousarray(a, np.float32).copy() for a in sc.params()]
    m = [np.zeros_like(a) for a in params]
    v = [np.zeros_like(a) for a in params]
    vis, gnorm, max2d = (np.zeros(sc.n, np.float32) for _ in range(3))
    want = ("out_img", "radii", "v_xy", "v_conic", "v_rgb", "v_opacity", "v_mean3d", "v_scale", "v_quat",
            "v_rendered", "err_raster", "grad", "grad_err")
    loss, o = orc.train_step(cam, params, m, v, orc.adam_hparams(LRS, 1), gt, 0.2, vis, gnorm, max2d, want=want)
    out = dict(
        # inputs
        means=sc.means, scales=sc.scales, quats=sc.quats, f_dc=sc.f_dc, f_rest=sc.f_rest,
        opacities=sc.opacities, gt=gt, background=BG, degree=np.int32(degree),
        width=np.int32(su.width), height=np.int32(su.height),
        fx=np.float32(su.fx), fy=np.float32(su.fy), cx=np.float32(su.cx), cy=np.float32(su.cy),
        viewmat=su.viewmat, projmat=su.projmat, cam_pos=su.cam_pos, lrs=np.array(LRS, np.float32),
        # forward outputs
        xys=p["xys"], depths=p["depths"], radii=p["radii"], conics=p["conics"], colors=p["colors"],
        aabb=p["aabb"], num_tiles_hit=p["num_tiles_hit"], tile_counts=counts, tile_bins=tile_bins,
        gaussian_ids=ids, final_Ts=r["final_Ts"], final_index=r["final_index"], out_img=r["out_img"],
        # train step outputs
        loss=np.float32(loss), v_rendered=o["v_rendered"], v_xy=o["v_xy"], v_conic=o["v_conic"],
        v_rgb=o["v_rgb"], v_opacity=o["v_opacity"], v_mean3d=o["v_mean3d"], v_scale=o["v_scale"],
        v_quat=o["v_quat"], vis_counts=vis, xys_grad_norm=gnorm, max_2d_size=max2d,
        # the oracle's bounds on a GPU's difference (running error analysis)
        err_raster=o["err_raster"],
        **{f"grad{i}": o["grad"][i] for i in range(6)},
        **{f"grad_err{i}": o["grad_err"][i] for i in range(6)},
        **{f"param{i}_after": params[i] for i in range(6)},
        **{f"exp_avg{i}_after": m[i] for i in range(6)},
        **{f"exp_avg_sq{i}_after": v[i] for i in range(6)},
    )
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **{k: np.asarray(val) for k, val in out.items()})
    print(f"{path}: {len(ids)} intersections, loss {loss:.6f}, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    for name, args in CASES.items():
        make(name, *args)
