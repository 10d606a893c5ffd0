"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every stored output bit for bit (stages,
gradients, bounds, Adam state), so a change of the checker shows up here.
GPU: the HIP path reproduces the stored outputs directly, without running
the oracle: forward bit for bit, gradients within rel 1e-3 plus the stored
rounding bounds, Adam moments with those bounds carried through and the
update where the gradient's bound is the relative one.
"""
from __future__ import annotations

import glob
import os

import numpy as np
import pytest

import orc
from helpers import U, assert_bits_equal, bound_check
from msplat_amd import camera

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _setup(f):
    W, H = int(f["width"]), int(f["height"])
    return camera.CamSetup(float(f["fx"]), float(f["fy"]), float(f["cx"]), float(f["cy"]), H, W,
                           f["viewmat"], f["projmat"], f["cam_pos"], ((W + 15) // 16, (H + 15) // 16, 1))


def _params(f):
    return [f[k] for k in ("means", "scales", "quats", "f_dc", "f_rest", "opacities")]


def test_fixtures_present():
    names = {os.path.basename(p) for p in FIXTURES}
    assert {"sh3_small.npz", "sh1_dense.npz"} <= names


@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p))
def test_oracle_reproduces_golden(path):
    f = _load(path)
    su, deg = _setup(f), int(f["degree"])
    cam = orc.camera(su, deg, deg, f["background"])
    p = orc.project(cam, f["means"], f["scales"], f["quats"], f["f_dc"], f["f_rest"])
    vis = p["radii"] > 0
    assert_bits_equal(p["radii"], f["radii"], "radii")
    for k in ("xys", "depths", "conics", "colors", "aabb"):
        assert_bits_equal(p[k][vis], f[k][vis], k)
    counts, tb, ids = orc.bin_sort(cam, p)
    assert_bits_equal(tb, f["tile_bins"], "tile_bins")
    assert_bits_equal(ids, f["gaussian_ids"], "gaussian_ids")
    r = orc.rasterize(cam, p, f["opacities"], tb, ids)
    for k in ("final_Ts", "final_index", "out_img"):
        assert_bits_equal(r[k], f[k], k)
    params = [np.ascontiguousarray(a, np.float32).copy() for a in _params(f)]
    m = [np.zeros_like(a) for a in params]
    v = [np.zeros_like(a) for a in params]
    n = params[0].shape[0]
    vc, gn, mx = (np.zeros(n, np.float32) for _ in range(3))
    loss, o = orc.train_step(cam, params, m, v, orc.adam_hparams(list(f["lrs"]), 1), f["gt"], 0.2, vc, gn, mx,
                             want=("v_rendered", "v_xy", "v_conic", "v_rgb", "v_opacity", "v_mean3d", "v_scale",
                                   "v_quat", "err_raster", "grad", "grad_err"))
    assert np.float32(loss) == f["loss"]
    for k in ("v_rendered", "v_xy", "v_conic", "v_rgb", "v_opacity", "v_mean3d", "v_scale", "v_quat",
              "err_raster"):
        assert_bits_equal(o[k], f[k], k)
    for i in range(6):
        assert_bits_equal(o["grad"][i], f[f"grad{i}"], f"grad{i}")
        assert_bits_equal(o["grad_err"][i], f[f"grad_err{i}"], f"grad_err{i}")
        assert_bits_equal(params[i], f[f"param{i}_after"], f"param{i}")
        assert_bits_equal(m[i], f[f"exp_avg{i}_after"], f"exp_avg{i}")
        assert_bits_equal(v[i], f[f"exp_avg_sq{i}_after"], f"exp_avg_sq{i}")
    for k in ("vis_counts", "max_2d_size", "xys_grad_norm"):
        assert_bits_equal({"vis_counts": vc, "max_2d_size": mx, "xys_grad_norm": gn}[k], f[k], k)


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=lambda p: os.path.basename(p))
def test_gpu_matches_golden(path):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from msplat_amd import device
    device.init(0)
    f = _load(path)
    su, deg = _setup(f), int(f["degree"])
    bg = f["background"]
    n = f["means"].shape[0]
    g = device.DeviceGaussians.from_arrays(_params(f), deg, capacity=n)
    img = device.render(g, su, deg, bg).cpu().numpy()
    assert_bits_equal(img, f["out_img"], "out_img")
    assert_bits_equal(device.intermediate("tile_bins", np.int32).reshape(-1, 2), f["tile_bins"], "tile_bins")
    assert_bits_equal(device.intermediate("gaussian_ids", np.int32), f["gaussian_ids"], "gaussian_ids")
    H, W = su.height, su.width
    assert_bits_equal(device.intermediate("final_index", np.int32).reshape(H, W), f["final_index"], "final_index")
    grads = {k: torch.zeros((n, d), dtype=torch.float32, device="cuda") for k, d in
             (("v_mean3d", 3), ("v_scale", 3), ("v_quat", 4))}
    loss = device.train_step(g, su, deg, bg, device.to_dev(f["gt"]), 0.2, list(f["lrs"]), 1, grads_out=grads)
    assert abs(loss - float(f["loss"])) <= 1e-5 * abs(float(f["loss"]))
    assert_bits_equal(device.intermediate("v_rendered").reshape(H, W, 3), f["v_rendered"], "v_rendered")
    er = f["err_raster"]
    for k, q0, d in (("v_xy", 0, 2), ("v_conic", 2, 3), ("v_rgb", 5, 3), ("v_opacity", 8, 1)):
        got = device.intermediate(k).reshape(n, d)
        bound_check(got, f[k].reshape(n, d), er[:, q0:q0 + d], what=k)
    for i, k in enumerate(("v_mean3d", "v_scale", "v_quat")):
        bound_check(grads[k].cpu().numpy(), f[f"grad{i}"], f[f"grad_err{i}"], what=k)
    # Adam from zero moments: m = (1 - b1) g, and the update where the
    # gradient's bound is its relative term (then the update, about
    # -lr sign(g) at step 1, is fixed to its rounding)
    om1 = float(np.float32(1) - np.float32(0.9))
    params0 = _params(f)
    for i in range(6):
        go, ge = f[f"grad{i}"].astype(np.float64), f[f"grad_err{i}"].astype(np.float64)
        bound_check(g.m[i][:n].cpu().numpy(), f[f"exp_avg{i}_after"], om1 * ge + 6 * U * om1 * np.abs(go) + 1e-45,
                    what=f"exp_avg{i}")
        rd = (ge <= 1e-3 * np.abs(go)) & (go != 0)
        p0 = np.asarray(params0[i], np.float64)
        du = g.bufs[i][:n].cpu().numpy().astype(np.float64) - p0
        du_o = f[f"param{i}_after"].astype(np.float64) - p0
        ulp = np.spacing(np.abs(f[f"param{i}_after"]).astype(np.float32)).astype(np.float64)
        bound_check(du[rd], du_o[rd], 4 * ulp[rd] + 1e-3 * np.abs(du_o[rd]), rel=1e-5, what=f"update{i}")
        assert_bits_equal(g.bufs[i][:n].cpu().numpy()[go == 0] if i in (3, 4) else np.zeros(0),
                          f[f"param{i}_after"][go == 0] if i in (3, 4) else np.zeros(0), f"untouched {i}")
