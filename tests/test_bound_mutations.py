"""The gradient parity check at the benchmark's size, on the CPU.

helpers.bound_check accepts |gpu - orc| <= 1e-3 |orc| + err at every
element, where err is the oracle's running-error bound on the rounding
difference of the two evaluations (OrcTrainOut.err_raster / grad_err), and,
for the gradients summed straight from pixel terms, |gpu - orc| <= 1e-3
|orc| + 8 u sum|terms| at all but 0.01% of them.  Here the oracle's own
gradients of one config-2 train step (500k SH3 gaussians, 1297x840) stand in
for the GPU's and are perturbed: the check must pass differences of the size
rounding can make and reject each of
  * x1.01 on every 7th gaussian,
  * zeroing the elements below the median magnitude,
  * a sign flip of v_mean3d,
for every gradient the parity tests compare (the raster gradients, the
gradient of each Adam group, and the first moment after the step).
"""
from __future__ import annotations

import numpy as np
import pytest

import orc
from helpers import BG, LRS, bound_check
from msplat_amd import camera, synthetic

N_CONFIG2 = 500_000


@pytest.fixture(scope="module")
def step():
    sc = synthetic.config2(n=N_CONFIG2)
    cam_obj = sc.cameras[0]
    su = camera.prepare_cam(cam_obj)
    cam = orc.camera(su, 3, 3, BG)

    def render(s, c):
        return orc.render(orc.camera(camera.prepare_cam(c), 3, 3, BG), s.means, s.scales, s.quats, s.f_dc,
                          s.f_rest, s.opacities)[0]

    gt = synthetic.make_targets(sc, render)[0]
    ps = [np.ascontiguousarray(a, np.float32).copy() for a in sc.params()]
    m = [np.zeros_like(a) for a in ps]
    v = [np.zeros_like(a) for a in ps]
    vis, gn, mx = (np.zeros(N_CONFIG2, np.float32) for _ in range(3))
    want = ("radii", "v_xy", "v_conic", "v_rgb", "v_opacity", "mag_raster", "err_raster", "grad", "grad_mag",
            "grad_err")
    _, o = orc.train_step(cam, ps, m, v, orc.adam_hparams(LRS, 1), gt, 0.2, vis, gn, mx, want=want)
    n = N_CONFIG2
    er, mr = o["err_raster"], o["mag_raster"]
    f64 = lambda a: np.asarray(a, np.float64)
    cases = {}   # name: (gradient, tier-A bound, tier-B magnitude or None)
    for k, q0, d in (("v_xy", 0, 2), ("v_conic", 2, 3), ("v_rgb", 5, 3), ("v_opacity", 8, 1)):
        cases[k] = (f64(o[k].reshape(n, d)), f64(er[:, q0:q0 + d]), f64(mr[:, q0:q0 + d]))
    for i, k in enumerate(("v_mean3d", "v_scale", "v_quat", "grad f_dc", "grad f_rest", "grad opacity")):
        cases[k] = (f64(o["grad"][i].reshape(n, -1)), f64(o["grad_err"][i].reshape(n, -1)),
                    f64(o["grad_mag"][i].reshape(n, -1)) if i >= 3 else None)
    # first moment after step 1: (1 - b1) g, the bounds scaled alike
    om1 = float(np.float32(1) - np.float32(0.9))
    cases["exp_avg means"] = (om1 * cases["v_mean3d"][0], om1 * cases["v_mean3d"][1], None)
    cases["exp_avg f_rest"] = tuple(om1 * x for x in cases["grad f_rest"])
    assert int((o["radii"] > 0).sum()) > 100_000
    return cases


NAMES = ("v_xy", "v_conic", "v_rgb", "v_opacity", "v_mean3d", "v_scale", "v_quat", "grad f_dc", "grad f_rest",
         "grad opacity", "exp_avg means", "exp_avg f_rest")


@pytest.mark.parametrize("name", NAMES)
def test_accepts_rounding_sized_differences(step, name):
    """The oracle's gradient moved by up to 90% of its rounding bound and by
    up to 5e-4 relative (both at random) passes; the statistics show how
    the check decides at this size."""
    g, e, mg = step[name]
    rng = np.random.default_rng(7)
    # tier A alone: up to 90% of the rounding bound
    moved = g + e * rng.uniform(-0.9, 0.9, g.shape) + g * rng.uniform(-5e-4, 5e-4, g.shape)
    st = bound_check(moved, g, e, what=name, log=print)
    if mg is not None:   # both tiers: up to 90% of the smaller of the bound and 8 u sum|terms|
        w = np.minimum(e, 8 * 2.0 ** -24 * mg)
        moved = g + w * rng.uniform(-0.9, 0.9, g.shape) + g * rng.uniform(-5e-4, 5e-4, g.shape)
        bound_check(moved, g, e, what=name, log=print, mag=mg)
    # the bound binds: returning zero fails almost everywhere
    assert st["zero_pass"] < 0.02, st


def _rejected(moved, g, e, mg, name):
    """Elements the check rejects (tier A, else tier B's excess)."""
    with pytest.raises(AssertionError) as exc:
        bound_check(moved, g, e, what=name, mag=mg)
    return int(str(exc.value).split(":")[1].split(" of ")[0])


@pytest.mark.parametrize("name", NAMES)
def test_rejects_one_percent_on_every_seventh_gaussian(step, name):
    g, e, mg = step[name]
    moved = g.copy()
    moved[::7] *= 1.01
    nbad = _rejected(moved, g, e, mg, name)
    changed = int(np.count_nonzero(g[::7]))
    print(f"{name}: x1.01 on every 7th gaussian caught at {nbad} of {changed} changed elements")
    assert nbad > 0.1 * changed


@pytest.mark.parametrize("name", NAMES)
def test_rejects_zeroing_below_the_median(step, name):
    g, e, mg = step[name]
    mag = np.abs(g)
    med = np.median(mag[mag > 0])
    moved = np.where(mag < med, 0.0, g)
    nbad = _rejected(moved, g, e, mg, name)
    changed = int(np.count_nonzero((mag < med) & (mag > 0)))
    print(f"{name}: zeroing below the median caught at {nbad} of {changed} changed elements")
    assert nbad > 0.9 * changed


@pytest.mark.parametrize("name", ("v_mean3d", "exp_avg means"))
def test_rejects_sign_flip(step, name):
    g, e, mg = step[name]
    nbad = _rejected(-g, g, e, mg, name)
    changed = int(np.count_nonzero(g))
    print(f"{name}: sign flip caught at {nbad} of {changed} nonzero elements")
    assert nbad > 0.95 * changed
