"""GPU-vs-oracle comparison routines shared by the parity tests.

Each routine runs one render / train step / densify through the C ABI
(msplat_amd.device) and the same step on the CPU oracle (tests/orc.py) from
identical inputs, then compares:
  * projection outputs, tile counts / offsets / sorted id lists, the raster
    forward (final T, final index, image) and the loss gradient image: bit for
    bit;
  * raster / projection gradients, Adam-updated parameters and moments:
    relative 1e-3 with an absolute floor of 1e-4 of the tensor's largest
    value (grad_close), since float atomics sum in another order than the
    oracle's fixed-order sums;
  * densify counts, order and values on identical statistics and random
    samples: bit for bit.
Progress lines are printed (and flushed) before each GPU step, so that a run
that ends early names the case it was in.
"""
from __future__ import annotations

import time

import numpy as np

import orc
from helpers import BG, LRS, assert_bits_equal, grad_close
from msplat_amd import camera

PARAM_NAMES = ("means", "scales", "quats", "f_dc", "f_rest", "opacities")


def say(msg):
    print(f"[parity {time.strftime('%H:%M:%S')}] {msg}", flush=True)


def render_and_compare(dev, params, degree, cam_obj, dtu=None, bg=BG, label=""):
    """Render through the C ABI and compare every forward stage with the oracle.
    params: six host float32 arrays.  Returns (meta, tile counts)."""
    dtu = degree if dtu is None else dtu
    su = camera.prepare_cam(cam_obj)
    means, scales, quats, f_dc, f_rest, opac = params
    n = int(means.shape[0])
    say(f"render {label}: {n} gaussians, {su.width}x{su.height}, SH {degree}/{dtu}")
    g = dev.DeviceGaussians.from_arrays(params, degree)
    img = dev.render(g, su, dtu, bg).cpu().numpy()
    say(f"render {label}: GPU done, oracle projection")
    cam = orc.camera(su, degree, dtu, bg)
    p = orc.project(cam, means, scales, quats, f_dc, f_rest)
    assert_bits_equal(dev.intermediate("radii", np.int32), p["radii"], "radii")
    assert_bits_equal(dev.intermediate("num_tiles_hit", np.int32), p["num_tiles_hit"], "num_tiles_hit")
    vis = p["radii"] > 0
    assert vis.sum() > 0
    assert_bits_equal(dev.intermediate("xys").reshape(n, 2)[vis], p["xys"][vis], "xys")
    assert_bits_equal(dev.intermediate("depths")[vis], p["depths"][vis], "depths")
    assert_bits_equal(dev.intermediate("aabb").reshape(n, 2)[vis], p["aabb"][vis], "aabb")
    assert_bits_equal(dev.intermediate("conics").reshape(n, 3)[vis], p["conics"][vis], "conics")
    assert_bits_equal(dev.intermediate("colors").reshape(n, 3)[vis], p["colors"][vis], "colors")
    say(f"render {label}: oracle binning")
    counts, tile_bins, ids = orc.bin_sort(cam, p)
    assert_bits_equal(dev.intermediate("tile_bins", np.int32).reshape(-1, 2), tile_bins, "tile_bins")
    assert_bits_equal(dev.intermediate("gaussian_ids", np.int32), ids, "gaussian_ids")
    say(f"render {label}: {int(counts.sum())} intersections, largest tile {int(counts.max())}; oracle raster")
    r = orc.rasterize(cam, p, opac, tile_bins, ids)
    H, W = su.height, su.width
    assert_bits_equal(dev.intermediate("final_Ts").reshape(H, W), r["final_Ts"], "final_Ts")
    assert_bits_equal(dev.intermediate("final_index", np.int32).reshape(H, W), r["final_index"], "final_index")
    assert_bits_equal(img, r["out_img"], "out_img")
    work = dev.raster_work()
    assert [work[k] for k in dev.RASTER_WORK_KEYS[:3]] == orc.raster_counts()[:3], (work, orc.raster_counts())
    say(f"render {label}: bit-exact")
    return dev.meta(), counts


class TrainResult:
    """GPU state (DeviceGaussians) and oracle state after train_compare."""

    def __init__(self, g, params, m, v, vis, gnorm, max2d, loss_gpu, loss_orc):
        self.g, self.params, self.m, self.v = g, params, m, v
        self.vis, self.gnorm, self.max2d = vis, gnorm, max2d
        self.loss_gpu, self.loss_orc = loss_gpu, loss_orc


def train_compare(dev, params, degree, cam_obj, gt, steps=1, dtu=None, check_grads=True, capacity=None,
                  bg=BG, label=""):
    """`steps` train steps through the C ABI and on the oracle from the same
    parameters and target (host float32 [H,W,3]); compares the first step's
    forward, loss image, gradients and work counts, and every parameter,
    moment and statistic after the last step."""
    import torch
    dtu = degree if dtu is None else dtu
    su = camera.prepare_cam(cam_obj)
    H, W = su.height, su.width
    n = int(params[0].shape[0])
    say(f"train {label}: {n} gaussians, {W}x{H}, {steps} step(s)")
    g = dev.DeviceGaussians.from_arrays(params, degree, capacity=capacity or n)
    gt_d = dev.to_dev(np.ascontiguousarray(gt, np.float32))
    grads = {k: torch.zeros((n, d), dtype=torch.float32, device="cuda") for k, d in
             (("v_mean3d", 3), ("v_scale", 3), ("v_quat", 4))}
    ps = [np.ascontiguousarray(a, np.float32).copy() for a in params]
    m = [np.zeros_like(a) for a in ps]
    v = [np.zeros_like(a) for a in ps]
    vis, gnorm, max2d = (np.zeros(n, np.float32) for _ in range(3))
    cam = orc.camera(su, degree, dtu, bg)
    loss_g = loss_o = None
    for step in range(1, steps + 1):
        say(f"train {label}: GPU step {step}")
        loss_g = dev.train_step(g, su, dtu, bg, gt_d, 0.2, LRS, step, grads_out=grads)
        want = ("out_img", "radii", "v_xy", "v_conic", "v_rgb", "v_opacity", "v_mean3d", "v_scale", "v_quat",
                "v_rendered")
        say(f"train {label}: oracle step {step}")
        loss_o, o = orc.train_step(cam, ps, m, v, orc.adam_hparams(LRS, step), gt, 0.2, vis, gnorm, max2d,
                                   want=want)
        assert abs(loss_g - loss_o) <= 1e-5 * abs(loss_o), (loss_g, loss_o)
        if step == 1:
            work = dev.raster_work()
            assert [work[k] for k in dev.RASTER_WORK_KEYS] == orc.raster_counts(), (work, orc.raster_counts())
            assert_bits_equal(dev.intermediate("out_img").reshape(H, W, 3), o["out_img"], "out_img")
            assert_bits_equal(dev.intermediate("v_rendered").reshape(H, W, 3), o["v_rendered"], "v_rendered")
            assert_bits_equal(dev.intermediate("radii", np.int32), o["radii"], "radii")
        if check_grads and step == 1:
            for k, d in (("v_xy", 2), ("v_conic", 3), ("v_rgb", 3), ("v_opacity", 1)):
                grad_close(dev.intermediate(k).reshape(n, d) if d > 1 else dev.intermediate(k),
                           o[k], what=k)
            for k in ("v_mean3d", "v_scale", "v_quat"):
                grad_close(grads[k].cpu().numpy(), o[k], what=k)
    gp = g.numpy()
    for i in range(6):
        grad_close(gp[i], ps[i], rtol=1e-3, floor=1e-6, what=f"param {PARAM_NAMES[i]}")
        grad_close(g.m[i][:n].cpu().numpy(), m[i], what=f"exp_avg {PARAM_NAMES[i]}")
        grad_close(g.v[i][:n].cpu().numpy(), v[i], rtol=2e-3, what=f"exp_avg_sq {PARAM_NAMES[i]}")
    grad_close(g.vis[:n].cpu().numpy(), vis, rtol=0, floor=0, what="vis_counts")
    grad_close(g.gnorm[:n].cpu().numpy(), gnorm, what="xys_grad_norm")
    grad_close(g.max2d[:n].cpu().numpy(), max2d, rtol=0, floor=0, what="max_2d_size")
    say(f"train {label}: within tolerance (loss {loss_g:.6f} vs {loss_o:.6f})")
    return TrainResult(g, ps, m, v, vis, gnorm, max2d, loss_g, loss_o)


def densify_compare(dev, g, rnd, half_max_dim, grad_thresh=2e-4, size_thresh=0.01, screen_thresh=0.05,
                    check_screen=True, cull_alpha=0.005, cull_scale=0.5, cull_screen=0.15, check_huge=False,
                    label=""):
    """Densify the GPU state g (DeviceGaussians, statistics included) on the
    GPU and a host copy of the same state on the oracle, with the same random
    samples rnd (device [2N*3]); counts, flags, order and values bit for bit.
    Returns (new count, splits, duplicates, culled)."""
    n = g.n
    say(f"densify {label}: copying {n} gaussians (capacity {g.capacity}) to the host")
    bufs = [b.cpu().numpy().copy() for b in g.bufs]
    ms = [b.cpu().numpy().copy() for b in g.m]
    vs = [b.cpu().numpy().copy() for b in g.v]
    gnorm = g.gnorm[:n].cpu().numpy().copy()
    vis = g.vis[:n].cpu().numpy().copy()
    max2d = g.max2d[:n].cpu().numpy().copy()
    rnd_h = rnd.cpu().numpy()
    oa = orc.OrcDensifyArgs()
    oa.N = n
    oa.grad_thresh, oa.size_thresh, oa.screen_thresh, oa.check_screen = (grad_thresh, size_thresh, screen_thresh,
                                                                         int(check_screen))
    oa.cull_alpha_thresh, oa.cull_scale_thresh, oa.cull_screen_size, oa.check_huge = (cull_alpha, cull_scale,
                                                                                      cull_screen, int(check_huge))
    oa.half_max_dim, oa.fr_stride = half_max_dim, g.rest_bases() * 3
    say(f"densify {label}: oracle")
    nn_o, split, dup, keep = orc.densify(oa, gnorm, vis, max2d, bufs, ms, vs, rnd_h)
    say(f"densify {label}: GPU")
    nn_g = dev.densify(g, grad_thresh=grad_thresh, size_thresh=size_thresh, screen_thresh=screen_thresh,
                       check_screen=int(check_screen), cull_alpha=cull_alpha, cull_scale=cull_scale,
                       cull_screen=cull_screen, check_huge=int(check_huge), half_max_dim=half_max_dim,
                       random_samples=rnd)
    assert nn_g == nn_o, (nn_g, nn_o)
    for i in range(6):
        assert_bits_equal(g.bufs[i][:nn_o].cpu().numpy(), bufs[i][:nn_o], f"densified {PARAM_NAMES[i]}")
        assert_bits_equal(g.m[i][:nn_o].cpu().numpy(), ms[i][:nn_o], f"densified exp_avg {PARAM_NAMES[i]}")
        assert_bits_equal(g.v[i][:nn_o].cpu().numpy(), vs[i][:nn_o], f"densified exp_avg_sq {PARAM_NAMES[i]}")
    n_split, n_dup = int(split.sum()), int(dup.sum())
    culled = n + n_split * 2 + n_dup - nn_o
    say(f"densify {label}: {n} -> {nn_o} ({n_split} split, {n_dup} duplicated, {culled} culled), bit-exact")
    return nn_o, n_split, n_dup, culled
