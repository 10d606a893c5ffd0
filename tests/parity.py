"""GPU-vs-oracle comparison routines shared by the parity tests.

Each routine runs one render / train step / densify through the C ABI
(msplat_amd.device) and the same step on the CPU oracle (tests/orc.py) from
identical inputs, then compares:
  * projection outputs, tile counts / offsets / sorted id lists, the raster
    forward (final T, final index, image) and the loss gradient image: bit for
    bit;
  * raster / projection gradients, Adam updates and moments: relative 1e-3
    plus the oracle's running-error bound of the two evaluations (float
    atomics sum in another order than the oracle's fixed-order sums, the
    kernels use hardware reciprocals); the projection backward and Adam
    again on the GPU's own inputs, to their arithmetic's rounding;
  * densify counts, order and values on identical statistics and random
    samples: bit for bit.
Progress lines are printed (and flushed) before each GPU step, so that a run
that ends early names the case it was in.
"""
from __future__ import annotations

import time

import numpy as np

import orc
from helpers import BG, LRS, U, assert_bits_equal, bound_check
from msplat_amd import camera

PARAM_NAMES = ("means", "scales", "quats", "f_dc", "f_rest", "opacities")


def say(msg):
    print(f"[parity {time.strftime('%H:%M:%S')}] {msg}", flush=True)


def render_and_compare(dev, params, degree, cam_obj, dtu=None, bg=BG, label="", clip=0.01):
    """Render through the C ABI and compare every forward stage with the oracle.
    params: six host float32 arrays.  Returns (meta, tile counts)."""
    dtu = degree if dtu is None else dtu
    su = camera.prepare_cam(cam_obj)
    means, scales, quats, f_dc, f_rest, opac = params
    n = int(means.shape[0])
    say(f"render {label}: {n} gaussians, {su.width}x{su.height}, SH {degree}/{dtu}")
    g = dev.DeviceGaussians.from_arrays(params, degree)
    img = dev.render(g, su, dtu, bg, clip=clip).cpu().numpy()
    say(f"render {label}: GPU done, oracle projection")
    cam = orc.camera(su, degree, dtu, bg, clip=clip)
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
    """GPU state (DeviceGaussians) after train_compare and the oracle's
    outputs of the last step."""

    def __init__(self, g, loss_gpu, loss_orc, stats):
        self.g = g
        self.loss_gpu, self.loss_orc = loss_gpu, loss_orc
        self.stats = stats   # what each bound check decided, by name


def _host_state(g, n):
    """Host copies of the GPU's parameters, moments and statistics."""
    return ([b[:n].cpu().numpy().copy() for b in g.bufs], [b[:n].cpu().numpy().copy() for b in g.m],
            [b[:n].cpu().numpy().copy() for b in g.v],
            [x[:n].cpu().numpy().copy() for x in (g.vis, g.gnorm, g.max2d)])


def _as_group(g, shape):
    """A gradient array in its parameter group's shape."""
    return np.asarray(g, np.float32).reshape(shape)


def _ulp(x):
    """Spacing of float32 at |x| (one unit in the last place)."""
    x = np.abs(np.asarray(x, np.float32))
    return np.spacing(x).astype(np.float64)


def _adam_ref(p, m, v, g, step_size, bc2_sqrt, b1=0.9, b2=0.999, eps=1e-8):
    """fused_adam (.metal:1666-1689) in float64 from float32 state and
    constants: new m, new v, the update and d(update)/dg."""
    f = np.float32
    b1, b2, eps = f(b1), f(b2), f(eps)
    omb1, omb2 = f(1) - b1, f(1) - b2
    b1, b2, omb1, omb2, eps = (float(x) for x in (b1, b2, omb1, omb2, eps))
    m, v, g = (np.asarray(a, np.float64) for a in (m, v, g))
    mn = b1 * m + omb1 * g
    vn = b2 * v + omb2 * g * g
    sq = np.sqrt(vn)
    D = sq / bc2_sqrt + eps
    upd = -step_size * mn / D
    dsq = np.where(sq > 0, omb2 * g / np.maximum(sq, 1e-300), 0.0)
    dupd = -step_size * (omb1 / D - mn * dsq / (bc2_sqrt * D * D))
    rnd_m = b1 * np.abs(m) + omb1 * np.abs(g)
    rnd_v = b2 * np.abs(v) + omb2 * g * g
    return mn, vn, upd, dupd, rnd_m, rnd_v


def train_compare(dev, params, degree, cam_obj, gt, steps=1, dtu=None, check_grads=True, capacity=None,
                  bg=BG, label=""):
    """`steps` train steps through the C ABI, each also run on the oracle from
    the GPU's own state before it (parameters, moments, statistics), so every
    step is checked the same way (host float32 [H,W,3] target):
      * forward stages, loss gradient image and work counts bit for bit;
      * raster gradients and the gradients fed to Adam against the oracle's
        within rel 1e-3 + the oracle's running-error bound of the two
        evaluations (bound_check);
      * the projection backward again on the GPU's own raster gradients, and
        the Adam update, moments and statistics on the GPU's own gradients,
        to their arithmetic's rounding bound (the update within rel 1e-5 plus
        the parameter's last-place rounding): each kernel's arithmetic alone;
      * Adam moments and statistics against the oracle's (the gradient bound
        carried through), the update against the oracle's where the gradient
        bound is the relative one, and untouched elements bit for bit."""
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
    cam = orc.camera(su, degree, dtu, bg)
    rest_bases = g.rest_bases()
    nb_use = min(rest_bases, (min(dtu, 3) + 1) ** 2 - 1)
    inv_max_dim = np.float32(1.0) / np.float32(max(H, W))
    stats = {}
    loss_g = loss_o = None
    for step in range(1, steps + 1):
        pb, mb, vb, (visb, gnb, mxb) = _host_state(g, n)
        say(f"train {label}: GPU step {step}")
        loss_g = dev.train_step(g, su, dtu, bg, gt_d, 0.2, LRS, step, grads_out=grads)
        work = dev.raster_work()
        gi = {k: dev.intermediate(k) for k in ("out_img", "v_rendered")}
        radii = dev.intermediate("radii", np.int32)
        conics = dev.intermediate("conics").reshape(n, 3)
        rg = {k: dev.intermediate(k).reshape(n, d) for k, d in (("v_xy", 2), ("v_conic", 3), ("v_rgb", 3),
                                                                ("v_opacity", 1))}
        gg = {k: grads[k].cpu().numpy() for k in grads}
        pa, ma, va, (visa, gna, mxa) = _host_state(g, n)
        say(f"train {label}: oracle step {step} (from the GPU's state)")
        ps, m, v = [a.copy() for a in pb], [a.copy() for a in mb], [a.copy() for a in vb]
        vis, gnorm, max2d = visb.copy(), gnb.copy(), mxb.copy()
        want = ("out_img", "radii", "v_xy", "v_conic", "v_rgb", "v_opacity", "v_rendered", "mag_raster",
                "err_raster", "grad", "grad_mag", "grad_err")
        loss_o, o = orc.train_step(cam, ps, m, v, orc.adam_hparams(LRS, step), gt, 0.2, vis, gnorm, max2d,
                                   want=want)
        tag = f"{label} step {step}"
        assert abs(loss_g - loss_o) <= 1e-5 * abs(loss_o), (loss_g, loss_o)
        assert [work[k] for k in dev.RASTER_WORK_KEYS] == orc.raster_counts(), (work, orc.raster_counts())
        assert_bits_equal(gi["out_img"].reshape(H, W, 3), o["out_img"], "out_img")
        assert_bits_equal(gi["v_rendered"].reshape(H, W, 3), o["v_rendered"], "v_rendered")
        assert_bits_equal(radii, o["radii"], "radii")
        vis_mask = radii > 0

        def chk(name, a, b, e, rel=1e-3, mag=None):
            stats[f"{name} (step {step})"] = bound_check(a, b, e, rel=rel, what=f"{tag} {name}", log=say, mag=mag)

        er, mr = o["err_raster"], o["mag_raster"]
        if check_grads:
            for k, q0, d in (("v_xy", 0, 2), ("v_conic", 2, 3), ("v_rgb", 5, 3), ("v_opacity", 8, 1)):
                chk(k, rg[k], o[k].reshape(n, d), er[:, q0:q0 + d], mag=mr[:, q0:q0 + d])
            for i, k in enumerate(("v_mean3d", "v_scale", "v_quat")):
                chk(k, gg[k], o["grad"][i], o["grad_err"][i])
        # projection backward on the GPU's own raster gradients: rounding only
        vm, vs_, vq, perr = orc.project_backward(cam, pb[0], pb[1], pb[2], radii, conics, rg["v_xy"], rg["v_conic"])
        for k, ref, sl in (("v_mean3d", vm, slice(0, 3)), ("v_scale", vs_, slice(3, 6)), ("v_quat", vq, slice(6, 10))):
            chk(f"{k} | GPU raster gradients", gg[k], ref, perr[:, sl], rel=0.0)
        # Adam on the GPU's own gradients, and against the oracle
        v_dc, v_rest = orc.sh_backward(cam, pb[0], radii, rg["v_rgb"], rest_bases)
        ggpu = [gg["v_mean3d"], gg["v_scale"], gg["v_quat"], v_dc, v_rest, rg["v_opacity"].reshape(n)]
        upd_mask = [None, None, None, np.repeat(vis_mask[:, None], 3, 1), None, None]
        if rest_bases:
            bm = np.zeros((n, rest_bases, 3), bool)
            bm[:, :nb_use] = vis_mask[:, None, None]
            upd_mask[4] = bm
        ss, bc = dev.adam_constants(LRS, step)
        for i in range(6):
            if pb[i].size == 0:
                continue
            msk = np.ones(pb[i].shape, bool) if upd_mask[i] is None else upd_mask[i]
            name = PARAM_NAMES[i]
            for arr_a, arr_b, what in ((pa[i], pb[i], "param"), (ma[i], mb[i], "exp_avg"), (va[i], vb[i], "exp_avg_sq")):
                assert_bits_equal(arr_a[~msk], arr_b[~msk], f"{tag} {name} {what} outside the update")
            gk = ggpu[i].reshape(pb[i].shape)[msk]
            mn, vn, upd, _, rnd_m, rnd_v = _adam_ref(pb[i][msk], mb[i][msk], vb[i][msk], gk, ss[i], bc[i])
            du = pa[i][msk].astype(np.float64) - pb[i][msk].astype(np.float64)
            # the update's own rounding, the first moment's rounding carried
            # through, and the stored parameter's last place
            d_mn = np.abs(upd) / np.maximum(np.abs(mn), 1e-300) * 3 * U * rnd_m
            chk(f"{name} update | GPU gradients", du, upd, d_mn + 2 * _ulp(pa[i][msk]), rel=1e-5)
            chk(f"{name} exp_avg | GPU gradients", ma[i][msk], mn, 3 * U * rnd_m + 1e-45, rel=0.0)
            chk(f"{name} exp_avg_sq | GPU gradients", va[i][msk], vn, 4 * U * rnd_v + 1e-45, rel=0.0)
            if not check_grads:
                continue
            go, ge = o["grad"][i][msk].astype(np.float64), o["grad_err"][i][msk].astype(np.float64)
            # tier B for the gradients summed straight from pixel terms
            # (f_dc, f_rest: the colour gradient times a basis value; opacity)
            gm = o["grad_mag"][i][msk].astype(np.float64) if i in (3, 4, 5) else None
            if i in (3, 4):
                chk(f"grad {name}", _as_group(ggpu[i], pb[i].shape)[msk], go, ge, mag=gm)
            mn_o, _, upd_o, dupd, rnd_mo, rnd_vo = _adam_ref(pb[i][msk], mb[i][msk], vb[i][msk], go, ss[i], bc[i])
            om1, om2 = float(np.float32(1) - np.float32(0.9)), float(np.float32(1) - np.float32(0.999))
            # m = b1 m + (1 - b1) g: the gradient's bound scaled by 1 - b1
            # (its relative part too where b1 m cancels part of the new term),
            # and both sides' rounding
            mo = m[i][msk].astype(np.float64)
            chk(f"{name} exp_avg", ma[i][msk], mo, om1 * ge + 1e-3 * np.maximum(0.0, om1 * np.abs(go) - np.abs(mo))
                + 6 * U * rnd_mo + 1e-45, mag=None if gm is None else om1 * gm + rnd_mo)
            chk(f"{name} exp_avg_sq", va[i][msk], v[i][msk], om2 * (2 * np.abs(go) * ge + ge * ge) + 6 * U * rnd_vo
                + 1e-45, rel=2e-3)
            # the update against the oracle's where the gradient bound is the
            # relative term (first order in the gradient's difference)
            rd = (ge <= 1e-3 * np.abs(go)) & (go != 0)
            du_o = ps[i][msk].astype(np.float64) - pb[i][msk].astype(np.float64)
            tol_u = (2.0 * np.abs(dupd) * (2e-3 * np.abs(go)) + 2 * _ulp(pa[i][msk]) + 2 * _ulp(ps[i][msk]) +
                     2 * np.abs(upd_o) / np.maximum(np.abs(mn_o), 1e-300) * 3 * U * rnd_mo)
            chk(f"{name} update (gradient rel-decided)", du[rd], du_o[rd], tol_u[rd], rel=1e-5)
        # statistics: exact counts and sizes, the norm to its rounding
        assert_bits_equal(visa, (visb + vis_mask.astype(np.float32)).astype(np.float32), f"{tag} vis_counts")
        assert_bits_equal(mxa, np.where(vis_mask, np.maximum(mxb, radii.astype(np.float32) * inv_max_dim), mxb)
                          .astype(np.float32), f"{tag} max_2d_size")
        vx = rg["v_xy"].astype(np.float64)
        nrm = np.where(vis_mask, np.sqrt(vx[:, 0] ** 2 + vx[:, 1] ** 2), 0.0)
        chk("xys_grad_norm | GPU v_xy", gna.astype(np.float64) - gnb, nrm, 4 * U * (np.abs(gnb) + nrm) + 1e-45,
            rel=0.0)
        if check_grads:
            # |norm(a) - norm(b)| <= |a - b|, whose relative part is at most
            # sqrt(2) 1e-3 of the norm
            chk("xys_grad_norm", gna.astype(np.float64) - gnb, gnorm.astype(np.float64) - gnb,
                er[:, 0] + er[:, 1] + 8 * U * (np.abs(gnb) + nrm) + 1e-45, rel=1.5e-3)
            assert_bits_equal(visa, vis, f"{tag} vis_counts vs oracle")
            assert_bits_equal(mxa, max2d, f"{tag} max_2d_size vs oracle")
    say(f"train {label}: within bounds (loss {loss_g:.6f} vs {loss_o:.6f})")
    return TrainResult(g, loss_g, loss_o, stats)


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
