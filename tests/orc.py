"""ctypes binding of the CPU oracle (oracle/liboracle.so) for the tests.

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this, and only as the checker.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int32, c_int64, c_uint32

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# MSPLAT_ORACLE_LIB points the tests at another build of the oracle (used to
# check that the pins fail on a deliberately mutated copy).
LIB = os.environ.get("MSPLAT_ORACLE_LIB") or os.path.join(ROOT, "oracle", "liboracle.so")


class OrcCamera(ctypes.Structure):
    _fields_ = [
        ("viewmat", c_float * 16), ("projmat", c_float * 16),
        ("fx", c_float), ("fy", c_float), ("cx", c_float), ("cy", c_float),
        ("width", c_int32), ("height", c_int32),
        ("cam_pos", c_float * 3),
        ("clip_thresh", c_float), ("glob_scale", c_float),
        ("degree", c_int32), ("degrees_to_use", c_int32),
        ("background", c_float * 3),
    ]


class OrcAdam(ctypes.Structure):
    _fields_ = [("step_size", c_float * 6), ("bc2_sqrt", c_float * 6),
                ("beta1", c_float), ("beta2", c_float), ("eps", c_float)]


class OrcTrainOut(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("out_img", "radii", "v_xy", "v_conic", "v_rgb", "v_opacity", "v_mean3d", "v_scale", "v_quat",
                 "v_rendered", "mag_raster", "err_raster")] + [
        ("grad", ctypes.c_void_p * 6), ("grad_mag", ctypes.c_void_p * 6), ("grad_err", ctypes.c_void_p * 6)]


class OrcDensifyArgs(ctypes.Structure):
    _fields_ = [("N", c_int32),
                ("grad_thresh", c_float), ("size_thresh", c_float), ("screen_thresh", c_float),
                ("check_screen", c_int32),
                ("cull_alpha_thresh", c_float), ("cull_scale_thresh", c_float), ("cull_screen_size", c_float),
                ("check_huge", c_int32),
                ("half_max_dim", c_float), ("fr_stride", c_int32)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} missing: run make -C oracle")
        L = ctypes.CDLL(LIB)
        L.orc_expf.restype = c_float
        L.orc_expf.argtypes = [c_float]
        L.orc_expf_raster.restype = c_float
        L.orc_expf_raster.argtypes = [c_float]
        L.orc_bin_sort.restype = c_int64
        L.orc_ssim_loss.restype = c_double
        L.orc_train_step.restype = c_float
        L.orc_densify.restype = c_int32
        L.orc_tile_chunks.restype = c_int32
        L.orc_num_threads.restype = c_int32
        _lib = L
    return _lib


def P(a: np.ndarray):
    """Pointer to a C-contiguous numpy array (None passes through)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def camera(setup, degree: int, degrees_to_use: int, background=(0.6130, 0.0101, 0.3984),
           clip: float = 0.01, glob_scale: float = 1.0) -> OrcCamera:
    c = OrcCamera()
    c.viewmat[:] = [float(v) for v in np.asarray(setup.viewmat, np.float32).reshape(16)]
    c.projmat[:] = [float(v) for v in np.asarray(setup.projmat, np.float32).reshape(16)]
    c.fx, c.fy, c.cx, c.cy = setup.fx, setup.fy, setup.cx, setup.cy
    c.width, c.height = setup.width, setup.height
    c.cam_pos[:] = [float(v) for v in setup.cam_pos]
    c.clip_thresh, c.glob_scale = clip, glob_scale
    c.degree, c.degrees_to_use = degree, min(degrees_to_use, degree)
    c.background[:] = [float(v) for v in background]
    return c


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def project(cam: OrcCamera, means, scales, quats, f_dc, f_rest):
    n = means.shape[0]
    out = dict(xys=np.zeros((n, 2), np.float32), depths=np.zeros(n, np.float32),
               radii=np.zeros(n, np.int32), conics=np.zeros((n, 3), np.float32),
               num_tiles_hit=np.zeros(n, np.int32), colors=np.zeros((n, 3), np.float32),
               aabb=np.zeros((n, 2), np.float32))
    means, scales, quats, f_dc, f_rest = map(f32, (means, scales, quats, f_dc, f_rest))
    lib().orc_project_forward(ctypes.byref(cam), n, P(means), P(scales), P(quats), P(f_dc), P(f_rest),
                              P(out["xys"]), P(out["depths"]), P(out["radii"]), P(out["conics"]),
                              P(out["num_tiles_hit"]), P(out["colors"]), P(out["aabb"]))
    return out


def bin_sort(cam: OrcCamera, proj: dict):
    n = proj["xys"].shape[0]
    tbx, tby = (cam.width + 15) // 16, (cam.height + 15) // 16
    cap = int(proj["num_tiles_hit"].astype(np.int64).sum())
    counts = np.zeros(tbx * tby, np.int32)
    tile_bins = np.zeros((tbx * tby, 2), np.int32)
    ids = np.zeros(max(cap, 1), np.int32)
    tot = lib().orc_bin_sort(ctypes.byref(cam), n, P(proj["xys"]), P(proj["depths"]), P(proj["radii"]),
                             P(proj["aabb"]), cap, P(counts), P(tile_bins), P(ids))
    assert tot == cap, (tot, cap)
    return counts, tile_bins, ids[:tot]


def rasterize(cam: OrcCamera, proj: dict, opac_logits, tile_bins, ids, v_out=None):
    n = proj["xys"].shape[0]
    H, W = cam.height, cam.width
    out = dict(final_Ts=np.zeros((H, W), np.float32), final_index=np.zeros((H, W), np.int32),
               out_img=np.zeros((H, W, 3), np.float32))
    grads = None
    if v_out is not None:
        grads = dict(v_xy=np.zeros((n, 2), np.float32), v_conic=np.zeros((n, 3), np.float32),
                     v_rgb=np.zeros((n, 3), np.float32), v_opacity=np.zeros(n, np.float32))
    op = f32(opac_logits).reshape(-1)
    ids = np.ascontiguousarray(ids, np.int32)
    if ids.size == 0:
        ids = np.zeros(1, np.int32)
    lib().orc_rasterize(ctypes.byref(cam), n, P(proj["xys"]), P(proj["conics"]), P(proj["colors"]), P(op),
                        P(np.ascontiguousarray(tile_bins, np.int32)), P(ids),
                        P(out["final_Ts"]), P(out["final_index"]), P(out["out_img"]),
                        P(f32(v_out)) if v_out is not None else None,
                        *( [P(grads[k]) for k in ("v_xy", "v_conic", "v_rgb", "v_opacity")] if grads else [None] * 4))
    if grads:
        out.update(grads)
    return out


def project_backward(cam: OrcCamera, means, scales, quats, radii, conics, v_xy, v_conic, err_xy=None,
                     err_conic=None):
    """Projection backward of the given raster gradients: (v_mean3d, v_scale,
    v_quat, err[N,10]) where err bounds |GPU - oracle| of the three outputs
    (v_mean3d 3, v_scale 3, v_quat 4) given inputs that err by err_xy /
    err_conic (None: exact inputs, the bound is the arithmetic's own)."""
    n = means.shape[0]
    means, scales, quats, conics, v_xy, v_conic = map(f32, (means, scales, quats, conics, v_xy, v_conic))
    radii = np.ascontiguousarray(radii, np.int32)
    vm, vs, vq = np.zeros((n, 3), np.float32), np.zeros((n, 3), np.float32), np.zeros((n, 4), np.float32)
    err = np.zeros((n, 10), np.float32)
    L = lib()
    L.orc_project_backward(ctypes.byref(cam), n, P(means), P(scales), P(quats), P(radii), P(conics), P(v_xy),
                           P(v_conic), P(vm), P(vs), P(vq))
    L.orc_project_backward_err(ctypes.byref(cam), n, P(means), P(scales), P(quats), P(radii), P(conics), P(v_xy),
                               P(v_conic), P(f32(err_xy)) if err_xy is not None else None,
                               P(f32(err_conic)) if err_conic is not None else None, P(err))
    return vm, vs, vq, err


def sh_backward(cam: OrcCamera, means, radii, v_rgb, rest_bases: int):
    """(v_dc [N,3], v_rest [N,rest_bases,3]) of the given colour gradients."""
    n = means.shape[0]
    nb = max(rest_bases, 0)
    full = (((cam.degree + 1) ** 2) - 1)
    v_dc = np.zeros((n, 3), np.float32)
    v_rest = np.zeros((n, full, 3), np.float32)
    lib().orc_sh_backward(ctypes.byref(cam), n, P(f32(means)), P(np.ascontiguousarray(radii, np.int32)),
                          P(f32(v_rgb)), P(v_dc), P(v_rest))
    return v_dc, np.ascontiguousarray(v_rest[:, :nb])


def raster_counts():
    """Pair counts of the last orc_rasterize call (fwd tested/in range/composited, bwd tested/in range/grad)."""
    out = (c_int64 * 6)()
    lib().orc_raster_counts(out)
    return [int(v) for v in out]


def ssim_loss(img, gt, ssim_weight=0.2, inv_n=None, want_bufs=False):
    H, W = img.shape[:2]
    if inv_n is None:
        inv_n = np.float32(1.0) / np.float32(H * W * 3)
    v = np.zeros((H, W, 3), np.float32)
    hb = np.zeros((H, W, 15), np.float32) if want_bufs else None
    db = np.zeros((H, W, 15), np.float32) if want_bufs else None
    s = lib().orc_ssim_loss(H, W, P(f32(img)), P(f32(gt)), c_float(ssim_weight), c_float(inv_n), P(v), P(hb), P(db))
    return float(s), v, hb, db


def render(cam: OrcCamera, means, scales, quats, f_dc, f_rest, opac_logits):
    H, W = cam.height, cam.width
    img = np.zeros((H, W, 3), np.float32)
    Ts = np.zeros((H, W), np.float32)
    idx = np.zeros((H, W), np.int32)
    rc = lib().orc_render(ctypes.byref(cam), means.shape[0], P(f32(means)), P(f32(scales)), P(f32(quats)),
                          P(f32(f_dc)), P(f32(f_rest)), P(f32(opac_logits).reshape(-1)), P(img), P(Ts), P(idx))
    assert rc == 0
    return img, Ts, idx


def image_metrics(img, gt, window_size=11, sigma=1.5) -> dict:
    """psnr / ssim_eval / l1_loss of two (H, W, 3) float32 images."""
    img, gt = f32(img), f32(gt)
    out = np.zeros(3, np.float32)
    lib().orc_image_metrics(c_int32(img.shape[0]), c_int32(img.shape[1]), P(img), P(gt),
                            c_int32(window_size), c_float(sigma), P(out))
    return {"psnr": float(out[0]), "ssim": float(out[1]), "l1": float(out[2])}


def image_to_rgba8(img) -> np.ndarray:
    img = f32(img)
    n = img.size // 3
    out = np.zeros(img.shape[:-1] + (4,), np.uint8)
    lib().orc_image_to_rgba8(c_int64(n), P(img), P(out))
    return out


def knn_mean_dist(xyz) -> np.ndarray:
    xyz = f32(xyz)
    out = np.zeros(xyz.shape[0], np.float32)
    lib().orc_knn_mean_dist(c_int64(xyz.shape[0]), P(xyz), P(out))
    return out


def resize_area(img, dw: int, dh: int) -> np.ndarray:
    img = f32(img)
    sh, sw = img.shape[:2]
    out = np.zeros((dh, dw, 3), np.float32)
    lib().orc_resize_area(c_int32(sw), c_int32(sh), P(img), c_int32(dw), c_int32(dh), P(out))
    return out


def _cam_arrays(intr, dist):
    return np.ascontiguousarray(intr, np.float32), np.ascontiguousarray(dist, np.float32)


def undistort_roi(w: int, h: int, intr, dist) -> np.ndarray:
    i, d = _cam_arrays(intr, dist)
    roi = np.zeros(4, np.int32)
    lib().orc_undistort_roi(c_int32(w), c_int32(h), P(i), P(d), P(roi))
    return roi


def undistort(img, intr, dist):
    """(cropped undistorted image, roi) of an [h,w,3] image."""
    img = f32(img)
    h, w = img.shape[:2]
    i, d = _cam_arrays(intr, dist)
    roi = np.zeros(4, np.int32)
    buf = np.zeros(h * w * 3, np.float32)
    lib().orc_undistort(c_int32(w), c_int32(h), P(img), P(i), P(d), P(roi), P(buf))
    return buf[: roi[2] * roi[3] * 3].reshape(roi[3], roi[2], 3).copy(), roi


def adam_hparams(lrs, step: int, beta1=0.9, beta2=0.999, eps=1e-8) -> OrcAdam:
    """fullIteration's bias corrections (model.cpp:558-571), fp32 like the reference."""
    a = OrcAdam()
    bc1 = np.float32(1.0) - np.float32(beta1) ** np.float32(step)
    bc2 = np.float32(1.0) - np.float32(beta2) ** np.float32(step)
    for g in range(6):
        a.step_size[g] = float(np.float32(lrs[g]) / bc1)
        a.bc2_sqrt[g] = float(np.sqrt(bc2))
    a.beta1, a.beta2, a.eps = beta1, beta2, eps
    return a


def train_step(cam: OrcCamera, params, m, v, adam: OrcAdam, gt, ssim_weight, vis, gnorm, max2d, want=()):
    """One oracle train step; params/m/v are lists of 6 float32 arrays updated in place.

    want names the outputs to return: the fields of OrcTrainOut
    (out_img, radii, v_xy ... v_rendered, mag_raster, err_raster: arrays) and
    grad / grad_mag / grad_err (lists of six arrays shaped like params)."""
    n = params[0].shape[0]
    H, W = cam.height, cam.width
    rest_bases = params[4].shape[1] if params[4].ndim == 3 else 0
    outs = {}
    shapes = dict(out_img=((H, W, 3), np.float32), radii=((n,), np.int32), v_xy=((n, 2), np.float32),
                  v_conic=((n, 3), np.float32), v_rgb=((n, 3), np.float32), v_opacity=((n,), np.float32),
                  v_mean3d=((n, 3), np.float32), v_scale=((n, 3), np.float32), v_quat=((n, 4), np.float32),
                  v_rendered=((H, W, 3), np.float32), mag_raster=((n, 9), np.float32),
                  err_raster=((n, 9), np.float32))
    to = OrcTrainOut()
    for k in want:
        if k in ("grad", "grad_mag", "grad_err"):
            outs[k] = [np.zeros(a.shape, np.float32) for a in params]
            arr = getattr(to, k)
            for i in range(6):
                arr[i] = P(outs[k][i]).value
            continue
        shp, dt = shapes[k]
        outs[k] = np.zeros(shp, dt)
        setattr(to, k, P(outs[k]).value)
    parr = (ctypes.c_void_p * 6)(*[P(a).value for a in params])
    marr = (ctypes.c_void_p * 6)(*[P(a).value for a in m])
    varr = (ctypes.c_void_p * 6)(*[P(a).value for a in v])
    loss = lib().orc_train_step(ctypes.byref(cam), n, rest_bases, parr, marr, varr, ctypes.byref(adam),
                                P(f32(gt)), c_float(ssim_weight), P(vis), P(gnorm), P(max2d), ctypes.byref(to))
    return float(loss), outs


def densify(args: OrcDensifyArgs, gnorm, vis, max2d, bufs, m, v, rnd):
    n = args.N
    split = np.zeros(n, np.int32)
    dup = np.zeros(n, np.int32)
    keep = np.zeros(3 * n, np.int32)
    barr = (ctypes.c_void_p * 6)(*[P(a).value for a in bufs])
    marr = (ctypes.c_void_p * 6)(*[P(a).value for a in m])
    varr = (ctypes.c_void_p * 6)(*[P(a).value for a in v])
    nn = lib().orc_densify(ctypes.byref(args), P(gnorm), P(vis), P(max2d), barr, marr, varr, P(f32(rnd)),
                           P(split), P(dup), P(keep))
    return int(nn), split, dup, keep
