"""Pins of the CPU oracle (oracle/liboracle.so) by mathematics, not by retyping.

The reference ships no golden vectors, known-answer tests or fixtures for the
splatting path (its tests are end-to-end smoke tests on Apple hardware), and
its Metal code cannot run here.  Each oracle function is therefore checked
against what the mathematics fixes: libm, closed forms, orthogonality,
brute-force enumeration, float64 re-derivations and float64 central finite
differences, chosen so that a dropped term, a wrong sign or index or a
transposed operand fails.  Where the reference computes something that is not
a true derivative (documented quirks), the finite difference is taken of the
surrogate the reference differentiates, and the test says so.

CPU only; runs in the default `-m "not gpu"` suite.
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np
import pytest

import orc
from helpers import BG, small_scene
from msplat_amd import camera

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
F32 = np.float32


def _cam(width=64, height=48, pos=(0.3, -0.2, 4.0), fov=60.0, degree=3, dtu=3, bg=BG):
    cam = camera.pinhole(width, height, fov, camera.look_at(pos))
    su = camera.prepare_cam(cam)
    return su, orc.camera(su, degree, dtu, bg)


# ---------------------------------------------------------------- exp --------

def test_exp_against_libm():
    """Cody-Waite exp within 2 ulp of the correctly rounded exp over [-87, 88]."""
    rng = np.random.default_rng(1)
    x = np.concatenate([np.linspace(-87.0, 88.0, 400001, dtype=F32),
                        rng.uniform(-6.0, 0.0, 200000).astype(F32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 1.0, -1.0, 0.5, -5.55], F32)])
    y = np.empty_like(x)
    orc.lib().orc_expf_n(x.size, orc.P(x), orc.P(y))
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(F32)).astype(np.float64)
    err = np.abs(y.astype(np.float64) - ref) / ulp
    assert err.max() <= 2.0, (float(err.max()), float(x[np.argmax(err)]))
    assert orc.lib().orc_expf(0.0) == 1.0
    # specials: no subnormal results below -87, +inf above 88, NaN propagates
    assert orc.lib().orc_expf(-87.5) == 0.0
    assert math.isinf(orc.lib().orc_expf(88.5))
    assert math.isnan(orc.lib().orc_expf(float("nan")))


def test_exp_raster_against_libm():
    """The rasteriser's exp (Remez degree-6) within 1.05 ulp of the correctly
    rounded exp over the range of -sigma it is used on, [-5.6, 0], including
    every float in [-1, 0] near the reduction boundaries."""
    rng = np.random.default_rng(2)
    x = np.concatenate([np.linspace(-5.6, 0.0, 1000001, dtype=F32),
                        rng.uniform(-5.6, 0.0, 500000).astype(F32),
                        # arguments around multiples of ln2/2, where k changes
                        (np.arange(-17, 1, dtype=np.float64)[:, None] * math.log(2) / 2 +
                         np.linspace(-1e-5, 1e-5, 2001)[None, :]).astype(F32).ravel(),
                        np.array([0.0, -0.0, -1e-30, -5.55, -5.5499997], F32)])
    x = x[(x >= -5.6) & (x <= 0.0)]
    y = np.empty_like(x)
    orc.lib().orc_expf_raster_n(x.size, orc.P(x), orc.P(y))
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(F32)).astype(np.float64)
    err = np.abs(y.astype(np.float64) - ref) / ulp
    assert err.max() <= 1.05, (float(err.max()), float(x[np.argmax(err)]))
    assert orc.lib().orc_expf_raster(0.0) == 1.0
    assert math.isnan(orc.lib().orc_expf_raster(float("nan")))
    # monotone over the used range (alpha thresholds are decided on it)
    xs = np.sort(x)
    ys = np.empty_like(xs)
    orc.lib().orc_expf_raster_n(xs.size, orc.P(xs), orc.P(ys))
    assert np.all(np.diff(ys.astype(np.float64)) >= 0)


def test_sigma_clamp_rejects_through_alpha():
    """The raster kernels fold the range early-out (skip sigma < 0 or >= 5.55)
    into the alpha test by clamping sigma's bits to those of 5.55f with an
    unsigned min.  That rejects exactly the out-of-range pairs because
    min(0.999, o exp(-5.55)) < 1/255 for every opacity in [0, 1] (float32
    arithmetic, the largest opacity below 1 and 1 itself), while every sigma
    in [+0, 5.55) keeps its bits; -0, negatives, >= 5.55, inf and NaN clamp."""
    e = np.float32(orc.lib().orc_expf_raster(-5.55))
    thr = np.float32(1.0) / np.float32(255.0)
    for o in (np.float32(1.0), np.nextafter(np.float32(1.0), np.float32(0.0)), np.float32(0.5)):
        assert np.minimum(np.float32(0.999), o * e) < thr
    cap = np.uint32(0x40B1999A)
    assert np.array([5.55], F32).view(np.uint32)[0] == cap
    s = np.array([0.0, 1e-30, 1.0, 5.5499997, 5.55, 6.0, np.inf, np.nan, -0.0, -1e-30, -1.0, -np.inf],
                 F32)
    clamped = np.minimum(s.view(np.uint32), cap).view(F32)
    ref_in = ~((s < 0) | (s >= F32(5.55)))            # the reference's test (NaN passes it)
    kept = s.view(np.uint32) < cap                    # below the cap: sigma keeps its bits
    assert np.array_equal(clamped[kept].view(np.uint32), s[kept].view(np.uint32))
    # identical for every sigma but -0 and NaN, which the clamp rejects
    special = (np.signbit(s) & (s == 0)) | np.isnan(s)
    assert np.array_equal(kept[~special], ref_in[~special])
    assert not kept[special].any()
    assert np.all(clamped[~kept] == F32(5.55))


# ---------------------------------------------------------------- SH ---------

SH_CLOSED = [
    1 / (2 * math.sqrt(math.pi)),                         # C0
    math.sqrt(3) / (2 * math.sqrt(math.pi)),              # C1
    # C2
    math.sqrt(15) / (2 * math.sqrt(math.pi)), -math.sqrt(15) / (2 * math.sqrt(math.pi)),
    math.sqrt(5) / (4 * math.sqrt(math.pi)), -math.sqrt(15) / (2 * math.sqrt(math.pi)),
    math.sqrt(15) / (4 * math.sqrt(math.pi)),
    # C3
    -math.sqrt(35 / (2 * math.pi)) / 4, math.sqrt(105) / (2 * math.sqrt(math.pi)),
    -math.sqrt(21 / (2 * math.pi)) / 4, math.sqrt(7) / (4 * math.sqrt(math.pi)),
    -math.sqrt(21 / (2 * math.pi)) / 4, math.sqrt(105) / (4 * math.sqrt(math.pi)),
    -math.sqrt(35 / (2 * math.pi)) / 4,
]


def test_sh_constants_closed_form():
    """SH_C0..C3 against Sloan's closed forms ("Stupid SH Tricks")."""
    out = np.zeros(25, F32)
    orc.lib().orc_sh_consts(orc.P(out))
    np.testing.assert_allclose(out[:14].astype(np.float64), SH_CLOSED, rtol=2e-7, atol=0)


def _sh_basis(degree, dirs):
    """Basis values (n_dirs, K) from orc_sh_eval with one-hot coefficients."""
    K = (degree + 1) ** 2
    out = np.zeros((dirs.shape[0], K))
    col = np.zeros(3, F32)
    for b in range(K):
        dc = np.zeros(3, F32)
        rest = np.zeros(max(K - 1, 1) * 3, F32)
        if b == 0:
            dc[0] = 1.0
        else:
            rest[3 * (b - 1)] = 1.0
        for i, d in enumerate(dirs):
            dd = np.ascontiguousarray(d, F32)
            orc.lib().orc_sh_eval(degree, orc.P(dd), orc.P(dc), orc.P(rest), orc.P(col))
            out[i, b] = col[0]
    return out


def test_sh_basis_orthonormal_and_harmonic():
    """Bands 0..4 are orthonormal on the sphere (Gauss-Legendre x uniform
    quadrature) and each band-l function is a homogeneous harmonic polynomial
    of degree l (least-squares fit off the sphere, Laplacian of the fit = 0)."""
    deg = 4
    nt, nphi = 12, 24
    ct, wt = np.polynomial.legendre.leggauss(nt)
    phi = (np.arange(nphi) + 0.5) * 2 * math.pi / nphi
    st = np.sqrt(1 - ct ** 2)
    dirs = np.stack([np.outer(st, np.cos(phi)).ravel(), np.outer(st, np.sin(phi)).ravel(),
                     np.repeat(ct, nphi)], axis=1)
    w = np.repeat(wt, nphi) * (2 * math.pi / nphi)
    Y = _sh_basis(deg, dirs)
    G = (Y * w[:, None]).T @ Y
    np.testing.assert_allclose(G, np.eye(G.shape[0]), atol=2e-6)
    # r^l Y(p / r) must be a homogeneous harmonic polynomial of degree l (the
    # band-4 formulas use x^2 + y^2 + z^2 = 1, so evaluate on the sphere)
    rng = np.random.default_rng(3)
    pts = rng.normal(size=(80, 3)) * rng.uniform(0.5, 1.5, size=(80, 1))
    rad = np.linalg.norm(pts, axis=1)
    Yp = _sh_basis(deg, pts / rad[:, None])
    for l in range(1, deg + 1):
        Yp[:, l * l:(l + 1) ** 2] *= rad[:, None] ** l
        monos = [(i, j, l - i - j) for i in range(l + 1) for j in range(l + 1 - i)]
        A = np.stack([pts[:, 0] ** i * pts[:, 1] ** j * pts[:, 2] ** k for i, j, k in monos], axis=1)
        for b in range(l * l, (l + 1) ** 2):
            coef, *_ = np.linalg.lstsq(A, Yp[:, b], rcond=None)
            assert np.abs(A @ coef - Yp[:, b]).max() < 1e-5, (l, b)   # homogeneous of degree l
            lap = {}
            for c, (i, j, k) in zip(coef, monos):
                for (e, n) in ((0, i), (1, j), (2, k)):
                    if n >= 2:
                        key = [i, j, k]
                        key[e] -= 2
                        lap[tuple(key)] = lap.get(tuple(key), 0.0) + c * n * (n - 1)
            assert max([abs(v) for v in lap.values()] + [0.0]) < 1e-4, (l, b, lap)


def test_sh_band1_convention():
    """Band 1 is C1 * (-y, z, -x) (the 3DGS real-SH sign convention, .metal:604-606)."""
    d = np.array([[0.2, -0.5, 0.7]], F32)
    Y = _sh_basis(1, d)
    c1 = SH_CLOSED[1]
    np.testing.assert_allclose(Y[0, 1:], [-c1 * -0.5, c1 * 0.7, -c1 * 0.2], rtol=1e-6)


# ------------------------------------------------------- SSIM window ---------

def test_gauss1d_window():
    """GAUSS_1D: the normalised 11-tap Gaussian with sigma 1.5, and, where the
    reference's createSSIMWindow (core/src/ssim.cpp:7-24) could be compiled
    into oracle/_ref/ssim_window, its taps to within 2 ulp per factor."""
    g = np.zeros(11, F32)
    orc.lib().orc_gauss1d(orc.P(g))
    x = np.arange(11) - 5.0
    ref = np.exp(-x * x / (2 * 1.5 ** 2))
    ref /= ref.sum()
    np.testing.assert_allclose(g.astype(np.float64), ref, rtol=3e-7)
    exe = os.path.join(ROOT, "oracle", "_ref", "ssim_window")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/ssim_window not built (needs /root/reference)")
    import subprocess
    taps = [float.fromhex(t) for t in subprocess.check_output([exe], text=True).split()]
    assert len(taps) == 121
    w2 = np.array(taps, F32).reshape(11, 11)
    # the reference's 2D window is the fp32 outer product of its computed 1D
    # taps; the training kernels use the 10-digit decimal taps of .metal:3041-3045
    # (GAUSS_1D), which reproduce all 121 products to within 4 ulp (2 per factor)
    prod = np.outer(g, g).astype(F32)
    ulps = np.abs(w2.astype(np.float64) - prod) / np.spacing(prod).astype(np.float64)
    assert ulps.max() <= 4.0, ulps.max()
    np.testing.assert_array_equal(w2, w2.T)


# -------------------------------------------------- rotation / cov3d ---------

def _rot64(q):
    w, x, y, z = np.asarray(q, np.float64) / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def test_quat_to_rotmat():
    """Orthonormal, det 1, rotates by the quaternion's axis-angle (Rodrigues),
    unnormalised input handled by normalisation."""
    rng = np.random.default_rng(5)
    R = np.zeros(9, F32)
    for _ in range(200):
        q = rng.normal(size=4).astype(F32) * F32(rng.uniform(0.2, 3.0))
        orc.lib().orc_quat_to_rotmat(orc.P(q), orc.P(R))
        M = R.reshape(3, 3).astype(np.float64)
        np.testing.assert_allclose(M @ M.T, np.eye(3), atol=3e-6)
        assert abs(np.linalg.det(M) - 1) < 3e-6
        qn = q.astype(np.float64) / np.linalg.norm(q)
        ang = 2 * math.atan2(np.linalg.norm(qn[1:]), qn[0])
        axis = qn[1:] / np.linalg.norm(qn[1:])
        K = np.array([[0, -axis[2], axis[1]], [axis[2], 0, -axis[0]], [-axis[1], axis[0], 0]])
        rod = np.eye(3) + math.sin(ang) * K + (1 - math.cos(ang)) * K @ K
        np.testing.assert_allclose(M, rod, atol=3e-6)


def test_cov3d_eigen():
    """cov3d = R diag(glob*s)^2 R^T: symmetric PSD with eigenvalues (glob*s)^2
    and eigenvectors the columns of R."""
    rng = np.random.default_rng(6)
    cov = np.zeros(6, F32)
    for _ in range(200):
        s = np.exp(rng.uniform(-5, 1, 3)).astype(F32)
        q = rng.normal(size=4).astype(F32)
        glob = F32(rng.uniform(0.5, 2.0))
        orc.lib().orc_cov3d(orc.P(s), ctypes.c_float(glob), orc.P(q), orc.P(cov))
        C = np.array([[cov[0], cov[1], cov[2]], [cov[1], cov[3], cov[4]], [cov[2], cov[4], cov[5]]], np.float64)
        R = _rot64(q)
        ref = R @ np.diag((float(glob) * s.astype(np.float64)) ** 2) @ R.T
        np.testing.assert_allclose(C, ref, rtol=2e-5, atol=2e-6 * np.abs(ref).max())
        ev = np.sort(np.linalg.eigvalsh(ref))
        np.testing.assert_allclose(np.sort(np.linalg.eigvalsh(C)), ev, rtol=1e-4, atol=1e-6 * ev[-1])


# ------------------------------------------------------- projection ----------

def _ewa64(su, mean, log_s, q, clamp=True, normalize_q=True):
    """float64 EWA splat of one gaussian: camera-space mean, cov2d, conic."""
    V = np.asarray(su.viewmat, np.float64)
    t = V[:3, :3] @ mean + V[:3, 3]
    s = np.exp(log_s)
    if normalize_q:
        R = _rot64(q)
    else:
        w, x, y, z = q
        R = np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                      [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                      [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])
    S3 = R @ np.diag(s * s) @ R.T
    tx, ty, tz = t
    if clamp:
        limx, limy = 1.3 * 0.5 * su.width / su.fx, 1.3 * 0.5 * su.height / su.fy
        tx = tz * min(limx, max(-limx, tx / tz))
        ty = tz * min(limy, max(-limy, ty / tz))
    J = np.array([[su.fx / tz, 0, -su.fx * tx / tz ** 2], [0, su.fy / tz, -su.fy * ty / tz ** 2]])
    W = V[:3, :3]
    C2 = J @ W @ S3 @ W.T @ J.T + 0.3 * np.eye(2)
    det = C2[0, 0] * C2[1, 1] - C2[0, 1] ** 2
    conic = np.array([C2[1, 1] / det, -C2[0, 1] / det, C2[0, 0] / det])
    return t, C2, conic


def _scene_in_view(n, su, rng, depth=(2.5, 6.0), log_s=(-3.5, -1.5), margin=0.8):
    """Gaussians whose centres project inside the image (no FOV clamp)."""
    V = np.asarray(su.viewmat, np.float64)
    Rw, tw = V[:3, :3], V[:3, 3]
    z = rng.uniform(*depth, n)
    u = rng.uniform(-margin, margin, (n, 2))
    cam = np.stack([u[:, 0] * z * 0.5 * su.width / su.fx, u[:, 1] * z * 0.5 * su.height / su.fy, z], 1)
    means = (Rw.T @ (cam - tw).T).T
    scales = rng.uniform(*log_s, (n, 3))
    quats = rng.normal(size=(n, 4))
    quats /= np.linalg.norm(quats, axis=1, keepdims=True)
    return tuple(np.ascontiguousarray(a, F32) for a in (means, scales, quats))


def test_project_forward_against_float64_ewa():
    """Depth, pixel centre (pinhole: fx X/Z + cx - 0.5), conic = inv(J W S W^T
    J^T + 0.3 I), radius = ceil(3 sqrt(lambda_max)), extents = ceil(3 sqrt(diag))."""
    su, cam = _cam(96, 64, degree=0, dtu=0)
    rng = np.random.default_rng(7)
    n = 300
    means, scales, quats = _scene_in_view(n, su, rng)
    f_dc = rng.normal(0, 0.3, (n, 3)).astype(F32)
    f_rest = np.zeros((n, 0, 3), F32)
    p = orc.project(cam, means, scales, quats, f_dc, f_rest.reshape(n, 0))
    assert (p["radii"] > 0).all()
    for g in range(n):
        t, C2, conic = _ewa64(su, means[g].astype(np.float64), scales[g].astype(np.float64),
                              quats[g].astype(np.float64))
        assert abs(p["depths"][g] - t[2]) <= 1e-5 * t[2]
        px = su.fx * t[0] / t[2] + su.cx - 0.5
        py = su.fy * t[1] / t[2] + su.cy - 0.5
        assert abs(p["xys"][g, 0] - px) < 5e-3 and abs(p["xys"][g, 1] - py) < 5e-3, (g, p["xys"][g], px, py)
        np.testing.assert_allclose(p["conics"][g], conic, rtol=2e-4, atol=2e-5 * np.abs(conic).max())
        b = 0.5 * (C2[0, 0] + C2[1, 1])
        det = C2[0, 0] * C2[1, 1] - C2[0, 1] ** 2
        r = 3 * math.sqrt(b + math.sqrt(max(0.1, b * b - det)))
        assert abs(p["radii"][g] - math.ceil(r)) <= (1 if abs(r - round(r)) < 1e-3 else 0)
        for k in range(2):
            e = 3 * math.sqrt(C2[k, k])
            assert abs(p["aabb"][g, k] - math.ceil(e)) <= (1 if abs(e - round(e)) < 1e-3 else 0)
        # degree 0: colour = C0 * dc (raw, no +0.5)
        np.testing.assert_allclose(p["colors"][g], SH_CLOSED[0] * f_dc[g].astype(np.float64), rtol=1e-6)


def test_project_near_plane_cull():
    su, cam = _cam(64, 48, degree=0, dtu=0)
    V = np.asarray(su.viewmat, np.float64)
    z = np.array([0.005, 0.01, 0.011, -1.0])
    cam_pts = np.stack([0 * z, 0 * z, z], 1)
    means = ((V[:3, :3].T @ (cam_pts - V[:3, 3]).T).T).astype(F32)
    n = len(z)
    p = orc.project(cam, means, np.full((n, 3), -3, F32), np.tile(np.array([1, 0, 0, 0], F32), (n, 1)),
                    np.zeros((n, 3), F32), np.zeros((n, 0), F32))
    assert list(p["radii"] > 0) == [False, False, True, False]


def test_tile_rect_enumeration():
    """The tile rectangle is exactly the set of 16-px tiles whose column/row
    span meets [x - ext, x + ext] x [y - ext_y, y + ext_y], clipped to the grid."""
    su, cam = _cam(200, 120)
    tbx, tby = (200 + 15) // 16, (120 + 15) // 16
    rng = np.random.default_rng(8)
    rect = np.zeros(4, np.int32)
    for _ in range(3000):
        xy = rng.uniform(-60, 260, 2).astype(F32)
        ext = np.ceil(rng.uniform(0, 50, 2)).astype(F32)
        orc.lib().orc_tile_rect(ctypes.byref(cam), orc.P(xy), orc.P(ext), orc.P(rect))
        for a, (lo, hi, nt) in enumerate(((0, 2, tbx), (1, 3, tby))):
            c, e = float(xy[a]), float(ext[a])
            tiles = [t for t in range(nt) if (16 * t <= c + e) and (16 * (t + 1) > c - e)]
            want = (tiles[0], tiles[-1] + 1) if tiles else None
            got = (int(rect[lo]), int(rect[hi]))
            if want is None:
                assert got[1] <= got[0], (xy, ext, got)
            else:
                assert got == want, (xy, ext, got, want)


def test_bin_sort_brute_force():
    """Per-tile id lists: brute-force enumeration of (tile, depth bits, id)
    keys sorted lexicographically; tile_bins are the run boundaries."""
    sc = small_scene(n=1500, width=96, height=80, seed_off=201)
    su = camera.prepare_cam(sc.cameras[0])
    cam = orc.camera(su, 3, 3, BG)
    p = orc.project(cam, sc.means, sc.scales, sc.quats, sc.f_dc, sc.f_rest)
    counts, tile_bins, ids = orc.bin_sort(cam, p)
    keys = []
    rect = np.zeros(4, np.int32)
    tbx = (su.width + 15) // 16
    for g in np.nonzero(p["radii"] > 0)[0]:
        orc.lib().orc_tile_rect(ctypes.byref(cam), orc.P(np.ascontiguousarray(p["xys"][g])),
                                orc.P(np.ascontiguousarray(p["aabb"][g])), orc.P(rect))
        dbits = int(np.array(p["depths"][g], F32).view(np.uint32))
        for ty in range(rect[1], rect[3]):
            for tx in range(rect[0], rect[2]):
                keys.append((ty * tbx + tx, dbits, int(g)))
    keys.sort()
    assert len(keys) == ids.size
    np.testing.assert_array_equal(ids, [k[2] for k in keys])
    T = tile_bins.shape[0]
    bc = np.bincount([k[0] for k in keys], minlength=T)
    np.testing.assert_array_equal(counts, bc)
    ends = np.cumsum(bc)
    np.testing.assert_array_equal(tile_bins[:, 1], ends)
    np.testing.assert_array_equal(tile_bins[:, 0], ends - bc)


def test_tile_chunks_rule():
    """Chunk counts: one chunk per 512 entries below 400 tiles; above, one
    piece unless a tile exceeds 8192 entries; never truncated."""
    f = orc.lib().orc_tile_chunks
    for n in (0, 1, 511, 512, 513, 2048, 2049, 8192, 8193, 20000):
        assert f(n, 256) == max(1, -(-n // 512))
        assert f(n, 4000) == (1 if n <= 8192 else -(-n // 512))


# --------------------------------------------------- raster forward ----------

def _composite64(su, proj, opac_logits, tile_bins, ids, bg):
    """float64 per-pixel front-to-back compositing over each tile's sorted list
    (monolithic semantics), with the reference's skip / stop rules."""
    H, W = su.height, su.width
    tbx = (W + 15) // 16
    img = np.zeros((H, W, 3))
    Tf = np.ones((H, W))
    o = 1 / (1 + np.exp(-opac_logits.astype(np.float64).reshape(-1)))
    for t in range(tile_bins.shape[0]):
        s, e = tile_bins[t]
        g = ids[s:e]
        if g.size == 0:
            x0, y0 = (t % tbx) * 16, (t // tbx) * 16
            img[y0:y0 + 16, x0:x0 + 16] = bg
            continue
        xy = proj["xys"][g].astype(np.float64)
        a, b, c = (proj["conics"][g, k].astype(np.float64) for k in range(3))
        col = np.maximum(proj["colors"][g].astype(np.float64) + 0.5, 0)
        og = o[g]
        x0, y0 = (t % tbx) * 16, (t // tbx) * 16
        for i in range(y0, min(y0 + 16, H)):
            for j in range(x0, min(x0 + 16, W)):
                dx, dy = xy[:, 0] - j, xy[:, 1] - i
                sig = 0.5 * (a * dx * dx + c * dy * dy) + b * dx * dy
                al = np.minimum(0.999, og * np.exp(-sig))
                ok = (sig >= 0) & (sig < 5.55) & (al >= 1 / 255)
                T, C = 1.0, np.zeros(3)
                for k in np.nonzero(ok)[0]:
                    nT = T * (1 - al[k])
                    if nT <= 1e-4:
                        break
                    C += col[k] * al[k] * T
                    T = nT
                img[i, j] = np.clip(bg * T + C, 0, 1)
                Tf[i, j] = T
    return img, Tf


def test_raster_single_gaussian_closed_form():
    """One gaussian: out = clamp(bg (1 - a) + a max(c + 0.5, 0)), a = min(0.999, o e^-sigma)."""
    su, cam = _cam(32, 32, degree=0, dtu=0)
    xy = np.array([[13.3, 17.6]], F32)
    conic = np.array([[0.05, 0.012, 0.08]], F32)
    col = np.array([[0.2, -0.1, 0.35]], F32)
    logit = np.array([0.7], F32)
    proj = dict(xys=xy, conics=conic, colors=col)
    tb = np.zeros(((32 // 16) ** 2, 2), np.int32)
    ids = []
    for t in range(4):
        tb[t] = (len(ids), len(ids) + 1)
        ids.append(0)
    r = orc.rasterize(cam, proj, logit, tb, np.array(ids, np.int32))
    o = 1 / (1 + math.exp(-0.7))
    jj, ii = np.meshgrid(np.arange(32), np.arange(32))
    dx, dy = 13.3 - jj, 17.6 - ii
    sig = 0.5 * (0.05 * dx * dx + 0.08 * dy * dy) + 0.012 * dx * dy
    al = np.minimum(0.999, o * np.exp(-sig))
    hit = (sig < 5.55) & (al >= 1 / 255)
    al = np.where(hit, al, 0)
    ref = np.clip(BG[None, None, :].astype(np.float64) * (1 - al[..., None]) +
                  al[..., None] * np.maximum(col[0].astype(np.float64) + 0.5, 0), 0, 1)
    np.testing.assert_allclose(r["out_img"], ref, atol=2e-6)
    np.testing.assert_allclose(r["final_Ts"], 1 - al, atol=2e-6)
    assert (r["final_index"][hit] >= 0).all() and (r["final_index"][~hit] == np.array(tb)[
        (ii // 16 * 2 + jj // 16)[~hit], 0] - 1).all()


def test_raster_stop_rule():
    """Opaque stack at one pixel: the entry that would take T to <= 1e-4 is
    not composited and final_index points at the entry before it."""
    su, cam = _cam(16, 16, degree=0, dtu=0)
    n = 4
    xy = np.tile(np.array([[8.0, 8.0]], F32), (n, 1))
    conic = np.tile(np.array([[1e-4, 0.0, 1e-4]], F32), (n, 1))
    col = np.array([[0.1, 0, 0], [0, 0.2, 0], [0, 0, 0.3], [0.4, 0.4, 0.4]], F32)
    logit = np.full(n, 5.0, F32)   # o = 0.9933, alpha = o (sigma ~ 0 at the centre)
    proj = dict(xys=xy, conics=conic, colors=col)
    r = orc.rasterize(cam, proj, logit, np.array([[0, n]], np.int32), np.arange(n, dtype=np.int32))
    o = 1 / (1 + math.exp(-5.0))
    a = o * math.exp(-0.0)
    # T after one entry 6.7e-3, after two 4.5e-5 <= 1e-4 -> stop before the second
    assert r["final_index"][8, 8] == 0
    assert abs(r["final_Ts"][8, 8] - (1 - a)) < 1e-6
    ref = np.clip(BG * (1 - a) + a * (col[0] + 0.5), 0, 1)
    np.testing.assert_allclose(r["out_img"][8, 8], ref, atol=2e-6)


def test_raster_forward_against_float64_compositing():
    """Random small scene (monolithic tiles, >= 400 tiles is not needed: every
    tile holds < 512 entries so chunked == one piece): the oracle image within
    2e-5 of a float64 per-pixel compositing except where a skip / stop
    threshold flips (at most 0.1% of pixels)."""
    sc = small_scene(n=600, width=64, height=48, seed_off=202)
    su = camera.prepare_cam(sc.cameras[0])
    cam = orc.camera(su, 3, 3, BG)
    p = orc.project(cam, sc.means, sc.scales, sc.quats, sc.f_dc, sc.f_rest)
    counts, tb, ids = orc.bin_sort(cam, p)
    r = orc.rasterize(cam, p, sc.opacities, tb, ids)
    ref, Tf = _composite64(su, p, sc.opacities, tb, ids, BG.astype(np.float64))
    bad = np.abs(r["out_img"] - ref).max(axis=2) > 2e-5
    assert bad.mean() <= 1e-3, (bad.sum(), np.abs(r["out_img"] - ref).max())


def test_chunked_forward_close_to_monolithic():
    """A dense scene below 400 tiles takes the 512-entry chunked path with
    chunk-local stops and the merge; it stays within 3e-4 of float64
    monolithic compositing (the difference is bounded by the stop threshold)."""
    sc = small_scene(n=12000, width=48, height=48, seed_off=203, spread=0.5)
    su = camera.prepare_cam(sc.cameras[0])
    cam = orc.camera(su, 3, 3, BG)
    p = orc.project(cam, sc.means, sc.scales, sc.quats, sc.f_dc, sc.f_rest)
    counts, tb, ids = orc.bin_sort(cam, p)
    assert counts.max() > 1024
    r = orc.rasterize(cam, p, sc.opacities, tb, ids)
    ref, _ = _composite64(su, p, sc.opacities, tb, ids, BG.astype(np.float64))
    diff = np.abs(r["out_img"] - ref).max(axis=2)
    assert (diff > 3e-4).mean() <= 2e-3, (int((diff > 3e-4).sum()), float(diff.max()))


# --------------------------------------------------- raster backward ---------

def _raster_loss64(su, xy, conic, col, logit, v_out, bg):
    """float64 sum(v_out * image) for one tile list holding every gaussian in
    depth order (no stop, no clamp active in the test scene)."""
    H, W = su.height, su.width
    jj, ii = np.meshgrid(np.arange(W, dtype=np.float64), np.arange(H, dtype=np.float64))
    T = np.ones((H, W))
    C = np.zeros((H, W, 3))
    o = 1 / (1 + np.exp(-logit))
    for k in range(xy.shape[0]):
        dx, dy = xy[k, 0] - jj, xy[k, 1] - ii
        sig = 0.5 * (conic[k, 0] * dx * dx + conic[k, 2] * dy * dy) + conic[k, 1] * dx * dy
        al = np.minimum(0.999, o[k] * np.exp(-sig))
        al = np.where((sig >= 0) & (sig < 5.55) & (al >= 1 / 255), al, 0.0)
        C += (al * T)[..., None] * np.maximum(col[k] + 0.5, 0)
        T = T * (1 - al)
    img = bg * T[..., None] + C
    assert img.min() > 0 and img.max() < 1
    return float((v_out * img).sum())


def test_raster_backward_finite_differences():
    """v_xy, v_conic (a, b/2, c: the symmetric-matrix convention), v_rgb and
    v_opacity (w.r.t. the logit) against float64 central differences of
    sum(v_out * image) on a scene where no stop, clamp or alpha cap triggers."""
    su, cam = _cam(32, 32, degree=0, dtu=0)
    rng = np.random.default_rng(9)
    n = 12
    xy = rng.uniform(4, 28, (n, 2)).astype(F32)
    A = rng.uniform(0.02, 0.12, n)
    Cc = rng.uniform(0.02, 0.12, n)
    B = rng.uniform(-0.5, 0.5, n) * np.sqrt(A * Cc)
    conic = np.stack([A, B, Cc], 1).astype(F32)
    col = rng.uniform(-0.3, 0.2, (n, 3)).astype(F32)
    logit = rng.uniform(-2.0, 0.5, n).astype(F32)
    bg = np.array([0.3, 0.4, 0.5], F32)
    cam.background[:] = [float(v) for v in bg]
    proj = dict(xys=xy, conics=conic, colors=col)
    tb = np.array([[0, n]] * 4, np.int32)
    tb = np.array([[k * n, (k + 1) * n] for k in range(4)], np.int32)
    ids = np.tile(np.arange(n, dtype=np.int32), 4)
    v_out = rng.normal(size=(32, 32, 3)).astype(F32)
    r = orc.rasterize(cam, proj, logit, tb, ids, v_out=v_out)
    args = [a.astype(np.float64) for a in (xy, conic, col, logit)]

    def f(i, idx, h):
        a = [x.copy() for x in args]
        a[i][idx] += h
        return _raster_loss64(su, *a, v_out.astype(np.float64), bg.astype(np.float64))

    def fd(i, idx, h):
        return (f(i, idx, h) - f(i, idx, -h)) / (2 * h)

    for k in range(n):
        for d in range(2):
            g = fd(0, (k, d), 1e-4)
            assert abs(r["v_xy"][k, d] - g) <= 2e-3 * abs(g) + 2e-4, ("v_xy", k, d, r["v_xy"][k, d], g)
        for d, half in ((0, 1.0), (1, 0.5), (2, 1.0)):
            g = half * fd(1, (k, d), 1e-6)
            assert abs(r["v_conic"][k, d] - g) <= 2e-3 * abs(g) + 2e-2, ("v_conic", k, d, r["v_conic"][k, d], g)
        for d in range(3):
            g = fd(2, (k, d), 1e-4)
            assert abs(r["v_rgb"][k, d] - g) <= 2e-3 * abs(g) + 1e-4, ("v_rgb", k, d, r["v_rgb"][k, d], g)
        g = fd(3, (k,), 1e-4)
        assert abs(r["v_opacity"][k] - g) <= 2e-3 * abs(g) + 1e-4, ("v_opacity", k, r["v_opacity"][k], g)


# ------------------------------------------------ projection backward --------

def test_project_backward_finite_differences():
    """v_mean3d / v_scale (w.r.t. log scale) / v_quat against float64 central
    differences of L = v_xy . xy + v_a a + 2 v_b b + v_c c.  The reference
    differentiates a surrogate, and the difference is taken of that surrogate:
    the pixel centre's 1/w is held at its value (project_pix_vjp drops the
    w-row, .metal:1216-1234) and the quaternion enters the rotation
    unnormalised (no normalisation Jacobian, .metal:1409-1452; evaluated at
    |q| = 1).  Centres are inside the 1.3 tan(fov) clamp."""
    su, cam = _cam(96, 64, degree=0, dtu=0)
    rng = np.random.default_rng(10)
    n = 24
    means, scales, quats = _scene_in_view(n, su, rng, log_s=(-2.5, -1.0), margin=0.6)
    p = orc.project(cam, means, scales, quats, np.zeros((n, 3), F32), np.zeros((n, 0), F32))
    assert (p["radii"] > 0).all()
    v_xy = rng.normal(size=(n, 2)).astype(F32)
    v_conic = (rng.normal(size=(n, 3)) * 10).astype(F32)
    vm, vs, vq = np.zeros((n, 3), F32), np.zeros((n, 3), F32), np.zeros((n, 4), F32)
    orc.lib().orc_project_backward(ctypes.byref(cam), n, orc.P(means), orc.P(scales), orc.P(quats),
                                   orc.P(p["radii"]), orc.P(p["conics"]), orc.P(v_xy), orc.P(v_conic),
                                   orc.P(vm), orc.P(vs), orc.P(vq))
    Pm = np.asarray(su.projmat, np.float64)

    def loss(g, mean, ls, q):
        hw0 = Pm[3, :3] @ means[g].astype(np.float64) + Pm[3, 3]
        rw0 = 1.0 / (hw0 + 1e-6)
        hx = Pm[0, :3] @ mean + Pm[0, 3]
        hy = Pm[1, :3] @ mean + Pm[1, 3]
        x = 0.5 * su.width * hx * rw0 + su.cx - 0.5
        y = 0.5 * su.height * hy * rw0 + su.cy - 0.5
        _, _, con = _ewa64(su, mean, ls, q, clamp=False, normalize_q=False)
        va, vb, vc = (float(v) for v in v_conic[g])
        return float(v_xy[g, 0]) * x + float(v_xy[g, 1]) * y + va * con[0] + 2 * vb * con[1] + vc * con[2]

    for g in range(n):
        base = [means[g].astype(np.float64), scales[g].astype(np.float64), quats[g].astype(np.float64)]
        for which, out, h in ((0, vm, 1e-5), (1, vs, 1e-5), (2, vq, 1e-6)):
            for d in range(base[which].size):
                hi = [b.copy() for b in base]
                lo = [b.copy() for b in base]
                hi[which][d] += h
                lo[which][d] -= h
                fdv = (loss(g, *hi) - loss(g, *lo)) / (2 * h)
                got = float(out[g, d])
                tol = 3e-3 * abs(fdv) + 3e-4 * (np.abs(out[g]).max() + 1e-3)
                assert abs(got - fdv) <= tol, (("mean", "scale", "quat")[which], g, d, got, fdv)


def test_sh_backward_is_basis_times_v_rgb():
    """v_dc / v_rest = basis value x v_rgb (the colour is linear in the
    coefficients), for bands up to degrees_to_use and zero above."""
    su, cam = _cam(64, 48, degree=3, dtu=2)
    rng = np.random.default_rng(11)
    n = 40
    means, _, _ = _scene_in_view(n, su, rng)
    radii = np.ones(n, np.int32)
    radii[::7] = 0
    v_rgb = rng.normal(size=(n, 3)).astype(F32)
    v_dc = np.zeros((n, 3), F32)
    v_rest = np.zeros((n, 15, 3), F32)
    orc.lib().orc_sh_backward(ctypes.byref(cam), n, orc.P(means), orc.P(radii), orc.P(v_rgb),
                              orc.P(v_dc), orc.P(v_rest))
    cpos = np.asarray(su.cam_pos, np.float64)
    for g in range(n):
        if radii[g] == 0:
            assert not v_dc[g].any() and not v_rest[g].any()
            continue
        d = means[g].astype(np.float64) - cpos
        d /= np.linalg.norm(d)
        Y = _sh_basis(3, d[None, :].astype(F32))[0]
        np.testing.assert_allclose(v_dc[g], Y[0] * v_rgb[g], rtol=1e-5, atol=1e-7)
        ref = Y[1:, None] * v_rgb[g][None, :]
        ref[8:] = 0.0   # bands 3 above degrees_to_use = 2
        np.testing.assert_allclose(v_rest[g], ref, rtol=1e-4, atol=1e-6)


# ------------------------------------------------------------- SSIM ----------

def _ssim_loss64(img, gt, w):
    """float64 training loss value: sum over pixels of w (1 - mean_c SSIM) +
    (1 - w) mean_c |gt - img|, divided by H W; 11x11 Gaussian window
    (sigma 1.5), zero padding, C1 = 1e-4, C2 = 9e-4."""
    from scipy.signal import convolve2d
    x = np.arange(11) - 5.0
    g1 = np.exp(-x * x / 4.5)
    g1 /= g1.sum()
    win = np.outer(g1, g1)
    H, W = img.shape[:2]
    tot = 0.0
    ssim = np.zeros((H, W))
    for c in range(3):
        X, Y = gt[..., c], img[..., c]
        f = lambda a: convolve2d(a, win, mode="same", boundary="fill")
        mx, my = f(X), f(Y)
        sxx, syy, sxy = f(X * X) - mx * mx, f(Y * Y) - my * my, f(X * Y) - mx * my
        ssim += ((2 * mx * my + 1e-4) * (2 * sxy + 9e-4)) / ((mx * mx + my * my + 1e-4) * (sxx + syy + 9e-4))
    tot = (w * (1 - ssim / 3) + (1 - w) * np.abs(gt - img).mean(axis=2)).sum()
    return tot / (H * W)


def test_ssim_forward_brute_force():
    rng = np.random.default_rng(12)
    H, W = 30, 37
    img = rng.uniform(0.05, 0.95, (H, W, 3)).astype(F32)
    gt = np.clip(img + rng.normal(0, 0.1, img.shape), 0, 1).astype(F32)
    s, v, _, _ = orc.ssim_loss(img, gt, 0.2)
    ref = _ssim_loss64(img.astype(np.float64), gt.astype(np.float64), 0.2)
    assert abs(s / (H * W) - ref) <= 2e-6 * abs(ref), (s / (H * W), ref)


def test_ssim_backward_finite_differences():
    """v_rendered = d loss / d img at pixels >= 5 columns from the left and
    right edges; nearer the side edges the reference's horizontal-halo quirk
    (out-of-image window centres are not excluded, .metal:3243-3299) makes it
    differ from the true gradient, which is the reference's semantics."""
    rng = np.random.default_rng(13)
    H, W = 20, 24
    img = rng.uniform(0.1, 0.9, (H, W, 3)).astype(F32)
    gt = np.clip(img + rng.normal(0, 0.15, img.shape), 0, 1).astype(F32)
    _, v, _, _ = orc.ssim_loss(img, gt, 0.2)
    base = img.astype(np.float64)
    gt64 = gt.astype(np.float64)
    h = 1e-6
    checked = 0
    for i in range(0, H, 3):
        for j in range(5, W - 5, 2):
            for c in range(3):
                if abs(base[i, j, c] - gt64[i, j, c]) < 10 * h:
                    continue
                a, b = base.copy(), base.copy()
                a[i, j, c] += h
                b[i, j, c] -= h
                fdv = (_ssim_loss64(a, gt64, 0.2) - _ssim_loss64(b, gt64, 0.2)) / (2 * h)
                assert abs(v[i, j, c] - fdv) <= 2e-3 * abs(fdv) + 2e-7, (i, j, c, v[i, j, c], fdv)
                checked += 1
    assert checked > 100


# ------------------------------------------------------------- Adam ----------

def test_adam_matches_torch():
    """fused_adam with step_size = lr / (1 - b1^t), bc2_sqrt = sqrt(1 - b2^t)
    reproduces torch.optim.Adam over five steps."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(14)
    n = 1000
    p0 = rng.normal(size=n).astype(F32)
    grads = [rng.normal(size=n).astype(F32) * F32(10 ** rng.uniform(-4, 1)) for _ in range(5)]
    lr = 0.01
    tp = torch.tensor(p0.copy(), requires_grad=True)
    opt = torch.optim.Adam([tp], lr=lr, betas=(0.9, 0.999), eps=1e-8)
    p, m, v = p0.copy(), np.zeros(n, F32), np.zeros(n, F32)
    for t, g in enumerate(grads, start=1):
        tp.grad = torch.tensor(g)
        opt.step()
        a = orc.adam_hparams([lr] * 6, t)
        orc.lib().orc_adam(n, orc.P(p), orc.P(g), orc.P(m), orc.P(v), ctypes.c_float(a.step_size[0]),
                           ctypes.c_float(0.9), ctypes.c_float(0.999), ctypes.c_float(a.bc2_sqrt[0]),
                           ctypes.c_float(1e-8))
    np.testing.assert_allclose(p, tp.detach().numpy(), rtol=2e-6, atol=2e-7)


def test_grad_stats_closed_form():
    rng = np.random.default_rng(15)
    n = 50
    radii = rng.integers(0, 30, n).astype(np.int32)
    v_xy = rng.normal(size=(n, 2)).astype(F32)
    vis, gn, mx = np.ones(n, F32), np.full(n, 0.5, F32), np.full(n, 0.01, F32)
    orc.lib().orc_grad_stats(n, orc.P(radii), orc.P(v_xy), orc.P(vis), orc.P(gn), orc.P(mx),
                             ctypes.c_float(1.0 / 97))
    on = radii > 0
    np.testing.assert_array_equal(vis, np.where(on, 2.0, 1.0).astype(F32))
    np.testing.assert_allclose(gn, np.where(on, 0.5 + np.hypot(v_xy[:, 0], v_xy[:, 1]), 0.5), rtol=1e-6)
    np.testing.assert_allclose(mx, np.where(on, np.maximum(0.01, radii / 97.0), 0.01), rtol=1e-6)


# ------------------------------------------------------------ densify --------

def test_densify_hand_cases():
    """Four gaussians with known outcomes: 0 high-grad large -> split into two
    children at mean + R (eps * s) with log-scale - ln 1.6 (parent culled);
    1 high-grad small -> duplicated; 2 low-grad transparent -> culled;
    3 low-grad -> kept.  Survivors are stably compacted."""
    N, cap = 4, 12
    fr = 3
    bufs = [np.zeros(cap * k, F32) for k in (3, 3, 4, 3, fr, 1)]
    bufs[0][:12] = np.arange(12, dtype=F32)
    bufs[1][:12] = np.log([0.2, 0.1, 0.05, 0.001, 0.002, 0.003, 0.001, 0.001, 0.001, 0.001, 0.001, 0.001]).astype(F32)
    q0 = np.array([0.9, 0.1, -0.3, 0.2], F32)
    bufs[2][:16] = np.concatenate([q0, [1, 0, 0, 0], [1, 0, 0, 0], [1, 0, 0, 0]]).astype(F32)
    bufs[3][:12] = np.arange(12, dtype=F32) * 0.1
    bufs[4][:12] = np.arange(12, dtype=F32) * 0.01
    bufs[5][:4] = np.array([0.5, 0.3, -8.0, 0.2], F32)
    m = [np.full_like(b, 7.0) for b in bufs]
    v = [np.full_like(b, 9.0) for b in bufs]
    gnorm = np.array([1.0, 1.0, 0.0, 0.0], F32)
    vis = np.ones(4, F32)
    max2d = np.zeros(4, F32)
    rnd = np.array([[0.5, -1.0, 2.0], [-0.25, 0.75, 1.5]], F32).reshape(-1)
    args = orc.OrcDensifyArgs(N=N, grad_thresh=0.0002, size_thresh=0.01, screen_thresh=0.05, check_screen=0,
                              cull_alpha_thresh=0.005, cull_scale_thresh=0.5, cull_screen_size=0.15,
                              check_huge=0, half_max_dim=50.0, fr_stride=fr)
    nn, split, dup, keep = orc.densify(args, gnorm, vis, max2d, bufs, m, v, rnd)
    assert list(split) == [1, 0, 0, 0] and list(dup) == [0, 1, 0, 0]
    # grown set: 0 1 2 3 | child0 child1 | dup(1); keep: parent 0 and transparent 2 culled
    assert list(keep[:7]) == [0, 1, 0, 1, 1, 1, 1]
    assert nn == 5
    R = _rot64(q0.astype(np.float64))
    s0 = np.array([0.2, 0.1, 0.05])
    means = bufs[0][:15].reshape(5, 3)
    np.testing.assert_array_equal(means[0], [3, 4, 5])        # gaussian 1
    np.testing.assert_array_equal(means[1], [9, 10, 11])      # gaussian 3
    for k, ch in enumerate((2, 3)):
        want = np.array([0, 1, 2.0]) + R @ (rnd.reshape(2, 3)[k].astype(np.float64) * s0)
        np.testing.assert_allclose(means[ch], want, rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(bufs[1][3 * ch:3 * ch + 3], np.log(s0) - math.log(1.6), rtol=1e-5)
        np.testing.assert_array_equal(bufs[5][ch], F32(0.5))
        assert not m[0][3 * ch:3 * ch + 3].any() and not v[5][ch]
    np.testing.assert_array_equal(means[4], [3, 4, 5])        # duplicate of 1
    assert m[0][3 * 4] == 0.0 and m[0][0] == 7.0              # fresh Adam state only for new entries


def test_knn_mean_dist_against_kdtree():
    """orc_knn_mean_dist: the mean distance to the three nearest other points,
    as a float64 kd-tree (scipy's cKDTree, k=4 with the point itself first)
    gives it, on a blob with exact duplicates and on a plane; and a planted
    mistake (averaging the 1st..3rd instead of the 2nd..4th) fails."""
    from scipy.spatial import cKDTree
    rng = np.random.default_rng(11)
    blob = rng.normal(0, 1, (3000, 3))
    blob[200:300] = blob[0:100]
    plane = np.c_[rng.uniform(-2, 2, (2000, 2)), np.zeros(2000)]
    for x in (blob, plane):
        x = x.astype(np.float32)
        got = orc.knn_mean_dist(x)
        d, _ = cKDTree(x.astype(np.float64)).query(x.astype(np.float64), k=4)
        want = d[:, 1:].mean(axis=1)
        assert np.allclose(got, want, rtol=2e-6, atol=1e-7)
        assert not np.allclose(d[:, :3].mean(axis=1), want, rtol=2e-6, atol=1e-7)


def test_train_step_stage_times():
    """orc_stage_times: one train step's reference-named stages add up to
    about its wall time, and the sums reset."""
    import time
    sc = small_scene(n=800, width=64, height=48, seed_off=250)
    su = camera.prepare_cam(sc.cameras[0])
    cam = orc.camera(su, 3, 3, BG)
    gt = np.zeros((su.height, su.width, 3), F32)
    params = [np.ascontiguousarray(a, F32).copy() for a in sc.params()]
    m = [np.zeros_like(a) for a in params]
    v = [np.zeros_like(a) for a in params]
    z = [np.zeros(sc.n, F32) for _ in range(3)]
    ms = (ctypes.c_double * 8)()
    steps = ctypes.c_int64(0)
    orc.lib().orc_stage_times(ms, ctypes.byref(steps))
    t0 = time.perf_counter()
    orc.train_step(cam, params, m, v, orc.adam_hparams([1e-3] * 6, 1), gt, 0.2, *z)
    wall = 1e3 * (time.perf_counter() - t0)
    orc.lib().orc_stage_times(ms, ctypes.byref(steps))
    assert steps.value == 1
    tot = sum(ms)
    assert all(x >= 0 for x in ms) and ms[1] > 0 and ms[3] > 0 and ms[5] > 0
    assert 0.5 * wall <= tot <= wall, (tot, wall)
    orc.lib().orc_stage_times(ms, ctypes.byref(steps))
    assert steps.value == 0 and sum(ms) == 0.0
