"""Pins of the oracle's reference-specific branches by mathematics.

Where the reference's backward is not the derivative of its own forward, it is
still the exact derivative of a function that can be written down in closed
form.  Each test below states that function, evaluates it in float64, takes
central finite differences and compares them with the oracle's gradients;
each also checks that the oracle is far from the derivative of the plain
forward, so that an oracle which dropped the reference's branch fails.

* alpha cap (.metal:1049, 2992): a (pixel, gaussian) pair whose alpha is
  capped at 0.999 is skipped in the backward, with no gradient and no
  transmittance recovery through it.  The backward is then the gradient of
  the pixel with every capped pair removed and the whole composite
  (colours and background) scaled by the constant (1 - 0.999) per capped
  pair: every transmittance the backward recovers is off by that factor.
* saturate (.metal:580): the forward clamps the output to [0, 1], the
  backward ignores the clamp: the gradient of the unclamped bg T + C.
* SSIM halo (.metal:3243-3299, 3430-3435): window centres in the five
  columns left and right of the image carry derivative fields computed from
  all-zero statistics (f1 = 0, f2 = -2/C2, f3 = 2/C2); the gradient is that
  of the zero-padded training loss plus, for each such centre q in an image
  row, -w inv_n sum_p K(q - p) (-y_p^2 + 2 x_p y_p) / C2 per channel
  (x = target, y = render, K the 11x11 window).
* chunks (.metal:2633-2741, 2764-2799, 2804-2840, 2884-3031): every chunk
  of 512 entries composites from T = 1 and stops on its own; the merge
  folds chunks front to back and cuts off once T <= 1e-4; the backward's
  suffix sums every chunk, also those past the cutoff, and chunks past the
  cutoff get no gradient.  The backward is the gradient of
  sum_k pT_k C_k + T_final bg over all chunks with the entries of chunks past
  the cutoff frozen.
* sparse SH Adam (.metal:1846-1848 vs 1666-1689): culled gaussians' f_dc,
  f_rest and their moments are untouched by a step, while the dense groups
  (means, scales, quats, opacities) of the same gaussians still move.
CPU only.
"""
from __future__ import annotations

import math

import numpy as np

import orc
from helpers import LRS, small_scene, target_for
from msplat_amd import camera

F32 = np.float32
CAP = float(F32(0.999))
KAPPA = 1.0 - CAP                 # the (1 - alpha) of a capped pair, fp32 cap
C2 = float(F32(0.03) * F32(0.03))  # SSIM C2 as the kernels hold it (9e-4)


def _cam16(bg):
    cam = camera.pinhole(16, 16, 60.0, camera.look_at((0.0, 0.0, 4.0)))
    su = camera.prepare_cam(cam)
    c = orc.camera(su, 0, 0, bg)
    return su, c


def _alpha64(xy, conic, logit, j, i):
    """float64 sigma and unclamped alpha of each gaussian at pixel (column j, row i)."""
    dx, dy = xy[:, 0] - j, xy[:, 1] - i
    sig = 0.5 * (conic[:, 0] * dx * dx + conic[:, 2] * dy * dy) + conic[:, 1] * dx * dy
    o = 1.0 / (1.0 + np.exp(-logit))
    return sig, o * np.exp(-sig)


def _valid(sig, au):
    return (sig >= 0) & (sig < 5.55) & (np.minimum(CAP, au) >= 1 / 255)


def _fd_check(oracle, f, args, n, tol, what_rgb=True):
    """Central differences of f(args) against the oracle's v_xy, v_conic
    (symmetric-matrix convention: half of d/db), v_rgb, v_opacity."""
    def fd(i, idx, h):
        a = [x.copy() for x in args]
        b = [x.copy() for x in args]
        a[i][idx] += h
        b[i][idx] -= h
        return (f(a) - f(b)) / (2 * h)

    for k in range(n):
        for d in range(2):
            g = fd(0, (k, d), 1e-4)
            assert abs(oracle["v_xy"][k, d] - g) <= tol * abs(g) + 2e-4, ("v_xy", k, d, oracle["v_xy"][k, d], g)
        for d, half in ((0, 1.0), (1, 0.5), (2, 1.0)):
            g = half * fd(1, (k, d), 1e-6)
            assert abs(oracle["v_conic"][k, d] - g) <= tol * abs(g) + 2e-2, ("v_conic", k, d,
                                                                            oracle["v_conic"][k, d], g)
        if what_rgb:
            for d in range(3):
                g = fd(2, (k, d), 1e-4)
                assert abs(oracle["v_rgb"][k, d] - g) <= tol * abs(g) + 1e-4, ("v_rgb", k, d,
                                                                              oracle["v_rgb"][k, d], g)
        g = fd(3, (k,), 1e-4)
        assert abs(oracle["v_opacity"][k] - g) <= tol * abs(g) + 1e-4, ("v_opacity", k, oracle["v_opacity"][k], g)


# ------------------------------------------------------------ alpha cap ------

def _capped_scene():
    """Three gaussians over one 16x16 tile, depth order 0, 1, 2.  Gaussian 1
    is nearly opaque (sigmoid(12)) and wide: its alpha reaches the 0.999 cap
    at the pixels within sqrt(5) of its centre (8, 8), and stays below it
    elsewhere, with a margin far above rounding and the finite-difference
    steps.  Opacities keep T above the 1e-4 stop everywhere."""
    xy = np.array([[7.3, 8.6], [8.0, 8.0], [8.9, 7.4]], np.float64)
    conic = np.array([[0.035, 0.004, 0.03], [0.00036, 0.0, 0.00036], [0.03, -0.005, 0.04]], np.float64)
    col = np.array([[0.1, -0.2, 0.25], [-0.15, 0.3, 0.05], [0.2, 0.1, -0.3]], np.float64)
    logit = np.array([0.0, 12.0, 0.4], np.float64)
    return xy, conic, col, logit


def _cap_surrogate(args, caps, v_out, bg):
    """sum(v_out * image') with image' = kappa^(capped pairs) (C' + T' bg), the
    capped pairs (fixed set `caps`) removed from C' and T'."""
    xy, conic, col, logit = args
    tot = 0.0
    for i in range(16):
        for j in range(16):
            sig, au = _alpha64(xy, conic, logit, j, i)
            ok = _valid(sig, au)
            T, C, kap = 1.0, np.zeros(3), 1.0
            for k in range(xy.shape[0]):
                if not ok[k]:
                    continue
                if (i, j, k) in caps:
                    kap *= KAPPA
                    continue
                a = min(CAP, au[k])
                C += np.maximum(col[k] + 0.5, 0) * a * T
                T *= 1 - a
            tot += float(np.dot(v_out[i, j], kap * (C + T * bg)))
    return tot


def _plain_loss(args, v_out, bg):
    """sum(v_out * unclamped image) of the plain forward (capped pairs composite
    with alpha = 0.999, no skip)."""
    xy, conic, col, logit = args
    tot = 0.0
    for i in range(16):
        for j in range(16):
            sig, au = _alpha64(xy, conic, logit, j, i)
            ok = _valid(sig, au)
            T, C = 1.0, np.zeros(3)
            for k in range(xy.shape[0]):
                if ok[k]:
                    a = min(CAP, au[k])
                    C += np.maximum(col[k] + 0.5, 0) * a * T
                    T *= 1 - a
            tot += float(np.dot(v_out[i, j], C + T * bg))
    return tot


def _run_oracle(cam, xy, conic, col, logit, v_out, ids=None, n_entries=None):
    n = xy.shape[0]
    proj = dict(xys=xy.astype(F32), conics=conic.astype(F32), colors=col.astype(F32))
    if ids is None:
        ids = np.arange(n, dtype=np.int32)
    tb = np.array([[0, len(ids)]], np.int32)
    return orc.rasterize(cam, proj, logit.astype(F32), tb, ids, v_out=v_out.astype(F32))


def test_alpha_cap_skip_is_gradient_of_scaled_surrogate():
    bg = np.array([0.3, 0.4, 0.5], F32)
    su, cam = _cam16(bg)
    xy, conic, col, logit = _capped_scene()
    caps = set()
    margin = 1.0
    for i in range(16):
        for j in range(16):
            sig, au = _alpha64(xy, conic, logit, j, i)
            assert _valid(sig, au).all()
            margin = min(margin, abs(au[1] - CAP))
            if au[1] >= CAP:
                caps.add((i, j, 1))
            assert au[0] < CAP and au[2] < CAP
    assert len(caps) == 21 and margin > 5e-5, (len(caps), margin)   # d^2 <= 5: 1 + 4 + 4 + 4 + 8
    rng = np.random.default_rng(21)
    v_out = rng.normal(size=(16, 16, 3))
    r = _run_oracle(cam, xy, conic, col, logit, v_out)
    # no stop anywhere: every pixel's final index is the last entry
    assert (r["final_index"] == 2).all() and r["final_Ts"].min() > 1e-4
    args = [a.astype(F32).astype(np.float64) for a in (xy, conic, col, logit)]
    bg64 = bg.astype(np.float64)
    v64 = v_out.astype(F32).astype(np.float64)
    _fd_check(r, lambda a: _cap_surrogate(a, caps, v64, bg64), args, 3, 2e-3)
    # The plain forward's derivative is far from it: the capped gaussian's
    # colour (alpha T v at its capped pixels) and the front gaussian's
    # colour (whose transmittance the backward takes 1000x too small there).
    h = 1e-4
    for k in (0, 1):
        a, b = [x.copy() for x in args], [x.copy() for x in args]
        a[2][k, 0] += h
        b[2][k, 0] -= h
        plain = (_plain_loss(a, v64, bg64) - _plain_loss(b, v64, bg64)) / (2 * h)
        assert abs(r["v_rgb"][k, 0] - plain) > 0.05, (k, r["v_rgb"][k, 0], plain)


# ------------------------------------------------------------- saturate ------

def test_no_gradient_mask_for_saturated_pixels():
    """Bright, dense colours push C + T bg above 1 at the centre; the forward
    saturates there, the backward is the gradient of the unclamped image."""
    bg = np.array([0.9, 0.8, 0.95], F32)
    su, cam = _cam16(bg)
    xy = np.array([[7.5, 8.2], [8.4, 7.7], [8.0, 8.9]], np.float64)
    conic = np.array([[0.03, 0.002, 0.035], [0.025, -0.004, 0.03], [0.04, 0.0, 0.03]], np.float64)
    col = np.array([[0.7, 0.6, 0.8], [0.65, 0.75, 0.6], [0.8, 0.7, 0.7]], np.float64)
    logit = np.array([1.2, 0.8, 1.0], np.float64)
    rng = np.random.default_rng(22)
    v_out = rng.normal(size=(16, 16, 3))
    r = _run_oracle(cam, xy, conic, col, logit, v_out)
    args = [a.astype(F32).astype(np.float64) for a in (xy, conic, col, logit)]
    bg64, v64 = bg.astype(np.float64), v_out.astype(F32).astype(np.float64)

    def image(a):
        x, c, cl, lg = a
        img = np.zeros((16, 16, 3))
        for i in range(16):
            for j in range(16):
                sig, au = _alpha64(x, c, lg, j, i)
                ok = _valid(sig, au)
                T, C = 1.0, np.zeros(3)
                for k in range(3):
                    if ok[k]:
                        al = min(CAP, au[k])
                        C += np.maximum(cl[k] + 0.5, 0) * al * T
                        T *= 1 - al
                img[i, j] = C + T * bg64
        return img

    base = image(args)
    sat = base > 1.0
    # no pixel within the finite-difference steps (about 2e-5 of image) of the clamp
    assert sat.sum() >= 20 and np.abs(base - 1.0).min() > 1e-4, (sat.sum(), np.abs(base - 1.0).min())
    np.testing.assert_allclose(r["out_img"], np.clip(base, 0, 1), atol=2e-6)
    _fd_check(r, lambda a: float((v64 * image(a)).sum()), args, 3, 2e-3)
    # the clamped image's derivative differs: saturated channels pass nothing
    h = 1e-4
    a, b = [x.copy() for x in args], [x.copy() for x in args]
    a[3][0] += h
    b[3][0] -= h
    clamped = float((v64 * (np.clip(image(a), 0, 1) - np.clip(image(b), 0, 1))).sum()) / (2 * h)
    assert abs(r["v_opacity"][0] - clamped) > 0.05, (r["v_opacity"][0], clamped)


# ------------------------------------------------------------ SSIM halo ------

def _gauss11():
    x = np.arange(11) - 5.0
    g = np.exp(-x * x / 4.5)
    return g / g.sum()


def _ssim_true64(img, gt, w):
    from test_oracle_pins import _ssim_loss64
    return _ssim_loss64(img, gt, w)


def _halo_term64(img, gt, w):
    """Frozen-statistics contribution of the out-of-image window centres in
    the five columns left and right of the image (rows inside it)."""
    H, W = img.shape[:2]
    g = _gauss11()
    inv_n = 1.0 / (3.0 * H * W)
    tot = 0.0
    cols = list(range(-5, 0)) + list(range(W, W + 5))
    for qy in range(H):
        for qx in cols:
            for py in range(max(0, qy - 5), min(H, qy + 6)):
                for px in range(max(0, qx - 5), min(W, qx + 6)):
                    k = g[py - qy + 5] * g[px - qx + 5]
                    y, x = img[py, px], gt[py, px]
                    tot += k * float(np.sum(-y * y + 2.0 * x * y)) / C2
    return -w * inv_n * tot


def test_ssim_halo_is_gradient_of_frozen_centre_term():
    rng = np.random.default_rng(23)
    H, W = 14, 21
    img = rng.uniform(0.1, 0.9, (H, W, 3)).astype(F32)
    gt = np.clip(img + rng.normal(0, 0.15, img.shape), 0, 1).astype(F32)
    _, v, _, _ = orc.ssim_loss(img, gt, 0.2)
    base, gt64 = img.astype(np.float64), gt.astype(np.float64)
    h = 1e-6

    def total(a):
        return _ssim_true64(a, gt64, 0.2) + _halo_term64(a, gt64, 0.2)

    checked = far = near = 0
    for i in range(0, H, 2):
        for j in list(range(0, 5)) + list(range(W - 5, W)):
            for c in range(3):
                if abs(base[i, j, c] - gt64[i, j, c]) < 10 * h:
                    continue
                a, b = base.copy(), base.copy()
                a[i, j, c] += h
                b[i, j, c] -= h
                fdv = (total(a) - total(b)) / (2 * h)
                assert abs(v[i, j, c] - fdv) <= 2e-3 * abs(fdv) + 2e-7, (i, j, c, v[i, j, c], fdv)
                checked += 1
                if j in (0, 1, W - 2, W - 1):
                    # next to the edge the halo term dominates the plain gradient
                    plain = (_ssim_true64(a, gt64, 0.2) - _ssim_true64(b, gt64, 0.2)) / (2 * h)
                    far += abs(v[i, j, c] - plain) > 0.1 * abs(plain) + 1e-6
                    near += 1
    # (the halo gradient is proportional to target - render: nearly equal
    # pairs can leave it small)
    assert checked > 150 and near > 60 and far >= 0.95 * near, (checked, near, far)


# ---------------------------------------------------------------- chunks -----

CHUNK = 512
KEY = (0, 1, 512, 1024)   # list positions (= gaussian ids) of the four visible gaussians


def _chunk_scene():
    """One 16x16 tile (fewer than 400 tiles: chunk mode) holding 1025
    entries, so three chunks of 512, 512 and 1.  Only the entries at positions
    0, 1 (chunk 0), 512 (chunk 1) and 1024 (chunk 2) are visible; the rest are
    transparent (alpha < 1/255 at every pixel).  Near the centre the two
    nearly opaque gaussians of chunk 0 take the chunk's own T below 1e-4, so
    the second is not composited (a chunk-local stop the monolithic forward
    would turn into the pixel's end), and chunk 1 takes the merged T below
    1e-4, cutting off chunk 2."""
    n = 1025
    xy = np.tile(np.array([[8.0, 8.0]]), (n, 1))
    conic = np.tile(np.array([[0.05, 0.0, 0.05]]), (n, 1))
    col = np.zeros((n, 3))
    logit = np.full(n, -10.0)
    xy[list(KEY)] = [[7.6, 8.3], [8.4, 7.7], [8.1, 8.6], [7.9, 7.5]]
    conic[list(KEY)] = [[0.0015, 0.0002, 0.0018], [0.0017, -0.0002, 0.0015], [0.020, 0.0, 0.022],
                        [0.020, 0.002, 0.025]]
    # chunk 2's gaussian is bright (colours are not clamped before the
    # output), so that its contribution past the cutoff is well above rounding
    col[list(KEY)] = [[0.1, -0.2, 0.25], [0.3, 0.2, -0.1], [-0.2, 0.1, 0.2], [2.5, 2.4, 2.6]]
    # opacities 0.9985, 0.9985 (below the 0.999 cap), 0.99, 0.9
    logit[list(KEY)] = [6.5, 6.5, 4.6, 2.2]
    return xy, conic, col, logit


def _chunk_pixel(args, i, j, bg, decide=None, frozen_args=None):
    """float64 chunked forward of one pixel.  With decide=None returns the
    decisions (per chunk: index where the chunk stops or None; the merge
    cutoff); with decisions given, evaluates the backward's surrogate
    sum_k pT_k C_k + T_final bg, chunks past the cutoff taken from
    frozen_args.  Also returns the forward's (image, T_final, final index)."""
    xy, conic, col, logit = args
    n = xy.shape[0]
    K = (n + CHUNK - 1) // CHUNK
    stops, cT, cC, cidx = [], [], [], []
    for k in range(K):
        a = args if (decide is None or k < decide[1] or frozen_args is None) else frozen_args
        s, e = k * CHUNK, min((k + 1) * CHUNK, n)
        sig, au = _alpha64(a[0][s:e], a[1][s:e], a[3][s:e], j, i)
        ok = _valid(sig, au)
        T, C, last, stop = 1.0, np.zeros(3), s - 1, None
        for q in np.nonzero(ok)[0]:
            al = min(CAP, au[q])
            nT = T * (1 - al)
            forced = decide is not None and decide[0][k] == s + q
            if (decide is None and nT <= 1e-4) or forced:
                stop = s + q
                break
            C += np.maximum(a[2][s + q] + 0.5, 0) * al * T
            T = nT
            last = s + q
        stops.append(stop)
        cT.append(T)
        cC.append(C)
        cidx.append(last)
    Tr, Cr, li, cut = 1.0, np.zeros(3), -1, K
    for k in range(K):
        Cr = Cr + cC[k] * Tr
        Tr *= cT[k]
        li = cidx[k]
        if Tr <= 1e-4:
            cut = k + 1
            break
    fwd = (Cr + Tr * bg, Tr, li)
    if decide is None:
        return (stops, cut), fwd, cT
    pT, surr = 1.0, np.zeros(3)
    for k in range(K):
        surr = surr + pT * cC[k]
        pT *= cT[k]
    return surr + Tr * bg, fwd


def test_chunk_local_stop_merge_and_suffix():
    bg = np.array([0.3, 0.4, 0.5], F32)
    su, cam = _cam16(bg)
    xy, conic, col, logit = _chunk_scene()
    args = [a.astype(F32).astype(np.float64) for a in (xy, conic, col, logit)]
    bg64 = bg.astype(np.float64)
    rng = np.random.default_rng(24)
    v_out = rng.uniform(0.5, 1.5, size=(16, 16, 3))
    v64 = v_out.astype(F32).astype(np.float64)
    r = _run_oracle(cam, xy, conic, col, logit, v_out)
    decisions = {}
    n_stop = n_cut = 0
    for i in range(16):
        for j in range(16):
            d, (img, Tf, li), cT = _chunk_pixel(args, i, j, bg64)
            decisions[(i, j)] = d
            # the merge's cutoff decision keeps a margin wider than the steps
            assert abs(math.log(cT[0] * cT[1]) - math.log(1e-4)) > 1e-3, (i, j, cT)
            n_stop += d[0][0] is not None
            n_cut += d[1] < 3
            # forward: closed-form chunked compositing and merge
            np.testing.assert_allclose(r["out_img"][i, j], np.clip(img, 0, 1), atol=2e-6)
            assert abs(r["final_Ts"][i, j] - Tf) <= 2e-5 * Tf + 1e-10, (i, j, r["final_Ts"][i, j], Tf)
            assert r["final_index"][i, j] == li, (i, j, r["final_index"][i, j], li)
    assert n_stop >= 10 and n_cut >= 5 and n_cut < 256, (n_stop, n_cut)
    # at the centre chunk 0 stops before its second entry, yet chunk 1 still
    # composites: the final index is chunk 1's entry, not entry 0
    assert decisions[(8, 8)][0][0] == 1 and r["final_index"][8, 8] == 512
    # every stop and cutoff decision keeps a margin wider than the steps
    for (i, j), (stops, cut) in decisions.items():
        for k in range(3):
            s = k * CHUNK
            sig, au = _alpha64(args[0][s:s + 2], args[1][s:s + 2], args[3][s:s + 2], j, i)
            al = np.minimum(CAP, au)
            if k == 0:
                assert abs(math.log((1 - al[0]) * (1 - al[1])) - math.log(1e-4)) > 1e-3

    def total(a):
        t = 0.0
        for (i, j), d in decisions.items():
            surr, _ = _chunk_pixel(a, i, j, bg64, decide=d, frozen_args=args)
            t += float(np.dot(v64[i, j], surr))
        return t

    key = list(KEY)
    sub = {k: r[k][key] for k in ("v_xy", "v_conic", "v_rgb", "v_opacity")}
    fillers = np.setdiff1d(np.arange(1025), key)
    for k in ("v_xy", "v_conic", "v_rgb", "v_opacity"):
        assert (r[k][fillers] == 0).all()

    def f_key(a4):
        a = [x.copy() for x in args]
        for q in range(4):
            a[q][key] = a4[q]
        return total(a)

    _fd_check(sub, f_key, [x[key].copy() for x in args], 4, 2e-3)

    # The derivative of the forward's own image (suffix cut at the merge
    # cutoff) differs for the chunk-0 gaussians: the reference's suffix also
    # carries chunk 2's colour past the cutoff.
    def plain(a4):
        a = [x.copy() for x in args]
        for q in range(4):
            a[q][key] = a4[q]
        t = 0.0
        for (i, j), d in decisions.items():
            _, (img, _, _) = _chunk_pixel(a, i, j, bg64, decide=d, frozen_args=args)
            t += float(np.dot(v64[i, j], img))
        return t

    a4 = [x[key].copy() for x in args]
    worst = 0.0
    for q, name, steps, scale, abs_tol in ((0, "v_xy", 2, None, 2e-4), (1, "v_conic", 3, (1.0, 0.5, 1.0), 2e-2),
                                           (3, "v_opacity", 1, None, 1e-4)):
        for k in range(4):
            for d in range(steps):
                h = 1e-6 if q == 1 else 1e-4
                idx = (k, d) if q != 3 else (k,)
                up, dn = [x.copy() for x in a4], [x.copy() for x in a4]
                up[q][idx] += h
                dn[q][idx] -= h
                g = (plain(up) - plain(dn)) / (2 * h) * (scale[d] if scale else 1.0)
                o = sub[name][k, d] if q != 3 else sub[name][k]
                worst = max(worst, abs(o - g) / (2e-3 * abs(g) + abs_tol))
    # at least one component is several tolerances away from the plain derivative
    assert worst > 5, worst


# -------------------------------------------------------- sparse SH Adam -----

def test_sparse_sh_adam_leaves_culled_sh_untouched():
    sc = small_scene(n=400, width=64, height=48, seed_off=240)
    su = camera.prepare_cam(sc.cameras[0])
    c2w = np.asarray(sc.cameras[0].cam_to_world, np.float64)
    fwd = -c2w[:3, 2]
    # a quarter of the gaussians behind the camera: culled (radii 0)
    behind = np.arange(sc.n) % 4 == 0
    sc.means[behind] = (c2w[:3, 3] - 2.0 * fwd + 0.1 * sc.means[behind]).astype(F32)
    cam = orc.camera(su, 3, 3, orc.camera(su, 3, 3).background)
    gt = target_for(sc, (su.height, su.width))
    rng = np.random.default_rng(25)
    params = [np.ascontiguousarray(a, F32).copy() for a in sc.params()]
    m = [(rng.normal(size=a.shape) * 0.01).astype(F32) for a in params]
    v = [(np.abs(rng.normal(size=a.shape)) * 1e-4).astype(F32) for a in params]
    p0 = [a.copy() for a in params]
    m0 = [a.copy() for a in m]
    v0 = [a.copy() for a in v]
    z = [np.zeros(sc.n, F32) for _ in range(3)]
    _, o = orc.train_step(cam, params, m, v, orc.adam_hparams(LRS, 3), gt, 0.2, *z, want=("radii",))
    culled = o["radii"] == 0
    assert culled.sum() >= sc.n // 4 and (~culled).sum() > 100
    for g in (3, 4):   # f_dc, f_rest: sparse, bit-unchanged when culled
        for arr, ref in ((params, p0), (m, m0), (v, v0)):
            assert (arr[g][culled].view(np.uint32) == ref[g][culled].view(np.uint32)).all(), g
        assert (params[g][~culled] != p0[g][~culled]).any(axis=tuple(range(1, p0[g].ndim))).mean() > 0.9
    for g in (0, 1, 2, 5):   # dense groups: a zero gradient still moves them
        moved = (params[g][culled] != p0[g][culled]).reshape(int(culled.sum()), -1).any(axis=1)
        assert moved.all(), g
        np.testing.assert_array_equal(m[g][culled], (F32(0.9) * m0[g][culled]).astype(F32))


# ------------------------------------------------- EWA through the clamp -----

def test_ewa_backward_through_fov_clamp_is_unmasked():
    """Centres outside the 1.3 tan(fov) frustum (.metal:1351-1354): the
    forward evaluates the EWA Jacobian at the view position clamped to the
    frustum edge; the backward (.metal:1393-1407) differentiates J as if the
    clamped coordinate were free, with no zero through the clamp.  That is the
    exact derivative of the surrogate whose J is evaluated at t + D, D = (the
    clamped minus the raw view position) frozen at the base point.  Large
    gaussians just outside the frustum keep a footprint on the image, so they
    are not culled."""
    import ctypes
    from test_oracle_pins import _rot64
    cam_o = camera.pinhole(96, 64, 60.0, camera.look_at((0.3, -0.2, 4.0)))
    su = camera.prepare_cam(cam_o)
    cam = orc.camera(su, 0, 0)
    rng = np.random.default_rng(26)
    n = 16
    V = np.asarray(su.viewmat, np.float64)
    Rw, tw = V[:3, :3], V[:3, 3]
    limx, limy = 1.3 * 0.5 * su.width / su.fx, 1.3 * 0.5 * su.height / su.fy
    z = rng.uniform(2.5, 4.0, n)
    side = np.where(np.arange(n) % 2 == 0, 1.0, -1.0)
    ux = np.where(np.arange(n) % 4 < 2, side * rng.uniform(1.05, 1.15, n) * limx, rng.uniform(-0.5, 0.5, n) * limx)
    uy = np.where(np.arange(n) % 4 >= 2, side * rng.uniform(1.05, 1.15, n) * limy, rng.uniform(-0.5, 0.5, n) * limy)
    tcam = np.stack([ux * z, uy * z, z], 1)
    means = np.ascontiguousarray((Rw.T @ (tcam - tw).T).T, F32)
    scales = np.ascontiguousarray(rng.uniform(-0.9, -0.6, (n, 3)), F32)
    quats = rng.normal(size=(n, 4))
    quats = np.ascontiguousarray(quats / np.linalg.norm(quats, axis=1, keepdims=True), F32)
    p = orc.project(cam, means, scales, quats, np.zeros((n, 3), F32), np.zeros((n, 0), F32))
    assert (p["radii"] > 0).all(), p["radii"]
    v_xy = np.zeros((n, 2), F32)   # only the covariance path is under test
    v_conic = (rng.normal(size=(n, 3)) * 10).astype(F32)
    vm, vs, vq = np.zeros((n, 3), F32), np.zeros((n, 3), F32), np.zeros((n, 4), F32)
    orc.lib().orc_project_backward(ctypes.byref(cam), n, orc.P(means), orc.P(scales), orc.P(quats),
                                   orc.P(p["radii"]), orc.P(p["conics"]), orc.P(v_xy), orc.P(v_conic),
                                   orc.P(vm), orc.P(vs), orc.P(vq))

    def clamp_t(t):
        return np.array([t[2] * min(limx, max(-limx, t[0] / t[2])), t[2] * min(limy, max(-limy, t[1] / t[2])), t[2]])

    def conic_of(mean, ls, q, offset):
        """conic with J at (view position + offset); offset None: the clamped
        view position itself (the plain forward)."""
        t = Rw @ mean + tw
        tj = clamp_t(t) if offset is None else t + offset
        s = np.exp(ls)
        w, x, y, zq = q    # unnormalised, as the reference's rotation vjp
        R = np.array([[1 - 2 * (y * y + zq * zq), 2 * (x * y - w * zq), 2 * (x * zq + w * y)],
                      [2 * (x * y + w * zq), 1 - 2 * (x * x + zq * zq), 2 * (y * zq - w * x)],
                      [2 * (x * zq - w * y), 2 * (y * zq + w * x), 1 - 2 * (x * x + y * y)]])
        S3 = R @ np.diag(s * s) @ R.T
        tx, ty, tz = tj
        J = np.array([[su.fx / tz, 0, -su.fx * tx / tz ** 2], [0, su.fy / tz, -su.fy * ty / tz ** 2]])
        C = J @ Rw @ S3 @ Rw.T @ J.T + 0.3 * np.eye(2)
        det = C[0, 0] * C[1, 1] - C[0, 1] ** 2
        return np.array([C[1, 1] / det, -C[0, 1] / det, C[0, 0] / det])

    def loss(g, mean, ls, q, offset):
        con = conic_of(mean, ls, q, offset)
        va, vb, vc = (float(v) for v in v_conic[g])
        return va * con[0] + 2 * vb * con[1] + vc * con[2]

    far = 0
    for g in range(n):
        t0 = Rw @ means[g].astype(np.float64) + tw
        D = clamp_t(t0) - t0
        assert np.abs(D[:2]).max() > 1e-3 * t0[2]   # the clamp is active
        base = [means[g].astype(np.float64), scales[g].astype(np.float64), quats[g].astype(np.float64)]
        for which, out, h in ((0, vm, 1e-5), (1, vs, 1e-5), (2, vq, 1e-6)):
            for d in range(base[which].size):
                hi = [b.copy() for b in base]
                lo = [b.copy() for b in base]
                hi[which][d] += h
                lo[which][d] -= h
                fdv = (loss(g, *hi, D) - loss(g, *lo, D)) / (2 * h)
                got = float(out[g, d])
                tol = 3e-3 * abs(fdv) + 3e-4 * (np.abs(out[g]).max() + 1e-3)
                assert abs(got - fdv) <= tol, (("mean", "scale", "quat")[which], g, d, got, fdv)
                if which == 0:
                    plain = (loss(g, *hi, None) - loss(g, *lo, None)) / (2 * h)
                    far += abs(got - plain) > 10 * tol
    # the derivative through the clamp (zero along the clamped axis) differs
    assert far >= n, far
