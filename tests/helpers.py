"""Shared helpers for the parity tests: small scenes and comparison criteria."""
from __future__ import annotations

import numpy as np

from msplat_amd import camera, synthetic

BG = np.array([0.6130, 0.0101, 0.3984], np.float32)
LRS = [0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05]   # model.cpp:138


def small_scene(n=4000, width=160, height=112, degree=3, seed_off=50, dist=5.0, spread=1.5):
    """A config-2-like cloud at a reduced size (same distributions)."""
    st = synthetic.Stream(synthetic.BASE_SEED + seed_off)
    means = np.clip(st.normal(3 * n, 0.0, spread).reshape(n, 3), -4, 4)
    g = synthetic._gaussians(st, n, degree, means, 0.3, 0.05)
    d = st.normal(3).reshape(3)
    d /= np.linalg.norm(d)
    cam = camera.pinhole(width, height, 70.0, camera.look_at(dist * d))
    return synthetic.Scene(sh_degree=degree, cameras=[cam], name="small", **g)


def target_for(scene, setup_img_shape, seed_off=77):
    st = synthetic.Stream(synthetic.BASE_SEED + seed_off)
    H, W = setup_img_shape
    return st.uniform(H * W * 3).reshape(H, W, 3).astype(np.float32)


def assert_bits_equal(a, b, what):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, f"{what}: shape {a.shape} vs {b.shape}"
    if a.dtype.kind == "f":
        ne = a.view(np.uint32 if a.dtype == np.float32 else np.uint64) != b.view(
            np.uint32 if b.dtype == np.float32 else np.uint64)
    else:
        ne = a != b
    n = int(ne.sum())
    if n:
        idx = np.argwhere(ne)[:5]
        detail = ", ".join(f"{tuple(i)}: {a[tuple(i)]!r} vs {b[tuple(i)]!r}" for i in idx)
        raise AssertionError(f"{what}: {n} of {a.size} elements differ ({detail})")


U = 2.0 ** -24   # fp32 unit roundoff


def bound_check(gpu, orc, err, rel=1e-3, what="", log=None, mag=None, k=8.0, allow=1e-4) -> dict:
    """Two tiers of |gpu - orc| against the oracle.

    A (every element): |gpu - orc| <= rel |orc| + err, where err is the
    oracle's bound on the rounding difference of the two evaluations
    (running error analysis of the arithmetic both sides run:
    OrcTrainOut.err_raster / grad_err, orc_project_backward_err), absolute.
    Rounding cannot break it, and it binds at every element: the relative
    tolerance wherever rounding cannot reach it, the arithmetic's own bound
    where the element's terms cancel.
    B (with mag, the sum of the magnitudes of the terms the element is summed
    from): |gpu - orc| <= rel |orc| + k u mag for all but a share `allow` of
    the elements (those still pass A).  Measured rounding differences of the
    raster gradients stay below 4.3 u mag, so k = 8 is a tight, not a
    worst-case, bound.

    Returns and logs, over the elements where either side is nonzero:
      rel_decided  share whose relative term is the larger (tier B's when
                   mag is given, else tier A's);
      zero_pass    share that would still pass A if the GPU returned 0;
      max_used     largest |gpu - orc| / tier-A tolerance (< 1 passes);
      worst_rel    largest |gpu - orc| / |orc| over the rel-decided ones;
      b_exceed     share outside tier B."""
    a = np.asarray(gpu, np.float64).reshape(-1)
    b = np.asarray(orc, np.float64).reshape(-1)
    e = np.asarray(err, np.float64).reshape(-1)
    assert a.shape == b.shape == e.shape, f"{what}: shapes {a.shape} {b.shape} {e.shape}"
    d = np.abs(a - b)
    relt = rel * np.abs(b)
    tol = relt + e
    bad = d > tol
    nz = (a != 0) | (b != 0)
    st = {"n": int(nz.sum())}
    tight = e
    if mag is not None:
        mg = np.asarray(mag, np.float64).reshape(-1)
        assert mg.shape == a.shape, f"{what}: mag shape {mg.shape}"
        tight = k * U * mg
        st["b_exceed"] = float((nz & (d > relt + tight)).sum() / max(int(nz.sum()), 1))
    if nz.any():
        rd = nz & (relt >= tight)
        st.update(rel_decided=float(rd.sum() / nz.sum()),
                  zero_pass=float((nz & (np.abs(b) <= tol)).sum() / nz.sum()),
                  max_used=float(np.max(d[nz] / np.maximum(tol[nz], 1e-300))),
                  worst_rel=float(np.max(d[rd] / np.abs(b[rd]))) if rd.any() else 0.0)
    if log:
        tier = f"tier B (k={k:g}) " if mag is not None else ""
        extra = f", outside tier B {100 * st['b_exceed']:.4f}%" if mag is not None else ""
        log(f"{what}: {st['n']} nonzero, {tier}rel-decided {100 * st.get('rel_decided', 1):.2f}%, zero-pass "
            f"{100 * st.get('zero_pass', 0):.3f}%, max |d|/tol {st.get('max_used', 0):.3g}, worst rel err "
            f"(rel-decided) {st.get('worst_rel', 0):.3g}{extra}")
    n = int(bad.sum())
    if n:
        i = np.argwhere(bad).reshape(-1)[:5]
        detail = ", ".join(f"{j}: {a[j]:.8g} vs {b[j]:.8g} (tol {tol[j]:.3g})" for j in i)
        raise AssertionError(f"{what}: {n} of {a.size} outside rel {rel} + rounding bound ({detail})")
    if mag is not None and st["b_exceed"] > allow:
        nb = int(round(st["b_exceed"] * st["n"]))
        raise AssertionError(f"{what}: {nb} of {a.size} outside rel {rel} + {k:g} u sum|terms| "
                             f"(more than {allow:g} of the elements)")
    return st


def grad_close(a, b, rtol=1e-3, floor=1e-4, what=""):
    """|a - b| <= rtol |b| + floor * max|b| elementwise (D5: relative 1e-3 with an
    absolute floor scaled to the tensor's largest gradient)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, f"{what}: shape {a.shape} vs {b.shape}"
    scale = float(np.max(np.abs(b))) if b.size else 0.0
    tol = rtol * np.abs(b) + floor * scale
    bad = np.abs(a - b) > tol
    n = int(bad.sum())
    if n:
        i = np.argwhere(bad)[:5]
        detail = ", ".join(f"{tuple(j)}: {a[tuple(j)]:.6g} vs {b[tuple(j)]:.6g}" for j in i)
        raise AssertionError(f"{what}: {n} of {a.size} outside rtol={rtol} floor={floor}*{scale:.3g} ({detail})")
