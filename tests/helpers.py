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
