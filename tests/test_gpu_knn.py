"""Nearest-neighbour initial scales on the GPU (msplat_hip_knn_mean_dist) and
the initial gaussians of a COLMAP point cloud.

The GPU grid search must return, bit for bit, the brute-force oracle's mean
of sqrt over the 2nd..4th smallest squared distances (the reference's
nanoflann query, kdtree_tensor.hpp:26-40; the oracle itself is pinned
against scipy's cKDTree in tests/test_oracle_pins.py) on clouds that stress
the grid: gaussian blobs, exact duplicates, a plane, a line, isolated
outliers far outside the cluster, an offset far from the origin, and the
4-point minimum.  The dataset's initial gaussians follow Model::Model
(model.cpp:59-110): log of those distances, DC from colour, logit(0.1),
unit quaternions, zero higher bands.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import orc
from helpers import assert_bits_equal

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mods():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from msplat_amd import _abi, device
    device.init(0)
    return torch, device, _abi


def _clouds():
    rng = np.random.default_rng(7)
    blob = rng.normal(0, 1.0, (20000, 3))
    dup = rng.normal(0, 0.5, (3000, 3))
    dup[1000:1500] = dup[0:500]                    # exact duplicates
    plane = np.c_[rng.uniform(-3, 3, (5000, 2)), np.zeros(5000)]
    line = np.c_[np.linspace(0, 10, 2000), np.zeros((2000, 2))]
    outl = np.r_[rng.normal(0, 0.2, (4000, 3)), [[50, 0, 0], [0, -40, 3], [30, 30, 30]]]
    offset = rng.normal(1000.0, 0.01, (3000, 3))
    tiny = rng.normal(0, 1, (4, 3))
    clusters = np.r_[rng.normal(0, 0.01, (2000, 3)), rng.normal(5, 0.01, (2000, 3))]
    return {"blob": blob, "duplicates": dup, "plane": plane, "line": line, "outliers": outl,
            "offset": offset, "four": tiny, "two_clusters": clusters}


@pytest.mark.parametrize("name", list(_clouds().keys()))
def test_knn_matches_oracle(mods, name):
    torch, device, _abi = mods
    xyz = np.ascontiguousarray(_clouds()[name], np.float32)
    print(f"knn {name} n={len(xyz)}", flush=True)
    d_xyz = torch.from_numpy(xyz).cuda()
    out = torch.empty(len(xyz), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    _abi.check(device.init().msplat_hip_knn_mean_dist(device.ptr(d_xyz), len(xyz), device.ptr(out)))
    device.sync()
    assert_bits_equal(out.cpu().numpy(), orc.knn_mean_dist(xyz), f"knn {name}")


def test_knn_rejects_bad_input(mods):
    torch, device, _abi = mods
    lib = device.init()
    x = torch.zeros((3, 3), dtype=torch.float32, device="cuda")
    o = torch.empty(3, dtype=torch.float32, device="cuda")
    assert lib.msplat_hip_knn_mean_dist(device.ptr(x), 3, device.ptr(o)) == -1
    y = torch.zeros((5, 3), dtype=torch.float32, device="cuda")
    y[2, 1] = float("nan")
    torch.cuda.synchronize()
    assert lib.msplat_hip_knn_mean_dist(device.ptr(y), 5, device.ptr(o)) == -1


def test_dataset_initial_gaussians(mods, tmp_path):
    from test_dataset_cpu import _write_model
    from msplat_amd import dataset
    _write_model(str(tmp_path), n_points=3000, seed=3)
    ds = dataset.Dataset(str(tmp_path))
    xyz, rgb = ds.points()
    g = ds.init_gaussians(sh_degree=3)
    assert_bits_equal(g[0], xyz, "means")
    libm = ctypes.CDLL("libm.so.6")
    libm.logf.restype, libm.logf.argtypes = ctypes.c_float, [ctypes.c_float]
    want_s = np.array([libm.logf(float(v)) for v in orc.knn_mean_dist(xyz)], np.float32)
    assert_bits_equal(g[1], np.repeat(want_s[:, None], 3, axis=1), "log scales")
    assert np.allclose(np.linalg.norm(g[2], axis=1), 1.0, atol=1e-6)
    dc = ((rgb.astype(np.float64) / 255.0 - 0.5) / 0.28209479177387814).astype(np.float32)
    assert_bits_equal(g[3], dc, "f_dc")
    assert g[4].shape == (3000, 15, 3) and not g[4].any()
    assert (g[5] == np.float32(libm.logf(float(np.float32(0.1) / np.float32(0.9))))).all()
    again = ds.init_gaussians(sh_degree=3)
    for a, b in zip(g, again):
        assert_bits_equal(a, b, "deterministic")
