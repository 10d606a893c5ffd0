"""GPU parity at the full benchmark workloads (configurations 2-5).

Each test runs the HIP path through the C ABI on one configuration at its full
size and checks it against the CPU oracle (OpenMP over the host's threads) on
identical inputs, with the bars of tests/parity.py: projection, binning, sort
and raster forward bit for bit, gradients / Adam state within rel 1e-3 (D5),
densify bit for bit.  Gaussians of configs 2, 3 and 5 are drawn on the GPU by
the library's counter-based generator (as bench.py draws them) and copied to
the host for the oracle; config 4 is the numpy scene of synthetic.config4.
Targets are renders of the cloud with means jittered by N(0, 0.02) plus
N(0, 0.01) pixel noise, as in the benchmark.
"""
from __future__ import annotations

import numpy as np
import pytest

import parity
from helpers import BG
from msplat_amd import synthetic

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from msplat_amd import device
    device.init(0)
    return device


def _host(params):
    return [p.detach().cpu().numpy().astype(np.float32, copy=True) for p in params]


def _target(params, cam, seed):
    return synthetic.device_targets(params, [cam], 3, BG, seed)[0].cpu().numpy()


@pytest.mark.timeout(900)
def test_config2_train_step(dev):
    """Config 2: 500k SH3 gaussians, 1297x840 (82 x 53 tiles, partial last
    column and row), one full train step."""
    parity.say("config2: generating 500k gaussians on the GPU")
    params = synthetic.device_cloud(500_000, 3, synthetic.BASE_SEED + 2)
    cam = synthetic.config2_cameras()[0]
    gt = _target(params, cam, synthetic.BASE_SEED + 2)
    parity.train_compare(dev, _host(params), 3, cam, gt, label="config2")
    m = dev.meta()
    assert m["n_chunked_tiles"] == 0 and m["total_isect"] > 1_000_000


@pytest.mark.timeout(900)
def test_config3_train_step_and_densify(dev):
    """Config 3: the benchmark's 1.5M cloud and first camera, one full train
    step, then one densify of the resulting state with the config-3
    thresholds at a step of the refinement schedule before 3000 (grad 2e-4,
    size 0.01, split-screen 0.05 checked, cull opacity < 0.005, no huge-cull)."""
    n = 1_500_000
    parity.say("config3: generating 1.5M gaussians on the GPU")
    params = synthetic.device_cloud(n, 3, synthetic.BASE_SEED + 3)
    cam = synthetic.config3_cameras()[0]
    gt = synthetic.device_targets(params, synthetic.config3_cameras()[:1], 3, BG,
                                  synthetic.BASE_SEED + 3)[0].cpu().numpy()
    res = parity.train_compare(dev, _host(params), 3, cam, gt, capacity=3 * n, label="config3")
    del params
    rnd = synthetic.device_randn(2 * n * 3, synthetic.BASE_SEED + 300)
    nn, n_split, n_dup, culled = parity.densify_compare(dev, res.g, rnd, half_max_dim=0.5 * 1297,
                                                        label="config3")
    # split parents are culled; the rest of the culls are opacity < 0.005
    assert n_split > 100 and n_dup > 10 and culled >= n_split, (n_split, n_dup, culled)
    assert nn > n


@pytest.mark.timeout(900)
def test_config3_densify_heavy(dev):
    """Densify of the 1.5M config-3 cloud with statistics that send about a
    third of the gaussians to split, a third to duplicate and a few percent
    to the opacity cull, so the compaction handles close to its 3N-row worst
    case; counts, order and values bit for bit."""
    import torch
    n = 1_500_000
    parity.say("config3 heavy densify: generating 1.5M gaussians on the GPU")
    params = synthetic.device_cloud(n, 3, synthetic.BASE_SEED + 3)
    g = dev.DeviceGaussians.from_tensors(params, 3, capacity=3 * n)
    del params
    st = synthetic.Stream(synthetic.BASE_SEED + 301)
    vis = np.floor(st.uniform(n) * 4).astype(np.float32)
    gnorm = (st.uniform(n) * 2e-3 * vis).astype(np.float32)
    max2d = (st.uniform(n) * 0.1).astype(np.float32)
    g.vis[:n].copy_(torch.from_numpy(vis))
    g.gnorm[:n].copy_(torch.from_numpy(gnorm))
    g.max2d[:n].copy_(torch.from_numpy(max2d))
    # a third of the gaussians large (max scale > 0.01), the rest small (of
    # which the half with max2d > 0.05 split by screen size), 4% nearly
    # transparent: about 750k splits, 375k duplicates, 810k culls
    big = torch.from_numpy(st.uniform(n) < 1.0 / 3.0).cuda()
    g.bufs[1][:n] += torch.where(big, 1.5, -1.5).unsqueeze(1)
    faint = torch.from_numpy(st.uniform(n) < 0.04).cuda()
    g.bufs[5][:n][faint] = -6.0
    for i in range(6):
        g.m[i][:n].copy_(synthetic.device_randn(g.m[i][:n].numel(), 310 + i, 0.0, 0.01).view_as(g.m[i][:n]))
        g.v[i][:n].copy_(synthetic.device_randn(g.v[i][:n].numel(), 320 + i, 0.0, 0.01).abs_().view_as(g.v[i][:n]))
    rnd = synthetic.device_randn(2 * n * 3, synthetic.BASE_SEED + 302)
    nn, n_split, n_dup, culled = parity.densify_compare(dev, g, rnd, half_max_dim=0.5 * 1297,
                                                        label="config3 heavy")
    assert n_split > 200_000 and n_dup > 200_000 and culled > n_split + 20_000, (n_split, n_dup, culled)


@pytest.mark.timeout(900)
def test_config4_heavy_tile_train_step(dev):
    """Config 4: 1M SH3 gaussians, 70% in a tight blob 1.5 units ahead of the
    camera, 2594x1680; tiles of more than 10k entries take the chunked
    forward, merge and prefix / suffix backward."""
    parity.say("config4: generating the scene (numpy)")
    sc = synthetic.config4()
    params = [dev.to_dev(a) for a in sc.params()]
    gt = _target(params, sc.cameras[0], synthetic.BASE_SEED + 4)
    del params
    parity.train_compare(dev, sc.params(), 3, sc.cameras[0], gt, label="config4")
    m = dev.meta()
    assert m["max_count"] > 10_000 and m["n_chunked_tiles"] > 0, m


@pytest.mark.timeout(900)
def test_config5_render(dev):
    """Config 5: one render of 6M SH3 gaussians at 4946x3286 (the first of
    the benchmark's 100 poses)."""
    parity.say("config5: generating 6M gaussians on the GPU")
    params = synthetic.device_cloud(6_000_000, 3, synthetic.BASE_SEED + 5)
    host = _host(params)
    del params
    meta, counts = parity.render_and_compare(dev, host, 3, synthetic.config5_cameras()[0], label="config5")
    assert meta["total_isect"] == int(counts.sum()) > 50_000_000
