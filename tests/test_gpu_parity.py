"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Forward stages (projection, tile counts / offsets / sorted id lists, raster
forward, SSIM and its input gradient) must be bit-exact; gradients and
Adam-updated parameters match to rel 1e-3 with an absolute floor (float
atomics sum in a different order than the oracle's fixed-order fp64 sums).
"""
from __future__ import annotations

import numpy as np
import pytest

import orc
import parity
from helpers import BG, LRS, assert_bits_equal, small_scene, target_for
from msplat_amd import camera, synthetic

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from msplat_amd import device
    device.init(0)
    return device


def _render_and_compare(dev, scene, dtu=None, cam_idx=0):
    return parity.render_and_compare(dev, scene.params(), scene.sh_degree, scene.cameras[cam_idx], dtu=dtu,
                                     label=scene.name)


def test_render_config1(dev):
    """Config 1 (10k SH0, 256x256, 256 tiles -> reference chunk mode)."""
    meta, counts = _render_and_compare(dev, synthetic.config1())
    assert meta["total_isect"] == int(counts.sum())


def test_render_sh3_small(dev):
    """Config-2 distributions at 4k gaussians, 160x112 (70 tiles, chunk mode)."""
    _render_and_compare(dev, small_scene())


def test_render_sh_degrees(dev):
    for deg, dtu in ((1, 1), (2, 1), (3, 2), (4, 4)):
        _render_and_compare(dev, small_scene(n=1500, degree=deg, seed_off=60 + deg), dtu=dtu)


def test_render_monolithic_tiles(dev):
    """>= 400 tiles: the monolithic kernel (reference selector, .mm:876),
    uncapped up to 8192 entries per tile."""
    meta, counts = _render_and_compare(dev, small_scene(n=20000, width=400, height=272, seed_off=70))
    assert meta["n_chunked_tiles"] == int((counts > 8192).sum())


def test_render_heavy_chunked_tiles(dev):
    """Dense scene in chunk mode: tiles of several 512-entry chunks + merge."""
    meta, counts = _render_and_compare(dev, small_scene(n=60000, width=128, height=96, seed_off=71, spread=0.6))
    assert counts.max() > 1024 and meta["n_chunked_tiles"] > 0


def test_render_large_and_huge_tiles(dev):
    """Tiles of more than 16384 entries (the reference caps tiles at 2048)."""
    sc = small_scene(n=40000, width=48, height=32, seed_off=72, spread=0.3, dist=6.0)
    meta, counts = _render_and_compare(dev, sc)
    assert counts.max() > 16384, counts.max()
    assert meta["max_count"] == int(counts.max())
    assert meta["n_chunked_tiles"] == int((counts > 512).sum())


def test_render_empty_and_culled(dev):
    """No gaussian in front of the camera: every pixel is background."""
    sc = small_scene(n=500, seed_off=73)
    su = camera.prepare_cam(sc.cameras[0])
    fwd = -np.asarray(sc.cameras[0].cam_to_world)[:3, 2]
    sc.means = (np.asarray(sc.cameras[0].cam_to_world)[:3, 3] - 3.0 * fwd + 0.01 * sc.means).astype(np.float32)
    g = dev.DeviceGaussians.from_arrays(sc.params(), 3)
    img = dev.render(g, su, 3, BG).cpu().numpy()
    assert dev.meta()["total_isect"] == 0
    assert np.all(img == np.clip(BG, 0, 1)[None, None, :])


def _train_compare(dev, scene, steps=1, dtu=None, check_grads=True):
    su = camera.prepare_cam(scene.cameras[0])
    gt = target_for(scene, (su.height, su.width))
    return parity.train_compare(dev, scene.params(), scene.sh_degree, scene.cameras[0], gt, steps=steps, dtu=dtu,
                                check_grads=check_grads, label=scene.name)


def test_train_step_small(dev):
    _train_compare(dev, small_scene(n=3000, seed_off=80))


def test_train_step_chunked(dev):
    """Chunk mode with multi-chunk tiles: prefix/suffix backward."""
    _train_compare(dev, small_scene(n=30000, width=96, height=64, seed_off=81, spread=0.6))


def test_train_step_deep_chunks_past_zero_transmittance(dev):
    """Tiles of more than 16 depth chunks (20k gaussians of scale about 1 in a
    64x64 image: 16 tiles of 18k-20k entries, all chunked).  Twelve tiles
    reach a running transmittance of exactly 0 at every pixel within their
    first 16 chunks, so their later chunks are not rasterised; the four
    corner tiles do not, and theirs are.  Image, T, final index, gradients
    and the Adam step still equal the oracle's, which rasterises every
    chunk."""
    sc = small_scene(n=20000, width=64, height=64, seed_off=86, spread=0.2)
    sc.scales = sc.scales + np.float32(4.5)      # log scales N(0, 0.5^2)
    _train_compare(dev, sc)
    tb = dev.intermediate("tile_bins", np.int32).reshape(-1, 2)
    counts = tb[:, 1] - tb[:, 0]
    assert (counts > 16 * 512).all(), counts
    done = dev.intermediate("tile_done", np.int32)[: counts.size]
    # both launches of the chunked forward ran: skipped and computed tails
    assert set(np.nonzero(done == 0)[0]) == {0, 3, 12, 15}, done


def _far_scene(seed_off):
    """A small scene whose first 400 gaussians sit at depths 700..3200 (five
    to twelve binades above the rest, 18 above the 0.01 clip), each about a
    pixel across; gaussians 400..439 repeat the positions of 0..39 (equal
    depths, ordered by id)."""
    sc = small_scene(n=3000, seed_off=seed_off)
    c2w = np.asarray(sc.cameras[0].cam_to_world, np.float64)
    pos, right, up, fwd = c2w[:3, 3], c2w[:3, 0], c2w[:3, 1], -c2w[:3, 2]
    st = synthetic.Stream(synthetic.BASE_SEED + seed_off + 1)
    k = 400
    far = st.uniform(k) * 2500.0 + 700.0
    lat = (st.uniform(2 * k).reshape(k, 2) - 0.5) * 0.8       # inside the 70 degree view
    pts = pos + far[:, None] * (fwd + lat[:, :1] * right + lat[:, 1:] * up)
    sc.means[:k] = pts.astype(np.float32)
    sc.scales[:k] = np.log(0.01 * far)[:, None].astype(np.float32) + np.zeros((1, 3), np.float32)
    sc.means[k:k + 40] = sc.means[:40]
    return sc


def test_render_far_depths_and_ties(dev):
    """Depths over 18 binades with ties: the depth order (all 32 key bits)
    and every forward stage bit-exact."""
    sc = _far_scene(74)
    _render_and_compare(dev, sc)
    far_vis = dev.intermediate("radii", np.int32)[:400] > 0
    assert far_vis.sum() > 100, far_vis.sum()


def test_render_zero_clip(dev):
    """clip_thresh 0: every gaussian in front of the camera is kept, however
    near; equal depths ordered by id."""
    sc = small_scene(n=3000, seed_off=76)
    sc.means[100:140] = sc.means[:40]
    parity.render_and_compare(dev, sc.params(), sc.sh_degree, sc.cameras[0], clip=0.0, label="clip 0")


def test_train_step_far_depths_and_ties(dev):
    """A train step over the far scene (depths over 18 binades, ties)."""
    _train_compare(dev, _far_scene(78))


def test_train_step_monolithic(dev):
    _train_compare(dev, small_scene(n=12000, width=336, height=208, seed_off=82))


def test_train_step_large_tiles_monolithic_and_chunked(dev):
    """>= 400 tiles (336x320, 420 tiles): tiles of 2049..8192 entries are
    rasterised in one piece, uncapped (the reference's monolithic kernel
    keeps at most 2048), and the tiles above 8192 in 512-entry chunks, in
    one train step."""
    _train_compare(dev, small_scene(n=80000, width=336, height=320, seed_off=91, spread=0.5))
    tb = dev.intermediate("tile_bins", np.int32).reshape(-1, 2)
    counts = tb[:, 1] - tb[:, 0]
    assert ((counts > 2048) & (counts <= 8192)).sum() > 10, counts.max()
    assert (counts > 8192).sum() > 0, counts.max()
    assert dev.meta()["n_chunked_tiles"] == int((counts > 8192).sum())


def test_render_partial_edge_tiles(dev):
    """167x93: W % 16, W % 32, H % 16 and H % 32 all nonzero, so the last tile
    column and row are partial (pixels outside the image in every wave of
    them, and quadrants with no pixel at all)."""
    _render_and_compare(dev, small_scene(n=5000, width=167, height=93, seed_off=90))


def test_train_step_partial_edge_tiles(dev):
    """Train step at 167x93: partial raster tiles in the forward and backward,
    and SSIM windows cut by the right and bottom image edges (rows and
    columns past the image contribute zero statistics, D14)."""
    _train_compare(dev, small_scene(n=5000, width=167, height=93, seed_off=91))


@pytest.mark.parametrize("width,height", [(7, 5), (13, 9), (43, 11), (33, 47)])
def test_train_step_tiny_odd_images(dev, width, height):
    """Train steps at images smaller than or just past one SSIM tile (32 x 32)
    and its window: odd widths, so that the horizontal sums' position pairs
    end half inside the image, heights that cut the vertical pass's row pairs,
    and a single raster tile; the loss gradient image must stay bit-exact."""
    _train_compare(dev, small_scene(n=300, width=width, height=height, seed_off=95 + width))


def test_train_step_partial_edge_tiles_chunked(dev):
    """Partial edge tiles in chunk mode (fewer than 400 tiles) with
    multi-chunk tiles: prefix / suffix backward at the image border."""
    _train_compare(dev, small_scene(n=30000, width=101, height=75, seed_off=92, spread=0.6))


def test_render_benchmark_resolution_small_cloud(dev):
    """The benchmark image size 1297x840 (82 x 53 tiles, partial last column
    and row) at 20k gaussians."""
    sc = small_scene(n=20000, width=1297, height=840, seed_off=93)
    _render_and_compare(dev, sc)


def test_raster_counters_match_work(dev):
    """The rasteriser's in-kernel pair counters (used for the roofline) equal
    the per-pixel work walk, which the train tests pin against the oracle."""
    torch = pytest.importorskip("torch")
    for sc in (small_scene(n=3000, seed_off=84), small_scene(n=30000, width=96, height=64, seed_off=85, spread=0.6)):
        su = camera.prepare_cam(sc.cameras[0])
        gt = dev.to_dev(target_for(sc, (su.height, su.width)))
        g = dev.DeviceGaussians.from_arrays(sc.params(), 3, capacity=sc.n)
        lib = dev.init()
        dev._abi.check(lib.msplat_hip_enable_stage_timing(1))
        try:
            dev.train_step(g, su, 3, BG, gt, 0.2, LRS, 1)
            counters = dev.drain_raster_counters()
            work = dev.raster_work()
        finally:
            dev._abi.check(lib.msplat_hip_enable_stage_timing(0))
        assert counters[:2] == (work["fwd_composited"], work["bwd_with_grad"]), (counters, work)
        assert counters[1] > 0 and 64 * counters[3] >= counters[1] and 64 * counters[2] >= counters[0]
        torch.cuda.synchronize()


def _drain_stages(dev):
    import ctypes
    lib = dev.init()
    ms = (ctypes.c_double * 16)()
    cnt = (ctypes.c_int64 * 16)()
    names = (ctypes.c_char_p * 16)()
    n, calls = ctypes.c_int(0), ctypes.c_int64(0)
    dev._abi.check(lib.msplat_hip_drain_stage_times(ms, cnt, names, 16, ctypes.byref(n), ctypes.byref(calls)))
    return {names[i].decode(): (ms[i], cnt[i]) for i in range(n.value)}


def test_stage_timing_mask(dev):
    """msplat_hip_set_stage_timing_mask: only the selected stages are timed
    (one bracketing pair of events each), all eight with the full mask; the
    step's results do not depend on what is timed."""
    sc = small_scene(n=3000, seed_off=86)
    su = camera.prepare_cam(sc.cameras[0])
    gt = dev.to_dev(target_for(sc, (su.height, su.width)))
    lib = dev.init()
    outs = []
    try:
        for mask in (1 << 5, 0xFFFFFFFF, (1 << 0) | (1 << 3) | (1 << 7)):
            g = dev.DeviceGaussians.from_arrays(sc.params(), 3, capacity=sc.n)
            dev._abi.check(lib.msplat_hip_set_stage_timing_mask(mask))
            dev._abi.check(lib.msplat_hip_enable_stage_timing(1))
            dev.train_step(g, su, 3, BG, gt, 0.2, LRS, 1)
            dev.train_step(g, su, 3, BG, gt, 0.2, LRS, 2)
            dev.sync()
            st = _drain_stages(dev)
            timed = {k for k, (ms, c) in st.items() if c}
            want = {k for i, k in enumerate(STAGE_NAMES) if (mask >> i) & 1}
            assert timed == want, (hex(mask), timed)
            assert all(st[k][1] == 2 and st[k][0] > 0 for k in want)
            outs.append([b[: sc.n].cpu().numpy().copy() for b in g.bufs])
    finally:
        dev._abi.check(lib.msplat_hip_set_stage_timing_mask(0xFFFFFFFF))
        dev._abi.check(lib.msplat_hip_enable_stage_timing(0))
        dev.drain_raster_counters()
    for o in outs[1:]:
        for x, y in zip(outs[0], o):
            assert np.allclose(x, y, rtol=1e-4, atol=1e-6)


# the eight stages of a train step, in the order of their timing-mask bits
# (bit 8, densify, brackets densification calls)
STAGE_NAMES = ["proj_sh_fwd", "prefix_sort_pack.depth_sort", "prefix_sort_pack.tile_lists", "rast_fwd",
               "loss_fwd_bwd", "rast_bwd", "proj_sh_bwd_adam.sh_rest", "proj_sh_bwd_adam.dense"]


def test_densify_stage_timing(dev):
    """A densification call is bracketed as the "densify" stage (timing bit
    8), one timed instance per call, and brackets nothing else."""
    torch = pytest.importorskip("torch")
    sc = small_scene(n=3000, seed_off=87)
    n = sc.n
    g = dev.DeviceGaussians.from_arrays(sc.params(), 3, capacity=3 * n)
    g.vis[:n].fill_(1.0)
    g.gnorm[:n].fill_(1e-3)
    lib = dev.init()
    try:
        dev._abi.check(lib.msplat_hip_set_stage_timing_mask(1 << 8))
        dev._abi.check(lib.msplat_hip_enable_stage_timing(1))
        nn = dev.densify(g, grad_thresh=2e-4, size_thresh=0.01, screen_thresh=0.05, check_screen=1,
                         cull_alpha=0.005, cull_scale=0.5, cull_screen=0.15, check_huge=0, half_max_dim=80.0,
                         seed=5)
        st = _drain_stages(dev)
    finally:
        dev._abi.check(lib.msplat_hip_set_stage_timing_mask(0xFFFFFFFF))
        dev._abi.check(lib.msplat_hip_enable_stage_timing(0))
    assert nn > n
    assert st["densify"][1] == 1 and st["densify"][0] > 0, st
    assert all(c == 0 for k, (ms, c) in st.items() if k != "densify"), st
    torch.cuda.synchronize()


def test_train_three_steps(dev):
    """Adam state carried over three steps (bias corrections t = 1, 2, 3):
    each step checked in full from the GPU's state before it (forward bit
    for bit, gradients and updates within their bounds)."""
    _train_compare(dev, small_scene(n=2000, seed_off=83), steps=3)


def test_unsynchronised_loss_reads(dev):
    """msplat_hip_last_loss without a wait returns the loss of the latest
    step known to have completed: after a train step whose loss was not
    requested, the previous step's (the step's own totals wait has passed
    it).  With zero learning rates the parameters stay as they are, so each
    step's loss depends only on its target; six targets give six losses, read
    once with a stream sync per step and once without any sync."""
    import ctypes
    sc = small_scene(n=3000, seed_off=80)
    su = camera.prepare_cam(sc.cameras[0])
    g = dev.DeviceGaussians.from_arrays(sc.params(), 3)
    tg = [dev.to_dev(target_for(sc, (su.height, su.width), seed_off=500 + k)) for k in range(6)]
    lr0 = [0.0] * 6
    synced = [dev.train_step(g, su, 3, BG, tg[k], 0.2, lr0, k + 1) for k in range(6)]
    assert len(set(synced)) == 6, synced
    lib = dev.init()
    got = []
    for k in range(6):
        dev.train_step(g, su, 3, BG, tg[k], 0.2, lr0, 7 + k, want_loss=False)
        v = ctypes.c_float(0.0)
        dev._abi.check(lib.msplat_hip_last_loss(ctypes.byref(v), 0))
        got.append(v.value)
    # the first read sees the last synced step's loss, then each the step before
    assert got == [synced[5]] + synced[:5], (got, synced)
    v = ctypes.c_float(0.0)
    dev._abi.check(lib.msplat_hip_last_loss(ctypes.byref(v), 1))
    assert v.value == synced[5]


def _misalign(t):
    """A copy of device tensor t whose data starts 4 bytes past a 16-byte
    boundary (one float into a larger allocation)."""
    import torch
    flat = torch.zeros(t.numel() + 1, dtype=t.dtype, device=t.device)
    out = flat[1:].view(t.shape)
    out.copy_(t)
    assert out.data_ptr() % 16 == 4
    return out


@pytest.mark.parametrize("misaligned", [False, True], ids=["aligned", "misaligned"])
def test_densify_parity(dev, misaligned):
    """Identical statistics and random samples -> identical densify result
    (counts, order, values).  The misaligned case puts every parameter and
    moment buffer 4 bytes off a 16-byte boundary, which takes the scalar
    copy-back path of the compaction instead of float4 stores."""
    torch = pytest.importorskip("torch")
    sc = small_scene(n=5000, seed_off=84)
    n = sc.n
    cap = 3 * n
    g = dev.DeviceGaussians.from_arrays(sc.params(), 3, capacity=cap)
    if misaligned:
        g.bufs = [_misalign(b) for b in g.bufs]
        g.m = [_misalign(b) for b in g.m]
        g.v = [_misalign(b) for b in g.v]
    st = synthetic.Stream(synthetic.BASE_SEED + 85)
    vis = np.floor(st.uniform(n) * 4).astype(np.float32)
    gnorm = (st.uniform(n) * 4e-3 * vis).astype(np.float32)
    max2d = (st.uniform(n) * 0.2).astype(np.float32)
    sc_logs = sc.scales.copy()
    sc_logs[: n // 3] += 1.5   # some large gaussians
    sc.scales = sc_logs
    g.bufs[1][:n].copy_(torch.from_numpy(sc_logs))
    m0 = [(st.uniform(b.numel()).reshape(tuple(b.shape)) * 0.1).astype(np.float32) for b in g.bufs]
    for i in range(6):
        g.m[i].copy_(torch.from_numpy(m0[i]))
        g.v[i].copy_(torch.from_numpy(m0[i] * 0.5))
    g.vis[:n].copy_(torch.from_numpy(vis))
    g.gnorm[:n].copy_(torch.from_numpy(gnorm))
    g.max2d[:n].copy_(torch.from_numpy(max2d))
    rnd = torch.empty(2 * n * 3, dtype=torch.float32, device="cuda")
    dev.init()
    from msplat_amd import _abi
    _abi.check(dev.init().msplat_hip_randn(dev.ptr(rnd), rnd.numel(), 1234))
    rnd_h = rnd.cpu().numpy()
    kw = dict(grad_thresh=2e-4, size_thresh=0.01, screen_thresh=0.05, check_screen=1, cull_alpha=0.005,
              cull_scale=0.5, cull_screen=0.15, check_huge=1, half_max_dim=0.5 * 160)
    # oracle
    bufs = [b.cpu().numpy().copy() for b in g.bufs]
    ms = [a.copy() for a in m0]
    vs = [(a * 0.5).astype(np.float32) for a in m0]
    oa = orc.OrcDensifyArgs()
    oa.N = n
    oa.grad_thresh, oa.size_thresh, oa.screen_thresh, oa.check_screen = 2e-4, 0.01, 0.05, 1
    oa.cull_alpha_thresh, oa.cull_scale_thresh, oa.cull_screen_size, oa.check_huge = 0.005, 0.5, 0.15, 1
    oa.half_max_dim, oa.fr_stride = 0.5 * 160, 45
    nn_o, split, dup, keep = orc.densify(oa, gnorm, vis, max2d, bufs, ms, vs, rnd_h)
    nn_g = dev.densify(g, random_samples=rnd, **kw)
    assert split.sum() > 0 and dup.sum() > 0 and (keep == 0).sum() > split.sum()
    assert nn_g == nn_o, (nn_g, nn_o)
    for i in range(6):
        assert_bits_equal(g.bufs[i][:nn_o].cpu().numpy(), bufs[i][:nn_o], f"densified param {i}")
        assert_bits_equal(g.m[i][:nn_o].cpu().numpy(), ms[i][:nn_o], f"densified exp_avg {i}")
        assert_bits_equal(g.v[i][:nn_o].cpu().numpy(), vs[i][:nn_o], f"densified exp_avg_sq {i}")


def test_randn_statistics(dev):
    torch = pytest.importorskip("torch")
    from msplat_amd import _abi
    x = torch.empty(1 << 20, dtype=torch.float32, device="cuda")
    _abi.check(dev.init().msplat_hip_randn(dev.ptr(x), x.numel(), 99))
    h = x.cpu().numpy().astype(np.float64)
    assert abs(h.mean()) < 5e-3 and abs(h.std() - 1.0) < 5e-3
    assert abs(((h > 1.0).mean()) - 0.158655) < 3e-3


def test_scratch_reuse_across_sizes(dev):
    """Regression: the sort / binning scratch is cleared by the kernels that
    use it (radix digit totals, tile run edges, intersection counters) rather
    than by memsets, so consecutive frames with fewer gaussians, fewer
    intersections and fewer tiles must still be bit-exact.  Renders a large
    scene, a much smaller one, then the large one again."""
    big = small_scene(n=6000, width=192, height=128, seed_off=820)
    little = small_scene(n=700, width=64, height=48, seed_off=821)
    m1, _ = _render_and_compare(dev, big)
    m2, _ = _render_and_compare(dev, little)
    m3, _ = _render_and_compare(dev, big)
    assert m2["total_isect"] < m1["total_isect"] == m3["total_isect"]
