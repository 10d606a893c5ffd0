"""Benchmark of the splatting hot path on one MI355X.

Workload (BASELINE.json metric "train iters/sec + render FPS, 1.5M Gaussians
SH3 @1297x840, 1xMI355X"; configuration 3): 1.5M SH-degree-3 gaussians with
config-2 distributions, 1297x840, 32 seeded cameras on a radius 4..6 shell
cycled in order, full train step (forward + SSIM/L1 + backward + Adam) with
GPU densification by the reference's afterTrain policy every 100 steps
(grad 2e-4, size 0.01, split-screen 0.05, cull opacity < 0.005).  Targets are
renders of the cloud with means jittered by N(0, 0.02) plus N(0, 0.01) pixel
noise.  All inputs are synthetic and resident in HBM before timing starts.

value = train iterations / s over the timed steps; render_fps = renders / s
over `--frames` poses.  Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "train iters/sec + render FPS, 1.5M Gaussians SH3 @1297×840, 1×MI355X"
HBM_PEAK = 8.0e12
FP32_PEAK = 157.3e12


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def config3_cameras(n_cams=32, width=1297, height=840):
    from msplat_amd import camera, synthetic
    st = synthetic.Stream(synthetic.BASE_SEED + 3 + 1000)
    dirs = synthetic._sphere_dirs(st, n_cams)
    radii = 4.0 + 2.0 * st.uniform(n_cams)
    return [camera.pinhole(width, height, 70.0, camera.look_at(r * d)) for r, d in zip(radii, dirs)]


def make_targets(params, cams, degree, bg):
    """Render of the cloud with means jittered by N(0,0.02) plus N(0,0.01) pixel noise."""
    from msplat_amd import camera, device, synthetic
    seed = synthetic.BASE_SEED + 3
    jit = [p for p in params]
    jit[0] = params[0] + synthetic.device_randn(params[0].numel(), seed * 7 + 11, 0.0, 0.02).view_as(params[0])
    g = device.DeviceGaussians.from_tensors(jit, degree)
    out = []
    for i, c in enumerate(cams):
        s = camera.prepare_cam(c)
        img = device.render(g, s, degree, bg).clone()
        img += synthetic.device_randn(img.numel(), seed * 13 + i, 0.0, 0.01).view_as(img)
        out.append(img)
    del g
    return out


def stage_times(lib):
    import ctypes
    from msplat_amd import _abi
    ms = (ctypes.c_double * 16)()
    cnt = (ctypes.c_int64 * 16)()
    names = (ctypes.c_char_p * 16)()
    n = ctypes.c_int(0)
    calls = ctypes.c_int64(0)
    _abi.check(lib.msplat_hip_drain_stage_times(ms, cnt, names, 16, ctypes.byref(n), ctypes.byref(calls)))
    return {names[i].decode(): (ms[i], cnt[i]) for i in range(n.value)}, calls.value


def cpu_baseline(params_dev, cams, targets, degree, bg, n_steps):
    """The CPU oracle (oracle/liboracle.so, OpenMP) on a bounded sample of the
    same workload: n_steps full train steps at the full 1.5M / 1297x840 size."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import orc
    from msplat_amd import camera
    params = [p.detach().cpu().numpy().astype(np.float32).copy() for p in params_dev]
    m = [np.zeros_like(a) for a in params]
    v = [np.zeros_like(a) for a in params]
    n = params[0].shape[0]
    z = [np.zeros(n, np.float32) for _ in range(3)]
    lrs = [0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05]
    t0 = time.perf_counter()
    for s in range(n_steps):
        su = camera.prepare_cam(cams[s % len(cams)])
        cam = orc.camera(su, degree, degree, bg)
        gt = targets[s % len(cams)].cpu().numpy()
        orc.train_step(cam, params, m, v, orc.adam_hparams(lrs, s + 1), gt, 0.2, *z)
    dt = time.perf_counter() - t0
    return n_steps / dt, int(orc.lib().orc_num_threads()), dt


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--frames", type=int, default=200)
    ap.add_argument("--n", type=int, default=1_500_000)
    ap.add_argument("--cpu-steps", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); "
              "this build has no multi-GPU path.", file=sys.stderr)
        sys.exit(2)

    import torch
    from msplat_amd import camera, device, synthetic
    from msplat_amd.trainer import GaussianTrainer, TrainingConfig

    lib = device.init(0)
    bg = np.array([0.6130, 0.0101, 0.3984], np.float32)
    degree = 3
    t = time.perf_counter()
    params = device_params = synthetic.device_cloud(args.n, degree, synthetic.BASE_SEED + 3)
    cams = config3_cameras()
    targets = make_targets(params, cams, degree, bg)
    torch.cuda.synchronize()
    log(f"setup: {args.n} gaussians, {len(cams)} cameras, targets ready in {time.perf_counter() - t:.1f}s")

    cfg = TrainingConfig(iterations=30000, sh_degree=degree, sh_degree_interval=0, num_downscales=0,
                         warmup_length=0, cull_alpha_thresh=0.005, shuffle_cameras=False)
    tr = GaussianTrainer(params, cams, targets, cfg)
    for _ in range(args.warmup):
        tr.step()
    device.sync()
    _abi = device._abi
    _abi.check(lib.msplat_hip_enable_stage_timing(1))
    n_start = tr.splat_count()
    device.sync()
    t0 = time.perf_counter()
    counts = []
    for _ in range(args.steps):
        st = tr.step()
        counts.append(st.splat_count)
    device.sync()
    t1 = time.perf_counter()
    stages, calls = stage_times(lib)
    train_s = t1 - t0
    its = args.steps / train_s
    log(f"train: {args.steps} steps in {train_s:.3f}s = {its:.1f} it/s; gaussians {n_start} -> {tr.splat_count()}")
    for k, (ms, c) in stages.items():
        if c:
            log(f"  {k:18s} {ms / c:8.3f} ms/call  ({c} calls, {100 * ms / (train_s * 1e3):5.1f}% of wall)")

    # render FPS over the 32 camera poses
    setups = [camera.prepare_cam(c) for c in cams]
    out = torch.empty((setups[0].height, setups[0].width, 3), dtype=torch.float32, device="cuda")
    g = tr.model.g
    for i in range(5):
        device.render(g, setups[i % len(setups)], degree, bg, out=out)
    _abi.check(lib.msplat_hip_enable_stage_timing(1))
    device.sync()
    r0 = time.perf_counter()
    for i in range(args.frames):
        device.render(g, setups[i % len(setups)], degree, bg, out=out)
    device.sync()
    r1 = time.perf_counter()
    rstages, _ = stage_times(lib)
    fps = args.frames / (r1 - r0)
    log(f"render: {args.frames} frames in {r1 - r0:.3f}s = {fps:.1f} FPS at N={tr.splat_count()}")
    for k, (ms, c) in rstages.items():
        if c:
            log(f"  {k:18s} {ms / c:8.3f} ms/call")

    cpu = None
    if not args.no_cpu and args.cpu_steps > 0:
        rate, cores, dt = cpu_baseline(device_params, cams, targets, degree, bg, args.cpu_steps)
        cpu = {"value": rate, "unit": "it/s", "cores": cores, "kind": "port",
               "sample": f"{args.cpu_steps} full train steps of the same 1.5M SH3 1297x840 workload "
                         f"(initial parameters, cameras 0..{args.cpu_steps - 1}), {dt:.1f}s"}
        log(f"cpu baseline: {rate:.4f} it/s on {cores} threads")

    res = {
        "metric": METRIC, "value": its, "unit": "it/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": 1e3 * train_s / args.steps, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "config3: 1.5M SH3 gaussians, 1297x840, 32 cameras cycled, densify every 100 steps",
                   "gaussians_start": n_start, "gaussians_end": tr.splat_count(), "render_frames": args.frames},
        "render_fps": fps,
        "stage_ms": {k: ms / c for k, (ms, c) in stages.items() if c},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
