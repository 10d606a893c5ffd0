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
over `--frames` poses.  Inside the timed loops HIP events bracket only the
roofline kernel (raster backward in training, raster forward in rendering);
the per-stage times come from `--stage-steps` further steps / frames with
every stage bracketed.  Prints one JSON line.
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
# The CPU baseline's OpenMP threads stay on the cores they start on (read by
# the OpenMP runtime when it loads, so set before torch or the oracle loads).
os.environ.setdefault("OMP_PROC_BIND", "close")
# CPUs this process may use, read before an OpenMP runtime binds the main
# thread to one of them.
try:
    USABLE_CPUS = len(os.sched_getaffinity(0))
except AttributeError:
    USABLE_CPUS = os.cpu_count()

METRIC = "train iters/sec + render FPS, 1.5M Gaussians SH3 @1297×840, 1×MI355X"
HBM_PEAK = 8.0e12
FP32_PEAK = 157.3e12

# Algorithmic fp32 operations per (pixel, entry) pair of the reference's
# per-pixel raster loops (.metal:472-585 forward, 898-1099 backward), counted
# as add/sub/mul/min/max = 1, fma = 2, exp and reciprocal = 1 each:
#   every evaluated pair   d = xy - p (2), sigma = 0.5 (a dx^2 + c dy^2) +
#                          b dx dy (9), alpha = min(0.999, o exp(-sigma)) (3)
#   forward, composited    next_T, vis, three colour fmas (9)
#   backward, with grad    1/(1-a), T, fac, v_rgb, three clamped colour terms,
#                          v_alpha, buffer fmas, v_sigma, v_conic, v_xy,
#                          v_opacity (55) + the nine gradient sums (9)
# Only pairs that composite (forward) or carry a gradient (backward) are
# counted, as the rasteriser's own GPU counters report them; pairs that are
# tested and rejected add nothing, so the figure is a lower bound.
FWD_PAIR_FLOPS = 11 + 3 + 9
BWD_PAIR_FLOPS = 11 + 3 + 64
# Timed train steps whose raster backward is bracketed with HIP events (and
# counted): every third, a stride coprime with the 32 config-3 cameras.
BWD_SAMPLE = 3
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "raster_bwd_config3_traffic.json")
# Stage names in the order of the library's stage-timing bits: the
# reference profiler's train stages (msplat_metal.mm:30-34), ".part" where a
# stage runs as two kernels, and densify.
STAGES = ["proj_sh_fwd", "prefix_sort_pack.depth_sort", "prefix_sort_pack.tile_lists", "rast_fwd",
          "loss_fwd_bwd", "rast_bwd", "proj_sh_bwd_adam.sh_rest", "proj_sh_bwd_adam.dense", "densify"]
# The reference's eight train stages; blit_zero runs inside proj_sh_fwd here
# (the projection zeroes the gradient accumulators) and grad_stats inside
# proj_sh_bwd_adam.dense.
REFERENCE_STAGES = ["blit_zero", "proj_sh_fwd", "prefix_sort_pack", "rast_fwd", "loss_fwd_bwd", "rast_bwd",
                    "proj_sh_bwd_adam", "grad_stats"]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


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


def cpu_baseline(state, cams, targets, degree, bg, n_steps, first_step):
    """The CPU oracle (oracle/liboracle.so, OpenMP) on a bounded sample of the
    same workload: n_steps full train steps at the full size, from the
    trainer's state after the timed steps (parameters and Adam moments, host
    copies), with the cameras and Adam step numbers that come next.  Returns
    the rate, the thread count, the seconds and the mean wall milliseconds per
    step of each reference train stage (the oracle's rast_bwd recomputes each
    pixel's forward before its backward)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import ctypes
    import orc
    from msplat_amd import camera
    params, m, v = state
    n = params[0].shape[0]
    z = [np.zeros(n, np.float32) for _ in range(3)]
    lrs = [0.00016, 0.005, 0.001, 0.0025, 0.000125, 0.05]
    orc.lib().orc_stage_times((ctypes.c_double * 8)(), None)
    t0 = time.perf_counter()
    for s in range(n_steps):
        ci = (first_step - 1 + s) % len(cams)
        su = camera.prepare_cam(cams[ci])
        cam = orc.camera(su, degree, degree, bg)
        gt = targets[ci].cpu().numpy()
        orc.train_step(cam, params, m, v, orc.adam_hparams(lrs, first_step + s), gt, 0.2, *z)
    dt = time.perf_counter() - t0
    ms = (ctypes.c_double * 8)()
    steps = ctypes.c_int64(0)
    orc.lib().orc_stage_times(ms, ctypes.byref(steps))
    stage_ms = {name: ms[i] / max(steps.value, 1) for i, name in enumerate(REFERENCE_STAGES)}
    return n_steps / dt, int(orc.lib().orc_num_threads()), dt, stage_ms


def trainer_state(tr, degree):
    """Host copies of a trainer's parameters and Adam moments in the oracle's
    layouts (f_rest [N, K-1, 3], opacities [N, 1])."""
    nb = (degree + 1) ** 2 - 1
    out = []
    for which in range(3):
        gs = [tr.group(g, which) for g in range(6)]
        gs[4] = gs[4].reshape(gs[4].shape[0], nb, 3)
        gs[5] = gs[5].reshape(-1, 1)
        out.append([np.ascontiguousarray(a, np.float32) for a in gs])
    return out


def rocprof_summary(d: str, first: int, count: int, command: str) -> str:
    """Markdown summary of a `rocprofv3 --kernel-trace --stats -f csv` output
    directory: kernels by total time, and the raster backward's average
    duration over all its dispatches and over dispatches [first, first +
    count) (in a default run: after the warmup steps, the timed train
    steps)."""
    import csv
    import glob
    import re
    stats = glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)
    trace = glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
    if not stats or not trace:
        raise SystemExit(f"no kernel_stats / kernel_trace csv under {d}")

    short = _kernel_name

    rows = sorted(csv.DictReader(open(stats[0])), key=lambda r: -float(r["TotalDurationNs"]))
    out = [f"Command: `{command}`", "",
           "| kernel | calls | avg us | min us | max us | % time |", "|---|---:|---:|---:|---:|---:|"]
    for r in rows[:20]:
        out.append(f"| {short(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                   f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.2f} |")
    tr = [r for r in csv.DictReader(open(trace[0])) if "k_raster_bwd" in r["Kernel_Name"]]
    tr.sort(key=lambda r: int(r["Start_Timestamp"]))
    dur = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in tr]
    if dur:
        sel = dur[first:first + count] if count > 0 else dur
        out += ["", f"k_raster_bwd: {len(dur)} dispatches, average {sum(dur) / len(dur):.1f} us; "
                    f"dispatches {first}..{first + len(sel) - 1} (the timed steps) average "
                    f"{sum(sel) / max(len(sel), 1):.1f} us"]
    return "\n".join(out) + "\n"


def _kernel_name(full: str) -> str:
    """This library's kernel name in a profiler's kernel name, with its
    template arguments (k_radix_scatter<true>); other names up to '('."""
    import re
    m = re.search(r"(k_\w+(?:<[^>(]*>)?)", full)
    return m.group(1) if m else full.split("(")[0][:60]


def _kernel_match(want: str, full: str) -> bool:
    """A library kernel name (k_...) matches that kernel exactly, every
    template instance when given without arguments; anything else is a
    regular expression searched in the profiler's name."""
    import re
    if not want.startswith("k_"):
        return re.search(want, full) is not None
    name = _kernel_name(full)
    return name == want or ("<" not in want and name.split("<")[0] == want)


def _pmc_mean(d: str, kernel_re: str, counter: str, last: int) -> tuple:
    """Mean of one counter over the dispatches of the kernel kernel_re (as
    _kernel_match reads it; the last `last` dispatches when last > 0) in a
    `rocprofv3 --pmc -f csv` directory."""
    import csv
    import glob
    f = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not f:
        raise SystemExit(f"no counter_collection csv under {d}")
    rows = [r for r in csv.DictReader(open(f[0]))
            if _kernel_match(kernel_re, r["Kernel_Name"]) and r["Counter_Name"] == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    v = [float(r["Counter_Value"]) for r in rows]
    if last > 0:
        v = v[-last:]
    if not v:
        raise SystemExit(f"no {counter} samples for /{kernel_re}/ under {d}")
    return sum(v) / len(v), len(v)


def traffic_summary(dirs: list, copy_mib: int, last: int, commands: str,
                    kernel: str = "k_raster_bwd") -> dict:
    """HBM bytes per launch of `kernel` from FETCH_SIZE / WRITE_SIZE runs
    (KiB per dispatch), each scaled so that a plain device copy of copy_mib MiB
    reads and writes exactly copy_mib MiB."""
    fetch_dir, write_dir, copy_fetch_dir, copy_write_dir = dirs
    fk, nf = _pmc_mean(fetch_dir, kernel, "FETCH_SIZE", last)
    wk, nw = _pmc_mean(write_dir, kernel, "WRITE_SIZE", last)
    cf, _ = _pmc_mean(copy_fetch_dir, "copyBuffer", "FETCH_SIZE", 0)
    cw, _ = _pmc_mean(copy_write_dir, "copyBuffer", "WRITE_SIZE", 0)
    fs, ws = copy_mib * 1024 / cf, copy_mib * 1024 / cw
    return {"kernel": kernel, "dispatches": [nf, nw],
            "fetch_kib_per_dispatch": fk, "write_kib_per_dispatch": wk,
            "copy_fetch_kib": cf, "copy_write_kib": cw, "copy_mib": copy_mib,
            "fetch_scale": fs, "write_scale": ws,
            "hbm_bytes_per_launch": 1024 * (fk * fs + wk * ws), "commands": commands}


def pmc_summary(d: str, kernels: list, last: int, command: str) -> str:
    """Markdown table of every counter in a `rocprofv3 --pmc -f csv` output
    directory for each kernel whose name matches one of `kernels`, averaged
    per dispatch over its last `last` dispatches (all when last <= 0)."""
    import csv
    import glob
    import re
    f = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not f:
        raise SystemExit(f"no counter_collection csv under {d}")
    rows = list(csv.DictReader(open(f[0])))
    names = sorted({r["Counter_Name"] for r in rows})
    out = [f"Command: `{command}`", "", "| kernel | dispatches | " + " | ".join(names) + " |",
           "|---|---:|" + "---:|" * len(names)]
    for k in kernels:
        vals = {}
        n = 0
        for c in names:
            rs = [r for r in rows if _kernel_match(k, r["Kernel_Name"]) and r["Counter_Name"] == c]
            rs.sort(key=lambda r: int(r["Dispatch_Id"]))
            v = [float(r["Counter_Value"]) for r in rs]
            if last > 0:
                v = v[-last:]
            if v:
                vals[c] = sum(v) / len(v)
                n = max(n, len(v))
        if vals:
            out.append(f"| {k} | {n} | " + " | ".join(f"{vals.get(c, float('nan')):.4g}" for c in names) + " |")
    return "\n".join(out) + "\n"


def _stage_line(stages):
    return {k: ms / c for k, (ms, c) in stages.items() if c}


def _reference_stages(parts: dict) -> dict:
    """Per-call milliseconds under the reference's stage names: the parts of a
    stage summed; the fused blit_zero and grad_stats are 0."""
    out = {}
    for name in REFERENCE_STAGES:
        tot = sum(v for k, v in parts.items() if k == name or k.startswith(name + "."))
        if tot or name in ("blit_zero", "grad_stats"):
            out[name] = tot
    return out


def cpu_description() -> dict:
    """Host CPU model, logical CPUs usable by this process and the OpenMP
    thread binding, for the CPU baseline."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "cpus_usable": USABLE_CPUS, "binding": os.environ.get("OMP_PROC_BIND", "unset"),
            "places": os.environ.get("OMP_PLACES", "unset")}


def proj_bytes(n_vis, n_cul):
    """Algorithmic bytes of the projection: read means, log-scales, quats,
    f_dc, f_rest (45), opacity = 236 B; write the 64-byte record, radii,
    tiles hit, depth key / value and the zeroed 36-byte gradient accumulator
    = 116 B (culled: 12 B read, 52 B written)."""
    return n_vis * (236 + 116) + n_cul * (12 + 52)


def bench_config4(args):
    """Config 4, heavy-tile stress: 1M SH3 gaussians (70% in a N(0, 0.05^2)
    blob 1.5 units in front of the camera, 30% U[-4,4]^3), 2594x1680, full
    train steps (forward + SSIM/L1 + backward + Adam) on one camera, target =
    render of the means jittered by N(0, 0.02) plus N(0, 0.01) pixel noise."""
    import torch
    from msplat_amd import camera, device, synthetic
    from msplat_amd.trainer import LR_INIT
    lib = device.init(0)
    bg = np.array([0.6130, 0.0101, 0.3984], np.float32)
    t = time.perf_counter()
    scene = synthetic.config4()
    params = [device.to_dev(a) for a in scene.params()]
    g = device.DeviceGaussians.from_tensors(params, 3)
    su = camera.prepare_cam(scene.cameras[0])
    seed = synthetic.BASE_SEED + 4
    jit = device.DeviceGaussians.from_tensors(params, 3)
    jit.bufs[0][: jit.n] += synthetic.device_randn(3 * jit.n, seed * 7 + 11, 0.0, 0.02).view(jit.n, 3)
    gt = device.render(jit, su, 3, bg).clone()
    gt += synthetic.device_randn(gt.numel(), seed * 13, 0.0, 0.01).view_as(gt)
    del jit
    torch.cuda.synchronize()
    m = device.meta()
    log(f"config4 setup {time.perf_counter() - t:.1f}s: {g.n} gaussians, {su.width}x{su.height}, "
        f"{m['total_isect']} intersections, largest tile {m['max_count']} entries, "
        f"{m['n_chunked_tiles']} chunked tiles, {m['n_items']} raster work items")
    for s in range(args.warmup):
        device.train_step(g, su, 3, bg, gt, 0.2, LR_INIT, s + 1, want_loss=False)
    device.sync()
    t0 = time.perf_counter()
    for s in range(args.steps):
        device.train_step(g, su, 3, bg, gt, 0.2, LR_INIT, args.warmup + s + 1, want_loss=False)
    device.sync()
    dt = time.perf_counter() - t0
    # per-stage breakdown over further steps, every stage bracketed by events
    n_staged = max(1, min(args.stage_steps, args.steps))
    _abi_check(lib.msplat_hip_set_stage_timing_mask(0xFFFFFFFF))
    _abi_check(lib.msplat_hip_enable_stage_timing(1))
    for s in range(n_staged):
        device.train_step(g, su, 3, bg, gt, 0.2, LR_INIT, args.warmup + args.steps + s + 1,
                          want_loss=False)
    device.sync()
    stages, _ = stage_times(lib)
    pairs = device.drain_raster_counters()
    _abi_check(lib.msplat_hip_enable_stage_timing(0))
    m = device.meta()
    its = args.steps / dt
    for k, v in _stage_line(stages).items():
        log(f"  {k:18s} {v:8.3f} ms/call")
    log(f"config4: {its:.1f} train it/s; largest tile {m['max_count']} entries")
    return {"metric": "train iters/sec, config 4 (1M heavy-tile blob SH3 @2594x1680), 1xMI355X",
            "value": its, "unit": "it/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": 1e3 * dt / args.steps, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "config4: 1M SH3, 70% blob 1.5 units ahead, 2594x1680, full train step",
                       "intersections": m["total_isect"], "largest_tile": m["max_count"],
                       "chunked_tiles": m["n_chunked_tiles"], "raster_items": m["n_items"]},
            "stage_ms": _stage_line(stages),
            "bwd_grad_pairs_per_step": pairs[1] / n_staged,
            "raster_per_step": {"fwd_composited": pairs[0] / n_staged, "bwd_with_grad": pairs[1] / n_staged,
                                "fwd_wave_steps": pairs[2] / n_staged, "bwd_wave_steps": pairs[3] / n_staged}}


def bench_config5(args):
    """Config 5, render only: 6M SH3 gaussians with config-2 distributions
    (generated on the GPU), 4946x3286, 100 poses on a radius-5 sphere; render
    FPS and the projection's HBM rate."""
    import torch
    from msplat_amd import camera, device, synthetic
    lib = device.init(0)
    bg = np.array([0.6130, 0.0101, 0.3984], np.float32)
    t = time.perf_counter()
    params = synthetic.device_cloud(6_000_000, 3, synthetic.BASE_SEED + 5)
    g = device.DeviceGaussians.from_tensors(params, 3)
    del params
    cams = synthetic.config5_cameras()
    setups = [camera.prepare_cam(c) for c in cams]
    out = torch.empty((setups[0].height, setups[0].width, 3), dtype=torch.float32, device="cuda")
    for i in range(3):
        device.render(g, setups[i], 3, bg, out)
    torch.cuda.synchronize()
    log(f"config5 setup {time.perf_counter() - t:.1f}s")
    vis = cul = 0
    isect = 0
    t0 = time.perf_counter()
    for i, su in enumerate(setups):
        device.render(g, su, 3, bg, out)
    device.sync()
    dt = time.perf_counter() - t0
    # per-stage breakdown over the same poses again, every stage bracketed
    _abi_check(lib.msplat_hip_set_stage_timing_mask(0xFFFFFFFF))
    _abi_check(lib.msplat_hip_enable_stage_timing(1))
    for su in setups:
        device.render(g, su, 3, bg, out)
    device.sync()
    stages, _ = stage_times(lib)
    _abi_check(lib.msplat_hip_enable_stage_timing(0))
    # visible counts per pose, outside the timed loop
    for su in setups[:10]:
        device.render(g, su, 3, bg, out)
        radii = device.intermediate("radii", np.int32)
        vis += int((radii > 0).sum())
        cul += int((radii <= 0).sum())
        isect += device.meta()["total_isect"]
    vis, cul, isect = vis / 10, cul / 10, isect / 10
    fps = len(setups) / dt
    st = _stage_line(stages)
    pb = proj_bytes(vis, cul)
    hbm = {"proj_sh_fwd": {"ms": st["proj_sh_fwd"], "bytes": pb,
                           "GBps": pb / (st["proj_sh_fwd"] * 1e-3) / 1e9,
                           "frac": pb / (st["proj_sh_fwd"] * 1e-3) / HBM_PEAK}}
    for k, v in st.items():
        log(f"  {k:18s} {v:8.3f} ms/call")
    log(f"config5: {fps:.1f} render FPS; projection {hbm['proj_sh_fwd']['GBps']:.0f} GB/s")
    return {"metric": "render FPS, config 5 (6M SH3 @4946x3286, 100 poses), 1xMI355X",
            "value": fps, "unit": "FPS", "n_gpus": 1, "steps": len(setups), "warmup": 3,
            "ms_per_step": 1e3 * dt / len(setups), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "config5: 6M SH3, 4946x3286, 100 poses on a radius-5 sphere, render only",
                       "visible_gaussians_mean": vis, "intersections_mean": isect},
            "stage_ms": st, "hbm_stages": hbm}


def _abi_check(rc):
    from msplat_amd import _abi
    _abi.check(rc)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--frames", type=int, default=200)
    ap.add_argument("--preroll", type=int, default=200,
                    help="untimed train steps before --warmup: through the opacity reset (step 100) "
                         "and the first densification (step 200) of the refinement policy")
    ap.add_argument("--train-only", action="store_true",
                    help="stop after the timed train steps (counter runs: the timed steps are then "
                         "the last dispatches of every train kernel)")
    ap.add_argument("--stage-steps", type=int, default=60,
                    help="untimed steps / frames with every stage bracketed, for the per-stage breakdown")
    ap.add_argument("--n", type=int, default=1_500_000)
    ap.add_argument("--cpu-steps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the config-4 train window and the config-5 render window that the "
                         "default run times after the headline and reports as extra keys")
    ap.add_argument("--c4-steps", type=int, default=50, help="timed config-4 train steps of the default run")
    ap.add_argument("--config", type=int, default=3, choices=(3, 4, 5),
                    help="3 (default): the headline train + render workload; 4: heavy-tile train "
                         "steps at 2594x1680; 5: 6M-gaussian render at 4946x3286 (extra lines, "
                         "not the headline metric)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB five times (calibrates "
                         "the FETCH_SIZE / WRITE_SIZE counters against known traffic) and exit")
    ap.add_argument("--rocprof-summary", default="",
                    help="only print a markdown summary of this rocprofv3 csv output directory and exit")
    ap.add_argument("--rocprof-command", default="", help="command line quoted in the summary")
    ap.add_argument("--pmc-summary", default="",
                    help="only print a markdown table of the counters of this rocprofv3 --pmc csv output "
                         "directory for --pmc-kernels (last --steps dispatches of each) and exit")
    ap.add_argument("--pmc-kernels", default="k_raster_fwd;k_raster_bwd;k_radix_hist<256>;k_radix_hist<512>;"
                                             "k_radix_scatter<false, 256>;k_radix_scatter<false, 512>;"
                                             "k_radix_scatter<true, 256>;k_lists_and_items;"
                                             "k_ssim_tile;k_project_fwd;k_sh_rest_adam;"
                                             "k_proj_bwd_adam",
                    help="semicolon-separated kernels for --pmc-summary (template arguments hold commas)")
    ap.add_argument("--traffic-summary", nargs=4, default=None,
                    metavar=("FETCH_DIR", "WRITE_DIR", "COPY_FETCH_DIR", "COPY_WRITE_DIR"),
                    help="only print the HBM traffic JSON of the raster backward from four "
                         "rocprofv3 --pmc csv directories (the copy runs use --copy-mib) and exit")
    ap.add_argument("--traffic-kernels", default="k_raster_bwd",
                    help="semicolon-separated kernels for --traffic-summary (one: a flat JSON object)")
    args = ap.parse_args()
    if args.traffic_summary:
        kernels = args.traffic_kernels.split(";")
        res = {k: traffic_summary(args.traffic_summary, args.copy_mib or 1024, args.steps,
                                  args.rocprof_command, k) for k in kernels}
        print(json.dumps(res[kernels[0]] if len(kernels) == 1 else res, indent=1))
        return
    if args.pmc_summary:
        print(pmc_summary(args.pmc_summary, args.pmc_kernels.split(";"), args.steps, args.rocprof_command), end="")
        return
    if args.rocprof_summary:
        print(rocprof_summary(args.rocprof_summary, args.preroll + args.warmup, args.steps,
                              args.rocprof_command), end="")
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); "
              "this build has no multi-GPU path.", file=sys.stderr)
        sys.exit(2)
    if args.config in (4, 5):
        if args.config == 4 and args.steps == 300:
            args.steps = 50
        res = bench_config4(args) if args.config == 4 else bench_config5(args)
        print(json.dumps(res), flush=True)
        return
    if args.copy_mib > 0:
        import torch
        n = args.copy_mib * (1 << 20) // 4
        a = torch.ones(n, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"copied {args.copy_mib} MiB x5")
        return

    import torch
    from msplat_amd import camera, device, synthetic
    from msplat_amd.trainer import GaussianTrainer, TrainingConfig

    lib = device.init(0)
    bg = np.array([0.6130, 0.0101, 0.3984], np.float32)
    degree = 3
    t = time.perf_counter()
    params = synthetic.device_cloud(args.n, degree, synthetic.BASE_SEED + 3)
    cams = synthetic.config3_cameras()
    targets = synthetic.device_targets(params, cams, degree, bg, synthetic.BASE_SEED + 3)
    torch.cuda.synchronize()
    log(f"setup: {args.n} gaussians, {len(cams)} cameras, targets ready in {time.perf_counter() - t:.1f}s")

    cfg = TrainingConfig(iterations=30000, sh_degree=degree, sh_degree_interval=0, num_downscales=0,
                         warmup_length=0, cull_alpha_thresh=0.005, shuffle_cameras=False)
    tr = GaussianTrainer(params, cams, targets, cfg)
    _abi = device._abi
    # Pre-roll (untimed): through the opacity reset at step refine_every and
    # the first densification at 2 refine_every, so that the timed steps see
    # the post-reset cloud whatever --steps is.  Densification calls are
    # bracketed by HIP events from here on, so their cost is known even when
    # the timed window holds none.
    _abi.check(lib.msplat_hip_set_stage_timing_mask(1 << STAGES.index("densify")))
    _abi.check(lib.msplat_hip_enable_stage_timing(1))
    for _ in range(args.preroll):
        tr.step()
    device.sync()
    pre, _ = stage_times(lib)
    device.drain_raster_counters()
    pre_dens = pre["densify"]
    log(f"pre-roll: {args.preroll} steps, {pre_dens[1]} densification(s), gaussians {args.n} -> "
        f"{tr.splat_count()}")
    for _ in range(args.warmup):
        tr.step()
    device.sync()
    # The timed steps bracket densification calls and the raster backward (the
    # roofline kernel) of every BWD_SAMPLE-th step with HIP events: each event
    # leaves the GPU idle for about 4.5 us.  The stride is coprime with the 32
    # cameras, so the sampled launches visit every camera; the raster pair
    # counters run on exactly the sampled launches.
    mask_dens = 1 << STAGES.index("densify")
    mask_bwd = mask_dens | (1 << STAGES.index("rast_bwd"))
    _abi.check(lib.msplat_hip_set_stage_timing_mask(mask_dens))
    _abi.check(lib.msplat_hip_enable_stage_timing(1))
    n_start = tr.splat_count()
    first_step = args.preroll + args.warmup + 1
    device.sync()
    t0 = time.perf_counter()
    for i in range(args.steps):
        lib.msplat_hip_set_stage_timing_mask(mask_bwd if i % BWD_SAMPLE == 0 else mask_dens)
        tr.step()
    device.sync()
    t1 = time.perf_counter()
    timed, _ = stage_times(lib)
    train_pairs = device.drain_raster_counters()
    window_s = t1 - t0
    win_dens_ms, win_dens_n = timed["densify"]
    dens_n = pre_dens[1] + win_dens_n
    densify_ms = (pre_dens[0] + win_dens_ms) / dens_n if dens_n else 0.0
    # steady-state cost of a step: the timed steps without the densification
    # calls that fell inside them, plus one densification per refine_every steps
    step_ms_no_densify = (1e3 * window_s - win_dens_ms) / args.steps
    ms_per_step = step_ms_no_densify + densify_ms / cfg.refine_every
    its = 1e3 / ms_per_step
    cpu_state = None if args.no_cpu or args.cpu_steps <= 0 else trainer_state(tr, degree)
    log(f"train: steps {first_step}..{first_step + args.steps - 1} in {window_s:.3f}s "
        f"({args.steps / window_s:.1f} it/s wall, {win_dens_n} densification(s) inside); "
        f"{step_ms_no_densify:.3f} ms/step + densify {densify_ms:.2f} ms / {cfg.refine_every} "
        f"= {ms_per_step:.3f} ms/step = {its:.1f} it/s; gaussians {n_start} -> {tr.splat_count()}")
    if args.train_only:
        print(json.dumps({"metric": METRIC, "value": its, "unit": "it/s", "steps": args.steps,
                          "warmup": args.warmup, "preroll": args.preroll, "train_only": True}), flush=True)
        return
    # Per-stage breakdown: further steps with every stage bracketed.
    _abi.check(lib.msplat_hip_set_stage_timing_mask(0xFFFFFFFF))
    _abi.check(lib.msplat_hip_enable_stage_timing(1))
    for _ in range(args.stage_steps):
        tr.step()
    device.sync()
    stages, _ = stage_times(lib)
    device.drain_raster_counters()
    parts = _stage_line(stages)
    parts.pop("densify", None)
    ref_stages = _reference_stages(parts)
    step_ms = sum(parts.values())
    log(f"stage breakdown over {args.stage_steps} more steps (sum {step_ms:.3f} ms/step):")
    for k, v in parts.items():
        log(f"  {k:30s} {v:8.3f} ms/call  ({100 * v / step_ms:5.1f}% of stage sum)")

    # render FPS over the 32 camera poses (render_from_pose into a device buffer)
    out = torch.empty((cams[0].height, cams[0].width, 3), dtype=torch.float32, device="cuda")
    poses = [np.asarray(c.cam_to_world, np.float32) for c in cams]
    for i in range(5):
        tr.render_pose_device(poses[i % len(poses)], i % len(poses), out)
    # the FPS window runs with no events and no pair counters (neither is
    # part of a render); the render forward's kernel time and pairs come
    # from the bracketed frames after it
    _abi.check(lib.msplat_hip_enable_stage_timing(0))
    device.sync()
    r0 = time.perf_counter()
    for i in range(args.frames):
        tr.render_pose_device(poses[i % len(poses)], i % len(poses), out)
    device.sync()
    r1 = time.perf_counter()
    fps = args.frames / (r1 - r0)
    log(f"render: {args.frames} frames in {r1 - r0:.3f}s = {fps:.1f} FPS at N={tr.splat_count()}")
    _abi.check(lib.msplat_hip_set_stage_timing_mask(0xFFFFFFFF))
    _abi.check(lib.msplat_hip_enable_stage_timing(1))
    for i in range(args.stage_steps):
        tr.render_pose_device(poses[i % len(poses)], i % len(poses), out)
    device.sync()
    rstages, _ = stage_times(lib)
    render_pairs = device.drain_raster_counters()
    rtimed = rstages
    _abi.check(lib.msplat_hip_enable_stage_timing(0))
    rparts = _stage_line(rstages)
    for k, v in rparts.items():
        log(f"  {k:30s} {v:8.3f} ms/call")

    # Roofline of the dominant kernel (raster backward): algorithmic flops from
    # the GPU pair counters over exactly the timed launches, divided by those
    # launches' HIP-event durations on the context stream.
    bwd_ms, bwd_n = timed["rast_bwd"][0] / max(timed["rast_bwd"][1], 1), timed["rast_bwd"][1]
    bwd_flops = BWD_PAIR_FLOPS * train_pairs[1] / max(bwd_n, 1)
    achieved = bwd_flops / (bwd_ms * 1e-3)
    fwd_ms, fwd_n = rtimed["rast_fwd"][0] / max(rtimed["rast_fwd"][1], 1), rtimed["rast_fwd"][1]
    fwd_flops = FWD_PAIR_FLOPS * render_pairs[0] / max(fwd_n, 1)
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    roofline = {"bound": "mfma", "achieved": achieved / 1e12, "peak": FP32_PEAK / 1e12, "unit": "TFLOP/s",
                "frac": achieved / FP32_PEAK, "traffic": traffic,
                "kernel": "k_raster_bwd", "roof": "fp32 vector ALU (the kernel has no matrix-shaped work)",
                "launches": bwd_n, "launch_sample": f"1 in {BWD_SAMPLE} timed steps",
                "launch_ms": bwd_ms, "flops_per_launch": bwd_flops,
                "grad_pairs_per_launch": train_pairs[1] / max(bwd_n, 1),
                "lane_use": train_pairs[1] / max(64 * train_pairs[3], 1)}
    log(f"roofline k_raster_bwd: {bwd_flops / 1e9:.2f} GFLOP/launch ({train_pairs[1] / max(bwd_n, 1) / 1e6:.1f}M "
        f"gradient pairs) in {bwd_ms:.3f} ms = {achieved / 1e12:.2f} TFLOP/s ({100 * achieved / FP32_PEAK:.1f}% "
        f"of fp32 peak); render forward {fwd_flops / 1e9:.2f} GFLOP in {fwd_ms:.3f} ms = "
        f"{fwd_flops / fwd_ms / 1e9:.2f} TFLOP/s")
    log(f"  wave steps/launch: bwd {train_pairs[3] / max(bwd_n, 1) / 1e6:.2f}M (lanes with gradient "
        f"{100 * train_pairs[1] / max(64 * train_pairs[3], 1):.1f}%), render fwd "
        f"{render_pairs[2] / max(fwd_n, 1) / 1e6:.2f}M (lanes compositing "
        f"{100 * render_pairs[0] / max(64 * render_pairs[2], 1):.1f}%)")

    # HBM-bound stages: algorithmic bytes per launch (visible / culled
    # gaussians counted separately, from the last step's radii) over the
    # stages' HIP-event times.
    radii = device.intermediate("radii", np.int32)
    n_all = int(radii.size)
    n_vis = int((radii > 0).sum())
    n_cul = n_all - n_vis
    px = cams[0].width * cams[0].height
    algo_bytes = {
        "proj_sh_fwd": proj_bytes(n_vis, n_cul),
        # f_rest, its two moments read and written (1080 B), direction 16 B,
        # v_rgb 12 B, radii 4 B (culled: radii only)
        "proj_sh_bwd_adam.sh_rest": n_vis * (1080 + 16 + 12 + 4) + n_cul * 4,
        # dense Adam on means / scales / quats / opacity (11 floats x p, m, v
        # read + written = 264 B), f_dc Adam for visible (72 B), record 48 B,
        # gradient accumulator 36 B, radii 4 B, three statistics r + w 24 B
        "proj_sh_bwd_adam.dense": n_vis * (264 + 72 + 48 + 36 + 4 + 24) + n_cul * (264 + 4),
        # read render + target, write the loss gradient image: 36 B per pixel
        "loss_fwd_bwd": 36 * px,
    }
    hbm = {}
    for k, b in algo_bytes.items():
        ms = parts[k]
        hbm[k] = {"ms": ms, "bytes": b, "GBps": b / (ms * 1e-3) / 1e9, "frac": b / (ms * 1e-3) / HBM_PEAK}
        log(f"  {k:30s} {b / 1e6:8.1f} MB algorithmic in {ms:.3f} ms = {hbm[k]['GBps']:7.0f} GB/s "
            f"({100 * hbm[k]['frac']:.1f}% of HBM peak)")

    cpu = None
    if not args.no_cpu and args.cpu_steps > 0:
        nxt = first_step + args.steps
        rate, cores, dt, cpu_stage_ms = cpu_baseline(cpu_state, cams, targets, degree, bg, args.cpu_steps, nxt)
        cpu = {"value": rate, "unit": "it/s", "cores": cores, "kind": "port",
               "sample": f"{args.cpu_steps} full train steps of the same workload from the trainer's state "
                         f"after the timed steps ({cpu_state[0][0].shape[0]} gaussians, steps {nxt}.."
                         f"{nxt + args.cpu_steps - 1}), {dt:.1f}s",
               **cpu_description(), "stage_ms": cpu_stage_ms,
               "gpu_speedup_per_stage": {k: cpu_stage_ms[k] / ref_stages[k] for k in cpu_stage_ms
                                         if ref_stages.get(k)}}
        log(f"cpu baseline: {rate:.4f} it/s on {cores} threads ({cpu['cpu_model']}, "
            f"OMP_PROC_BIND={cpu['binding']})")

    # The other benchmark workloads on the same clock: a config-4 train
    # window (heavy tiles) and a config-5 render window (6M gaussians),
    # each on its own scene after the headline's state is released.
    extra = {}
    n_end = tr.splat_count()
    if not args.no_extra:
        del tr, params, targets, out, cpu_state
        import gc
        gc.collect()
        torch.cuda.empty_cache()
        c4 = bench_config4(argparse.Namespace(steps=args.c4_steps, warmup=10, stage_steps=20))
        torch.cuda.empty_cache()
        c5 = bench_config5(argparse.Namespace())
        torch.cuda.empty_cache()
        extra = {"config4_it_s": c4["value"], "config4_ms_per_step": c4["ms_per_step"],
                 "config4_steps": c4["steps"], "config4_workload": c4["config"],
                 "config4_stage_ms": c4["stage_ms"], "config4_raster_per_step": c4["raster_per_step"],
                 "config5_fps": c5["value"], "config5_ms_per_frame": c5["ms_per_step"],
                 "config5_frames": c5["steps"], "config5_workload": c5["config"],
                 "config5_stage_ms": c5["stage_ms"], "config5_hbm_stages": c5["hbm_stages"]}

    res = {
        "metric": METRIC, "value": its, "unit": "it/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "config3: 1.5M SH3 gaussians, 1297x840, 32 cameras cycled, densify every 100 "
                               "steps; timed after the opacity reset and the first densification",
                   "preroll_steps": args.preroll, "timed_steps": [first_step, first_step + args.steps - 1],
                   "gaussians_start": n_start, "gaussians_end": n_end, "render_frames": args.frames},
        "window_wall_it_s": args.steps / window_s,
        "step_ms_without_densify": step_ms_no_densify,
        "densify_ms": densify_ms, "densifies_measured": dens_n, "densifies_in_window": win_dens_n,
        "render_fps": fps,
        "stage_ms": ref_stages,
        "stage_parts_ms": parts,
        "render_stage_ms": _reference_stages(rparts),
        "rast_fwd_render_tflops": fwd_flops / fwd_ms / 1e9,
        "hbm_stages": hbm,
        "visible_gaussians": n_vis,
        "roofline": roofline,
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
