"""The bindings.h-shaped C++ shim (msplat_amd/host/bindings.hpp) on the GPU.

A C++ program compiled against bindings.hpp runs the call sequence of the
reference's Model::fullIteration (model.cpp:546-597): camera matrices and the
background in gpu_empty tensors written on the host through data<float>() (as
model.cpp writes its shared-storage buffers), then msplat_train_step's
MTensor overload.  Those small tensors are mapped host memory, so the step
reads them without a copy or a stream wait.  The same steps through the
float-array overloads (this build's own Model) give the same losses: the
first bit for bit, the later ones within float-atomic rounding.
"""
from __future__ import annotations

import os
import shutil
import subprocess

import numpy as np
import pytest

from helpers import BG, LRS, small_scene, target_for
from msplat_amd import camera

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROGRAM = r"""
#include "bindings.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

using namespace msplat;

static std::vector<float> rd(FILE* f, size_t n) {
    std::vector<float> v(n);
    if (std::fread(v.data(), 4, n, f) != n) { std::fprintf(stderr, "short read\n"); std::exit(3); }
    return v;
}

struct Cam { float vm[16], pm[16], fx, fy, cx, cy, pos[3]; int W, H; };

int main(int argc, char** argv) {
    FILE* f = std::fopen(argv[1], "rb");
    int hdr[4];
    if (std::fread(hdr, 4, 4, f) != 4) return 3;
    const int n = hdr[0], rest = hdr[1], W = hdr[2], H = hdr[3];
    std::vector<float> host[6] = {rd(f, n * 3), rd(f, n * 3), rd(f, n * 4), rd(f, n * 3), rd(f, (size_t)n * rest * 3),
                                  rd(f, n)};
    std::vector<float> gt_h = rd(f, (size_t)H * W * 3), bg_h = rd(f, 3), lrs = rd(f, 6);
    Cam cams[2];
    for (Cam& c : cams) {
        std::vector<float> v = rd(f, 39);
        std::memcpy(c.vm, v.data(), 64);
        std::memcpy(c.pm, v.data() + 16, 64);
        c.fx = v[32]; c.fy = v[33]; c.cx = v[34]; c.cy = v[35];
        std::memcpy(c.pos, v.data() + 36, 12);
        c.W = W; c.H = H;
    }
    std::fclose(f);
    check(msplat_hip_init(0), "init");
    const int64_t shapes[6][3] = {{n, 3, 0}, {n, 3, 0}, {n, 4, 0}, {n, 3, 0}, {n, rest, 3}, {n, 1, 0}};
    float losses[2][4];
    for (int path = 0; path < 2; ++path) {
        MTensor p[6], m[6], v[6];
        for (int g = 0; g < 6; ++g) {
            std::vector<int64_t> s = {shapes[g][0], shapes[g][1]};
            if (shapes[g][2]) s.push_back(shapes[g][2]);
            p[g] = gpu_empty(s, DType::Float32);
            p[g].copy_from_host(host[g].data(), host[g].size() * 4);
            m[g] = gpu_zeros(s, DType::Float32);
            v[g] = gpu_zeros(s, DType::Float32);
        }
        MTensor gt = gpu_empty({H, W, 3}, DType::Float32);
        gt.copy_from_host(gt_h.data(), gt_h.size() * 4);
        MTensor vis = gpu_zeros({n}, DType::Float32), gn = gpu_zeros({n}, DType::Float32),
                mx = gpu_zeros({n}, DType::Float32);
        // camera matrices and background: written on the host, as model.cpp does
        MTensor viewmat = gpu_empty({4, 4}, DType::Float32), projmat = gpu_empty({4, 4}, DType::Float32),
                background = gpu_empty({3}, DType::Float32), window2d;
        if (!viewmat.mapped() || !background.mapped() || p[0].mapped()) {
            std::fprintf(stderr, "small tensors must be mapped, parameters device-resident\n");
            return 4;
        }
        std::memcpy(background.data<float>(), bg_h.data(), 12);
        for (int step = 1; step <= 4; ++step) {
            const Cam& c = cams[(step - 1) % 2];
            std::memcpy(viewmat.data<float>(), c.vm, 64);
            std::memcpy(projmat.data<float>(), c.pm, 64);
            const float bc1 = 1.0f - std::pow(0.9f, (float)step), bc2 = 1.0f - std::pow(0.999f, (float)step);
            float ss[6], bc[6];
            for (int g = 0; g < 6; ++g) { ss[g] = lrs[g] / bc1; bc[g] = std::sqrt(bc2); }
            const auto tb = std::make_tuple((W + 15) / 16, (H + 15) / 16, 1);
            const float inv_n = 1.0f / (float)(H * W * 3), inv_md = 1.0f / (float)std::max(H, W);
            float pos[3] = {c.pos[0], c.pos[1], c.pos[2]};
            if (path == 0) {
                msplat_train_step(n, p[0], p[1], 1.0f, p[2], viewmat, projmat, c.fx, c.fy, c.cx, c.cy, H, W, tb,
                                  0.01f, 3, 3, pos, p[3], p[4], p[5], background, gt, window2d, 0.2f, inv_n, rest,
                                  6, p, m, v, ss, bc, 0.9f, 0.999f, 1e-8f, vis, gn, mx, inv_md);
            } else {
                msplat_train_step(n, p[0], p[1], 1.0f, p[2], c.vm, c.pm, c.fx, c.fy, c.cx, c.cy, H, W, tb, 0.01f,
                                  3, 3, c.pos, p[3], p[4], p[5], bg_h.data(), gt, 0.2f, inv_n, rest, 6, p, m, v,
                                  ss, bc, 0.9f, 0.999f, 1e-8f, vis, gn, mx, inv_md);
            }
            float l = 0.f;
            check(msplat_hip_last_loss(&l, 1), "loss");
            losses[path][step - 1] = l;
        }
    }
    for (int k = 0; k < 4; ++k) std::printf("%.9g %.9g\n", losses[0][k], losses[1][k]);
    cleanup_msplat();
    return 0;
}
"""


def test_reference_shaped_train_steps(tmp_path):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    cxx = shutil.which("g++")
    if not cxx:
        pytest.skip("no host C++ compiler")
    lib_dir = os.path.join(ROOT, "msplat_amd")
    src = tmp_path / "prog.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "prog"
    subprocess.check_call([cxx, "-std=c++17", "-O1", "-I", os.path.join(lib_dir, "host"), "-I",
                           os.path.join(ROOT, "include"), str(src), "-L", lib_dir, "-lmsplat_hip",
                           f"-Wl,-rpath,{lib_dir}", "-o", str(exe)])
    sc = small_scene(n=3000, seed_off=86)
    sc.cameras.append(camera.pinhole(sc.cameras[0].width, sc.cameras[0].height, 70.0,
                                     camera.look_at(np.array([4.0, 1.0, -2.5]))))
    sus = [camera.prepare_cam(c) for c in sc.cameras]
    H, W = sus[0].height, sus[0].width
    gt = target_for(sc, (H, W))
    params = [np.ascontiguousarray(a, np.float32) for a in sc.params()]
    rest = params[4].shape[1]
    with open(tmp_path / "scene.bin", "wb") as f:
        f.write(np.array([sc.n, rest, W, H], np.int32).tobytes())
        for a in params:
            f.write(a.tobytes())
        f.write(np.ascontiguousarray(gt, np.float32).tobytes())
        f.write(np.asarray(BG, np.float32).tobytes())
        f.write(np.asarray(LRS, np.float32).tobytes())
        for su in sus:
            f.write(np.concatenate([np.asarray(su.viewmat, np.float32).reshape(16),
                                    np.asarray(su.projmat, np.float32).reshape(16),
                                    np.array([su.fx, su.fy, su.cx, su.cy], np.float32),
                                    np.asarray(su.cam_pos, np.float32).reshape(3)]).tobytes())
    print("running the bindings.hpp program", flush=True)
    out = subprocess.run([str(exe), str(tmp_path / "scene.bin")], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    rows = [tuple(float(x) for x in line.split()) for line in out.stdout.strip().splitlines()]
    assert len(rows) == 4
    a, b = zip(*rows)
    assert all(np.isfinite(a)) and 0 < a[0] < 1
    assert a[0] == b[0], rows      # same inputs, bit-exact forward and loss
    assert a[1] != a[0]            # the second camera
    for x, y in zip(a[1:], b[1:]):
        assert abs(x - y) <= 1e-5 * abs(y), rows
