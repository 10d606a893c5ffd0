"""The C ABI (include/msplat_hip.h, libmsplat_hip.so) without a GPU.

Checks that the library loads, exports every function the header declares,
that the ctypes mirror in msplat_amd/_abi.py has the header's struct layouts
(sizes and field offsets compiled from the header by the host C compiler),
and that entry points called before msplat_hip_init fail with
MSPLAT_ERR_NOINIT instead of touching a device.  No compute call is made.
"""
from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess

import pytest

from msplat_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "msplat_hip.h")
TRAINER_HEADER = os.path.join(ROOT, "include", "msplat_trainer.h")
C_API_HEADER = os.path.join(ROOT, "include", "msplat_c_api.h")
HEADERS = (HEADER, C_API_HEADER, TRAINER_HEADER)
# every exported function starts with one of these
EXPORT_RE = r"msplat_(?:hip_|trainer_|scene_|dataset_|undistort_|prepare_cam|image_|sync|cleanup|set_)\w*"


def _declared():
    """Functions declared in the three headers (static inline helpers excluded)."""
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        text = re.sub(r"static inline[^{]*\{.*?\n\}", "", text, flags=re.S)
        names |= set(re.findall(r"\b(" + EXPORT_RE + r")\s*\(", text))
    return sorted(names)


def test_header_and_ctypes_signatures_agree():
    assert _declared() == sorted(n for n, _, _ in _abi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_abi.LIB_PATH):
        pytest.skip("libmsplat_hip.so not built")
    lib = ctypes.CDLL(_abi.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    nm = shutil.which("nm")
    if nm:
        out = subprocess.check_output([nm, "-D", "--defined-only", _abi.LIB_PATH], text=True)
        exported = set(re.findall(r"\bT (" + EXPORT_RE + ")", out))
        assert set(_declared()) <= exported


STRUCTS = {"MsplatConfig": _abi.Config, "MsplatRenderArgs": _abi.RenderArgs, "MsplatTrainArgs": _abi.TrainArgs,
           "MsplatDensifyArgs": _abi.DensifyArgs, "MsplatTrainerConfig": _abi.TrainerConfig,
           "MsplatTrainerCamera": _abi.TrainerCamera, "MsplatStats": _abi.Stats,
           "MsplatCamSetup": _abi.CamSetupC,
           "MsplatPixelBuffer": _abi.PixelBuffer, "MsplatImageMetrics": _abi.ImageMetrics,
           "MsplatEvalMetrics": _abi.EvalMetrics}


def test_struct_layouts_match_header(tmp_path):
    cc = shutil.which("gcc") or shutil.which("cc")
    if not cc:
        pytest.skip("no host C compiler")
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"',
             f'#include "{C_API_HEADER}"', f'#include "{TRAINER_HEADER}"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.check_call([cc, "-std=c99", "-o", str(exe), str(src)])
    got = dict(l.rsplit(" ", 1) for l in subprocess.check_output([str(exe)], text=True).splitlines())
    for cname, py in STRUCTS.items():
        assert int(got[f"{cname} size"]) == ctypes.sizeof(py), cname
        for fname, _ in py._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(py, fname).offset, (cname, fname)


def test_missing_library_raises(tmp_path):
    saved = _abi._lib
    _abi._lib = None
    try:
        with pytest.raises(RuntimeError, match="missing"):
            _abi.load(str(tmp_path / "nope.so"))
    finally:
        _abi._lib = saved


def test_calls_before_init_fail_cleanly():
    if not os.path.exists(_abi.LIB_PATH):
        pytest.skip("libmsplat_hip.so not built")
    from msplat_amd import device
    if device._initialised:
        pytest.skip("a context already exists in this process")
    lib = _abi.load()
    assert lib.msplat_hip_sync() == -3
    assert b"not initialised" in lib.msplat_hip_last_error()
    a = _valid_empty_render_args()
    assert lib.msplat_hip_render(ctypes.byref(a), None) == -3
    t = _abi.TrainArgs()
    t.r = _valid_empty_render_args()
    loss = ctypes.c_float(0)
    assert lib.msplat_hip_train_step(ctypes.byref(t), None, ctypes.byref(loss)) == -3
    n = ctypes.c_int32(0)
    d = _abi.DensifyArgs()
    assert lib.msplat_hip_densify(ctypes.byref(d), ctypes.byref(n)) == -3
    counts = (ctypes.c_int64 * 6)()
    assert lib.msplat_hip_raster_work(counts) == -3


def _valid_empty_render_args(n=0, w=16, h=16):
    a = _abi.RenderArgs()
    a.num_points = n
    a.img_width, a.img_height = w, h
    a.tile_bounds[:] = [(w + 15) // 16, (h + 15) // 16, 1]
    return a


def test_argument_errors_without_a_device():
    """Argument checks come before the context check: a gaussian count past
    the 32-bit accumulator addressing limit (36 bytes per gaussian), an empty
    image and mismatched tile bounds are rejected with MSPLAT_ERR_ARG (-1)
    without touching a device."""
    if not os.path.exists(_abi.LIB_PATH):
        pytest.skip("libmsplat_hip.so not built")
    lib = _abi.load()
    limit = 0x7FFFFFFF // 36
    a = _valid_empty_render_args(n=limit + 1)
    assert lib.msplat_hip_render(ctypes.byref(a), None) == -1
    assert b"exceeds the limit" in lib.msplat_hip_last_error()
    t = _abi.TrainArgs()
    t.r = _valid_empty_render_args(n=limit + 1)
    assert lib.msplat_hip_train_step(ctypes.byref(t), None, None) == -1
    assert b"exceeds the limit" in lib.msplat_hip_last_error()
    a = _valid_empty_render_args(w=0)
    assert lib.msplat_hip_render(ctypes.byref(a), None) == -1
    a = _valid_empty_render_args(w=33)
    a.tile_bounds[0] = 2
    assert lib.msplat_hip_render(ctypes.byref(a), None) == -1
    assert b"tile_bounds" in lib.msplat_hip_last_error()
