"""The reference-shaped C API (include/msplat_c_api.h) and the image reader,
without a GPU.

* Every function of the reference's core/include/msplat_c_api.h is declared
  in include/msplat_c_api.h with the same return type, name and parameter
  list, and the four structs have the same fields and layouts (sizes and
  offsets printed by the host C compiler from each header).  These two tests
  read the reference tree and are skipped where it is absent.
* msplat_image_read (the dataset's image decoder) equals Pillow's RGB
  decoding for PNG files of every colour type it writes; 16-bit grey takes
  the high byte.
* Calls that fail before any device work give the reference's empty results
  and a message.
"""
from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

from msplat_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OURS = os.path.join(ROOT, "include", "msplat_c_api.h")
REF = "/root/reference/core/include/msplat_c_api.h"


def _strip(text):
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return re.sub(r"static inline[^{]*\{.*?\n\}", "", text, flags=re.S)


def _norm(s):
    s = re.sub(r"\s+", " ", s).strip()
    return re.sub(r"\s*([*,()\[\]])\s*", r"\1", s)


def _prototypes(path):
    text = _strip(open(path).read())
    out = {}
    for ret, name, params in re.findall(r"([\w\s\*]+?)\b(msplat_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.S):
        ret = ret.strip().split("\n")[-1]
        out[name] = (_norm(ret), _norm(params))
    return out


def _structs(path):
    text = _strip(open(path).read())
    return {name: [_norm(f) for f in body.split(";") if f.strip()]
            for body, name in re.findall(r"typedef struct\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S)}


def _ref_or_skip():
    if not os.path.exists(REF):
        pytest.skip("reference tree absent")


def test_c_api_prototypes_match_reference():
    _ref_or_skip()
    ref, ours = _prototypes(REF), _prototypes(OURS)
    assert len(ref) == 22, sorted(ref)
    for name, sig in ref.items():
        assert name in ours, f"{name} missing from include/msplat_c_api.h"
        assert ours[name] == sig, (name, ours[name], sig)
    assert set(ours) == set(ref)
    # the other header declares none of these names with another signature
    trainer = _prototypes(os.path.join(ROOT, "include", "msplat_trainer.h"))
    assert not set(trainer) & set(ref), set(trainer) & set(ref)


def test_c_api_types_match_reference(tmp_path):
    _ref_or_skip()
    ref, ours = _structs(REF), _structs(OURS)
    for name in ("MsplatConfig", "MsplatStats", "MsplatEvalMetrics", "MsplatPixelBuffer"):
        assert ours[name] == ref[name], name
    cc = shutil.which("gcc") or shutil.which("cc")
    if not cc:
        pytest.skip("no host C compiler")
    fields = {n: [re.split(r"[\s\*]+", f.split("[")[0])[-1] for f in ref[n]] for n in
              ("MsplatConfig", "MsplatStats", "MsplatEvalMetrics", "MsplatPixelBuffer")}

    def layout(header):
        lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{header}"', "int main(void) {"]
        for n, fs in fields.items():
            lines.append(f'printf("{n} %zu\\n", sizeof({n}));')
            lines += [f'printf("{n}.{f} %zu\\n", offsetof({n}, {f}));' for f in fs]
        lines.append("MsplatConfig c = msplat_default_config();")
        lines.append('printf("default %d %d %g %d %g %d %g\\n", c.iterations, c.shDegreeInterval, '
                     'c.ssimWeight, c.warmupLength, c.densifyGradThresh, (int)c.keepCrs, c.bgColor[1]);')
        lines += ["return 0;", "}"]
        src = tmp_path / f"l{abs(hash(header))}.c"
        src.write_text("\n".join(lines))
        exe = str(src)[:-2]
        subprocess.check_call([cc, "-std=c99", "-o", exe, str(src)])
        return subprocess.check_output([exe], text=True)

    assert layout(OURS) == layout(REF)


def _lib():
    if not os.path.exists(_abi.LIB_PATH):
        pytest.skip("libmsplat_hip.so not built")
    return _abi.load()


def _read(lib, path):
    rgb = ctypes.POINTER(ctypes.c_float)()
    w, h = ctypes.c_int32(0), ctypes.c_int32(0)
    rc = lib.msplat_image_read(str(path).encode(), ctypes.byref(rgb), ctypes.byref(w), ctypes.byref(h))
    if rc != 0:
        return None, lib.msplat_trainer_last_error().decode()
    try:
        return np.ctypeslib.as_array(rgb, shape=(h.value, w.value, 3)).copy(), ""
    finally:
        ctypes.CDLL(None).free(ctypes.cast(rgb, ctypes.c_void_p))


@pytest.mark.parametrize("mode", ["RGB", "RGBA", "L", "LA", "P", "1", "P+tRNS", "L+tRNS", "RGB+tRNS"])
def test_png_decoder_matches_pillow(mode, tmp_path):
    """Opaque images decode to Pillow's RGB bit for bit.  Transparent ones
    (alpha channel or tRNS chunk) become the image drawn source-over black,
    as the reference's CoreGraphics context without alpha draws it
    (image_io.cpp:33-41): round(c * a / 255) of Pillow's RGBA samples."""
    Image = pytest.importorskip("PIL.Image")
    lib = _lib()
    rng = np.random.default_rng(31)
    h, w = 37, 53   # odd sizes: rows of sub-byte pixels end mid-byte
    rgb = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
    base = mode.split("+")[0]
    im = Image.fromarray(rgb, "RGB")
    im = im.convert(base) if base != "P" else im.quantize(colors=61)
    save_kw = {}
    if mode in ("RGBA", "LA"):
        alpha = Image.fromarray(rng.integers(0, 256, (h, w), dtype=np.uint8), "L")
        im.putalpha(alpha)
    elif mode == "P+tRNS":
        save_kw["transparency"] = bytes(rng.integers(0, 256, 40, dtype=np.uint8))   # 21 entries stay opaque
    elif mode == "L+tRNS":
        save_kw["transparency"] = int(np.asarray(im)[3, 4])
    elif mode == "RGB+tRNS":
        save_kw["transparency"] = tuple(int(v) for v in np.asarray(im)[5, 6])
    path = tmp_path / f"img_{mode}.png"
    im.save(path, format="PNG", **save_kw)
    with Image.open(path) as f:
        if mode in ("RGB", "L", "P", "1"):
            want8 = np.asarray(f.convert("RGB"), dtype=np.uint8)
        else:
            rgba = np.asarray(f.convert("RGBA"), dtype=np.uint32)
            assert (rgba[..., 3] < 255).any(), "the fixture must hold transparent pixels"
            want8 = ((rgba[..., :3] * rgba[..., 3:] + 127) // 255).astype(np.uint8)
    want = want8.astype(np.float32) / np.float32(255.0)
    got, err = _read(lib, path)
    assert got is not None, err
    assert got.shape == want.shape
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


def test_png_decoder_16_bit_grey_and_errors(tmp_path):
    Image = pytest.importorskip("PIL.Image")
    lib = _lib()
    rng = np.random.default_rng(32)
    v = rng.integers(0, 65536, (19, 23), dtype=np.uint16)
    path = tmp_path / "g16.png"
    Image.fromarray(v.astype(np.int32), "I").convert("I;16").save(path, format="PNG")
    with Image.open(path) as f:
        raw = np.asarray(f, dtype=np.uint16)
    got, err = _read(lib, path)
    assert got is not None, err
    want = ((raw >> 8).astype(np.float32) / np.float32(255.0))[..., None].repeat(3, axis=2)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    # a truncated file, a non-image file, a missing file
    data = open(path, "rb").read()
    (tmp_path / "cut.png").write_bytes(data[: len(data) // 2])
    (tmp_path / "text.png").write_bytes(b"not an image at all")
    for p, msg in ((tmp_path / "cut.png", "PNG"), (tmp_path / "text.png", "neither PNG nor JPEG"),
                   (tmp_path / "none.png", "")):
        got, err = _read(lib, p)
        assert got is None and msg in err, (p, err)


def _jpeg_fixture(h=61, w=83, seed=5):
    """A smooth gradient image with noise (odd sizes: partial MCUs)."""
    rng = np.random.default_rng(seed)
    yy, xx = np.mgrid[0:h, 0:w]
    base = np.stack([(xx * 3 + yy) % 256, (yy * 4) % 256, (xx * yy) % 256], -1).astype(np.float32)
    return np.clip(base + rng.normal(0, 20, base.shape), 0, 255).astype(np.uint8)


JPEG_CASES = {
    "444_q90": dict(quality=90, subsampling=0),
    "422_q75": dict(quality=75, subsampling=1),
    "420_q75": dict(quality=75, subsampling=2),
    "411_q75": dict(quality=75, subsampling="4:1:1"),
    "420_q50_optimized": dict(quality=50, subsampling=2, optimize=True),
    "420_q100": dict(quality=100, subsampling=2),
    "420_progressive": dict(quality=95, subsampling=2, progressive=True),
    "420_progressive_optimized": dict(quality=80, subsampling=2, progressive=True, optimize=True),
    "444_progressive": dict(quality=85, subsampling=0, progressive=True),
    "420_restarts": dict(quality=85, subsampling=2, restart_marker_blocks=3),
    "422_progressive_restarts": dict(quality=85, subsampling=1, progressive=True, restart_marker_rows=1),
    "grey": dict(quality=80, mode="L"),
    "grey_progressive": dict(quality=80, mode="L", progressive=True),
}


@pytest.mark.parametrize("case", sorted(JPEG_CASES))
def test_jpeg_decoder_matches_pillow(case, tmp_path):
    """The library's JPEG decoder against Pillow's (libjpeg-turbo, default
    settings) on baseline / progressive, 4:4:4 / 4:2:2 / 4:2:0 / 4:1:1 /
    grey, optimised Huffman tables and restart intervals: equal samples."""
    Image = pytest.importorskip("PIL.Image")
    lib = _lib()
    kw = dict(JPEG_CASES[case])
    mode = kw.pop("mode", "RGB")
    img = _jpeg_fixture()
    im = Image.fromarray(img if mode == "RGB" else img[..., 0], mode)
    path = tmp_path / f"{case}.jpg"
    im.save(path, "JPEG", **kw)
    data = open(path, "rb").read()
    if "restart" in case:
        assert b"\xff\xd0" in data and b"\xff\xdd" in data, "the file must use restart markers"
    if "progressive" in case:
        assert b"\xff\xc2" in data
    with Image.open(path) as f:
        want = np.asarray(f.convert("RGB"), dtype=np.uint8).astype(np.float32) / np.float32(255.0)
    got, err = _read(lib, path)
    assert got is not None, err
    assert got.shape == want.shape
    assert (got.view(np.uint32) == want.view(np.uint32)).all(), \
        f"{int((got != want).sum())} samples differ, max {float(np.abs(got - want).max()) * 255:.1f} levels"


def test_jpeg_decoder_errors(tmp_path):
    """Truncated data, CMYK and non-image files fail with a message."""
    Image = pytest.importorskip("PIL.Image")
    lib = _lib()
    p = tmp_path / "a.jpg"
    Image.fromarray(_jpeg_fixture(), "RGB").save(p, "JPEG", quality=90)
    data = open(p, "rb").read()
    (tmp_path / "cut.jpg").write_bytes(data[: len(data) // 3])
    Image.new("CMYK", (20, 16), (10, 20, 30, 40)).save(tmp_path / "cmyk.jpg", "JPEG")
    (tmp_path / "soi_only.jpg").write_bytes(b"\xff\xd8\xff\xd9")
    (tmp_path / "text.jpg").write_bytes(b"not an image at all")
    for name, msg in (("cut.jpg", ""), ("cmyk.jpg", "4 components"), ("soi_only.jpg", "JPEG"),
                      ("text.jpg", "neither PNG nor JPEG")):
        got, err = _read(lib, tmp_path / name)
        assert got is None and msg in err, (name, err)


def test_c_api_calls_that_fail_before_device_work(tmp_path):
    """Failures give the reference's empty results (NULL handles, -1
    counts, zero-sized buffers) with a message, and touch no device."""
    lib = _lib()
    assert not lib.msplat_dataset_create(str(tmp_path / "missing").encode(), 1.0, False, 8)
    assert lib.msplat_trainer_last_error()
    assert lib.msplat_dataset_num_train(None) == -1 and lib.msplat_dataset_num_test(None) == -1
    assert not lib.msplat_trainer_create(None, _abi.default_config())
    assert b"null dataset" in lib.msplat_trainer_last_error()
    buf = lib.msplat_trainer_render(None, 0, False)
    assert not buf.data and buf.width == 0 and buf.height == 0
    pose = (ctypes.c_float * 16)(*np.eye(4, dtype=np.float32).reshape(16))
    w, h = ctypes.c_int(7), ctypes.c_int(7)
    lib.msplat_trainer_render_pose_to_buffer(None, pose, 0, None, ctypes.byref(w), ctypes.byref(h))
    assert w.value == 0 and h.value == 0
    lib.msplat_set_metallib_path(b"/nonexistent/default.metallib")
    lib.msplat_dataset_camera_pose(None, 0, pose)
    assert list(pose) == list(np.eye(4, dtype=np.float32).reshape(16))


REF_BINDINGS = "/root/reference/core/metal/bindings.h"


def test_bindings_shim_has_every_reference_prototype(tmp_path):
    """Each function of the reference's core/metal/bindings.h exists in
    msplat_amd/host/bindings.hpp with the same type: the C++ compiler takes a
    pointer of the reference's exact type to it (an overload that differs in
    any parameter or the return type does not convert)."""
    if not os.path.exists(REF_BINDINGS):
        pytest.skip("reference tree absent")
    cxx = shutil.which("g++")
    if not cxx:
        pytest.skip("no host C++ compiler")
    text = open(REF_BINDINGS).read()
    text = re.sub(r"#ifdef __OBJC__.*?#else(.*?)#endif", r"\1", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    text = re.sub(r"#[^\n]*", "", text)
    protos = re.findall(r"([\w:<>,\s\*&]+?[\s\*&])(\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.S)
    names = [n for _, n, _ in protos]
    assert len(protos) >= 12 and "msplat_densify" in names and "msplat_train_step" in names, names
    lines = ['#include "bindings.hpp"', "using namespace msplat;"]
    for k, (ret, name, params) in enumerate(protos):
        ret = " ".join(ret.split())
        lines.append(f"static {ret} (*p{k})({' '.join(params.split())}) = &msplat::{name};")
    lines.append("int main() { return 0; }")
    src = tmp_path / "shim.cpp"
    src.write_text("\n".join(lines))
    host = os.path.join(ROOT, "msplat_amd", "host")
    subprocess.check_call([cxx, "-std=c++17", "-fsyntax-only", "-I", host, "-I", os.path.join(ROOT, "include"),
                           str(src)])
