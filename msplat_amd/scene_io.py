"""Gaussian scene files in host memory: PLY / .splat export and PLY import
(core/src/loaders/save_gaussians.cpp), through the library's host-only
functions msplat_scene_write_ply / write_splat / read_ply
(include/msplat_trainer.h).  No GPU is touched.

params: [means (N,3), scales (N,3) log, quats (N,4) wxyz, f_dc (N,3),
f_rest (N,K-1,3), opacities (N,) or (N,1) logits] float32 numpy arrays.
crs: optional (scale, (tx, ty, tz)) dataset normalisation, undone on export
and applied on import (keepCrs).
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Tuple

import numpy as np

from . import _abi

Crs = Optional[Tuple[float, Tuple[float, float, float]]]


def _crs_args(crs: Crs):
    if crs is None:
        return 1.0, (ctypes.c_float * 3)(0.0, 0.0, 0.0), 0
    scale, t = crs
    return float(scale), (ctypes.c_float * 3)(*[float(v) for v in t]), 1


def _pack(params):
    ps = [np.ascontiguousarray(p, np.float32) for p in params]
    n = int(ps[0].shape[0])
    rest_bases = int(ps[4].size // (3 * n)) if n else 0
    return ps, n, rest_bases, (ctypes.c_void_p * 6)(*[p.ctypes.data for p in ps])


def _check(lib, rc):
    if rc != 0:
        raise _abi.MsplatError(lib.msplat_trainer_last_error().decode())


def write_ply(path: str, params, step: int = 0, crs: Crs = None) -> None:
    lib = _abi.load()
    ps, n, rb, pp = _pack(params)
    scale, t, keep = _crs_args(crs)
    _check(lib, lib.msplat_scene_write_ply(str(path).encode(), n, rb, pp, scale, t, keep, step))


def write_splat(path: str, params, crs: Crs = None) -> None:
    lib = _abi.load()
    ps, n, rb, pp = _pack(params)
    scale, t, keep = _crs_args(crs)
    _check(lib, lib.msplat_scene_write_splat(str(path).encode(), n, rb, pp, scale, t, keep))


def read_ply(path: str, crs: Crs = None) -> Tuple[List[np.ndarray], int]:
    """Returns ([means, scales, quats, f_dc, f_rest, opacities (N,1)], step)."""
    lib = _abi.load()
    scale, t, keep = _crs_args(crs)
    n, rb, step = ctypes.c_int64(0), ctypes.c_int32(0), ctypes.c_int32(0)
    _check(lib, lib.msplat_scene_read_ply(str(path).encode(), scale, t, keep, ctypes.byref(n),
                                          ctypes.byref(rb), ctypes.byref(step), None))
    N, K1 = n.value, rb.value
    out = [np.empty((N, 3), np.float32), np.empty((N, 3), np.float32), np.empty((N, 4), np.float32),
           np.empty((N, 3), np.float32), np.empty((N, K1, 3), np.float32), np.empty((N, 1), np.float32)]
    pp = (ctypes.c_void_p * 6)(*[a.ctypes.data for a in out])
    _check(lib, lib.msplat_scene_read_ply(str(path).encode(), scale, t, keep, ctypes.byref(n),
                                          ctypes.byref(rb), ctypes.byref(step), pp))
    return out, int(step.value)
