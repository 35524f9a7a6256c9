"""ctypes wrapper of the brute-force C oracle (msda_brute.c) — TEST INFRASTRUCTURE ONLY.

Inputs are converted to contiguous float64 numpy arrays; outputs are float64. See
msda_brute.c for the restated algorithm and its reference citations.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_SO = _HERE / "_build" / "libmsda_brute.so"
_lib = None

_d = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.POINTER(ctypes.c_int64)


def build() -> Path:
    """Compile msda_brute.c with gcc (via oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _SO


def _load():
    global _lib
    if _lib is None:
        if not _SO.exists():
            build()
        lib = ctypes.CDLL(str(_SO))
        common = [ctypes.c_int, ctypes.c_int, ctypes.c_long, ctypes.c_int, ctypes.c_int,
                  ctypes.c_int, ctypes.c_int, ctypes.c_int, _i64, _d, _d, _d, ctypes.c_int,
                  ctypes.c_double, ctypes.c_int]
        lib.msda_brute_fwd.argtypes = common + [_d]
        lib.msda_brute_fwd.restype = None
        lib.msda_brute_bwd.argtypes = common + [_d, _d, _d, _d]
        lib.msda_brute_bwd.restype = None
        lib.msda_brute_coords.argtypes = [ctypes.c_int] * 6 + [_i64, _d, ctypes.c_int,
                                                                ctypes.c_double, ctypes.c_int, _d]
        lib.msda_brute_coords.restype = None
        _lib = lib
    return _lib


def _f64(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().cpu().double().numpy()
    return np.ascontiguousarray(x, dtype=np.float64)


def _ptr(a: np.ndarray, t=_d):
    return a.ctypes.data_as(t)


def _dims(value, shapes, loc):
    B, K, H, C = value.shape
    _, Q, _, L, P, dim = loc.shape
    assert shapes.shape == (L, dim)
    return dim, B, K, H, C, Q, L, P


def fwd(value, shapes, loc, attn, clamp_grid=True, clamp_eps=1e-4, coord_f32=False):
    """Forward in float64: returns (B, Q, H*C)."""
    v, lo, at = _f64(value), _f64(loc), _f64(attn)
    sh = np.ascontiguousarray(np.asarray(shapes.cpu() if hasattr(shapes, "cpu") else shapes),
                              dtype=np.int64)
    dim, B, K, H, C, Q, L, P = _dims(v, sh, lo)
    out = np.zeros((B, Q, H * C), dtype=np.float64)
    _load().msda_brute_fwd(dim, B, K, H, C, Q, L, P, _ptr(sh, _i64), _ptr(v), _ptr(lo), _ptr(at),
                           int(bool(clamp_grid)), float(clamp_eps), int(bool(coord_f32)),
                           _ptr(out))
    return out


def bwd(value, shapes, loc, attn, grad_out, clamp_grid=True, clamp_eps=1e-4, coord_f32=False):
    """Backward in float64: returns (grad_value, grad_loc, grad_attn)."""
    v, lo, at, go = _f64(value), _f64(loc), _f64(attn), _f64(grad_out)
    sh = np.ascontiguousarray(np.asarray(shapes.cpu() if hasattr(shapes, "cpu") else shapes),
                              dtype=np.int64)
    dim, B, K, H, C, Q, L, P = _dims(v, sh, lo)
    gv = np.zeros_like(v)
    gl = np.zeros_like(lo)
    ga = np.zeros_like(at)
    _load().msda_brute_bwd(dim, B, K, H, C, Q, L, P, _ptr(sh, _i64), _ptr(v), _ptr(lo), _ptr(at),
                           int(bool(clamp_grid)), float(clamp_eps), int(bool(coord_f32)),
                           _ptr(go), _ptr(gv), _ptr(gl), _ptr(ga))
    return gv, gl, ga


def coords(shapes, loc, clamp_grid=True, clamp_eps=1e-4, coord_f32=False):
    """Pixel coordinate u of every (sample, axis), shaped like loc."""
    lo = _f64(loc)
    sh = np.ascontiguousarray(np.asarray(shapes.cpu() if hasattr(shapes, "cpu") else shapes),
                              dtype=np.int64)
    B, Q, H, L, P, dim = lo.shape
    u = np.zeros_like(lo)
    _load().msda_brute_coords(dim, B, H, Q, L, P, _ptr(sh, _i64), _ptr(lo), int(bool(clamp_grid)),
                              float(clamp_eps), int(bool(coord_f32)), _ptr(u))
    return u


def edge_mask(shapes, loc, tol, clamp_grid=True, clamp_eps=1e-4):
    """True where a sample's pixel coordinate lies within `tol` of a cell edge (an integer).

    There the bilinear derivative is discontinuous and one ulp of coordinate rounding
    selects a different cell, so gradient comparisons for those samples are not
    meaningful. Returned per sample (shape loc.shape[:-1]).
    """
    u = coords(shapes, loc, clamp_grid, clamp_eps, coord_f32=False)
    near = np.abs(u - np.round(u)) < tol
    return near.any(axis=-1)
