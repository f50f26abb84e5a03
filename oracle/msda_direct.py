"""TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

ctypes/numpy front end of oracle/msda_direct.c, the float64 direct-loop
restatement of MSDA and its analytic gradients.
"""

from __future__ import annotations

import ctypes
import subprocess
from functools import lru_cache
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "build" / "libmsda_direct.so"


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


@lru_cache(maxsize=1)
def _lib() -> ctypes.CDLL:
    if not LIBRARY.is_file() or LIBRARY.stat().st_mtime < (HERE / "msda_direct.c").stat().st_mtime:
        build()
    lib = ctypes.CDLL(str(LIBRARY))
    p, i = ctypes.c_void_p, ctypes.c_int64
    lib.msda_direct_forward.argtypes = [p] * 6 + [i] * 7
    lib.msda_direct_forward.restype = None
    lib.msda_direct_backward.argtypes = [p] * 9 + [i] * 7
    lib.msda_direct_backward.restype = None
    return lib


def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def _i64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64))


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _dims(value, spatial_shapes, loc):
    bs, nv, heads, channels = value.shape
    _, nq, _, levels, points, _ = loc.shape
    assert spatial_shapes.shape == (levels, 2)
    return bs, nv, heads, channels, levels, nq, points


def level_starts(spatial_shapes) -> np.ndarray:
    shapes = _i64(spatial_shapes)
    sizes = shapes[:, 0] * shapes[:, 1]
    return _i64(np.concatenate([[0], np.cumsum(sizes)[:-1]]) if len(sizes) else np.zeros(0))


def forward(value, spatial_shapes, sampling_locations, attention_weights, level_start_index=None):
    value, shapes = _f64(value), _i64(spatial_shapes)
    loc, attn = _f64(sampling_locations), _f64(attention_weights)
    starts = level_starts(shapes) if level_start_index is None else _i64(level_start_index)
    bs, nv, heads, channels, levels, nq, points = _dims(value, shapes, loc)
    out = np.zeros((bs, nq, heads * channels), dtype=np.float64)
    _lib().msda_direct_forward(
        _ptr(value), _ptr(shapes), _ptr(starts), _ptr(loc), _ptr(attn), _ptr(out),
        bs, nv, heads, channels, levels, nq, points,
    )
    return out


def backward(value, spatial_shapes, sampling_locations, attention_weights, grad_output,
             level_start_index=None):
    """(grad_value, grad_sampling_locations, grad_attention_weights) in float64."""
    value, shapes = _f64(value), _i64(spatial_shapes)
    loc, attn, gout = _f64(sampling_locations), _f64(attention_weights), _f64(grad_output)
    starts = level_starts(shapes) if level_start_index is None else _i64(level_start_index)
    bs, nv, heads, channels, levels, nq, points = _dims(value, shapes, loc)
    gv = np.zeros_like(value)
    gl = np.zeros_like(loc)
    ga = np.zeros_like(attn)
    _lib().msda_direct_backward(
        _ptr(value), _ptr(shapes), _ptr(starts), _ptr(loc), _ptr(attn), _ptr(gout),
        _ptr(gv), _ptr(gl), _ptr(ga), bs, nv, heads, channels, levels, nq, points,
    )
    return gv, gl, ga
